"""Placeholder: the ensemble engine binding is added with the engine sources."""
