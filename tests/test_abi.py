"""The C-ABI library loads on a machine without a GPU and exports every
symbol that include/*.h declares (no compute calls are made here)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(hk_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_symbols():
    assert "hk_mlstm_step" in declared()


def test_library_exports_every_declared_symbol():
    from hackathon_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libhackathon_amd.so is not built (run __graft_entry__.build())")
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(handle, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_header():
    from hackathon_amd import _lib
    import hackathon_amd.engine  # noqa: F401  (registers the engine signatures)
    import hackathon_amd.weights  # noqa: F401  (registers the host-side helpers)

    assert set(declared()) <= set(_lib.declared_symbols())
    lib = _lib.lib()
    assert lib.hk_version() >= 1
    assert isinstance(lib.hk_last_error(), bytes)
