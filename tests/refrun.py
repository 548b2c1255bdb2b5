"""Helpers for the GPU parity tests: the reference's rounds on selected
symbols, run by the oracle (test infrastructure only).

Symbols are independent: rows never mix (example_model.py:422-427) and a
symbol's state advances only with its own requests, in order
(example_model.py:773-781). So the predictions the reference gives a symbol
over a run of ticks depend on that symbol's own request history alone, and
a handful of symbols can be replayed on the oracle as a small batch whatever
else the engine's ticks held.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import model as om


def zipf_tick(rng, n_symbols, batch, s=1.1):
    """Symbol ids of `batch` requests ~ Zipf(s) over n_symbols, grouped: the
    distinct ids in first-arrival order and their request counts."""
    p = np.arange(1, n_symbols + 1, dtype=np.float64) ** -s
    ids = rng.choice(n_symbols, size=batch, p=p / p.sum())
    uniq, first, counts = np.unique(ids, return_index=True, return_counts=True)
    order = np.argsort(first, kind="stable")
    return uniq[order].astype(np.int32), counts[order].astype(np.int64)


def to_device(state, dev):
    if isinstance(state, (list, tuple)):
        out = [to_device(s, dev) for s in state]
        return type(state)(out) if isinstance(state, tuple) else out
    return state.to(dev)


def reference_rounds(P: om.Params, cfg, histories, device="cpu"):
    """The reference's rounds over len(histories) rows: round k advances row
    i with histories[i][k] if it has more than k requests (a masked
    forward, example_model.py:885-899). Returns each row's predictions
    [len(history), 4] (float64, CPU) and the final state tree (CPU)."""
    B = len(histories)
    F = cfg.num_features
    state = to_device(om.init_state(cfg, B, P.dtype), device)
    preds = [np.zeros((len(h), 4)) for h in histories]
    with torch.inference_mode():
        for k in range(max(len(h) for h in histories)):
            x = torch.zeros(B, F, dtype=P.dtype)
            mask = torch.zeros(B, dtype=torch.bool)
            for i, h in enumerate(histories):
                if len(h) > k:
                    x[i] = torch.as_tensor(h[k], dtype=P.dtype)
                    mask[i] = True
            out, state = om.forward(P, cfg, x.to(device), state, mask.to(device))
            out = out.double().cpu().numpy()
            for i, h in enumerate(histories):
                if len(h) > k:
                    preds[i][k] = out[i]
    return preds, to_device(state, "cpu")


def rel_err(got, exact, floor=1e-2):
    """|got - exact| / max(|exact|, floor), elementwise."""
    got, exact = np.asarray(got, np.float64), np.asarray(exact, np.float64)
    return np.abs(got - exact) / np.maximum(np.abs(exact), floor)


def leaf_rel(got, exact):
    """Norm-wise relative distance of two state leaves (infinities, e.g. the
    sLSTM running max of an unused row, must match exactly)."""
    g, e = got.double().cpu(), exact.double().cpu()
    inf = torch.isinf(e)
    if inf.any():
        assert torch.equal(g[inf], e[inf]), "infinite entries differ"
        g, e = g[~inf], e[~inf]
    n = float(torch.linalg.vector_norm(e))
    return float(torch.linalg.vector_norm(g - e)) / max(n, 1e-30)
