"""The stress configuration on the GPU: 8192 resident symbols at a reduced
width (hidden 512, proj 1024, depth 12, 8 heads: 14.8 MB of state per
symbol, 121 GB for all of them; at the default dims 8192 symbols would need
1.26 TB), bf16 CastLinear weights, ticks of B ~ U(1..512) requests over
uniform symbol ids, features N(0, 1).

- Parity: four symbols that the ticks touch are replayed on the oracle from
  their own histories (symbols are independent), in fp32 and with the
  reference's bf16 CastLinear: over their predictions the engine's mean
  squared distance from the reference's bf16 result is at most 3% of that
  result's distance from fp32 (r_32), and its distance from fp32 at most
  r_32 (measured 1.95% and 0.84).
- Idle slots: a sample of slots the ticks never touch keeps every state leaf
  bit-identical (their initial values).
- Determinism: the last tick replayed from its imported start state gives
  bit-identical predictions and state for its slots.
- hipGraph replay for ticks of at most 64 requests, as the configuration
  asks: every third tick has B ~ U(1..64) and replays a captured graph, so
  the parity sample above covers replayed ticks too.
"""

import numpy as np
import pytest
import torch

from hackathon_amd import spec, weights
from oracle import model as om
from refrun import reference_rounds

pytestmark = pytest.mark.gpu

CFG = spec.ModelConfig(hidden_size=512, proj_size=1024, tower_depth=12, num_heads=8,
                       num_features=79)
S, BMAX = 8192, 512


def _tick(rng, bmax=BMAX):
    B = int(rng.integers(1, bmax + 1))
    ids = rng.integers(0, S, size=B)
    uniq, first, counts = np.unique(ids, return_index=True, return_counts=True)
    order = np.argsort(first, kind="stable")
    return uniq[order].astype(np.int32), counts[order].astype(np.int64)


def _rows(eng, slots):
    """State leaves of the given slots (reference tree, flattened)."""
    out = None
    for s in slots:
        leaves = list(om.flatten(eng.export_state(int(s), 1)))
        out = [[x] for x in leaves] if out is None else [o + [x] for o, x in zip(out, leaves)]
    return [torch.cat(o) for o in out]


def test_c5_reduced_width_8192_symbols(dev):
    from hackathon_amd.engine import Engine, pack_runs

    params = weights.generate(CFG, 0)
    eng = Engine(CFG, capacity=S, max_rows=BMAX, max_runs=BMAX, linear_dtype="bf16", device=dev)
    eng.load_weights(params)
    eng.graphs(max_rows=64)
    rng = np.random.default_rng(3)
    frng = np.random.default_rng(1)
    ticks = [_tick(rng, 64 if j % 3 == 2 else BMAX) for j in range(12)]
    n_small = sum(int(c.sum()) <= 64 for _, c in ticks)
    touched = np.unique(np.concatenate([t[0] for t in ticks]))
    seen_twice = [s for s in touched if sum(int(s in t[0]) for t in ticks) >= 2]
    small = [int(s) for j, (syms_j, _) in enumerate(ticks) if j % 3 == 2 for s in syms_j]
    sample = [int(s) for s in seen_twice[:3]]
    sample += [next(s for s in small if s not in sample)]  # advanced by a replayed graph
    untouched = np.setdiff1d(np.arange(S), touched)
    idle = rng.choice(untouched, size=16, replace=False)
    idle_before = _rows(eng, idle)

    hist = {s: [] for s in sample}
    got = {s: [] for s in sample}
    for j, (syms, counts) in enumerate(ticks):
        runs, order = pack_runs(syms, counts)
        x = frng.standard_normal((runs.n_rows, CFG.num_features), dtype=np.float32)
        feats = torch.from_numpy(x).to(dev)
        if j == len(ticks) - 1:
            start = [eng.export_state(int(s), 1) for s in syms]
        preds = eng.tick(runs, feats).clone()
        for pos, i in enumerate(order):
            s = int(syms[i])
            if s in hist:
                a, b = int(runs.run_off[pos]), int(runs.run_off[pos + 1])
                hist[s].extend(x[a:b])
                got[s].extend(preds[a:b].cpu().numpy())
    eng.check()
    assert eng.graph_info()["replays"] == n_small >= 4
    after = _rows(eng, syms)
    # determinism: the last tick again from its start state
    for s, tree in zip(syms, start):
        eng.import_state(tree, int(s))
    preds2 = eng.tick(runs, feats)
    assert torch.equal(preds, preds2), "predictions differ between replays"
    for i, (a, b) in enumerate(zip(after, _rows(eng, syms))):
        assert torch.equal(a, b), f"leaf {i} differs between replays"
    for i, (a, b) in enumerate(zip(idle_before, _rows(eng, idle))):
        assert torch.equal(a, b), f"leaf {i}: an untouched slot changed"
    eng.check()
    eng.close()
    torch.cuda.empty_cache()

    histories = [hist[s] for s in sample]
    assert all(len(h) >= 1 for h in histories)
    p32, _ = reference_rounds(om.Params(params), CFG, histories)
    plp, _ = reference_rounds(om.Params(params, lp="bf16"), CFG, histories)
    cat = lambda v: np.concatenate([np.asarray(a, np.float64) for a in v])
    g_, r_lp, r32 = cat([got[s] for s in sample]), cat(plp), cat(p32)
    e_lp = float(((g_ - r_lp) ** 2).mean())
    e_32 = float(((g_ - r32) ** 2).mean())
    r_32 = float(((r_lp - r32) ** 2).mean())
    print(f"C5 sample {sample} ({[len(h) for h in histories]} requests): MSE engine-vs-bf16-ref "
          f"{e_lp:.3e}, engine-vs-fp32 {e_32:.3e}, bf16-ref-vs-fp32 {r_32:.3e}; "
          f"e_lp/r_32 {e_lp / r_32:.4f}, e_32/r_32 {e_32 / r_32:.4f}")
    # measured e_lp/r_32 0.0195, e_32/r_32 0.844
    assert e_lp <= 0.03 * r_32
    assert e_32 <= 1.0 * r_32
