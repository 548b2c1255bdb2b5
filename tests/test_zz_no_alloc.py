"""hk_engine_load_param_noalloc (binds a weight slot with no device
allocation, staging CastLinear weights through the library's per-GPU
16 MiB array in 4 Mi-value chunks) against hk_engine_load_param: two engines
bound through the two entry points give bit-identical predictions, at a
width where CastLinear slots span one full chunk (4 Mi values exactly) and
more than one (4.46 Mi values); then two calls in a row on each engine, a
two-chunk slot followed by a smaller one (new values), and the engines still
agree bit for bit. bf16 and fp16 modes (the staging is used only there)."""

import numpy as np
import pytest
import torch

from hackathon_amd import spec, weights

pytestmark = pytest.mark.gpu

CFG = spec.ModelConfig(hidden_size=1024, proj_size=2048, tower_depth=1, num_heads=8,
                       num_features=79)


def _tick(engines, dev, rng):
    from hackathon_amd.engine import pack_runs

    runs, _ = pack_runs(np.arange(4, dtype=np.int32), np.array([3, 1, 2, 1]))
    x = torch.from_numpy(rng.standard_normal((runs.n_rows, CFG.num_features)).astype(np.float32)).to(dev)
    return [e.tick(runs, x).cpu() for e in engines]


@pytest.mark.parametrize("lp", ["bf16", "fp16"])
def test_load_param_noalloc_matches_load_param(dev, lp):
    from hackathon_amd.engine import Engine

    params = weights.generate(CFG, 0)
    ref = Engine(CFG, capacity=4, max_rows=16, linear_dtype=lp, device=dev)
    na = Engine(CFG, capacity=4, max_rows=16, linear_dtype=lp, device=dev)
    ref.load_weights(params)
    na.load_weights(params, noalloc=True)
    rng = np.random.default_rng(0)
    a, b = _tick([ref, na], dev, rng)
    assert torch.isfinite(a).all() and torch.equal(a, b)

    # Two calls in a row, the second smaller: Mamba2's packed projection
    # (slot 6 of tower 1: 4352 x 1024 = 4.46 Mi values, two chunks), then
    # RetNet's out_proj (slot 7 of tower 2: 1 Mi values), new values.
    new = weights.generate(CFG, 1)
    I, bc = CFG.inner, CFG.mamba_bc_size
    pre = "towers.1.blocks.0.layer."
    proj = torch.cat([new[pre + n].reshape(-1) for n in
                      ("input_proj.weight", "b_proj.weight", "c_proj.weight", "z_proj.weight")])
    assert proj.numel() == (2 * I + 2 * bc) * CFG.hidden_size > 4 << 20
    out = new["towers.2.blocks.0.layer.out_proj.weight"]
    for e, noalloc in ((ref, False), (na, True)):
        e.load_param(1, 0, 6, proj, noalloc=noalloc)
        e.load_param(2, 0, 7, out, noalloc=noalloc)
    a2, b2 = _tick([ref, na], dev, rng)
    assert torch.equal(a2, b2)
    assert not torch.equal(a2[:, 1:3], a[:, 1:3])  # the new weights took effect
    ref.check()
    na.check()
    ref.close()
    na.close()


def test_load_param_noalloc_refuses_wrong_size(dev):
    from hackathon_amd import _lib
    from hackathon_amd.engine import Engine

    e = Engine(spec.SMALL, capacity=2, max_rows=8, linear_dtype="bf16", device=dev)
    with pytest.raises(ValueError):
        e.load_param(0, 0, 2, torch.zeros(5), noalloc=True)
    st = _lib.lib().hk_engine_load_param_noalloc(e._h, 0, 0, 2, torch.zeros(5).data_ptr(), 5)
    assert st == _lib.HK_ERR_ARG and b"expects" in _lib.lib().hk_last_error()
    e.close()
