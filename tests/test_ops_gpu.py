"""GPU parity of the towers' other per-step operators (causal conv,
BlockLinear, RG-LRU step, sLSTM cell) through the C-ABI, against the
oracle's functions on the same seeded inputs:

- idle state rows bit-identical, idle outputs exactly zero, masks mixed /
  all-true / all-false / None;
- the conv's state shift is exact (a copy); its 4-term sums within 1e-5
  relative, 1e-6 absolute;
- BlockLinear's 512-term fp32 contractions (matrix-core path) and 4-term
  ones (small-block kernel) within the kernel API's bar, rtol 1e-4 /
  atol 1e-5 (check_kernels.py:78-87);
- RG-LRU and sLSTM elementwise results within 1e-5 relative, 1e-6 absolute
  (powf / expf / tanhf differ from torch's CPU routines by a few ulp);
- composed steps (RGLRU.forward = two BlockLinears + the step, an sLSTM
  block's gates = input + state BlockLinears + the cell) over several steps.
"""

import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5       # contractions
E_RTOL, E_ATOL = 1e-5, 1e-6   # elementwise


def _masks(batch, g):
    mixed = torch.rand(batch, generator=g) < 0.5
    mixed[0] = True
    mixed[-1] = False
    yield "mixed", mixed
    yield "all", torch.ones(batch, dtype=torch.bool)
    yield "none", torch.zeros(batch, dtype=torch.bool)
    yield "None", None


def _live(mask, batch):
    return torch.ones(batch, dtype=torch.bool) if mask is None else mask


@pytest.mark.parametrize("batch,channels,taps", [(39, 4096, 4), (256, 512, 4), (6, 48, 4),
                                                 (5, 17, 2), (3, 33, 8), (4, 10, 1)])
def test_conv1d_step(dev, batch, channels, taps):
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(100 + channels)
    w = torch.randn(channels, 1, taps, generator=g) / taps ** 0.5
    b = torch.randn(channels, generator=g) * 0.05
    for name, mask in _masks(batch, g):
        state0 = torch.randn(batch, channels, taps - 1, generator=g)
        x = torch.randn(batch, channels, generator=g)
        want, want_state = om.causal_conv(x, state0, w, b)
        got_state = state0.to(dev)
        got = hk.causal_conv1d_step(got_state, x.to(dev), w.to(dev), b.to(dev),
                                    None if mask is None else mask.to(dev))
        torch.cuda.synchronize()
        got, got_state = got.cpu(), got_state.cpu()
        live = _live(mask, batch)
        assert torch.equal(got_state[~live], state0[~live]), f"{name}: idle rows changed"
        assert torch.equal(got_state[live], want_state[live]), f"{name}: state shift"
        torch.testing.assert_close(got[live], want[live], rtol=E_RTOL, atol=E_ATOL)
        assert bool(torch.all(got[~live] == 0.0)), f"{name}: idle outputs not zero"


def test_conv1d_steps_in_sequence_without_bias(dev):
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(5)
    B, C = 8, 256
    w = torch.randn(C, 1, 4, generator=g) / 2
    zero_b = torch.zeros(C)
    st_ref = torch.zeros(B, C, 3)
    st_gpu = st_ref.to(dev)
    for _ in range(6):
        x = torch.randn(B, C, generator=g)
        want, st_ref = om.causal_conv(x, st_ref, w, zero_b)
        got = hk.causal_conv1d_step(st_gpu, x.to(dev), w.to(dev), None)
        torch.testing.assert_close(got.cpu(), want, rtol=E_RTOL, atol=E_ATOL)
    assert torch.equal(st_gpu.cpu(), st_ref)


@pytest.mark.parametrize("batch,blocks,bs,bias", [(39, 4, 512, False), (39, 4, 512, True),
                                                  (256, 8, 64, True), (6, 1024, 4, False),
                                                  (5, 3, 48, True), (7, 2, 20, True),
                                                  (1, 4, 16, False), (16, 2, 256, True),
                                                  (17, 2, 256, True), (3, 1, 1024, True)])
def test_block_linear(dev, batch, blocks, bs, bias):
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(200 + bs)
    w = (torch.rand(blocks, bs, bs, generator=g) * 2 - 1) / bs ** 0.5
    b = torch.randn(blocks * bs, generator=g) * 0.05 if bias else None
    x = torch.randn(batch, blocks * bs, generator=g)
    want = om.block_linear(x, w, b)
    got = hk.block_linear(x.to(dev), w.to(dev), None if b is None else b.to(dev))
    torch.cuda.synchronize()
    assert got.shape == want.shape and got.is_contiguous()
    torch.testing.assert_close(got.cpu(), want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("batch,width", [(39, 2048), (256, 512), (5, 33)])
def test_rglru_step(dev, batch, width):
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(300 + width)
    a = torch.rand(width, generator=g) * 0.8 + 0.1   # U(0.1, 0.9), the init range
    for name, mask in _masks(batch, g):
        h0 = torch.randn(batch, width, generator=g)
        x, gi, gr = (torch.randn(batch, width, generator=g) * 2 for _ in range(3))
        want = om.rglru(x, h0, gi, gr, a)
        got_h = h0.to(dev)
        got = hk.rglru_step(got_h, x.to(dev), gi.to(dev), gr.to(dev), a.to(dev), 8.0,
                            None if mask is None else mask.to(dev))
        torch.cuda.synchronize()
        got, got_h = got.cpu(), got_h.cpu()
        live = _live(mask, batch)
        assert torch.equal(got_h[~live], h0[~live]), f"{name}: idle rows changed"
        torch.testing.assert_close(got_h[live], want[live], rtol=E_RTOL, atol=E_ATOL)
        assert torch.equal(got[live], got_h[live])
        assert bool(torch.all(got[~live] == 0.0)), f"{name}: idle outputs not zero"


@pytest.mark.parametrize("batch,width", [(39, 2048), (64, 512), (5, 33)])
def test_slstm_step(dev, batch, width):
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(400 + width)
    for name, mask in _masks(batch, g):
        c0 = torch.randn(batch, width, generator=g)
        n0 = torch.rand(batch, width, generator=g) * 2 + 0.5
        m0 = torch.randn(batch, width, generator=g)
        m0[0, : width // 2] = float("-inf")   # rows that have never stepped
        c0[0, : width // 2] = 0.0
        n0[0, : width // 2] = 0.0
        i, f, z, o = (torch.randn(batch, width, generator=g) * 2 for _ in range(4))
        y_want, (c_want, n_want, m_want) = om.slstm_cell(i, f, z, o, c0, n0, m0)
        st = [t.to(dev) for t in (c0, n0, m0)]
        y = hk.slstm_step(st, i.to(dev), f.to(dev), z.to(dev), o.to(dev),
                          None if mask is None else mask.to(dev))
        torch.cuda.synchronize()
        y, st = y.cpu(), [t.cpu() for t in st]
        live = _live(mask, batch)
        for got, init, want, what in zip(st, (c0, n0, m0), (c_want, n_want, m_want), "cnm"):
            assert torch.equal(got[~live], init[~live]), f"{name}: idle {what} changed"
            torch.testing.assert_close(got[live], want[live], rtol=E_RTOL, atol=E_ATOL)
        torch.testing.assert_close(y[live], y_want[live], rtol=E_RTOL, atol=E_ATOL)
        assert bool(torch.all(y[~live] == 0.0)), f"{name}: idle outputs not zero"


def test_rglru_forward_composed_over_steps(dev):
    # RGLRU.forward (model/hawk.py:18-39) at the default width, 2048 channels
    # in 4 blocks of 512: BlockLinear x2 on the matrix cores, then the step.
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(9)
    B, H, nb = 16, 2048, 4
    bs = H // nb
    wi, wr = ((torch.rand(nb, bs, bs, generator=g) * 2 - 1) / bs ** 0.5 for _ in range(2))
    a = torch.rand(H, generator=g) * 0.8 + 0.1
    wi_d, wr_d, a_d = wi.to(dev), wr.to(dev), a.to(dev)
    h_ref = torch.zeros(B, H)
    h_gpu = h_ref.to(dev)
    for _ in range(8):
        x = torch.randn(B, H, generator=g)
        h_ref = om.rglru(x, h_ref, om.block_linear(x, wi), om.block_linear(x, wr), a)
        xd = x.to(dev)
        hk.rglru_step(h_gpu, xd, hk.block_linear(xd, wi_d), hk.block_linear(xd, wr_d), a_d)
    torch.testing.assert_close(h_gpu.cpu(), h_ref, rtol=RTOL, atol=ATOL)


def test_slstm_gates_composed_over_steps(dev):
    # The sLSTM block's recurrence (model/xlstm.py:319-324) at the default
    # width, 4 heads of 512: i, f, z, o = input BlockLinear + state BlockLinear
    # (+ bias) of h_{t-1}, then the cell; h_t = y.
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(10)
    B, H, nh = 16, 2048, 4
    bs = H // nh
    w_in = [(torch.rand(nh, bs, bs, generator=g) * 2 - 1) / bs ** 0.5 for _ in range(4)]
    w_st = [(torch.rand(nh, bs, bs, generator=g) * 2 - 1) / bs ** 0.5 for _ in range(4)]
    b_st = [(torch.rand(H, generator=g) * 2 - 1) * 0.05 for _ in range(4)]
    w_in_d, w_st_d, b_st_d = ([t.to(dev) for t in ts] for ts in (w_in, w_st, b_st))
    h = torch.zeros(B, H)
    c, n, m = torch.zeros(B, H), torch.zeros(B, H), torch.full((B, H), float("-inf"))
    h_d = h.to(dev)
    st_d = [t.to(dev) for t in (c, n, m)]
    for _ in range(6):
        x = torch.randn(B, H, generator=g)
        gates = [om.block_linear(x, w_in[j]) + om.block_linear(h, w_st[j], b_st[j])
                 for j in range(4)]
        h, (c, n, m) = om.slstm_cell(*gates, c, n, m)
        xd = x.to(dev)
        gd = [hk.block_linear(xd, w_in_d[j]) + hk.block_linear(h_d, w_st_d[j], b_st_d[j])
              for j in range(4)]
        h_d = hk.slstm_step(st_d, *gd)
    torch.testing.assert_close(h_d.cpu(), h, rtol=RTOL, atol=ATOL)
    for got, want in zip(st_d, (c, n, m)):
        torch.testing.assert_close(got.cpu(), want, rtol=RTOL, atol=ATOL)


def test_refusal_guards(dev):
    from hackathon_amd import _lib
    from hackathon_amd import kernels as hk

    st = torch.zeros(4, 8, 3, device=dev)
    x = torch.zeros(4, 8, device=dev)
    w = torch.zeros(8, 1, 4, device=dev)
    with pytest.raises(AssertionError):
        hk.causal_conv1d_step(st.double(), x, w, None)
    with pytest.raises(AssertionError):
        hk.causal_conv1d_step(st, x[:, :4], w, None)
    with pytest.raises(AssertionError):
        hk.causal_conv1d_step(st, x, torch.zeros(8, 1, 3, device=dev), None)
    with pytest.raises(_lib.HipLibraryError):
        hk.causal_conv1d_step(st.cpu(), x.cpu(), w.cpu(), None)
    with pytest.raises(AssertionError):
        hk.block_linear(x, torch.zeros(2, 4, 5, device=dev))
    with pytest.raises(AssertionError):
        hk.rglru_step(x.t(), x, x, x, torch.zeros(8, device=dev))
    with pytest.raises(AssertionError):
        hk.slstm_step([x, x, x[:2]], x, x, x, x)
    with pytest.raises(AssertionError):
        hk.rglru_step(x, x, x, x, torch.zeros(8, device=dev),
                      mask=torch.ones(4, dtype=torch.int32, device=dev))


def _ulp(v, dtype):
    # spacing of the 16-bit format at |v| (normal range; fp16 subnormal step below)
    mant = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2(v.abs().clamp_min(1e-30)))
    if dtype == torch.float16:
        e = e.clamp_min(-14)
    return torch.pow(2.0, e - mant)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 4096, 2048), (37, 2048, 4096), (5, 8448, 2048), (1, 64, 64)])
def test_cast_linear_matches_castlinear(dev, dtype, M, N, K):
    """hk_cast_linear (the engine's projection GEMM) against CastLinear's
    expression F.linear(x.to(lp), W_lp, b_lp).to(float32)
    (example_model.py:92-95) as a GPU BLAS evaluates it: the sum and the bias
    accumulated in fp32, one rounding to the 16-bit format. Against the
    float64 sum rounded once, an element may differ by one rounding step
    plus the fp32 accumulation error, bounded here by sixteen fp32 rounding
    steps of the sum of the terms' magnitudes (16 * 2^-24 * sum_k |x_k w_k|,
    which dominates only for outputs near zero); at least 98% of them must
    be exact. torch's CPU kernel (which may round the product and the bias sum
    separately) stays within two steps. With and without a split-K
    workspace."""
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g)
    w = (torch.rand(N, K, generator=g) * 2 - 1) * K ** -0.5
    b = (torch.rand(N, generator=g) * 0.1 - 0.05)
    xl, wl, bl = x.to(dtype), w.to(dtype), b.to(dtype)
    exact = (xl.double() @ wl.double().T + bl.double()).to(dtype).to(torch.float32)
    acc = 16 * 2.0 ** -24 * (xl.double().abs() @ wl.double().abs().T + bl.double().abs()).float()
    cpu = torch.nn.functional.linear(xl, wl, bl).to(torch.float32)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    for workspace in (None, ws):
        got = hk.cast_linear(x.to(dev), wl.to(dev), bl.to(dev), workspace=workspace).cpu()
        d = (got - exact).abs()
        ulp = _ulp(torch.maximum(got.abs(), exact.abs()), dtype)
        assert bool((d <= ulp + acc).all()), float((d / (ulp + acc)).max())
        assert float((d == 0).float().mean()) >= 0.98
        assert bool(((got - cpu).abs() <= 2 * (_ulp(torch.maximum(got.abs(), cpu.abs()), dtype) + acc)).all())
    # the workspace is left zeroed (its arrival counters) for the next call
    assert int(ws[: 1 << 18].sum()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 8192, 2048), (256, 4096, 2048), (256, 2048, 2048),
                                   (179, 8448, 2048), (77, 2048, 4096), (37, 2048, 4096),
                                   (5, 8448, 2048), (1, 64, 64), (100, 320, 640), (300, 1024, 192),
                                   (16, 2048, 4096), (12, 320, 640), (17, 2048, 2048)])
def test_cast_linear_packed_matches_castlinear(dev, dtype, M, N, K):
    """The engine's projection kernel (hk_cast_linear_packed, the weight
    rearranged by hk_pack_cast_weight) against CastLinear's expression at the
    bar of test_cast_linear_matches_castlinear. The shapes cover every tile
    of the kernel (64x128, 64x64, 32x64, 32x32; rows past M, split K when the
    tiles cannot fill the device; at most 16 rows, the one-fragment form
    that takes all of K per work-group) and the tick's projections, under the tile
    rule of a lone GEMM, of the engine's ticks (112 work-groups) and one no
    shape meets (always the smallest tile, K split); the packed result also
    equals the row-major kernel's within the same bound."""
    from hackathon_amd import kernels as hk

    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g)
    w = (torch.rand(N, K, generator=g) * 2 - 1) * K ** -0.5
    b = (torch.rand(N, generator=g) * 0.1 - 0.05)
    xl, wl, bl = x.to(dtype), w.to(dtype), b.to(dtype)
    exact = (xl.double() @ wl.double().T + bl.double()).to(dtype).to(torch.float32)
    acc = 16 * 2.0 ** -24 * (xl.double().abs() @ wl.double().abs().T + bl.double().abs()).float()
    wd = wl.to(dev)
    packed = hk.pack_cast_weight(wd)
    assert not torch.equal(packed, wd) or N * K <= 64 * 64
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    for workspace, mwg in ((None, 0), (ws, 0), (ws, 112), (ws, 1 << 20)):
        got = hk.cast_linear(x.to(dev), packed, bl.to(dev), workspace=workspace, packed=True,
                             min_work_groups=mwg).cpu()
        d = (got - exact).abs()
        ulp = _ulp(torch.maximum(got.abs(), exact.abs()), dtype)
        assert bool((d <= ulp + acc).all()), float((d / (ulp + acc)).max())
        assert float((d == 0).float().mean()) >= 0.98
        rm = hk.cast_linear(x.to(dev), wd, bl.to(dev), workspace=workspace).cpu()
        assert bool(((got - rm).abs() <= 2 * (_ulp(torch.maximum(got.abs(), rm.abs()), dtype) + acc)).all())
    assert int(ws[: 1 << 18].sum()) == 0


def test_pack_cast_weight_layout(dev):
    """hk_pack_cast_weight moves element (n, k) of W to
    ((((n/32)*(K/32) + k/32)*2 + (n%32)/16)*64 + n%16 + 16*((k%32)/8))*8 + k%8:
    a permutation, checked element by element against that formula."""
    from hackathon_amd import kernels as hk

    N, K = 96, 192
    w = torch.arange(N * K, dtype=torch.int32).remainder(65521).to(torch.int16).view(torch.bfloat16)
    w = w.reshape(N, K).contiguous()
    p = hk.pack_cast_weight(w.to(dev)).cpu().view(torch.int16).reshape(-1)
    n = torch.arange(N).view(N, 1).expand(N, K)
    k = torch.arange(K).view(1, K).expand(N, K)
    lane = n % 16 + 16 * ((k % 32) // 8)
    idx = ((((n // 32) * (K // 32) + k // 32) * 2 + (n % 32) // 16) * 64 + lane) * 8 + k % 8
    assert torch.equal(p[idx.reshape(-1)], w.view(torch.int16).reshape(-1))
