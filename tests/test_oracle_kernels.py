"""Pin the oracle's three state steps (oracle/kernels.py) on the CPU.

What pins them (none of this retypes the oracle's own expression):
- fp64 brute force with explicit Python loops over every index, written from
  the recurrences' textbook definitions (mLSTM C' = f C + i k v^T, h = C'^T q;
  RetNet S' = gamma S + k v^T, o = S'^T q; Mamba2 h' = e^{A dt} h + dt x b^T,
  y = h' c), on tiny ragged shapes;
- library routines: torch.einsum over the same contraction;
- special cases: zero state -> out = (q.k) v scaled (closed form); all-false
  mask leaves the state bit-identical and the output zero; decay 0 forgets.
A transposed contraction axis (the reference's own warning, retnet.py:297-301)
fails the brute-force check because h != k in the ragged shapes.
"""

import itertools

import pytest
import torch

from oracle import kernels as ok


def _gen(seed):
    g = torch.Generator().manual_seed(seed)
    return lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)


def test_mlstm_brute_force():
    r = _gen(0)
    B, n, H, K = 3, 2, 5, 7
    C, q, k, v = r(B, n, H, K), r(B, n, H), r(B, n, H), r(B, n, K)
    ig, fg = r(B, n).abs(), r(B, n).abs()
    want_C = C.clone()
    want_o = torch.zeros(B, n, K, dtype=torch.float64)
    for b, h in itertools.product(range(B), range(n)):
        for i in range(H):
            for j in range(K):
                want_C[b, h, i, j] = fg[b, h] * C[b, h, i, j] + ig[b, h] * k[b, h, i] * v[b, h, j]
        for j in range(K):
            want_o[b, h, j] = sum(q[b, h, i] * want_C[b, h, i, j] for i in range(H))
    got_C = C.clone()
    got_o = ok.mlstm_step(got_C, q, k, v, ig, fg, None)
    torch.testing.assert_close(got_C, want_C, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got_o, want_o, rtol=1e-12, atol=1e-12)


def test_retnet_brute_force_contracts_h_not_k():
    r = _gen(1)
    B, n, H, K = 2, 3, 4, 6
    S, kr, v, qs = r(B, n, H, K), r(B, n, H), r(B, n, K), r(B, n, H)
    dec = torch.rand(n, dtype=torch.float64)
    want_S = torch.empty_like(S)
    want_o = torch.zeros(B, n, K, dtype=torch.float64)
    for b, h, i, j in itertools.product(range(B), range(n), range(H), range(K)):
        want_S[b, h, i, j] = S[b, h, i, j] * dec[h] + kr[b, h, i] * v[b, h, j]
    for b, h, j in itertools.product(range(B), range(n), range(K)):
        want_o[b, h, j] = sum(qs[b, h, i] * want_S[b, h, i, j] for i in range(H))
    got_S = S.clone()
    got_o = ok.retnet_step(got_S, kr, v, qs, dec, None)
    torch.testing.assert_close(got_S, want_S, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got_o, want_o, rtol=1e-12, atol=1e-12)
    # library routine: the same contraction through einsum
    torch.testing.assert_close(got_o, torch.einsum("bnh,bnhk->bnk", qs, want_S))


def test_mamba2_brute_force_contracts_c():
    r = _gen(2)
    B, n, H, Cc = 2, 3, 5, 7
    h0, x, b, c = r(B, n, H, Cc), r(B, n, H), r(B, Cc), r(B, Cc)
    dt = torch.rand(B, n, dtype=torch.float64)
    A = -torch.rand(n, dtype=torch.float64) * 4
    decay = torch.exp(A[None] * dt)
    want_h = torch.empty_like(h0)
    want_y = torch.zeros(B, n, H, dtype=torch.float64)
    for bb, hh, i, j in itertools.product(range(B), range(n), range(H), range(Cc)):
        want_h[bb, hh, i, j] = decay[bb, hh] * h0[bb, hh, i, j] + dt[bb, hh] * x[bb, hh, i] * b[bb, j]
    for bb, hh, i in itertools.product(range(B), range(n), range(H)):
        want_y[bb, hh, i] = sum(c[bb, j] * want_h[bb, hh, i, j] for j in range(Cc))
    got_h = h0.clone()
    got_y = ok.mamba2_step(got_h, x, b, c, dt, decay, None)
    torch.testing.assert_close(got_h, want_h, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got_y, want_y, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got_y, torch.einsum("bc,bnhc->bnh", c, want_h))


def test_zero_state_closed_form():
    # From zero state the mLSTM output is i * (q . k) * v, exactly.
    r = _gen(3)
    B, n, H, K = 2, 2, 8, 4
    q, k, v = r(B, n, H), r(B, n, H), r(B, n, K)
    ig, fg = torch.rand(B, n, dtype=torch.float64), torch.rand(B, n, dtype=torch.float64)
    C = torch.zeros(B, n, H, K, dtype=torch.float64)
    out = ok.mlstm_step(C, q, k, v, ig, fg, None)
    want = ig[:, :, None] * (q * k).sum(-1)[:, :, None] * v
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("which", ["mlstm", "retnet", "mamba2"])
def test_mask_semantics(which):
    r = _gen(4)
    B, n, H, K = 4, 2, 6, 5
    mask = torch.tensor([True, False, True, False])
    if which == "mlstm":
        S = r(B, n, H, K)
        args = (r(B, n, H), r(B, n, H), r(B, n, K), torch.rand(B, n, dtype=torch.float64),
                torch.rand(B, n, dtype=torch.float64))
        fn = ok.mlstm_step
    elif which == "retnet":
        S = r(B, n, H, K)
        args = (r(B, n, H), r(B, n, K), r(B, n, H), torch.rand(n, dtype=torch.float64))
        fn = ok.retnet_step
    else:
        S = r(B, n, H, K)
        args = (r(B, n, H), r(B, K), r(B, K), torch.rand(B, n, dtype=torch.float64),
                torch.rand(B, n, dtype=torch.float64))
        fn = ok.mamba2_step
    s_mask, s_all = S.clone(), S.clone()
    out_mask = fn(s_mask, *args, mask)
    out_all = fn(s_all, *args, None)
    assert torch.equal(s_mask[~mask], S[~mask])
    assert torch.equal(s_mask[mask], s_all[mask])
    assert torch.all(out_mask[~mask] == 0)
    assert torch.equal(out_mask[mask], out_all[mask])
    s_none = S.clone()
    out_none = fn(s_none, *args, torch.zeros(B, dtype=torch.bool))
    assert torch.equal(s_none, S) and torch.all(out_none == 0)


def test_zero_decay_forgets():
    r = _gen(5)
    B, n, H, K = 2, 2, 3, 3
    S = r(B, n, H, K)
    kr, v, qs = r(B, n, H), r(B, n, K), r(B, n, H)
    S1 = S.clone()
    ok.retnet_step(S1, kr, v, qs, torch.zeros(n, dtype=torch.float64), None)
    torch.testing.assert_close(S1, kr[..., None] * v[:, :, None, :])
