"""Fused recurrent state steps on gfx950, behind the reference's kernel API.

Drop-in for `model/kernels.py:346-401` (`mlstm_step`, `retnet_step`,
`mamba2_step`) with the same contract (`model/kernels.py:28-34`), plus the
towers' other per-step operators under the same contract: the causal conv
(`model/modules.py:45-49`), BlockLinear (`model/modules.py:71-79`), the
RG-LRU step (`model/hawk.py:31-37`) and the sLSTM cell
(`model/xlstm.py:247-274`):

- the state is updated IN PLACE; rows whose mask is False end bit-identical,
  rows whose mask is True hold the new value;
- the returned output is a fresh contiguous fp32 tensor, zero on idle rows;
- `mask=None` means every row is active;
- nothing is data-dependent on the host.

Argument checks follow `model/kernels.py:85-121`: wrong dtype, shape, device
or a non-contiguous state raise AssertionError and are never repaired. Unlike
the reference there is no torch fallback: the state must live on a GPU and
the HIP library must be present, or the call raises.
"""

from __future__ import annotations

import torch

from . import _lib


def _state_ok(state: torch.Tensor, name: str) -> None:
    # model/kernels.py:116-121
    assert state.dtype == torch.float32, f"{name} must be fp32, got {state.dtype}"
    assert state.is_contiguous(), f"{name} must be contiguous, it is written in place"
    assert state.dim() == 4, f"{name} must be 4-D, got {tuple(state.shape)}"
    if state.device.type != "cuda":
        raise _lib.HipLibraryError(f"{name} is on {state.device}; the HIP kernels need a GPU tensor")


def _small(t: torch.Tensor, shape: tuple, name: str, device) -> torch.Tensor:
    # model/kernels.py:85-98
    assert t.dtype == torch.float32, f"{name} must be fp32, got {t.dtype}"
    assert tuple(t.shape) == shape, f"{name} must be {shape}, got {tuple(t.shape)}"
    assert t.device == device, f"{name} must be on {device}, it is on {t.device}"
    return t.contiguous()


def _mask_u8(mask, batch: int, device):
    # model/kernels.py:101-113; None stays None (every row active).
    if mask is None:
        return None
    assert mask.dtype == torch.bool, f"mask must be bool, got {mask.dtype}"
    assert mask.shape == (batch,), f"mask must be ({batch},), got {tuple(mask.shape)}"
    assert mask.device == device, f"mask must be on {device}, it is on {mask.device}"
    return mask.contiguous().view(torch.uint8)


def mlstm_step(cell, q, k, v, i_gate, f_gate, mask):
    """cell <- f*cell + (i*k) outer v on active rows; returns sum_h q*cell_new.

    Reference: model/kernels.py:346-360 (Triton) and :143-151 (torch twin).
    """
    _state_ok(cell, "cell")
    batch, heads, size_h, size_k = (int(s) for s in cell.shape)
    dev = cell.device
    q = _small(q, (batch, heads, size_h), "q", dev)
    k = _small(k, (batch, heads, size_h), "k", dev)
    v = _small(v, (batch, heads, size_k), "v", dev)
    i_gate = _small(i_gate, (batch, heads), "i_gate", dev)
    f_gate = _small(f_gate, (batch, heads), "f_gate", dev)
    m = _mask_u8(mask, batch, dev)
    out = torch.empty((batch, heads, size_k), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_mlstm_step(
        cell.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), i_gate.data_ptr(),
        f_gate.data_ptr(), _lib.ptr(m), out.data_ptr(), batch, heads, size_h, size_k,
        _lib.current_stream(dev),
    )
    _lib.check(st, "hk_mlstm_step")
    return out


def retnet_step(state, k_rope, v, q_scaled, decay, mask):
    """state <- decay[head]*state + k_rope outer v; returns sum_h q_scaled*state_new.

    Reference: model/kernels.py:363-376 (Triton) and :154-160 (torch twin).
    """
    _state_ok(state, "recurrent_state")
    batch, heads, size_h, size_k = (int(s) for s in state.shape)
    dev = state.device
    k_rope = _small(k_rope, (batch, heads, size_h), "k_rope", dev)
    v = _small(v, (batch, heads, size_k), "v", dev)
    q_scaled = _small(q_scaled, (batch, heads, size_h), "q_scaled", dev)
    decay = _small(decay, (heads,), "decay", dev)
    m = _mask_u8(mask, batch, dev)
    out = torch.empty((batch, heads, size_k), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_retnet_step(
        state.data_ptr(), k_rope.data_ptr(), v.data_ptr(), q_scaled.data_ptr(), decay.data_ptr(),
        _lib.ptr(m), out.data_ptr(), batch, heads, size_h, size_k, _lib.current_stream(dev),
    )
    _lib.check(st, "hk_retnet_step")
    return out


def mamba2_step(ssm, x, b, c, dt, decay, mask):
    """ssm <- decay*ssm + (dt*b) outer x on active rows; returns sum_c c*ssm_new.

    Reference: model/kernels.py:379-401 (Triton) and :163-171 (torch twin).
    """
    _state_ok(ssm, "ssm_state")
    batch, heads, size_h, size_c = (int(s) for s in ssm.shape)
    dev = ssm.device
    x = _small(x, (batch, heads, size_h), "x", dev)
    b = _small(b, (batch, size_c), "b", dev)
    c = _small(c, (batch, size_c), "c", dev)
    dt = _small(dt, (batch, heads), "dt", dev)
    decay = _small(decay, (batch, heads), "decay", dev)
    m = _mask_u8(mask, batch, dev)
    y = torch.empty((batch, heads, size_h), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_mamba2_step(
        ssm.data_ptr(), x.data_ptr(), b.data_ptr(), c.data_ptr(), dt.data_ptr(),
        decay.data_ptr(), _lib.ptr(m), y.data_ptr(), batch, heads, size_h, size_c,
        _lib.current_stream(dev),
    )
    _lib.check(st, "hk_mamba2_step")
    return y


def _dense(t: torch.Tensor, shape: tuple, name: str, device) -> None:
    # In-place operands: fp32, contiguous, on the GPU (model/kernels.py:116-121).
    assert t.dtype == torch.float32, f"{name} must be fp32, got {t.dtype}"
    assert t.is_contiguous(), f"{name} must be contiguous, it is written in place"
    assert tuple(t.shape) == shape, f"{name} must be {shape}, got {tuple(t.shape)}"
    if t.device.type != "cuda":
        raise _lib.HipLibraryError(f"{name} is on {t.device}; the HIP kernels need a GPU tensor")
    assert t.device == device, f"{name} must be on {device}, it is on {t.device}"


def causal_conv1d_step(state, x, weight, bias, mask=None):
    """CausalConv1d.forward (model/modules.py:45-49) as a masked in-place step.

    state [B, C, K-1] is advanced in place on active rows; weight is the
    conv's [C, 1, K] (or [C, K]); bias [C] or None. Returns out [B, C], zero
    on idle rows.
    """
    assert state.dim() == 3, f"state must be 3-D, got {tuple(state.shape)}"
    batch, channels, hist = (int(s) for s in state.shape)
    _dense(state, (batch, channels, hist), "state", state.device)
    dev = state.device
    taps = hist + 1
    if weight.dim() == 3:
        assert weight.shape[1] == 1, f"weight must be [C, 1, K], got {tuple(weight.shape)}"
        weight = weight.reshape(weight.shape[0], weight.shape[2])
    weight = _small(weight, (channels, taps), "weight", dev)
    bias = None if bias is None else _small(bias, (channels,), "bias", dev)
    x = _small(x, (batch, channels), "x", dev)
    m = _mask_u8(mask, batch, dev)
    out = torch.empty((batch, channels), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_conv1d_step(
        state.data_ptr(), x.data_ptr(), weight.data_ptr(), _lib.ptr(bias), _lib.ptr(m),
        out.data_ptr(), batch, channels, taps, _lib.current_stream(dev),
    )
    _lib.check(st, "hk_conv1d_step")
    return out


def block_linear(x, weight, bias=None):
    """BlockLinear.forward (model/modules.py:71-79): weight [blocks, bs, bs]
    as (blocks, out, in), x [B, blocks*bs]; returns a fresh [B, blocks*bs]."""
    assert weight.dim() == 3 and weight.shape[1] == weight.shape[2], (
        f"weight must be [blocks, bs, bs], got {tuple(weight.shape)}")
    blocks, bs = int(weight.shape[0]), int(weight.shape[1])
    dev = weight.device
    if dev.type != "cuda":
        raise _lib.HipLibraryError(f"weight is on {dev}; the HIP kernels need a GPU tensor")
    assert x.dim() == 2, f"x must be 2-D, got {tuple(x.shape)}"
    batch = int(x.shape[0])
    x = _small(x, (batch, blocks * bs), "x", dev)
    weight = _small(weight, (blocks, bs, bs), "weight", dev)
    bias = None if bias is None else _small(bias, (blocks * bs,), "bias", dev)
    out = torch.empty((batch, blocks * bs), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_block_linear(
        x.data_ptr(), weight.data_ptr(), _lib.ptr(bias), out.data_ptr(), batch, blocks, bs,
        _lib.current_stream(dev),
    )
    _lib.check(st, "hk_block_linear")
    return out


def rglru_step(state, x, gate_i, gate_r, a, c=8.0, mask=None):
    """RGLRU.forward after its BlockLinears (model/hawk.py:31-37): gate_i =
    input_gate(x), gate_r = recurrence_gate(x). state [B, H] is advanced in
    place on active rows; returns the new state rows, zero on idle rows."""
    assert state.dim() == 2, f"state must be 2-D, got {tuple(state.shape)}"
    batch, width = (int(s) for s in state.shape)
    dev = state.device
    _dense(state, (batch, width), "state", dev)
    x = _small(x, (batch, width), "x", dev)
    gate_i = _small(gate_i, (batch, width), "gate_i", dev)
    gate_r = _small(gate_r, (batch, width), "gate_r", dev)
    a = _small(a, (width,), "a", dev)
    m = _mask_u8(mask, batch, dev)
    out = torch.empty((batch, width), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_rglru_step(
        state.data_ptr(), x.data_ptr(), gate_i.data_ptr(), gate_r.data_ptr(), a.data_ptr(),
        float(c), _lib.ptr(m), out.data_ptr(), batch, width, _lib.current_stream(dev),
    )
    _lib.check(st, "hk_rglru_step")
    return out


def slstm_step(state, i, f, z, o, mask=None):
    """SLSTMCell.forward (model/xlstm.py:247-274) on gate pre-activations.

    state = (cell, norm, max) [B, H] each, advanced in place on active rows
    (max starts at -inf). Returns y [B, H], zero on idle rows.
    """
    c_st, n_st, m_st = state
    assert c_st.dim() == 2, f"cell state must be 2-D, got {tuple(c_st.shape)}"
    batch, width = (int(s) for s in c_st.shape)
    dev = c_st.device
    for t, name in ((c_st, "cell_state"), (n_st, "norm_state"), (m_st, "max_state")):
        _dense(t, (batch, width), name, dev)
    i, f, z, o = (_small(t, (batch, width), name, dev)
                  for t, name in ((i, "i"), (f, "f"), (z, "z"), (o, "o")))
    m = _mask_u8(mask, batch, dev)
    y = torch.empty((batch, width), dtype=torch.float32, device=dev)
    st = _lib.lib().hk_slstm_step(
        c_st.data_ptr(), n_st.data_ptr(), m_st.data_ptr(), i.data_ptr(), f.data_ptr(),
        z.data_ptr(), o.data_ptr(), _lib.ptr(m), y.data_ptr(), batch, width,
        _lib.current_stream(dev),
    )
    _lib.check(st, "hk_slstm_step")
    return y


_LP = {torch.bfloat16: 0, torch.float16: 1}


def pack_cast_weight(weight):
    """A CastLinear weight [N, K] (bf16/fp16, N a multiple of 32, K of 64)
    rearranged into the matrix-core layout the engine's projection GEMM
    streams (hk_pack_cast_weight). The result has the same dtype and shape;
    only cast_linear(..., packed=True) reads it."""
    assert weight.dtype in _LP, f"weight must be bf16 or fp16, got {weight.dtype}"
    assert weight.dim() == 2 and weight.is_contiguous(), "weight must be a contiguous [N, K] matrix"
    N, K = weight.shape
    assert N % 32 == 0 and K % 64 == 0, f"packing needs N % 32 == 0 and K % 64 == 0, got {N} x {K}"
    if weight.device.type != "cuda":
        raise _lib.HipLibraryError("pack_cast_weight needs a GPU tensor")
    out = torch.empty_like(weight)
    _lib.check(_lib.lib().hk_pack_cast_weight(weight.data_ptr(), out.data_ptr(), N, K,
                                              _lib.current_stream(weight.device)),
               "hk_pack_cast_weight")
    return out


def cast_linear(x, weight, bias=None, workspace=None, packed=False, min_work_groups=0):
    """CastLinear.forward (example_model.py:92-95): F.linear(x.to(lp),
    weight, bias).to(float32) for a weight held in bf16 or fp16.

    x: fp32 [..., K] (cast to the weight's dtype, as CastLinear does);
    weight: [N, K] bf16/fp16 contiguous (with packed=True, the output of
    pack_cast_weight: the engine's kernel); bias: [N] in the weight's dtype
    or None; workspace: optional zero-filled uint8 CUDA tensor (>= 256 KiB)
    for split-K; min_work_groups: the packed kernel's tile rule (0: the
    device to itself). Returns fp32 [..., N]."""
    assert weight.dtype in _LP, f"weight must be bf16 or fp16, got {weight.dtype}"
    assert weight.dim() == 2 and weight.is_contiguous(), "weight must be a contiguous [N, K] matrix"
    N, K = weight.shape
    assert x.shape[-1] == K, f"x must end in {K}, got {tuple(x.shape)}"
    dev = weight.device
    if dev.type != "cuda":
        raise _lib.HipLibraryError("cast_linear needs GPU tensors")
    xl = x.reshape(-1, K).to(device=dev, dtype=weight.dtype).contiguous()
    b = None
    if bias is not None:
        assert bias.dtype == weight.dtype and tuple(bias.shape) == (N,), "bias must be [N] in the weight's dtype"
        b = bias.to(torch.float32).contiguous()
    out = torch.empty(xl.shape[0], N, dtype=torch.float32, device=dev)
    ws, ws_bytes = None, 0
    if workspace is not None:
        assert workspace.dtype == torch.uint8 and workspace.device == dev
        ws, ws_bytes = workspace.data_ptr(), workspace.numel()
    lib = _lib.lib()
    if packed:
        st = lib.hk_cast_linear_packed(xl.data_ptr(), weight.data_ptr(), _lib.ptr(b), out.data_ptr(),
                                       xl.shape[0], N, K, _LP[weight.dtype], int(min_work_groups),
                                       ws, ws_bytes, _lib.current_stream(dev))
        _lib.check(st, "hk_cast_linear_packed")
    else:
        st = lib.hk_cast_linear(xl.data_ptr(), weight.data_ptr(), _lib.ptr(b), out.data_ptr(),
                                xl.shape[0], N, K, _LP[weight.dtype], ws, ws_bytes,
                                _lib.current_stream(dev))
        _lib.check(st, "hk_cast_linear")
    return out.reshape(*x.shape[:-1], N)
