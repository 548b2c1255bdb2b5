"""Oracle for the 4-tower ensemble step (test infrastructure only).

A functional CPU restatement of the reference model, over a parameter dict
keyed by the reference's state_dict names:
- CausalConv1d       model/modules.py:36-49
- BlockLinear        model/modules.py:71-79
- SimpleMLP          model/modules.py:16-20
- Mamba2.forward     model/mamba2.py:62-168 (+ kernels.py:163-171 twin)
- RetNet.forward     model/retnet.py:38-172 (+ kernels.py:154-160 twin)
- Hawk/RGLRU         model/hawk.py:18-87
- MLSTMCell/Block    model/xlstm.py:33-236 (+ kernels.py:143-151 twin)
- SLSTMCell/Block    model/xlstm.py:247-329
- XLSTM.forward      model/xlstm.py:355-367
- Block/Tower/MultiTowerModel  model/inference_model.py:55-146
- CastLinear         example_model.py:68-101 (lp="bf16": weights, biases and
                     outputs rounded through bf16, inputs cast to bf16)
- _blend_state       example_model.py:907-949 (masked fold of every leaf)

`forward(P, cfg, x, state, mask=None, lp=None)` returns (preds [B,4],
new_state) with new_state in the reference's init_state tree. The dtype of
`x` and the params decides the arithmetic (fp32 for parity, fp64 for the
brute-force pinning tests). Nothing here is imported by the product.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

TOWERS = ("xlstm", "mamba2", "retnet", "hawk")
FP32_LINEAR_NAMES = ("dt_proj", "igate_proj", "fgate_proj", "output_proj")


class Params:
    """Parameter access with CastLinear emulation (example_model.py:68-148)."""

    def __init__(self, params: dict, lp: str | None = None, dtype=torch.float32):
        self.p = {k: v.to(dtype) for k, v in params.items()}
        self.lp = {"bf16": torch.bfloat16, "fp16": torch.float16, None: None}[lp]
        self.dtype = dtype
        self._cast = {}

    def __getitem__(self, name):
        return self.p[name]

    def linear(self, x, name, bias=True):
        """nn.Linear `name` (without .weight), CastLinear when converted."""
        w = self.p[name + ".weight"]
        b = self.p.get(name + ".bias") if bias else None
        owner = name.rsplit(".", 1)[-1]
        if self.lp is None or owner in FP32_LINEAR_NAMES:
            return F.linear(x, w, b)
        if name not in self._cast:
            self._cast[name] = (w.to(self.lp), None if b is None else b.to(self.lp))
        wl, bl = self._cast[name]
        return F.linear(x.to(self.lp), wl, bl).to(self.dtype)


def rms_norm(x, w, eps):
    # nn.RMSNorm: x * rsqrt(mean(x^2) + eps) * weight; eps None -> finfo eps.
    if eps is None:
        eps = torch.finfo(x.dtype).eps
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if w is None else y * w


def layer_norm(x, w):
    return F.layer_norm(x, (x.shape[-1],), w, None, 1e-5)


def group_norm(x, groups, w, b):
    return F.group_norm(x, groups, w, b, 1e-5)


def causal_conv(x, state, w, b):
    """model/modules.py:45-49: window [state, x], depthwise conv, shift."""
    win = torch.cat([state, x[:, :, None]], dim=-1)
    out = F.conv1d(win, w, b, groups=w.shape[0])
    return out.squeeze(-1), win[:, :, 1:]


def block_linear(x, w, b=None):
    """model/modules.py:71-79: out[b,n,k] = sum_h x[b,n,h] W[n,k,h] (+bias)."""
    B = x.shape[0]
    nb, bs = w.shape[0], w.shape[1]
    out = torch.einsum("bnh,nkh->bnk", x.view(B, nb, bs), w).reshape(B, nb * bs)
    return out if b is None else out + b


def rglru(x, h, gi, gr, a, c=8.0):
    """RGLRU.forward after its two BlockLinears (model/hawk.py:31-37):
    gi = input_gate(x), gr = recurrence_gate(x); returns the new state."""
    i_t = torch.sigmoid(gi)
    r_t = torch.sigmoid(gr)
    a_t = a ** (c * r_t)
    mult = torch.sqrt(1 - a_t ** 2)
    return (h * a_t) + (mult * (i_t * x))


def slstm_cell(gi, gf, gz, go, c, n, m):
    """SLSTMCell.forward (model/xlstm.py:258-274) on gate pre-activations;
    returns y and the new (c, n, m)."""
    lfm = m + F.logsigmoid(gf)
    m_new = torch.maximum(gi, lfm)
    o_gate = torch.sigmoid(go)
    i_gate = torch.exp(gi - m_new)
    f_gate = torch.exp(lfm - m_new)
    c_new = f_gate * c + i_gate * torch.tanh(gz)
    n_new = f_gate * n + i_gate
    y = o_gate * c_new / (n_new + 1e-6)
    return y, (c_new, n_new, m_new)


# ---- layers ----------------------------------------------------------------------


def mamba2(P: Params, pre, cfg, t, state):
    B = t.shape[0]
    nh, hs = cfg.mamba_heads, cfg.mamba_head_size
    x = P.linear(t, pre + "input_proj", bias=False)
    z = P.linear(t, pre + "z_proj", bias=False)
    b = P.linear(t, pre + "b_proj", bias=False)
    c = P.linear(t, pre + "c_proj", bias=False)
    dt = P.linear(t, pre + "dt_proj")
    xs, bs_, cs, ssm = state
    x, xs = causal_conv(x, xs, P[pre + "input_conv.conv.weight"], P[pre + "input_conv.conv.bias"])
    b, bs_ = causal_conv(b, bs_, P[pre + "b_conv.conv.weight"], P[pre + "b_conv.conv.bias"])
    c, cs = causal_conv(c, cs, P[pre + "c_conv.conv.weight"], P[pre + "c_conv.conv.bias"])
    x, b, c = F.silu(x), F.silu(b), F.silu(c)
    x = x.view(B, nh, hs)
    dt = F.softplus(dt)
    decay = torch.exp(P[pre + "a"][None] * dt)
    ssm_new = decay[:, :, None, None] * ssm + dt[:, :, None, None] * b[:, None, None] * x[:, :, :, None]
    contrib = (c[:, None, None, :] * ssm_new).sum(dim=-1)
    y = contrib + P[pre + "d"][None, :, None] * x
    y = y.view(B, cfg.inner) * F.silu(z)
    y = rms_norm(y, P[pre + "norm.weight"], 1e-5)
    return P.linear(y, pre + "out_proj", bias=False), [xs, bs_, cs, ssm_new]


def rotate_every_two(x):
    x1, x2 = x[..., ::2], x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(-2)


def retnet(P: Params, pre, cfg, x, state):
    B = x.shape[0]
    nh, hs = cfg.num_heads, cfg.retnet_head
    off, scales, S = state
    q = P.linear(x, pre + "q_proj", bias=False)
    k = P.linear(x, pre + "k_proj", bias=False)
    v = P.linear(x, pre + "v_proj", bias=False)
    g = P.linear(x, pre + "g_proj", bias=False)
    k = k * (hs ** -0.5)
    qh, kh, vh = q.view(B, nh, hs), k.view(B, nh, hs), v.view(B, nh, hs)
    ang = P[pre + "angle"]
    sin = torch.sin(off[:, None, None] * ang[None, None, :])
    cos = torch.cos(off[:, None, None] * ang[None, None, :])
    q_rope = qh * cos + rotate_every_two(qh) * sin
    k_rope = kh * cos + rotate_every_two(kh) * sin
    decay = P[pre + "decay"]
    new_scales = scales * decay + 1.0
    q_scaled = q_rope * (1.0 / new_scales.sqrt())[:, :, None]
    S_new = S * decay[None, :, None, None] + k_rope[:, :, :, None] * vh[:, :, None, :]
    out = (q_scaled[:, :, :, None] * S_new).sum(dim=2)
    out = rms_norm(out, None, 1e-6).reshape(B, cfg.hidden_size)
    out = F.silu(g) * out
    return P.linear(out, pre + "out_proj", bias=False), (off + 1, new_scales, S_new)


def hawk(P: Params, pre, cfg, x, state):
    conv_state, h = state
    gate = F.gelu(P.linear(x, pre + "gate_proj", bias=False))
    x = P.linear(x, pre + "recurrent_proj", bias=False)
    x, conv_state = causal_conv(x, conv_state, P[pre + "conv.conv.weight"], P[pre + "conv.conv.bias"])
    h_new = rglru(x, h, block_linear(x, P[pre + "rglru.input_gate.weight"]),
                  block_linear(x, P[pre + "rglru.recurrence_gate.weight"]), P[pre + "rglru.a"])
    return P.linear(gate * h_new, pre + "out_proj", bias=False), [conv_state, h_new]


def slstm_block(P: Params, pre, cfg, x, state):
    conv_state, h, (c, n, m) = state
    skip = x
    xn = layer_norm(x, P[pre + "norm.weight"])
    xc, conv_state = causal_conv(xn, conv_state, P[pre + "conv1d.conv.weight"], P[pre + "conv1d.conv.bias"])
    xca = F.silu(xc)
    gi = block_linear(xca, P[pre + "igate_input.weight"]) + block_linear(h, P[pre + "igate_state.weight"], P[pre + "igate_state.bias"])
    gf = block_linear(xca, P[pre + "fgate_input.weight"]) + block_linear(h, P[pre + "fgate_state.weight"], P[pre + "fgate_state.bias"])
    gz = block_linear(xn, P[pre + "zgate_input.weight"]) + block_linear(h, P[pre + "zgate_state.weight"], P[pre + "zgate_state.bias"])
    go = block_linear(xn, P[pre + "ogate_input.weight"]) + block_linear(h, P[pre + "ogate_state.weight"], P[pre + "ogate_state.bias"])
    y, (c_new, n_new, m_new) = slstm_cell(gi, gf, gz, go, c, n, m)
    out = group_norm(y, cfg.slstm_heads, P[pre + "group_norm.weight"], P[pre + "group_norm.bias"])
    return out + skip, (conv_state, y, (c_new, n_new, m_new))


def mlstm_block(P: Params, pre, cfg, x, state):
    B = x.shape[0]
    nh, hs, I = cfg.num_heads, cfg.mlstm_head, cfg.inner
    conv_state, (C, n, m) = state
    skip = x
    xn = layer_norm(x, P[pre + "norm.weight"])
    x_m = P.linear(xn, pre + "x_proj", bias=False)
    x_g = P.linear(xn, pre + "gate_proj", bias=False)
    xc, conv_state = causal_conv(x_m, conv_state, P[pre + "conv1d.conv.weight"], P[pre + "conv1d.conv.bias"])
    xmc = F.silu(xc)
    q = block_linear(xmc, P[pre + "q_proj.weight"])
    k = block_linear(xmc, P[pre + "k_proj.weight"])
    v = block_linear(x_m, P[pre + "v_proj.weight"])
    cp = pre + "mlstm_cell."
    qkv = torch.cat([q, k, v], dim=-1)
    ipre = P.linear(qkv, cp + "igate_proj")
    fpre = P.linear(qkv, cp + "fgate_proj")
    q, k, v = q.view(B, nh, hs), k.view(B, nh, hs), v.view(B, nh, hs)
    log_f = F.logsigmoid(fpre)
    m_new = torch.maximum(ipre, m + log_f)
    i_gate = torch.exp(ipre - m_new)
    f_gate = torch.exp(log_f + m - m_new)
    k = k / math.sqrt(hs)
    n_new = f_gate[:, :, None] * n + i_gate[:, :, None] * k
    C_new = f_gate[:, :, None, None] * C + i_gate[:, :, None, None] * k[:, :, :, None] * v[:, :, None]
    num = (q[:, :, :, None] * C_new).sum(dim=2)
    qn = torch.einsum("bnh,bnh->bn", q, n_new)
    den = torch.maximum(qn.abs(), torch.exp(-m_new)) + 1e-6
    out = num / den[:, :, None]
    out = group_norm(out.reshape(B, I), nh, P[cp + "outnorm.weight"], P[cp + "outnorm.bias"])
    h = (out + P[pre + "learnable_skip"] * xmc) * F.silu(x_g)
    y = P.linear(h, pre + "proj_down", bias=False)
    return y + skip, (conv_state, (C_new, n_new, m_new))


def xlstm(P: Params, pre, cfg, x, state):
    s_state, m_state = state
    x, s_state = slstm_block(P, pre + "slstm.", cfg, x, s_state)
    x, m_state = mlstm_block(P, pre + "mlstm.", cfg, x, m_state)
    return layer_norm(x, P[pre + "final_norm.weight"]), (s_state, m_state)


LAYERS = {"xlstm": xlstm, "mamba2": mamba2, "retnet": retnet, "hawk": hawk}


def tower(P: Params, t, cfg, x, state):
    pre = f"towers.{t}."
    x = P.linear(x, pre + "input_up")
    x = F.relu(x)
    x = P.linear(x, pre + "input_down")
    new = []
    for b, bst in enumerate(state):
        bp = f"{pre}blocks.{b}."
        skip = x
        y, st = LAYERS[TOWERS[t]](P, bp + "layer.", cfg, rms_norm(x, P[bp + "norm1.weight"], None), bst)
        x = y + skip
        h = F.relu(P.linear(rms_norm(x, P[bp + "norm2.weight"], None), bp + "mlp.fc1"))
        x = x + P.linear(h, bp + "mlp.fc2")
        new.append(st)
    return x, new


def init_state(cfg, B, dtype=torch.float32):
    """MultiTowerModel.init_state (model/inference_model.py:145-146)."""
    H, I, z = cfg.hidden_size, cfg.inner, lambda *s: torch.zeros(*s, dtype=dtype)
    out = []
    for ttype in TOWERS:
        blocks = []
        for _ in range(cfg.tower_depth):
            if ttype == "xlstm":
                nh, hs = cfg.num_heads, cfg.mlstm_head
                blocks.append((
                    (z(B, H, 3), z(B, H), (z(B, H), z(B, H), z(B, H) - float("inf"))),
                    (z(B, I, 3), (z(B, nh, hs, hs), z(B, nh, hs), z(B, nh))),
                ))
            elif ttype == "mamba2":
                bc = cfg.mamba_bc_size
                blocks.append([z(B, I, 3), z(B, bc, 3), z(B, bc, 3),
                               z(B, cfg.mamba_heads, cfg.mamba_head_size, bc)])
            elif ttype == "retnet":
                nh, hs = cfg.num_heads, cfg.retnet_head
                blocks.append((torch.zeros(B, dtype=torch.int32), z(B, nh), z(B, nh, hs, hs)))
            else:
                blocks.append([z(B, H, 3), z(B, H)])
        out.append(blocks)
    return out


def blend(old, new, mask):
    """_blend_state (example_model.py:907-949), returning a fresh tree."""
    if isinstance(old, (list, tuple)):
        out = [blend(o, n, mask) for o, n in zip(old, new, strict=True)]
        return type(old)(out) if isinstance(old, tuple) else out
    return torch.where(mask.view(mask.shape[0], *(1,) * (old.dim() - 1)), new, old)


def forward(P: Params, cfg, x, state, mask=None):
    """MultiTowerModel.forward + the client's masked fold."""
    outs, new_state = [], []
    for t in range(4):
        y, st = tower(P, t, cfg, x, state[t])
        outs.append(P.linear(y, "output_proj"))
        new_state.append(st)
    preds = torch.cat(outs, dim=1)
    if mask is not None:
        new_state = blend(state, new_state, mask)
    return preds, new_state


def select_rows(state, idx):
    if isinstance(state, (list, tuple)):
        out = [select_rows(s, idx) for s in state]
        return type(state)(out) if isinstance(state, tuple) else out
    return state[idx]


def flatten(state):
    if isinstance(state, (list, tuple)):
        for s in state:
            yield from flatten(s)
    else:
        yield state
