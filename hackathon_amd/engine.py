"""Python binding of the ensemble engine (hk_engine_* in include/hackathon_amd.h).

The engine owns, on one GPU:
- the packed weights (bf16 for the CastLinear projections in reduced-precision
  mode, fp32 otherwise and for every fp32-kept parameter);
- a slot-indexed recurrent state store for `capacity` symbols;
- workspaces for ticks of up to `max_rows` requests.

`tick()` advances a batch of runs (one per symbol, requests in order) and
returns one 4-wide prediction per request row. `export_state` / `import_state`
move slots' state in the reference's init_state tree layout
(model/inference_model.py:145-146) for parity checks.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .spec import TOWER_TYPES, ModelConfig

c_int, c_int64, c_void_p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_lib.register("hk_engine_create", c_int, [ctypes.POINTER(c_int), c_int, ctypes.POINTER(c_void_p)])
_lib.register("hk_engine_destroy", c_int, [c_void_p])
_lib.register("hk_engine_param_numel", c_int, [c_void_p, c_int, c_int, c_int, ctypes.POINTER(c_int64)])
_lib.register("hk_engine_load_param", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_int64])
_lib.register("hk_engine_load_param_noalloc", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_int64])
_lib.register("hk_engine_state_numel", c_int, [c_void_p, c_int, c_int, ctypes.POINTER(c_int64)])
_lib.register(
    "hk_engine_state_copy", c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p]
)
_lib.register("hk_engine_reset_slots", c_int, [c_void_p, c_void_p, c_int, c_void_p])
_lib.register("hk_engine_log_fill", c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p])
_lib.register("hk_engine_tick", c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p])

_lib.register("hk_engine_check", c_int, [c_void_p, c_void_p])
_lib.register("hk_engine_graphs", c_int, [c_void_p, c_int, c_int])
_lib.register("hk_engine_graph_info", c_int, [c_void_p] + [ctypes.POINTER(c_int64)] * 3)
_lib.register("hk_engine_profile", c_int, [c_void_p, c_int])
_lib.register("hk_engine_profile_read", c_int, [c_void_p, c_int, ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_double)])

# CastLinear modes (example_model.py:150-157): the converted linears' storage
# and compute format; "fp32" leaves every linear in fp32.
LINEAR_DTYPES = {"fp32": 0, "bf16": 1, "fp16": 2}
SCAN_KINDS = {"mlstm": 0, "mamba2": 1, "retnet": 2, "slstm": 3, "gemm": 4}

# Slot order per tower type; must match the enums in csrc/engine.hip.
_COMMON = ["norm1.weight", "norm2.weight", "mlp.fc1.weight", "mlp.fc1.bias", "mlp.fc2.weight", "mlp.fc2.bias"]


def _conv_taps(*ws):
    """CausalConv1d weights [C,1,4] (one or more, concatenated over channels)
    -> tap-major [4, C]."""
    w = torch.cat([x[:, 0, :] for x in ws], dim=0)
    return w.t().contiguous()


def _cat(*ts):
    return torch.cat([t.reshape(-1) for t in ts])


def _layer_slots(cfg: ModelConfig, ltype: str, P: dict, pre: str):
    """Packed slot arrays for one block's layer, in engine slot order."""
    g = lambda n: P[pre + n]
    if ltype == "xlstm":
        return [
            g("slstm.norm.weight"),
            _conv_taps(g("slstm.conv1d.conv.weight")),
            g("slstm.conv1d.conv.bias"),
            _cat(*(g(f"slstm.{x}gate_input.weight") for x in "ifzo")),
            _cat(*(g(f"slstm.{x}gate_state.weight") for x in "ifzo")),
            _cat(*(g(f"slstm.{x}gate_state.bias") for x in "ifzo")),
            g("slstm.group_norm.weight"),
            g("slstm.group_norm.bias"),
            g("mlstm.norm.weight"),
            _cat(g("mlstm.x_proj.weight"), g("mlstm.gate_proj.weight")),
            _cat(g("mlstm.q_proj.weight"), g("mlstm.k_proj.weight"), g("mlstm.v_proj.weight")),
            _conv_taps(g("mlstm.conv1d.conv.weight")),
            g("mlstm.conv1d.conv.bias"),
            _cat(g("mlstm.mlstm_cell.igate_proj.weight"), g("mlstm.mlstm_cell.fgate_proj.weight")),
            _cat(g("mlstm.mlstm_cell.igate_proj.bias"), g("mlstm.mlstm_cell.fgate_proj.bias")),
            g("mlstm.mlstm_cell.outnorm.weight"),
            g("mlstm.mlstm_cell.outnorm.bias"),
            g("mlstm.proj_down.weight"),
            g("mlstm.learnable_skip"),
            g("final_norm.weight"),
        ]
    if ltype == "mamba2":
        return [
            _cat(g("input_proj.weight"), g("b_proj.weight"), g("c_proj.weight"), g("z_proj.weight")),
            g("dt_proj.weight"),
            g("dt_proj.bias"),
            _conv_taps(g("input_conv.conv.weight"), g("b_conv.conv.weight"), g("c_conv.conv.weight")),
            _cat(g("input_conv.conv.bias"), g("b_conv.conv.bias"), g("c_conv.conv.bias")),
            g("a"),
            g("d"),
            g("norm.weight"),
            g("out_proj.weight"),
        ]
    if ltype == "retnet":
        return [
            _cat(*(g(f"{x}_proj.weight") for x in "qkvg")),
            g("out_proj.weight"),
            g("decay"),
            g("angle"),
        ]
    return [
        _cat(g("gate_proj.weight"), g("recurrent_proj.weight")),
        _conv_taps(g("conv.conv.weight")),
        g("conv.conv.bias"),
        _cat(g("rglru.input_gate.weight"), g("rglru.recurrence_gate.weight")),
        g("rglru.a"),
        g("out_proj.weight"),
    ]


@dataclass
class Runs:
    """A tick's packing: runs sorted by non-increasing length."""

    slot_ids: np.ndarray   # int32 [n_runs]
    run_off: np.ndarray    # int32 [n_runs + 1]

    @property
    def n_rows(self) -> int:
        return int(self.run_off[-1])


def pack_runs(slots, lengths) -> tuple[Runs, np.ndarray]:
    """Order runs by non-increasing length (stable). Returns the packing and
    `order`, the input index of each packed run."""
    lengths = np.asarray(lengths, dtype=np.int64)
    order = np.argsort(-lengths, kind="stable")
    slot_ids = np.asarray(slots, dtype=np.int32)[order]
    run_off = np.zeros(len(order) + 1, dtype=np.int32)
    np.cumsum(lengths[order], out=run_off[1:])
    return Runs(np.ascontiguousarray(slot_ids), run_off), order


def pack_tick(item_slots, item_lens):
    """Native packing of one process_batch call (hk_pack_tick; the loops of
    example_model.py:819-905). Items are the batch's symbols in dict order,
    slot -1 meaning "no slot" (answered with zeros). Returns the runs for
    Engine.tick, `req_row` (each request's row in the tick, -1 if unslotted;
    requests numbered item by item) and `resp_req` (the request answered at
    each response position, in the reference's order)."""
    slots = np.ascontiguousarray(item_slots, dtype=np.int32)
    lens = np.ascontiguousarray(item_lens, dtype=np.int32)
    n_items = len(slots)
    if len(lens) != n_items:
        raise ValueError("pack_tick: item_slots and item_lens differ in length")
    n_req = int(lens.sum(dtype=np.int64)) if n_items else 0
    slot_ids = np.empty(max(n_items, 1), dtype=np.int32)
    run_off = np.empty(n_items + 1, dtype=np.int32)
    req_row = np.empty(max(n_req, 1), dtype=np.int32)
    resp_req = np.empty(max(n_req, 1), dtype=np.int32)
    n_runs = ctypes.c_int(0)
    n_rows = ctypes.c_int(0)
    _lib.check(_lib.lib().hk_pack_tick(
        slots.ctypes.data, lens.ctypes.data, n_items, slot_ids.ctypes.data, run_off.ctypes.data,
        req_row.ctypes.data, resp_req.ctypes.data, ctypes.byref(n_runs), ctypes.byref(n_rows)),
        "hk_pack_tick")
    runs = Runs(slot_ids[:n_runs.value].copy(), run_off[:n_runs.value + 1].copy())
    return runs, req_row[:n_req], resp_req[:n_req]


class Engine:
    def __init__(
        self,
        cfg: ModelConfig,
        capacity: int,
        max_rows: int = 1024,
        max_runs: int | None = None,
        linear_dtype: str = "bf16",
        device: str | torch.device = "cuda:0",
    ):
        if linear_dtype not in LINEAR_DTYPES:
            raise ValueError(f"linear_dtype must be one of {tuple(LINEAR_DTYPES)}")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise _lib.HipLibraryError("the engine needs a GPU device")
        self.cfg = cfg
        self.capacity = capacity
        self.max_rows = max_rows
        self.max_runs = max_runs or min(capacity, max_rows)
        self.linear_dtype = linear_dtype
        vals = [
            cfg.hidden_size, cfg.proj_size, cfg.tower_depth, cfg.num_heads, cfg.num_features,
            cfg.mamba_head_size, cfg.mamba_bc_size, capacity, max_rows, self.max_runs,
            LINEAR_DTYPES[linear_dtype],
        ]
        arr = (c_int * len(vals))(*vals)
        handle = c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().hk_engine_create(arr, len(vals), ctypes.byref(handle)), "hk_engine_create")
        self._h = handle
        self.reset_slots()
        self._loaded = False

    # -- lifecycle ---------------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().hk_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self):
        return _lib.current_stream(self.device)

    # -- weights -------------------------------------------------------------------
    def load_param(self, tower: int, layer: int, slot: int, t: torch.Tensor, noalloc: bool = False):
        """Bind one packed weight slot (hk_engine_load_param, or with noalloc
        hk_engine_load_param_noalloc, which allocates no device memory)."""
        t = t.detach().to(torch.float32).contiguous().cpu()
        n = c_int64()
        _lib.check(_lib.lib().hk_engine_param_numel(self._h, tower, layer, slot, ctypes.byref(n)), "param_numel")
        if t.numel() != n.value:
            raise ValueError(f"slot ({tower},{layer},{slot}) expects {n.value} values, got {t.numel()}")
        fn = "hk_engine_load_param_noalloc" if noalloc else "hk_engine_load_param"
        with torch.cuda.device(self.device):
            _lib.check(getattr(_lib.lib(), fn)(self._h, tower, layer, slot, t.data_ptr(), t.numel()), fn)

    def load_weights(self, params: dict[str, torch.Tensor], noalloc: bool = False):
        """Bind a full parameter set keyed by the reference's state_dict names
        (noalloc: through the entry point that allocates no device memory)."""
        cfg = self.cfg
        fpad = (cfg.num_features + 63) // 64 * 64
        for t, ltype in enumerate(TOWER_TYPES):
            pre = f"towers.{t}."
            up = params[pre + "input_up.weight"]
            up_pad = torch.zeros(up.shape[0], fpad, dtype=torch.float32)
            up_pad[:, : up.shape[1]] = up
            for i, arr in enumerate([up_pad, params[pre + "input_up.bias"], params[pre + "input_down.weight"],
                                     params[pre + "input_down.bias"]]):
                self.load_param(t, -1, i, arr, noalloc=noalloc)
            for b in range(cfg.tower_depth):
                bp = f"{pre}blocks.{b}."
                arrs = [params[bp + n] for n in _COMMON] + _layer_slots(cfg, ltype, params, bp + "layer.")
                for i, arr in enumerate(arrs):
                    self.load_param(t, b, i, arr, noalloc=noalloc)
        self.load_param(-1, -1, 0, params["output_proj.weight"].reshape(-1), noalloc=noalloc)
        self.load_param(-1, -1, 1, params["output_proj.bias"].reshape(-1), noalloc=noalloc)
        self._loaded = True

    # -- state -----------------------------------------------------------------------
    def reset_slots(self, slots=None):
        with torch.cuda.device(self.device):
            if slots is None:
                st = _lib.lib().hk_engine_reset_slots(self._h, None, -1, self._stream())
            else:
                arr = np.ascontiguousarray(np.asarray(slots, dtype=np.int32))
                st = _lib.lib().hk_engine_reset_slots(self._h, arr.ctypes.data, len(arr), self._stream())
        _lib.check(st, "hk_engine_reset_slots")

    def log_fill(self, slots, counts):
        """Append counts[i] zero-valued pending-update entries to every
        write-back log of slot slots[i] (up to the capacity of 8): the state
        is unchanged, and later ticks find the logs as full as after a long
        run (a benchmark starts at steady state with it)."""
        sl = np.ascontiguousarray(np.asarray(slots, dtype=np.int32))
        ct = np.ascontiguousarray(np.asarray(counts, dtype=np.int32))
        assert sl.shape == ct.shape and sl.ndim == 1
        with torch.cuda.device(self.device):
            st = _lib.lib().hk_engine_log_fill(self._h, sl.ctypes.data, ct.ctypes.data, len(sl),
                                              self._stream())
        _lib.check(st, "hk_engine_log_fill")

    def _leaf_numel(self, tower: int, leaf: int) -> int:
        n = c_int64()
        _lib.check(_lib.lib().hk_engine_state_numel(self._h, tower, leaf, ctypes.byref(n)), "state_numel")
        return n.value

    def _copy_leaf(self, tower, layer, leaf, slot0, nslots, buf, to_engine):
        _lib.check(
            _lib.lib().hk_engine_state_copy(self._h, tower, layer, leaf, slot0, nslots, buf.data_ptr(),
                                            1 if to_engine else 0, self._stream()),
            "hk_engine_state_copy",
        )

    def _raw_leaves(self, tower, layer, slot0, nslots):
        nleaves = {0: 9, 1: 2, 2: 3, 3: 2}[tower]
        out = []
        for leaf in range(nleaves):
            per = self._leaf_numel(tower, leaf)
            buf = torch.empty(nslots, per, dtype=torch.float32, device=self.device)
            self._copy_leaf(tower, layer, leaf, slot0, nslots, buf, False)
            out.append(buf)
        return out

    def copy_slots(self, src0: int, dst0: int, nslots: int):
        """Copy the state of slots [src0, src0+nslots) to [dst0, dst0+nslots)
        (ranges disjoint), stream-ordered: every leaf of every block, pending
        write-back entries applied (the source's value is unchanged)."""
        assert nslots >= 0 and 0 <= src0 and 0 <= dst0
        assert max(src0, dst0) + nslots <= self.capacity
        assert src0 + nslots <= dst0 or dst0 + nslots <= src0, "slot ranges overlap"
        for t in range(4):
            for b in range(self.cfg.tower_depth):
                for leaf, buf in enumerate(self._raw_leaves(t, b, src0, nslots)):
                    self._copy_leaf(t, b, leaf, dst0, nslots, buf, True)

    def export_state(self, slot0: int = 0, nslots: int | None = None):
        """State of slots [slot0, slot0+nslots) in the reference's init_state
        tree: [tower][block] -> the layer's nested leaves (conv windows as
        [B, C, 3], the Mamba2 ssm as [B, heads, head, bc], RetNet offsets int32)."""
        cfg = self.cfg
        n = self.capacity - slot0 if nslots is None else nslots
        H, I, bc = cfg.hidden_size, cfg.inner, cfg.mamba_bc_size
        tree = []
        for t in range(4):
            blocks = []
            for b in range(cfg.tower_depth):
                lv = self._raw_leaves(t, b, slot0, n)
                conv = lambda x, C: x.view(n, 3, C).transpose(1, 2).contiguous()
                if t == 0:
                    nh, hs = cfg.num_heads, cfg.mlstm_head
                    blocks.append((
                        (conv(lv[0], H), lv[1], (lv[2], lv[3], lv[4])),
                        (conv(lv[5], I), (lv[6].view(n, nh, hs, hs), lv[7].view(n, nh, hs), lv[8])),
                    ))
                elif t == 1:
                    C = I + 2 * bc
                    cw = conv(lv[0], C)
                    ssm = lv[1].view(n, cfg.mamba_heads, bc, cfg.mamba_head_size).transpose(2, 3).contiguous()
                    blocks.append([cw[:, :I].contiguous(), cw[:, I:I + bc].contiguous(),
                                   cw[:, I + bc:].contiguous(), ssm])
                elif t == 2:
                    nh, hs = cfg.num_heads, cfg.retnet_head
                    blocks.append((lv[0].view(torch.int32).view(n), lv[1], lv[2].view(n, nh, hs, hs)))
                else:
                    blocks.append([conv(lv[0], H), lv[1]])
            tree.append(blocks)
        return tree

    def import_state(self, tree, slot0: int = 0):
        """Inverse of export_state."""
        cfg = self.cfg
        H, I, bc = cfg.hidden_size, cfg.inner, cfg.mamba_bc_size
        dev = self.device
        unconv = lambda x: x.to(dev, torch.float32).transpose(1, 2).contiguous()
        for t in range(4):
            for b in range(cfg.tower_depth):
                st = tree[t][b]
                if t == 0:
                    (sc, sh, (c, nn, m)), (lc, (C, ln, lm)) = st
                    leaves = [unconv(sc), sh, c, nn, m, unconv(lc), C, ln, lm]
                elif t == 1:
                    xc, bcv, cc, ssm = st
                    leaves = [unconv(torch.cat([xc, bcv, cc], dim=1)), ssm.to(dev).transpose(2, 3)]
                elif t == 2:
                    off, scales, S = st
                    leaves = [off.to(dev, torch.int32).view(torch.float32), scales, S]
                else:
                    leaves = [unconv(st[0]), st[1]]
                n = leaves[0].shape[0]
                for leaf, arr in enumerate(leaves):
                    buf = arr.to(dev).contiguous().view(n, -1)
                    if buf.dtype != torch.float32:
                        buf = buf.view(torch.float32)
                    self._copy_leaf(t, b, leaf, slot0, n, buf, True)
        torch.cuda.synchronize(dev)

    # -- ticks ---------------------------------------------------------------------
    def tick(self, runs: Runs, features: torch.Tensor, preds: torch.Tensor | None = None) -> torch.Tensor:
        """Advance `runs` with `features` [n_rows, F] (fp32, on the engine's
        device, rows grouped by run in order). Returns preds [n_rows, 4]."""
        if not self._loaded:
            raise _lib.HipLibraryError("weights are not loaded")
        n = runs.n_rows
        assert features.dtype == torch.float32 and features.is_contiguous()
        assert features.device == self.device and tuple(features.shape) == (n, self.cfg.num_features)
        if preds is None:
            preds = torch.empty(n, 4, dtype=torch.float32, device=self.device)
        assert preds.is_contiguous() and tuple(preds.shape) == (n, 4)
        slot_ids = np.ascontiguousarray(runs.slot_ids, dtype=np.int32)
        run_off = np.ascontiguousarray(runs.run_off, dtype=np.int32)
        st = _lib.lib().hk_engine_tick(
            self._h, slot_ids.ctypes.data, run_off.ctypes.data, len(slot_ids), features.data_ptr(),
            preds.data_ptr(), self._stream(),
        )
        _lib.check(st, "hk_engine_tick")
        return preds

    def graphs(self, max_rows: int, max_graphs: int = 256):
        """Replay ticks of at most max_rows rows through cached hipGraphs
        (one capture per tick shape, at most max_graphs shapes cached); 0
        turns replay off (the reference's captured step,
        example_model.py:444-492)."""
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().hk_engine_graphs(self._h, max_rows, max_graphs), "hk_engine_graphs")

    def graph_info(self) -> dict:
        """{"cached", "captures", "replays"} of the graph cache."""
        vals = [c_int64() for _ in range(3)]
        _lib.check(_lib.lib().hk_engine_graph_info(self._h, *[ctypes.byref(v) for v in vals]),
                   "hk_engine_graph_info")
        return dict(zip(("cached", "captures", "replays"), (v.value for v in vals)))

    def check(self):
        """Wait for the current stream's work (every tick enqueued on it) and
        raise if any in-kernel step barrier timed out. Releases the GIL while
        it waits (ctypes does), so a receive thread keeps running."""
        _lib.check(_lib.lib().hk_engine_check(self._h, self._stream()), "hk_engine_check")

    # -- measurement ---------------------------------------------------------------
    def profile(self, kinds=True):
        """Time the launches of the given kinds (names of SCAN_KINDS; True =
        all, False or () = stop); clears earlier records."""
        if kinds is True:
            kinds = tuple(SCAN_KINDS)
        elif kinds is False:
            kinds = ()
        mask = 0
        for k in kinds:
            mask |= 1 << SCAN_KINDS[k]
        _lib.check(_lib.lib().hk_engine_profile(self._h, mask), "hk_engine_profile")

    def profile_read(self, kind: str) -> tuple[int, float]:
        """(launch count, summed ms) of the recorded launches of `kind`."""
        n, ms = c_int(), ctypes.c_double()
        _lib.check(_lib.lib().hk_engine_profile_read(self._h, SCAN_KINDS[kind], ctypes.byref(n), ctypes.byref(ms)),
                   "hk_engine_profile_read")
        return n.value, ms.value
