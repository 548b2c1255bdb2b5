"""The reference's model API (model/inference_model.py:103-146) on the engine.

`MultiTowerModel(config)` keeps the reference's call shape:
- `init_state(batch_size, device)` returns the state of `batch_size` fresh
  rows (the reference's init_state values);
- `forward(x, state, mask=None) -> (preds, new_state)`, also as
  `model(x, state, mask)`, advances row b of the state by one step with x[b]
  where mask[b] is True (every row for mask None) and returns one prediction
  per tower per row, [B, 4].

The state does not travel as a tree of tensors: it stays resident in the
engine's HBM store, and `init_state` hands out an `EngineState`, a handle on
`batch_size` consecutive slots of it. How the two mask forms map onto that:
- With a mask, the reference advances its three big leaves in place and
  returns them as the same objects (model/inference_model.py:120-131).
  Here every leaf is advanced in place on the active rows and
  `forward` returns the same handle; idle rows keep their state bit for bit,
  so the caller's where(mask, new, old) fold (example_model.py:907-949) is
  already done.
- With mask None the reference writes nothing in place and returns fresh
  tensors (model/inference_model.py:132-134), so the old state stays
  usable. Here too: the rows are copied to `batch_size` fresh slots, which
  then advance, and a new handle on them is returned; the old handle still
  holds the old state. Each handle gives its slots back when it is released
  or garbage-collected, as the reference's tensors are freed, so the model
  needs room for both states at once (2 x batch_size rows) during the call.

`EngineState.export()` gives the reference's init_state tree (tensors) for
inspection, and `EngineState.load(tree)` writes one in.

Two deliberate deviations:
- Rows whose mask is False come back as zero predictions (the reference
  returns the full model's output on those rows, computed with the matrix
  cells' outputs zeroed, and its client discards them). The engine runs
  only the active rows.
- The mask is read on the host, because the tick's launch shapes (rows,
  runs, steps) come from it: a CPU bool tensor, numpy array or sequence
  costs nothing; a mask on the GPU is copied to the host first, which waits
  for the work queued before it (the reference reads a device mask inside
  its captured step, example_model.py:865-871). The engine's own client
  (NnInferenceClient.process_batch) builds its runs on the host and never
  waits for a mask.

`load_state_dict(sd)` binds a reference state_dict (weights only, as the
reference client loads its checkpoint with torch.load(weights_only=True),
example_model.py:296-302); `from_checkpoint(path)` reads one from a local
file with that loader.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .engine import Engine, Runs
from .spec import DEFAULT, ModelConfig


class StaleStateError(RuntimeError):
    """A released state handle was used again."""


class EngineState:
    """`batch_size` consecutive slots of a model's HBM state store."""

    def __init__(self, model: "MultiTowerModel", slot0: int, batch_size: int):
        self._model = model
        self.slot0 = slot0
        self.batch_size = batch_size
        self._live = True

    def _check(self, model):
        if not self._live:
            raise StaleStateError("this state was released")
        if model is not self._model:
            raise ValueError("the state belongs to another model")

    def export(self):
        """The rows' state in the reference's init_state tree layout."""
        self._check(self._model)
        return self._model.engine.export_state(self.slot0, self.batch_size)

    def load(self, tree):
        """Write a state tree (the reference's layout, batch_size rows)."""
        self._check(self._model)
        self._model.engine.import_state(tree, self.slot0)

    def release(self):
        """Give the slots back to the model."""
        if self._live:
            self._live = False
            self._model._free(self.slot0, self.batch_size)

    def __del__(self):
        try:
            self.release()
        except Exception:  # interpreter shutdown: the model may be gone
            pass


class MultiTowerModel:
    """model/inference_model.py:103-146 on the HIP engine.

    `capacity` bounds the rows of all live states together; `linear_dtype`
    is the CastLinear mode ("fp32", "bf16" or "fp16", example_model.py:
    150-157). Weights come from `weights` (a reference state_dict) or, when
    None, from the init spec with `seed`.
    """

    def __init__(self, config: ModelConfig = DEFAULT, capacity: int = 64,
                 linear_dtype: str = "fp32", weights: dict | None = None, seed: int = 0,
                 device: str | torch.device = "cuda:0", max_rows: int | None = None):
        self.config = config
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.engine = Engine(config, capacity=capacity, max_rows=max_rows or capacity,
                             linear_dtype=linear_dtype, device=self.device)
        self._free_ranges = [(0, capacity)]  # (slot0, count), disjoint
        if weights is None:
            from .weights import generate

            weights = generate(config, seed)
        self.load_state_dict(weights)

    @classmethod
    def from_checkpoint(cls, path, config: ModelConfig = DEFAULT, **kw):
        """A model whose weights are read from a local state_dict file
        (torch.load with weights_only=True)."""
        from .weights import load_checkpoint

        return cls(config, weights=load_checkpoint(path, config), **kw)

    def load_state_dict(self, state_dict: dict, strict: bool = True):
        """Bind a reference state_dict (its parameter names). With strict,
        unexpected keys raise as well as missing ones, as torch's
        load_state_dict does."""
        from .weights import check_state_dict

        check_state_dict(self.config, state_dict, strict)
        self.engine.load_weights(state_dict)

    # -- state slots ----------------------------------------------------------------
    def _alloc(self, n: int) -> int:
        for i, (s0, cnt) in enumerate(self._free_ranges):
            if cnt >= n:
                self._free_ranges[i] = (s0 + n, cnt - n)
                return s0
        raise _lib.CapacityError(f"no {n} free state rows (model capacity {self.engine.capacity})")

    def _free(self, s0: int, n: int):
        self._free_ranges.append((s0, n))
        self._free_ranges.sort()
        merged = []
        for a, c in self._free_ranges:
            if c == 0:
                continue
            if merged and merged[-1][0] + merged[-1][1] == a:
                merged[-1] = (merged[-1][0], merged[-1][1] + c)
            else:
                merged.append((a, c))
        self._free_ranges = merged

    def init_state(self, batch_size: int, device=None) -> EngineState:
        """MultiTowerModel.init_state (model/inference_model.py:145-146):
        batch_size rows at the reference's initial values."""
        if device is not None:
            d = torch.device(device)
            if d.type != self.device.type or (d.index is not None and d.index != self.device.index):
                raise ValueError(f"the state lives on {self.device}")
        s0 = self._alloc(batch_size)
        self.engine.reset_slots(np.arange(s0, s0 + batch_size, dtype=np.int32))
        return EngineState(self, s0, batch_size)

    # -- step ---------------------------------------------------------------------------
    def forward(self, x: torch.Tensor, state: EngineState, mask=None):
        state._check(self)
        B = state.batch_size
        assert x.dtype == torch.float32 and tuple(x.shape) == (B, self.config.num_features), (
            f"x must be float32 [{B}, {self.config.num_features}]")
        if mask is None:
            # the reference leaves the old state as it was: advance a copy
            active = np.arange(B, dtype=np.int32)
            try:
                s0 = self._alloc(B)
            except _lib.CapacityError as exc:
                raise _lib.CapacityError(
                    f"a mask=None forward keeps the old state: it needs {B} more free rows "
                    f"(model capacity {self.engine.capacity})") from exc
            with torch.cuda.device(self.device):
                self.engine.copy_slots(state.slot0, s0, B)
            state = EngineState(self, s0, B)
        else:
            m = mask.detach().cpu().numpy() if isinstance(mask, torch.Tensor) else np.asarray(mask)
            assert m.dtype == np.bool_ and m.shape == (B,), "mask must be bool [B]"
            active = np.flatnonzero(m).astype(np.int32)
        x = x.to(self.device)
        out = torch.zeros(B, 4, dtype=torch.float32, device=self.device)
        if len(active):
            n = len(active)
            runs = Runs(np.ascontiguousarray(active + state.slot0, dtype=np.int32),
                        np.arange(n + 1, dtype=np.int32))
            if n == B:
                out = self.engine.tick(runs, x.contiguous(), out)
            else:
                idx = torch.from_numpy(active.astype(np.int64)).pin_memory().to(
                    self.device, non_blocking=True)
                preds = self.engine.tick(runs, x.index_select(0, idx).contiguous())
                out.index_copy_(0, idx, preds)
        return out, state

    __call__ = forward

    def close(self):
        self.engine.close()
