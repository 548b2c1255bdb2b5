"""process_batch() drop-in (example_model.py:769-905) on the HIP engine.

`NnInferenceClient.process_batch(requests_by_symbol)` keeps the reference's
response semantics exactly:
- one 4-float prediction per request (one per tower);
- each symbol's requests advance its state once each, in list order;
- responses are listed round by round (round k = the k-th request of every
  symbol with more than k), symbols in dict order within a round, after the
  answers for symbols that found no free row (example_model.py:826-846,
  :881-899);
- symbols receive a state slot on first sight and keep it; past capacity a
  symbol is answered with [0.0]*4 and nothing is staged, with a warning
  printed once per process (example_model.py:724-767, :830-839);
- an empty batch returns an empty response.

Where the reference runs one full-capacity forward per round, the engine
advances every symbol's whole run in one layer-major tick.

`PendingRequest` and `InferenceResponse` carry the same fields as the
reference's client.py:28-39 and protocol.py:38-43, so objects of either type
can be passed in and the response serialises the same way.
"""

from __future__ import annotations

import os
import time
from dataclasses import dataclass, field
from typing import Dict, List

import numpy as np
import torch

from .engine import LINEAR_DTYPES, Engine, pack_tick
from .spec import DEFAULT, ModelConfig

# The reference client's precision default and its override
# (example_model.py:150-157, :306-313).
DEFAULT_LINEAR_DTYPE = "fp16"


def requested_linear_dtype() -> str:
    """LINEAR_DTYPE from the environment as the reference reads it: case-
    and space-insensitive, an unknown value falls back to the default with a
    message (example_model.py:306-313)."""
    requested = os.environ.get("LINEAR_DTYPE", DEFAULT_LINEAR_DTYPE).strip().lower()
    if requested not in LINEAR_DTYPES:
        print(f"LINEAR_DTYPE={requested!r} is not one of {sorted(LINEAR_DTYPES)}; "
              f"falling back to {DEFAULT_LINEAR_DTYPE}")
        requested = DEFAULT_LINEAR_DTYPE
    return requested


@dataclass
class PendingRequest:
    unique_id: int
    symbol: str
    features: List[float]
    received_time: float = 0.0

    def age_ms(self) -> float:
        return (time.time() - self.received_time) * 1000


@dataclass
class InferenceResponse:
    unique_ids: list
    predictions: list
    client_timestamp: float
    message_type: str = field(default="inference_response")


class NnInferenceClient:
    """The inference client's model side, without the TCP runtime.

    `num_symbols` is a capacity of state slots, as in the reference
    (example_model.py:249-272). To serve over the reference's protocol, mix
    this class into its BaseInferenceClient.
    """

    _overflow_warned = False

    def __init__(
        self,
        num_symbols: int,
        engine: Engine | None = None,
        config: ModelConfig = DEFAULT,
        weights: dict | None = None,
        linear_dtype: str | None = None,
        max_rows: int = 1024,
        device: str = "cuda:0",
        seed: int = 0,
    ):
        if engine is None:
            if linear_dtype is None:
                linear_dtype = requested_linear_dtype()
            engine = Engine(config, capacity=num_symbols, max_rows=max(max_rows, num_symbols),
                            linear_dtype=linear_dtype, device=device)
            if weights is None:
                from .weights import generate

                weights = generate(config, seed)
            engine.load_weights(weights)
        self.engine = engine
        self.capacity = num_symbols
        if num_symbols > engine.capacity:
            raise ValueError("num_symbols exceeds the engine's slot capacity")
        if engine.max_rows < num_symbols:
            # One round holds at most one request per symbol; it must fit a tick.
            raise ValueError("the engine's max_rows must be at least num_symbols")
        self.symbol_to_idx: Dict[str, int] = {}
        self.num_outputs = 4
        self.num_features = engine.cfg.num_features
        self.device = engine.device
        n = engine.max_rows
        self._feat_host = torch.empty(n, self.num_features, dtype=torch.float32, pin_memory=True)
        self._feat_dev = torch.empty(n, self.num_features, dtype=torch.float32, device=self.device)
        self._preds_dev = torch.empty(n, 4, dtype=torch.float32, device=self.device)
        self._preds_host = torch.empty(n, 4, dtype=torch.float32, pin_memory=True)

    def _row_for(self, symbol: str) -> int | None:
        """example_model.py:724-767: slot on first sight, never reclaimed."""
        row = self.symbol_to_idx.get(symbol)
        if row is not None:
            return row
        row = len(self.symbol_to_idx)
        if row >= self.capacity:
            if not NnInferenceClient._overflow_warned:
                NnInferenceClient._overflow_warned = True
                print(
                    f"WARNING: out of state slots ({self.capacity} of them, all owned); "
                    f"{symbol!r} and every later new symbol are answered with zeros. "
                    f"This prints once."
                )
            return None
        self.symbol_to_idx[symbol] = row
        return row

    @torch.inference_mode()
    def process_batch(self, requests_by_symbol: Dict[str, List[PendingRequest]]) -> InferenceResponse:
        all_ids: list = []
        all_preds: list = []
        items = []  # (slot, reqs) in dict order
        for symbol, reqs in requests_by_symbol.items():
            if not reqs:
                continue
            slot = self._row_for(symbol)
            if slot is None:
                for req in reqs:
                    all_ids.append(req.unique_id)
                    all_preds.append([0.0] * self.num_outputs)
                continue
            items.append((slot, reqs))
        if not items:
            return InferenceResponse(all_ids, all_preds, time.time())

        if sum(len(r) for _, r in items) <= self.engine.max_rows:
            self._run_items(items, all_ids, all_preds)
        else:
            # Round-major chunks of at most max_rows requests: chunk j holds
            # rounds [k0, k1) of every symbol, which keeps each symbol's order
            # and the reference's response order.
            maxlen = max(len(r) for _, r in items)
            k0 = 0
            while k0 < maxlen:
                k1, rows = k0, 0
                while k1 < maxlen:
                    add = sum(1 for _, r in items if len(r) > k1)
                    if rows + add > self.engine.max_rows and k1 > k0:
                        break
                    rows += add
                    k1 += 1
                part = [(slot, reqs[k0:k1]) for slot, reqs in items if len(reqs) > k0]
                self._run_items(part, all_ids, all_preds)
                k0 = k1
        return InferenceResponse(all_ids, all_preds, time.time())

    def _run_items(self, items, all_ids, all_preds):
        """One engine tick over (slot, requests) pairs; appends the answers
        round by round."""
        flat = [q for _, reqs in items for q in reqs]
        feats = np.asarray([q.features for q in flat], dtype=np.float32)
        runs, req_row, resp_req = pack_tick([s for s, _ in items], [len(r) for _, r in items])
        preds = self._tick_rows(runs, req_row, feats)
        all_ids.extend(flat[j].unique_id for j in resp_req)
        all_preds.extend(preds[resp_req].tolist())

    def _tick_rows(self, runs, rows, feats):
        """One engine tick over packed runs: feats[j] goes to row rows[j]
        (pinned staging, one H2D copy), and the predictions come back in the
        same order as float64 [len(rows), 4] (one D2H copy)."""
        n = runs.n_rows
        self._feat_host.numpy()[rows] = feats
        self._feat_dev[:n].copy_(self._feat_host[:n], non_blocking=True)
        self.engine.tick(runs, self._feat_dev[:n], self._preds_dev[:n])
        self._preds_host[:n].copy_(self._preds_dev[:n], non_blocking=True)
        self.engine.check()  # synchronises; raises if an in-kernel barrier timed out
        return self._preds_host[:n].numpy()[rows].astype(np.float64)

    def process_arrays(self, symbols, counts, features):
        """process_batch for callers holding flat arrays: `symbols` in dict
        order with `counts[i]` requests each, `features` [sum(counts),
        num_features] float32 with each symbol's requests together, in
        order. Returns (resp_req, predictions): the request index answered at
        each response position (the reference's order) and a float64
        [n_req, 4] array in that order. Same slot assignment and zero
        answers as process_batch; at most max_rows slotted requests."""
        counts = np.asarray(counts, dtype=np.int64)
        feats = np.ascontiguousarray(features, dtype=np.float32)
        if feats.shape != (int(counts.sum()), self.num_features):
            raise ValueError(f"features {feats.shape} do not match counts (sum {counts.sum()})")
        slots = np.full(len(counts), -1, dtype=np.int32)
        for i, (sym, c) in enumerate(zip(symbols, counts)):
            if c > 0:
                row = self._row_for(sym)
                slots[i] = -1 if row is None else row
        runs, req_row, resp_req = pack_tick(slots, counts)
        if runs.n_rows > self.engine.max_rows:
            raise ValueError(f"process_arrays: more than {self.engine.max_rows} slotted requests")
        out = np.zeros((len(req_row), self.num_outputs), dtype=np.float64)
        if runs.n_rows:
            sel = np.flatnonzero(req_row >= 0)
            out[sel] = self._tick_rows(runs, req_row[sel], feats[sel])
        return resp_req, out[resp_req]
