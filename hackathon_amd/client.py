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

import array
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


def _feature_rows(requests, width: int) -> np.ndarray:
    """[len(requests), width] float32 of the requests' feature lists. The
    values go through one flat list and array.array (float32, round to
    nearest, as numpy converts): 0.42 against 1.02 ms for 256 lists of 79
    Python floats. Anything else (ragged rows, objects array.array does not
    take) goes through numpy as before, which raises for what it cannot
    convert, and process_arrays checks the shape."""
    vals: list = []
    ext = vals.extend
    try:
        for q in requests:
            f = q.features
            if len(f) != width:
                break
            ext(f)
        else:
            return np.frombuffer(array.array("f", vals), dtype=np.float32).reshape(len(requests), width)
    except TypeError:
        pass
    return np.asarray([q.features for q in requests], dtype=np.float32)


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
        weights_path: str | None = None,
        max_rows: int = 1024,
        device: str = "cuda:0",
        seed: int = 0,
    ):
        if engine is None:
            if linear_dtype is None:
                linear_dtype = requested_linear_dtype()
            engine = Engine(config, capacity=num_symbols, max_rows=max(max_rows, num_symbols),
                            linear_dtype=linear_dtype, device=device)
            if weights is None and weights_path is not None:
                # the reference's checkpoint, from a local file
                # (example_model.py:296-302 fetches it over the network)
                from .weights import load_checkpoint

                weights = load_checkpoint(weights_path, config)
            if weights is None:
                from .weights import generate

                weights = generate(config, seed)
            engine.load_weights(weights)
        self.engine = engine
        self.capacity = num_symbols
        if num_symbols > engine.capacity:
            raise ValueError("num_symbols exceeds the engine's slot capacity")
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
        symbols, counts, flat = [], [], []
        for symbol, reqs in requests_by_symbol.items():
            symbols.append(symbol)
            counts.append(len(reqs))
            flat.extend(reqs)
        if not flat:
            return InferenceResponse([], [], time.time())
        feats = _feature_rows(flat, self.num_features)
        order, preds = self.process_arrays(symbols, counts, feats)
        return InferenceResponse([flat[j].unique_id for j in order], preds.tolist(), time.time())

    @torch.inference_mode()
    def process_arrays(self, symbols, counts, features):
        """process_batch for callers holding flat arrays: `symbols` in dict
        order with `counts[i]` requests each, `features` [sum(counts),
        num_features] float32 with each symbol's requests together, in
        order. Returns (order, predictions): the request index answered at
        each response position (the reference's order) and a float64
        [n_req, 4] array in that order. Same slot assignment and zero
        answers as process_batch.

        A batch of more slotted requests than the engine's max_rows runs as
        several ticks, each a range of rounds (round k = the k-th request of
        every symbol with more than k), which keeps each symbol's order and
        the reference's response order."""
        counts = np.asarray(counts, dtype=np.int64)
        feats = np.ascontiguousarray(features, dtype=np.float32)
        if len(counts) != len(symbols):
            raise ValueError("symbols and counts differ in length")
        if feats.shape != (int(counts.sum()), self.num_features):
            raise ValueError(f"features {feats.shape} do not match counts (sum {counts.sum()})")
        slots = np.full(len(counts), -1, dtype=np.int32)
        for i, (sym, c) in enumerate(zip(symbols, counts)):
            if c > 0:
                row = self._row_for(sym)
                slots[i] = -1 if row is None else row
        n_req = int(counts.sum())
        out = np.zeros((n_req, self.num_outputs), dtype=np.float64)
        base = np.concatenate([[0], np.cumsum(counts)])
        parts = []
        # symbols without a slot are answered first, with zeros
        # (example_model.py:826-839)
        unslotted = np.flatnonzero((slots < 0) & (counts > 0))
        if len(unslotted):
            parts.append(np.concatenate([np.arange(base[i], base[i + 1]) for i in unslotted]))
        items = np.flatnonzero(slots >= 0)
        for k0, k1, part in self._round_chunks(counts[items]):
            sub = items if part is None else items[part]
            c = np.clip(counts[sub] - k0, 0, k1 - k0)
            keep = c > 0
            it, c = sub[keep], c[keep]
            runs, req_row, resp = pack_tick(slots[it], c)
            # the chunk's requests (numbered item by item) -> global request index
            sub0 = np.concatenate([[0], np.cumsum(c)[:-1]])
            glob = np.repeat(base[it] + k0 - sub0, c) + np.arange(int(c.sum()))
            out[glob] = self._tick_rows(runs, req_row, feats[glob])
            parts.append(glob[resp])
        order = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)
        return order, out[order]

    def _round_chunks(self, counts):
        """Ticks as (k0, k1, part): rounds [k0, k1) of the symbols `part`
        (indices into counts; None = all), each within max_rows requests.
        Whole rounds are grouped while they fit; a single round larger than
        max_rows is cut into runs of consecutive symbols (dict order), which
        keeps every symbol's order and the response order (symbols in a
        round are independent)."""
        if len(counts) == 0:
            return []
        maxlen = int(counts.max())
        R = self.engine.max_rows
        if int(counts.sum()) <= R:
            return [(0, maxlen, None)]
        # requests in round k: symbols with more than k requests
        per_round = np.cumsum(np.bincount(counts, minlength=maxlen + 1)[::-1])[::-1][1:]
        chunks, k0, rows = [], 0, 0
        for k in range(maxlen):
            n = int(per_round[k])
            if rows and rows + n > R:
                chunks.append((k0, k, None))
                k0, rows = k, 0
            if n > R:
                active = np.flatnonzero(counts > k)
                chunks.extend((k, k + 1, active[j:j + R]) for j in range(0, n, R))
                k0, rows = k + 1, 0
                continue
            rows += n
        if k0 < maxlen:
            chunks.append((k0, maxlen, None))
        return chunks

    def _tick_rows(self, runs, rows, feats):
        """One engine tick over packed runs: feats[j] goes to row rows[j]
        (pinned staging, one H2D copy), and the predictions come back in the
        same order as float64 [len(rows), 4] (one D2H copy, then a wait for
        this stream only)."""
        n = runs.n_rows
        self._feat_host.numpy()[rows] = feats
        self._feat_dev[:n].copy_(self._feat_host[:n], non_blocking=True)
        self.engine.tick(runs, self._feat_dev[:n], self._preds_dev[:n])
        self._preds_host[:n].copy_(self._preds_dev[:n], non_blocking=True)
        self.engine.check()  # waits for the stream; raises if an in-kernel barrier timed out
        return self._preds_host[:n].numpy()[rows].astype(np.float64)
