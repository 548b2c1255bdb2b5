"""Oracle for process_batch (test infrastructure only).

Restates NnInferenceClient.process_batch / run_round / _row_for
(example_model.py:724-767, :769-905) literally: rounds of at most one request
per symbol, each round one masked forward over every capacity row through
oracle.model.forward, predictions read back per round.
"""

from __future__ import annotations

import numpy as np
import torch

from . import model as om


def _to(tree, device):
    if isinstance(tree, (list, tuple)):
        out = [_to(t, device) for t in tree]
        return tuple(out) if isinstance(tree, tuple) else out
    return tree.to(device)


class OracleClient:
    """`device`: where the state and each round's inputs live (the params
    `P` must be there too); "cpu" by default."""

    def __init__(self, P: om.Params, cfg, capacity: int, device="cpu"):
        self.P, self.cfg, self.capacity = P, cfg, capacity
        self.device = torch.device(device)
        self.state = _to(om.init_state(cfg, capacity, P.dtype), self.device)
        self.symbol_to_idx = {}

    def _row_for(self, symbol):
        row = self.symbol_to_idx.get(symbol)
        if row is not None:
            return row
        row = len(self.symbol_to_idx)
        if row >= self.capacity:
            return None
        self.symbol_to_idx[symbol] = row
        return row

    @torch.inference_mode()
    def process_batch(self, requests_by_symbol):
        ids, preds = [], []
        items = []
        for symbol, reqs in requests_by_symbol.items():
            if not reqs:
                continue
            row = self._row_for(symbol)
            if row is None:
                for r in reqs:
                    ids.append(r.unique_id)
                    preds.append([0.0] * 4)
                continue
            items.append((row, reqs))
        if not items:
            return ids, preds
        for k in range(max(len(r) for _, r in items)):
            idx, feats, batch = [], [], []
            for row, reqs in items:
                if len(reqs) > k:
                    idx.append(row)
                    feats.append(reqs[k].features)
                    batch.append(reqs[k])
            x = torch.zeros(self.capacity, self.cfg.num_features, dtype=self.P.dtype)
            x[idx] = torch.as_tensor(np.asarray(feats), dtype=self.P.dtype)
            mask = torch.zeros(self.capacity, dtype=torch.bool)
            mask[idx] = True
            out, self.state = om.forward(self.P, self.cfg, x.to(self.device), self.state,
                                         mask.to(self.device))
            out = out.to(torch.float64).cpu()
            for r, row in zip(batch, idx):
                ids.append(r.unique_id)
                preds.append(out[row].tolist())
        return ids, preds


def response_order(item_slots, item_lens):
    """The answer order of process_batch without the model
    (example_model.py:826-839, :881-899): items are the batch's symbols in
    dict order (slot None or -1: no row), their requests numbered item by
    item. Returns the request index at each response position."""
    base = np.concatenate([[0], np.cumsum(item_lens)]).astype(np.int64)
    order, items = [], []
    for i, (slot, n) in enumerate(zip(item_slots, item_lens)):
        if n == 0:
            continue
        if slot is None or slot < 0:
            order.extend(range(base[i], base[i] + n))
            continue
        items.append(i)
    if not items:
        return order
    for k in range(max(item_lens[i] for i in items)):
        for i in items:
            if item_lens[i] > k:
                order.append(base[i] + k)
    return order
