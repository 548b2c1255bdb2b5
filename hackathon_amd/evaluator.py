"""The reference's local evaluator (local_evaluator.py:19-112) over this
build's client.

`LocalEvaluator(requests_file)` reads a requests parquet (feature_00 ..
feature_78, target_00 .. target_03, symbol) and sizes the symbol capacity
as the reference does: one more than the largest numeric suffix of the
symbol names (local_evaluator.py:20-23).

`evaluate_model(process_batch_fn, batch_size)` replays the requests in file
order in batches of `batch_size` consecutive rows, each grouped by symbol in
order of first appearance within the batch, timing each process_batch call
(local_evaluator.py:25-62); every response of a batch is charged that
batch's wall time. `evaluate_arrays(client, batch_size)` does the same
through `NnInferenceClient.process_arrays` (flat arrays, no per-request
objects).

`calculate_metrics` is the reference's metric (local_evaluator.py:64-101):
total requests and responses, response rate, mean latency (ms), and per
tower the max and mean absolute error against the targets of the requests
that were answered.
"""

from __future__ import annotations

import time
from collections import defaultdict

import numpy as np

from .client import PendingRequest

TOWER_NAMES = ("XLSTM", "Mamba2", "RetNet", "Hawk")


def calculate_metrics(targets: np.ndarray, predictions: dict, latencies: dict,
                      ids=None) -> dict:
    """targets [n, 4], row r the targets of request ids[r] (ids: the
    requests' unique ids in file order, the parquet's index labels; default
    0 .. n-1); predictions and latencies keyed by request id
    (local_evaluator.py:64-101)."""
    tower_err = defaultdict(list)
    lat = []
    for r, uid in enumerate(range(len(targets)) if ids is None else ids):
        if uid not in predictions:
            continue
        pred = predictions[uid]
        if len(pred) != targets.shape[1]:
            raise ValueError(f"request {uid}: {len(pred)} predictions for {targets.shape[1]} targets")
        for t, (p, y) in enumerate(zip(pred, targets[r])):
            tower_err[t].append(abs(float(p) - float(y)))
        lat.append(latencies[uid])
    out = {
        "total_requests": len(targets),
        "total_responses": len(predictions),
        "response_rate": len(predictions) / len(targets),
        "avg_latency_ms": float(np.mean(lat)) if lat else 0,
    }
    for t, errs in tower_err.items():
        out[f"tower_{t}"] = (max(errs), float(np.mean(errs)))
    return out


class LocalEvaluator:
    def __init__(self, requests_file):
        import pandas as pd

        self.requests_df = pd.read_parquet(requests_file)
        names = self.requests_df["symbol"].unique()
        self.num_symbols = max(int(s[-3:]) for s in names) + 1
        df = self.requests_df
        self.feature_cols = [c for c in df.columns if c.startswith("feature")]
        self.target_cols = [c for c in df.columns if c.startswith("target")]
        self.features = df[self.feature_cols].to_numpy(dtype=np.float32)
        self.targets = df[self.target_cols].to_numpy(dtype=np.float64)
        self.symbols = df["symbol"].tolist()
        # request ids: the index labels, as the reference's iterrows() gives
        # them (local_evaluator.py:26-35)
        self.ids = df.index.tolist()

    def _batches(self, batch_size):
        n = len(self.symbols)
        for i in range(0, n, batch_size):
            yield range(i, min(i + batch_size, n))

    def evaluate_model(self, process_batch_fn, batch_size: int) -> dict:
        predictions, latencies = {}, {}
        for rows in self._batches(batch_size):
            batch_by_symbol = {}
            for r in rows:
                req = PendingRequest(unique_id=self.ids[r], symbol=self.symbols[r],
                                     features=self.features[r].tolist(), received_time=time.time())
                batch_by_symbol.setdefault(req.symbol, []).append(req)
            t0 = time.perf_counter()
            resp = process_batch_fn(batch_by_symbol)
            ms = (time.perf_counter() - t0) * 1000
            for uid, pred in zip(resp.unique_ids, resp.predictions):
                predictions[uid] = pred
                latencies[uid] = ms
        return calculate_metrics(self.targets, predictions, latencies, self.ids)

    def evaluate_arrays(self, client, batch_size: int) -> dict:
        """evaluate_model through client.process_arrays: the batch's rows
        grouped by symbol (first appearance order), features as one array."""
        predictions, latencies = {}, {}
        for rows in self._batches(batch_size):
            groups = {}
            for r in rows:
                groups.setdefault(self.symbols[r], []).append(r)
            order = np.asarray([r for g in groups.values() for r in g], dtype=np.int64)
            t0 = time.perf_counter()
            resp, preds = client.process_arrays(list(groups), [len(g) for g in groups.values()],
                                                self.features[order])
            ms = (time.perf_counter() - t0) * 1000
            for j, p in zip(resp, preds):
                uid = self.ids[int(order[j])]
                predictions[uid] = p.tolist()
                latencies[uid] = ms
        return calculate_metrics(self.targets, predictions, latencies, self.ids)

    @staticmethod
    def print_report(metrics: dict):
        print(f"\nTotal requests: {metrics['total_requests']:,}")
        print(f"Total responses: {metrics['total_responses']:,}")
        print(f"Response rate: {metrics['response_rate']:.2%}")
        print(f"Average latency: {metrics['avg_latency_ms']:.1f} ms")
        print("Tower Accuracies:")
        for t, name in enumerate(TOWER_NAMES):
            if f"tower_{t}" in metrics:
                mx, mean = metrics[f"tower_{t}"]
                print(f"{name}: max_error = {mx:.4f}, mean_error = {mean:.4f}")


def main(argv=None) -> int:
    """python -m hackathon_amd.evaluator --requests-parquet-file tiny.parquet
    [--batch-size N] [--weights state_dict.pt] [--linear-dtype fp16]"""
    import argparse

    ap = argparse.ArgumentParser()
    ap.add_argument("--requests-parquet-file", default="tiny.parquet")
    ap.add_argument("--batch-size", type=int, default=1)
    ap.add_argument("--weights", default=None,
                    help="local state_dict file (torch.load weights_only); default: init spec")
    ap.add_argument("--linear-dtype", default=None, help="fp32 / bf16 / fp16 (default: LINEAR_DTYPE or fp16)")
    args = ap.parse_args(argv)
    from .client import NnInferenceClient

    ev = LocalEvaluator(args.requests_parquet_file)
    client = NnInferenceClient(ev.num_symbols, weights_path=args.weights,
                               linear_dtype=args.linear_dtype)
    ev.print_report(ev.evaluate_model(client.process_batch, args.batch_size))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
