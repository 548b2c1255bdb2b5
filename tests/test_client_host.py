"""NnInferenceClient's host logic without a GPU: slot assignment, the
round-major chunking of batches larger than a tick, and the response order
(example_model.py:724-767, :819-905), with the engine tick replaced by a
stand-in that checks each tick's packing and answers request j with its own
first four features. Expected: the oracle's answer order (pinned against the
oracle's literal process_batch in test_pack_tick.py), zeros for symbols past
capacity, each symbol's requests in order within every tick."""

from types import SimpleNamespace

import numpy as np
import pytest

from hackathon_amd.client import NnInferenceClient, PendingRequest
from oracle.client import response_order


def _client(capacity, max_rows, F=6):
    c = NnInferenceClient.__new__(NnInferenceClient)
    c.engine = SimpleNamespace(max_rows=max_rows)
    c.capacity = capacity
    c.symbol_to_idx = {}
    c.num_outputs = 4
    c.num_features = F
    c.ticks = []

    def fake_tick(runs, rows, feats):
        n = runs.n_rows
        assert n <= max_rows and len(rows) == n == len(feats)
        assert sorted(rows.tolist()) == list(range(n))
        lens = np.diff(runs.run_off)
        assert np.all(lens >= 1) and np.all(np.diff(lens) <= 0)      # sorted runs
        assert len(set(runs.slot_ids.tolist())) == len(runs.slot_ids)  # distinct slots
        by_row = np.empty_like(feats)
        by_row[rows] = feats
        c.ticks.append((runs, by_row))
        return feats[:, :4].astype(np.float64)

    c._tick_rows = fake_tick
    return c


@pytest.mark.parametrize("max_rows", [64, 7, 3, 2])
def test_process_arrays_order_chunks_and_overflow(max_rows):
    rng = np.random.default_rng(max_rows)
    capacity = 5
    client = _client(capacity, max_rows=max_rows)  # 2: a round may span several ticks
    seen = []
    for batch in range(4):
        names = [f"S{i}" for i in rng.permutation(8)[:6]]
        counts = rng.integers(0, 9, size=len(names))
        n = int(counts.sum())
        feats = rng.standard_normal((n, 6)).astype(np.float32)
        feats[:, 0] = np.arange(n)  # request id in column 0
        for s, c in zip(names, counts):
            if c and s not in seen:
                seen.append(s)
        order, preds = client.process_arrays(names, counts, feats)
        slots = [client.symbol_to_idx.get(s, -1) if c else -1 for s, c in zip(names, counts)]
        assert list(client.symbol_to_idx) == seen[:capacity]
        assert order.tolist() == list(response_order(slots, counts.tolist()))
        want = np.zeros((n, 4))
        base = np.concatenate([[0], np.cumsum(counts)])
        for i, sl in enumerate(slots):
            if sl >= 0:
                want[base[i]:base[i + 1]] = feats[base[i]:base[i + 1], :4]
        assert np.array_equal(preds, want[order])
    # every tick's runs hold a symbol's requests in order (ids in column 0)
    for runs, feats in client.ticks:
        for r in range(len(runs.slot_ids)):
            ids = feats[runs.run_off[r]:runs.run_off[r + 1], 0]
            assert np.all(np.diff(ids) == 1)


def test_process_batch_response_shape():
    client = _client(capacity=2, max_rows=4, F=3)
    reqs = {"A": [PendingRequest(10 + k, "A", [k, 0.5, 1.0]) for k in range(5)],
            "B": [PendingRequest(20, "B", [7.0, 0.0, 0.0])],
            "C": [PendingRequest(30, "C", [9.0, 9.0, 9.0])],   # past capacity: zeros
            "D": []}
    client.num_outputs = 4
    client.num_features = 3

    def tick(runs, rows, feats):
        return np.concatenate([feats, np.ones((len(feats), 1))], axis=1).astype(np.float64)

    client._tick_rows = tick
    resp = client.process_batch(reqs)
    assert resp.unique_ids == [30, 10, 20, 11, 12, 13, 14]
    assert resp.predictions[0] == [0.0] * 4
    assert resp.predictions[1] == [0.0, 0.5, 1.0, 1.0]
    assert resp.predictions[2] == [7.0, 0.0, 0.0, 1.0]
    assert client.process_batch({}).unique_ids == []
    assert client.process_batch({"E": []}).unique_ids == []


def test_round_chunks_cover_rounds_within_max_rows():
    rng = np.random.default_rng(0)
    for max_rows in (4, 9, 33):
        client = _client(capacity=64, max_rows=max_rows)
        for _ in range(20):
            counts = rng.integers(1, 12, size=rng.integers(1, 3 * max_rows))
            chunks = client._round_chunks(counts)
            # every (request round, symbol) pair exactly once, rounds in order
            seen = []
            for k0, k1, part in chunks:
                idx = np.arange(len(counts)) if part is None else part
                c = np.clip(counts[idx] - k0, 0, k1 - k0)
                assert 0 < int(c.sum()) <= max_rows
                seen.extend((k, int(i)) for i, ci in zip(idx, c) for k in range(k0, k0 + ci))
            want = [(k, i) for i in range(len(counts)) for k in range(counts[i])]
            assert sorted(seen) == sorted(want) and len(seen) == len(want)
            starts = [k0 for k0, _, _ in chunks]
            assert starts == sorted(starts)


def test_feature_rows_matches_numpy():
    """process_batch's feature conversion (flat list through array.array)
    against numpy's on every form a request's features may take; ragged or
    non-numeric rows still raise as numpy does."""
    from hackathon_amd.client import _feature_rows

    rng = np.random.default_rng(5)
    rows = [rng.standard_normal(6).tolist() for _ in range(5)]
    forms = [
        rows,                                               # lists of Python floats
        [tuple(r) for r in rows],                           # tuples
        [np.asarray(r, dtype=np.float64) for r in rows],    # float64 arrays
        [np.asarray(r, dtype=np.float32) for r in rows],    # float32 arrays
        [[int(10 * v) for v in r] for r in rows],           # ints
        [[1e-45, 3.4e38, -0.0, float("inf"), float("nan"), 1.0 + 2 ** -30]] * 2,  # rounding edges
    ]
    for f in forms:
        reqs = [PendingRequest(i, "S", r) for i, r in enumerate(f)]
        got = _feature_rows(reqs, 6)
        want = np.asarray([q.features for q in reqs], dtype=np.float32)
        assert got.dtype == np.float32 and got.shape == want.shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        _feature_rows([PendingRequest(0, "S", [1.0, 2.0]), PendingRequest(1, "S", [1.0])], 2)
    # ragged rows whose lengths add up to the full count are still ragged
    with pytest.raises(ValueError):
        _feature_rows([PendingRequest(0, "S", [1.0, 2.0, 3.0]), PendingRequest(1, "S", [1.0])], 2)
    with pytest.raises(ValueError):
        _feature_rows([PendingRequest(0, "S", ["a", "b"])], 2)
