"""Host-side tick packing (hk_pack_tick, through hackathon_amd.engine.pack_tick)
against the oracle's answer order, which is pinned here against the oracle's
literal process_batch (example_model.py:819-905). Integer work: bit-exact.
No GPU: hk_pack_tick touches host memory only."""

import numpy as np
import pytest

from hackathon_amd import _lib, spec, weights
from hackathon_amd.engine import pack_tick
from oracle import model as om
from oracle.client import OracleClient, response_order


class Req:
    def __init__(self, uid, feats):
        self.unique_id, self.features = uid, feats


def _random_items(rng, n_items, max_len, p_unslotted):
    lens = rng.integers(0, max_len + 1, size=n_items)
    slots = rng.permutation(4 * n_items + 1)[:n_items].astype(np.int32)
    slots[rng.random(n_items) < p_unslotted] = -1
    return slots, lens


def test_oracle_order_matches_literal_process_batch():
    """response_order against the ids OracleClient.process_batch answers with
    (capacity 5: later symbols overflow and are answered with zeros)."""
    cfg = spec.SMALL
    P = om.Params(weights.generate(cfg, 0))
    rng = np.random.default_rng(3)
    client = OracleClient(P, cfg, 5)
    for trial in range(3):
        lens = rng.integers(0, 4, size=7)
        batch, uid = {}, 0
        for i, n in enumerate(lens):
            batch[f"s{trial}_{i}" if trial else f"s{i}"] = [
                Req(uid + k, rng.standard_normal(cfg.num_features).tolist()) for k in range(n)]
            uid += n
        slots = [client._row_for(s) if batch[s] else -1 for s in batch]
        ids, _ = client.process_batch(batch)
        assert ids == response_order(slots, list(lens))


@pytest.mark.parametrize("seed", range(6))
def test_pack_tick_matches_oracle_order_and_invariants(seed):
    rng = np.random.default_rng(seed)
    n_items = [0, 1, 5, 40, 200, 1000][seed]
    slots, lens = _random_items(rng, n_items, [1, 3, 6, 12, 30, 3][seed], 0.2)
    runs, req_row, resp_req = pack_tick(slots, lens)
    assert resp_req.tolist() == response_order(slots.tolist(), lens.tolist())
    live = [i for i in range(n_items) if slots[i] >= 0 and lens[i] > 0]
    # runs: the slotted items with requests, by non-increasing length, stable
    want = sorted(live, key=lambda i: -lens[i])
    assert runs.slot_ids.tolist() == [int(slots[i]) for i in want]
    assert runs.run_off.tolist() == np.concatenate([[0], np.cumsum(lens[want])]).tolist()
    base = np.concatenate([[0], np.cumsum(lens)])
    for pos, i in enumerate(want):
        assert req_row[base[i]:base[i + 1]].tolist() == list(
            range(runs.run_off[pos], runs.run_off[pos + 1]))
    for i in range(n_items):
        if slots[i] < 0:
            assert (req_row[base[i]:base[i + 1]] == -1).all()
    rows = np.sort(req_row[req_row >= 0])
    assert rows.tolist() == list(range(runs.n_rows))


def test_pack_tick_single_hot_symbol_and_all_unslotted():
    runs, req_row, resp_req = pack_tick([7, 3], [256, 1])
    assert runs.slot_ids.tolist() == [7, 3] and runs.run_off.tolist() == [0, 256, 257]
    assert resp_req.tolist() == [0, 256] + list(range(1, 256))
    runs, req_row, resp_req = pack_tick([-1, -1], [2, 1])
    assert runs.n_rows == 0 and req_row.tolist() == [-1, -1, -1]
    assert resp_req.tolist() == [0, 1, 2]
    runs, req_row, resp_req = pack_tick([], [])
    assert runs.n_rows == 0 and len(resp_req) == 0


def test_pack_tick_refuses_bad_items():
    with pytest.raises(_lib.HipLibraryError, match="two items"):
        pack_tick([4, 4], [1, 2])
    with pytest.raises(_lib.HipLibraryError, match="len"):
        pack_tick([0, 1], [1, -2])
    with pytest.raises(ValueError):
        pack_tick([0, 1], [1])
