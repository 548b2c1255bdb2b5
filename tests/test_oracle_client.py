"""Pin the oracle's process_batch restatement (oracle/client.py) on the CPU by
what the reference's semantics fix, without retyping its round loop:

- rows never mix and a symbol's requests apply in list order
  (example_model.py:773-781, :422-427): the predictions of a multi-symbol
  batch equal those of each symbol's requests applied one at a time through
  the model with only that symbol's row active;
- response order is round-major in first-seen symbol order, after the
  overflow answers (example_model.py:819-839, :881-899);
- past capacity a symbol is answered with zeros and stages nothing
  (example_model.py:830-839): the other rows' state is unchanged by it;
- empty request lists are skipped and an empty batch answers nothing.
"""

import numpy as np
import torch

from hackathon_amd import spec, weights
from oracle import model as om
from oracle.client import OracleClient


class Req:
    def __init__(self, uid, symbol, feats):
        self.unique_id, self.symbol, self.features = uid, symbol, feats


CFG = spec.SMALL


def _params():
    return om.Params(weights.generate(CFG, 0))


def _batch(rng, counts, uid0=0):
    out, uid = {}, uid0
    for sym, n in counts.items():
        out[sym] = []
        for _ in range(n):
            out[sym].append(Req(uid, sym, rng.standard_normal(CFG.num_features).astype(np.float32).tolist()))
            uid += 1
    return out


def test_rounds_equal_per_symbol_sequences():
    P = _params()
    rng = np.random.default_rng(0)
    counts = {"A": 3, "B": 1, "C": 2, "D": 0}
    reqs = _batch(rng, counts)
    client = OracleClient(P, CFG, 4)
    ids, preds = client.process_batch(reqs)
    got = dict(zip(ids, preds))

    # Each symbol alone, request by request, only its row active.
    state = om.init_state(CFG, 4)
    rows = {"A": 0, "B": 1, "C": 2}
    want = {}
    with torch.inference_mode():
        for sym in ("C", "A", "B"):  # any symbol order: rows never mix
            for r in reqs[sym]:
                x = torch.zeros(4, CFG.num_features)
                x[rows[sym]] = torch.tensor(r.features)
                mask = torch.zeros(4, dtype=torch.bool)
                mask[rows[sym]] = True
                out, state = om.forward(P, CFG, x, state, mask)
                want[r.unique_id] = out[rows[sym]].double().tolist()
    assert sorted(got) == sorted(want)
    for uid in want:
        np.testing.assert_allclose(got[uid], want[uid], rtol=2e-6, atol=1e-7)
    for a, b in zip(om.flatten(client.state), om.flatten(state)):
        torch.testing.assert_close(a, b, rtol=2e-6, atol=1e-7, equal_nan=True)


def test_response_order_and_overflow():
    P = _params()
    rng = np.random.default_rng(1)
    reqs = _batch(rng, {"A": 2, "B": 1, "C": 2, "E": 0})
    client = OracleClient(P, CFG, 2)  # C has no row
    ids, preds = client.process_batch(reqs)
    a, b, c = ([r.unique_id for r in reqs[s]] for s in "ABC")
    # overflow answers first, then round 0 (A, B), then round 1 (A)
    assert ids == c + [a[0], b[0], a[1]]
    assert preds[0] == [0.0] * 4 and preds[1] == [0.0] * 4
    assert client.symbol_to_idx == {"A": 0, "B": 1}

    # The overflow symbol staged nothing: the same batch without it leaves
    # the same state and predictions.
    ref = OracleClient(P, CFG, 2)
    ids2, preds2 = ref.process_batch({k: v for k, v in reqs.items() if k != "C"})
    assert ids2 == ids[2:] and preds2 == preds[2:]
    for x, y in zip(om.flatten(client.state), om.flatten(ref.state)):
        assert torch.equal(x, y) or torch.equal(torch.nan_to_num(x), torch.nan_to_num(y))


def test_empty_batches():
    client = OracleClient(_params(), CFG, 2)
    assert client.process_batch({}) == ([], [])
    assert client.process_batch({"A": []}) == ([], [])
    assert client.symbol_to_idx == {}
