"""The wire loop end to end on the GPU: StreamClient around NnInferenceClient
on the HIP engine (small dims, fp32), served over loopback TCP by a test
server that speaks the reference's protocol (protocol.py:14-103), checked
against the oracle's literal client (OracleClient: process_batch with the
reference's rounds, example_model.py:769-905).

The server streams request messages over 10 symbols into a client of 8
slots (the last two symbols to arrive get none and are answered with
zeros). The client batches whatever has queued (client.py:239-260); which
requests share a batch depends on timing, so each response is taken as the
batch it answers: its requests, grouped by symbol in the client's
first-seen order, are fed to OracleClient.process_batch in the order the
responses arrive, and the oracle's answer order must equal the response's
and its predictions must agree at the fp32 bar (|d| <= 1e-6 + 1e-5 |ref|).
A message of 150 requests for one symbol, sent when its queue is empty,
fills the queue (100) and drops the other 50 (client.py:202-220): those are
never answered and never advance the symbol's state.
"""

import socket
import time

import numpy as np
import pytest
import torch

from hackathon_amd import spec, weights
from hackathon_amd.client import InferenceResponse, NnInferenceClient, PendingRequest
from hackathon_amd.serving import InferenceRequest, LineSocket, RegisterMessage, StreamClient, decode
from oracle import model as om
from oracle.client import OracleClient

pytestmark = pytest.mark.gpu

CAP = 8
SYMBOLS = [f"SYM_{i:03d}" for i in range(10)]


def test_stream_client_engine_vs_oracle(dev):
    from hackathon_amd.engine import Engine

    cfg = spec.SMALL
    params = weights.generate(cfg, 0)
    eng = Engine(cfg, capacity=CAP, max_rows=64, linear_dtype="fp32", device=dev)
    eng.load_weights(params)
    model = NnInferenceClient(CAP, engine=eng, config=cfg)
    oracle = OracleClient(om.Params(params), cfg, CAP)

    srv = socket.socket(socket.AF_INET, socket.SOCK_STREAM)
    srv.bind(("127.0.0.1", 0))
    srv.listen(1)
    client = StreamClient(model, "127.0.0.1", srv.getsockname()[1], max_queue_size=100,
                          heartbeat_s=60.0)
    assert client.start()
    sock, _ = srv.accept()
    conn = LineSocket(sock)

    rng = np.random.default_rng(5)
    sent = {}        # uid -> (symbol, features)
    first_seen = []  # the client's queue order
    uid = 0

    def send(symbols):
        nonlocal uid
        feats = np.clip(rng.standard_normal((len(symbols), cfg.num_features)), -5, 5)
        feats = feats.astype(np.float32).astype(np.float64)
        ids = list(range(uid, uid + len(symbols)))
        for i, s in zip(ids, symbols):
            sent[i] = (s, feats[ids.index(i)].tolist())
            if s not in first_seen:
                first_seen.append(s)
        uid += len(symbols)
        assert conn.send(InferenceRequest(ids, list(symbols), feats.tolist(), time.time()))
        return ids

    answered = {}
    n_batches = 0
    sizes = []

    def drain(want_ids, timeout=60.0):
        """Read responses until every id in want_ids is answered; check each
        response against the oracle as it arrives."""
        nonlocal n_batches
        t0 = time.time()
        while not set(want_ids) <= set(answered):
            assert time.time() - t0 < timeout, f"unanswered: {sorted(set(want_ids) - set(answered))[:8]}"
            lines = conn.read_lines()
            assert lines is not None, "the client closed the connection"
            for line in lines:
                msg = decode(line)
                if isinstance(msg, RegisterMessage):
                    continue
                if not isinstance(msg, InferenceResponse):
                    continue
                n_batches += 1
                by_sym = {}
                for i in sorted(msg.unique_ids):
                    s, f = sent[i]
                    by_sym.setdefault(s, []).append(PendingRequest(i, s, f))
                reqs = {s: by_sym[s] for s in first_seen if s in by_sym}
                ids, preds = oracle.process_batch(reqs)
                assert msg.unique_ids == ids, "answer order differs from the reference's rounds"
                got, want = np.asarray(msg.predictions), np.asarray(preds)
                bad = np.abs(got - want) - (1e-6 + 1e-5 * np.abs(want))
                assert bad.max() <= 0, f"batch {n_batches}: max |d| {np.abs(got - want).max():.3e}"
                for i, p in zip(msg.unique_ids, msg.predictions):
                    assert i not in answered, f"request {i} answered twice"
                    answered[i] = p
                sizes.append(len(msg.unique_ids))

    try:
        # every symbol once, in order: slots for the first 8, none for the rest
        drain(send(SYMBOLS))
        # bursts of random requests, sent without waiting
        ids = []
        for _ in range(30):
            n = int(rng.integers(1, 25))
            ids += send([SYMBOLS[j] for j in rng.integers(0, len(SYMBOLS), size=n)])
        drain(ids)
        # 150 requests for one symbol whose queue is empty: 50 dropped
        burst = send([SYMBOLS[2]] * 150)
        drain(burst[:100])
        more = send([SYMBOLS[0], SYMBOLS[9], SYMBOLS[2]])
        drain(more)
        time.sleep(0.5)
        for _ in conn.read_lines() or []:
            raise AssertionError("an answer beyond the kept requests")
        assert client.dropped == 50
        assert not set(burst[100:]) & set(answered)
        assert set(answered) == set(sent) - set(burst[100:])
        # symbols past the capacity are answered with zeros
        for i, p in answered.items():
            if sent[i][0] in SYMBOLS[CAP:]:
                assert p == [0.0] * 4
        assert model.symbol_to_idx == oracle.symbol_to_idx
        print(f"wire loop: {len(answered)} answers in {n_batches} responses "
              f"(sizes {sizes[:12]}...), 50 dropped")
        eng.check()
    finally:
        client.stop()
        sock.close()
        srv.close()
        eng.close()
    torch.cuda.synchronize()
