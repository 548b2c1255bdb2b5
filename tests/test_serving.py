"""The wire protocol and client loop (hackathon_amd.serving; the reference's
protocol.py and client.py:41-260) on the CPU, over loopback TCP with a
stand-in for the model (no GPU): byte-exact encoding of every message type,
decoding and its error answers, registration, one response per batch with
every request answered once, symbols in first-seen order, per-symbol queues
bounded at 100 with drops, heartbeats."""

import json
import socket
import threading
import time

import numpy as np
import pytest

from hackathon_amd.client import InferenceResponse
from hackathon_amd.serving import (ErrorMessage, Heartbeat, InferenceRequest, LineSocket,
                                   RegisterMessage, ScoreUpdate, StreamClient, decode, encode)


def test_encoding_is_the_reference_wire_format():
    # dataclasses.asdict order + json.dumps defaults, message_type last
    assert encode(RegisterMessage()) == b'{"message_type": "register"}\n'
    assert encode(InferenceResponse([7, 3], [[0.5, -1.0, 2.0, 0.0]], 12.5)) == (
        b'{"unique_ids": [7, 3], "predictions": [[0.5, -1.0, 2.0, 0.0]], '
        b'"client_timestamp": 12.5, "message_type": "inference_response"}\n')
    assert encode(Heartbeat(1.25)) == b'{"timestamp": 1.25, "message_type": "heartbeat"}\n'
    assert encode(ErrorMessage("boom")) == (
        b'{"error": "boom", "details": null, "message_type": "error"}\n')
    req = InferenceRequest([1], ["SYM_001"], [[0.25, 1.0]], 3.0)
    assert encode(req) == (b'{"unique_ids": [1], "symbols": ["SYM_001"], "features": [[0.25, 1.0]], '
                           b'"timestamp": 3.0, "message_type": "inference_request"}\n')
    for msg in (req, ScoreUpdate([1], [0.5], [1.0], [2.0]), Heartbeat(4.0), RegisterMessage()):
        back = decode(encode(msg))
        assert type(back) is type(msg) and back == msg
    assert isinstance(decode(b'{"message_type": "nope"}'), ErrorMessage)
    assert "Unknown message type" in decode(b'{"message_type": "nope"}').error
    assert isinstance(decode(b"not json"), ErrorMessage)


class FakeModel:
    """process_arrays stand-in: request j is answered with its first four
    features; the first call can be held until released."""

    def __init__(self):
        self.calls = []
        self.hold = threading.Event()
        self.hold.set()

    def process_arrays(self, symbols, counts, features):
        self.calls.append((list(symbols), list(counts)))
        self.hold.wait(5)
        order = np.arange(len(features))[::-1]
        return order, features[order, :4].astype(np.float64)


def _server():
    srv = socket.socket(socket.AF_INET, socket.SOCK_STREAM)
    srv.bind(("127.0.0.1", 0))
    srv.listen(1)
    return srv, srv.getsockname()[1]


def _request(uid0, symbols, F=6):
    n = len(symbols)
    feats = [[float(uid0 + i)] + [0.5] * (F - 1) for i in range(n)]
    return InferenceRequest(list(range(uid0, uid0 + n)), list(symbols), feats, time.time())


def _read_until(conn, pred, timeout=10.0):
    out, t0 = [], time.time()
    while time.time() - t0 < timeout:
        for line in conn.read_lines() or []:
            out.append(decode(line))
        if pred(out):
            return out
    raise AssertionError(f"timed out with {out}")


def test_client_loop_over_loopback():
    srv, port = _server()
    model = FakeModel()
    client = StreamClient(model, "127.0.0.1", port, max_queue_size=100, heartbeat_s=0.2)
    assert client.start()
    sock, _ = srv.accept()
    conn = LineSocket(sock)
    first = _read_until(conn, lambda m: len(m) >= 1)
    assert isinstance(first[0], RegisterMessage)

    # one request: answered alone; hold the model so that the next requests
    # queue up behind it
    model.hold.clear()
    conn.send(_request(0, ["A"]))
    t0 = time.time()
    while not model.calls and time.time() - t0 < 5:
        time.sleep(0.01)
    assert model.calls == [(["A"], [1])]
    # 150 requests for B (50 dropped: the queue holds 100), 3 for A after them
    conn.send(_request(1, ["B"] * 150))
    conn.send(_request(151, ["A", "C", "A"]))
    time.sleep(0.3)
    model.hold.set()
    resps = _read_until(conn, lambda m: sum(len(x.unique_ids) for x in m
                                            if isinstance(x, InferenceResponse)) >= 1 + 100 + 3)
    answers = [x for x in resps if isinstance(x, InferenceResponse)]
    got = {uid: p for a in answers for uid, p in zip(a.unique_ids, a.predictions)}
    want_ids = [0] + list(range(1, 101)) + [151, 152, 153]
    assert sorted(got) == want_ids and client.dropped == 50
    for uid in want_ids:
        assert got[uid][0] == float(uid)
    # the second batch lists symbols in first-seen order: A (seen first), B, C
    assert model.calls[1] == (["A", "B", "C"], [2, 100, 1])
    assert any(isinstance(x, Heartbeat) for x in resps) or \
        any(isinstance(x, Heartbeat) for x in _read_until(conn, lambda m: any(
            isinstance(x, Heartbeat) for x in m)))
    sock.close()
    t0 = time.time()
    while client.running and time.time() - t0 < 5:
        time.sleep(0.05)
    assert not client.running  # the server closing ends the loop
    client.stop()
    srv.close()
