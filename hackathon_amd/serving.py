"""The reference's wire protocol (protocol.py:14-103) and client loop
(client.py:41-260) around this build's client.

Protocol: newline-delimited JSON, one message per line, the message's
fields in declaration order with `message_type` last (dataclasses.asdict
order, json.dumps default separators), so an encoded message is
byte-for-byte what the reference writes. `decode` returns an `ErrorMessage`
for a line it cannot decode or an unknown message type, as the reference
does.

Client loop (`StreamClient`): the reference's behaviour
- registers on connect; answers each batch of pending requests with one
  InferenceResponse (process_batch over {symbol: requests});
- per-symbol request queues bounded at `max_queue_size` (100), a request
  arriving at a full queue is dropped with a message (client.py:202-220);
- a batch takes every queued request of every symbol, symbols in the order
  the client first saw them (client.py:239-260);
- a Heartbeat every 5 s; score updates ignored; server errors printed.
What is built differently, for rate:
- requests are decoded straight into arrays (ids, symbol names, a
  float32 feature matrix per message) and handed to
  `NnInferenceClient.process_arrays`, with no per-request Python objects;
- neither thread polls: the receive thread blocks on the socket and wakes
  the processing thread through a condition variable, where the reference
  sleeps 1 ms between polls in both loops (client.py:149, :193).
"""

from __future__ import annotations

import json
import socket
import threading
import time
from collections import OrderedDict
from dataclasses import dataclass, fields
from typing import List, Optional

import numpy as np

from .client import InferenceResponse

REGISTER = "register"
INFERENCE_REQUEST = "inference_request"
INFERENCE_RESPONSE = "inference_response"
SCORE_UPDATE = "score_update"
HEARTBEAT = "heartbeat"
ERROR = "error"


@dataclass
class RegisterMessage:
    message_type: str = REGISTER


@dataclass
class InferenceRequest:
    unique_ids: list
    symbols: list
    features: list
    timestamp: float
    message_type: str = INFERENCE_REQUEST


@dataclass
class ScoreUpdate:
    unique_ids: list
    trade_pnls: list
    accuracies: list
    latencies_ms: list
    message_type: str = SCORE_UPDATE


@dataclass
class Heartbeat:
    timestamp: float
    message_type: str = HEARTBEAT


@dataclass
class ErrorMessage:
    error: str
    details: Optional[str] = None
    message_type: str = ERROR


MESSAGE_CLASSES = {
    REGISTER: RegisterMessage,
    INFERENCE_REQUEST: InferenceRequest,
    INFERENCE_RESPONSE: InferenceResponse,
    SCORE_UPDATE: ScoreUpdate,
    HEARTBEAT: Heartbeat,
    ERROR: ErrorMessage,
}


def encode(message) -> bytes:
    """One protocol line: the message's fields in declaration order."""
    return (json.dumps({f.name: getattr(message, f.name) for f in fields(message)}) + "\n").encode()


def decode(line: bytes):
    """The message object of one line, or an ErrorMessage saying why not."""
    try:
        d = json.loads(line.decode("utf-8").strip())
        kind = d.get("message_type")
        if kind not in MESSAGE_CLASSES:
            raise ValueError(f"Unknown message type: {kind}")
        d.pop("message_type", None)
        msg = MESSAGE_CLASSES[kind](**d)
        msg.message_type = kind
        return msg
    except Exception as exc:  # the reference answers any failure the same way
        return ErrorMessage(error=str(exc))


class LineSocket:
    """Newline-delimited messages over a connected socket: blocking reads
    with a timeout (so a reader can notice a stop flag), whole-line writes
    under a lock (two threads send)."""

    def __init__(self, sock: socket.socket, timeout: float = 0.2):
        self.sock = sock
        self.sock.settimeout(timeout)
        self.buf = b""
        self.lock = threading.Lock()

    def read_lines(self) -> Optional[List[bytes]]:
        """The complete lines received so far (waiting up to the timeout for
        some); [] on a timeout, None once the peer has closed."""
        try:
            data = self.sock.recv(1 << 20)
        except socket.timeout:
            return []
        except OSError:
            return None
        if not data:
            return None
        self.buf += data
        if b"\n" not in self.buf:
            return []
        *lines, self.buf = self.buf.split(b"\n")
        return [ln for ln in lines if ln]

    def send(self, message) -> bool:
        data = encode(message)
        try:
            with self.lock:
                self.sock.sendall(data)
            return True
        except OSError:
            return False


class _SymbolQueue:
    __slots__ = ("ids", "rows")

    def __init__(self):
        self.ids: list = []
        self.rows: list = []


class StreamClient:
    """Runs `client` (anything with process_arrays(symbols, counts,
    features) -> (order, predictions)) against an inference server."""

    def __init__(self, client, server_host: str = "localhost", server_port: int = 8080,
                 max_queue_size: int = 100, heartbeat_s: float = 5.0):
        self.client = client
        self.server_host, self.server_port = server_host, server_port
        self.max_queue_size = max_queue_size
        self.heartbeat_s = heartbeat_s
        self.conn: Optional[LineSocket] = None
        self.queues: "OrderedDict[str, _SymbolQueue]" = OrderedDict()  # first-seen order
        self.cv = threading.Condition()
        self.running = False
        self.threads: list = []
        self.dropped = 0
        self.answered = 0
        self.on_score = None  # optional callback for ScoreUpdate messages

    # -- connection -------------------------------------------------------------
    def connect(self) -> bool:
        try:
            sock = socket.create_connection((self.server_host, self.server_port))
        except OSError as exc:
            print(f"Connection failed: {exc}")
            return False
        sock.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)
        self.conn = LineSocket(sock)
        if not self.conn.send(RegisterMessage()):
            print("Failed to send registration")
            return False
        print(f"Connected to {self.server_host}:{self.server_port}")
        return True

    def start(self) -> bool:
        if not self.connect():
            return False
        self.running = True
        self.threads = [threading.Thread(target=self._receive_loop, daemon=True),
                        threading.Thread(target=self._process_loop, daemon=True)]
        for t in self.threads:
            t.start()
        return True

    def run(self):
        """client.py:262-284: run until interrupted or the server closes."""
        if not self.start():
            return
        print("Client running. Press Ctrl+C to stop.")
        try:
            while self.running:
                time.sleep(0.5)
        except KeyboardInterrupt:
            print("\nShutting down...")
        finally:
            self.stop()

    def stop(self):
        self.running = False
        with self.cv:
            self.cv.notify_all()
        for t in self.threads:
            if t is not threading.current_thread():
                t.join(timeout=2)
        if self.conn is not None:
            try:
                self.conn.sock.close()
            except OSError:
                pass

    # -- receive ------------------------------------------------------------------
    def _receive_loop(self):
        last_beat = time.monotonic()
        while self.running:
            lines = self.conn.read_lines()
            if lines is None:  # the server closed the connection
                self.running = False
                with self.cv:
                    self.cv.notify_all()
                break
            for line in lines:
                msg = decode(line)
                if isinstance(msg, InferenceRequest):
                    try:
                        self._enqueue(msg)
                    except Exception as exc:  # a malformed request is logged, not fatal
                        print(f"Receive error: {exc}")
                elif isinstance(msg, ScoreUpdate):
                    if self.on_score is not None:
                        self.on_score(msg)
                elif isinstance(msg, ErrorMessage):
                    print(f"Server error: {msg.error}")
            now = time.monotonic()
            if now - last_beat >= self.heartbeat_s:
                self.conn.send(Heartbeat(timestamp=time.time()))
                last_beat = now

    def _enqueue(self, req: InferenceRequest):
        feats = np.asarray(req.features, dtype=np.float32)
        with self.cv:
            for i, (uid, sym) in enumerate(zip(req.unique_ids, req.symbols)):
                q = self.queues.get(sym)
                if q is None:
                    q = self.queues[sym] = _SymbolQueue()
                if len(q.ids) >= self.max_queue_size:
                    print(f"Queue full for symbol {sym}, dropping request")
                    self.dropped += 1
                    continue
                q.ids.append(uid)
                q.rows.append(feats[i])
            self.cv.notify()

    # -- process ------------------------------------------------------------------
    def _gather(self):
        """Every queued request, symbols in first-seen order (waits for some)."""
        with self.cv:
            while self.running and not any(q.ids for q in self.queues.values()):
                self.cv.wait(timeout=0.5)
            symbols, counts, ids, rows = [], [], [], []
            for sym, q in self.queues.items():
                if q.ids:
                    symbols.append(sym)
                    counts.append(len(q.ids))
                    ids.extend(q.ids)
                    rows.extend(q.rows)
                    q.ids, q.rows = [], []
        return symbols, counts, ids, rows

    def _process_loop(self):
        while self.running:
            symbols, counts, ids, rows = self._gather()
            if not ids:
                continue
            try:
                order, preds = self.client.process_arrays(symbols, counts, np.stack(rows))
                resp = InferenceResponse([ids[j] for j in order], preds.tolist(), time.time())
                if not self.conn.send(resp):
                    print(f"Failed to send response for {len(ids)} requests")
                self.answered += len(ids)
            except Exception as exc:  # the reference logs and goes on (client.py:195-200)
                print(f"Process error: {exc}")
                time.sleep(0.1)
