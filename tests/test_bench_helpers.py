"""bench.py's host replays of the write-back log rule (no GPU).

The steady-state window of the C4 benchmark starts from the log occupancy
that log_occupancy() computes for 10,000 ticks, and matrix_scan_bytes()
gives the matrix scans' algorithmic bytes the tick roofline uses. Both
restate the scan kernel's rule: a run of len steps on a slot whose log holds
n entries appends its steps when n + len <= 8, else writes the tile back and
empties the log. Checked on hand-worked sequences."""

import numpy as np

import bench


def _tick(*pairs):
    syms = np.array([s for s, _ in pairs], np.int32)
    counts = np.array([c for _, c in pairs], np.int64)
    return syms, counts


def test_log_occupancy_hand_sequence():
    ticks = [
        _tick((0, 3), (1, 8)),   # 0: 3      1: 8 (fits exactly)
        _tick((0, 4), (1, 1)),   # 0: 7      1: 9 > 8 -> written back, 0
        _tick((0, 2), (2, 9)),   # 0: 9 > 8 -> 0   2: 9 > 8 on an empty log -> 0
        _tick((0, 8), (1, 5)),   # 0: 8      1: 5
        _tick((0, 1),),          # 0: 9 > 8 -> 0
    ]
    assert bench.log_occupancy(ticks) == {0: 0, 1: 5, 2: 0}
    assert bench.log_occupancy(ticks[:2]) == {0: 7, 1: 0}
    # resuming from an occupancy continues the same rule
    assert bench.log_occupancy(ticks[2:], bench.log_occupancy(ticks[:2])) == {0: 0, 1: 5, 2: 0}


def test_matrix_scan_bytes_hand_sequence():
    T, E, R = 1000.0, 10.0, 1.0  # tile, log entry, request row bytes
    ticks = [
        _tick((0, 3), (1, 8)),
        _tick((0, 4), (1, 1)),
        _tick((0, 2),),
    ]
    # tick 0: sym 0 n=0 defer: T + 0 + 3E; sym 1 n=0 defer: T + 8E; rows 11
    # tick 1: sym 0 n=3 defer: T + 3E + 4E; sym 1 n=8, 8+1 > 8: T + 8E + T; rows 5
    # tick 2: sym 0 n=7, 7+2 > 8: T + 7E + T; rows 2
    t0 = (T + 3 * E) + (T + 8 * E) + 11 * R
    t1 = (T + 7 * E) + (T + 8 * E + T) + 5 * R
    t2 = (T + 7 * E + T) + 2 * R
    assert bench.matrix_scan_bytes(ticks, 0, 1, T, E, R) == t0 + t1 + t2
    assert bench.matrix_scan_bytes(ticks, 1, 3, T, E, R) == 3 * (t1 + t2)
    # starting occupancy: symbol 0 already holds 6 entries -> 6+3 > 8 writes back
    got = bench.matrix_scan_bytes(ticks[:1], 0, 1, T, E, R, n_log0={0: 6})
    assert got == (T + 6 * E + T) + (T + 8 * E) + 11 * R


def test_log_occupancy_is_bounded_on_zipf_ticks():
    ticks = bench.zipf_ticks(200, 64, 32, 1.1, seed=3)
    occ = bench.log_occupancy(ticks)
    assert all(0 <= n <= bench.LOG_CAP for n in occ.values())
    # every symbol that ever had a request has an entry
    seen = set(int(s) for syms, _ in ticks for s in syms)
    assert set(occ) == seen


def test_xlstm_split_point_hand_cases():
    """The replica of the engine's xLSTM group split (bench.xlstm_split_point):
    per group 3 us per sLSTM step of its longest run plus 5 us per symbol, a
    split charged one more read of a layer's weights."""
    one_each = lambda n: np.arange(n + 1)  # n runs of one request
    # four one-request symbols: 3 + 20 = 23 unsplit; two and two cost 13
    assert bench.xlstm_split_point(one_each(4)) == 2
    # ... plus a second fp32 weight read (41 us): 54 > 0.8 * 23, no split
    assert bench.xlstm_split_point(one_each(4), 40.5) == 4
    # 64 one-request symbols: 323 unsplit, 163 + 24 split at 32 < 258.4
    assert bench.xlstm_split_point(one_each(64), 23.7) == 32
    # a 40-request run and 100 single ones: max(120 + 5k, 3 + 5(101 - k))
    # is least at k = 39 (315 against 318 at k = 38 and 320 at k = 40)
    run_off = np.concatenate([[0], np.cumsum([40] + [1] * 100)])
    assert bench.xlstm_split_point(run_off, 23.7) == 39
    assert bench.xlstm_split_point(np.array([0, 5])) == 1  # a single run
