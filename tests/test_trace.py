"""The trace ring and its latency report (include/trace.h). CPU only.

* trace_report_from prints the same text as the reference's own src/trace.c
  (compiled into oracle/_ref) on the same rings: random event streams,
  interleaved pairs, mismatched keys, timestamps running backwards, an empty
  ring and a ring whose head has passed its capacity.
* trace_pair_stats on streams whose latencies are known by construction.
* The clock map, the rebase and the merge.
"""
import ctypes as C
import os
import sys
import tempfile

import numpy as np
import pytest

CAP = 1 << 20
RING = 20971528
ENTRY = np.dtype([("tsc", "<u8"), ("type", "<u4"), ("rid", "<u4"), ("seq", "<u4")])
(ALLOC, FREE, POSTED, COMMITTED, CONSUMED, CPOSTED, POLLED, BATCH, RPOSTED, RSCORED, TDONE) = range(11)


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def _bind(lib):
    lib.trace_report_from.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_char_p]
    lib.trace_report_from.restype = C.c_int
    lib.trace_push_ts.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_uint32, C.c_uint32]
    lib.trace_push_ts.restype = None
    return lib


class _Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("n", "avg_ns", "p50_ns", "p90_ns", "p99_ns")]


class _Map(C.Structure):
    _fields_ = [("ns_per_tick", C.c_double), ("offset_ns", C.c_double)]


def _ring(entries, head=None):
    buf = np.zeros(RING, np.uint8)
    e = buf[:CAP * 20].view(ENTRY)
    e[:len(entries)] = entries
    buf[CAP * 20:].view(np.uint64)[0] = len(entries) if head is None else head
    return buf


def _capture(fn):
    """stdout of C code (fd 1) while fn runs."""
    libc = C.CDLL(None)
    sys.stdout.flush()
    saved = os.dup(1)
    with tempfile.TemporaryFile() as tf:
        os.dup2(tf.fileno(), 1)
        try:
            fn()
            libc.fflush(None)
        finally:
            os.dup2(saved, 1)
            os.close(saved)
        tf.seek(0)
        return tf.read().decode()


def _reports(rl, ref, buf, wall=123456789, prefix=b"T: "):
    mine, theirs = _bind(rl.lib()), _bind(ref)
    a = _capture(lambda: mine.trace_report_from(buf.ctypes.data, wall, 7, 3, prefix))
    b = _capture(lambda: theirs.trace_report_from(buf.ctypes.data, wall, 7, 3, prefix))
    return a, b


def _random_stream(rng, n, n_keys=3, back=0.05):
    e = np.zeros(n, ENTRY)
    e["type"] = rng.integers(0, 12, n)         # 11 is outside the enum
    e["rid"] = rng.integers(0, n_keys, n)
    e["seq"] = rng.integers(0, n_keys, n)
    step = rng.integers(0, 5000, n).astype(np.int64)
    step[rng.random(n) < back] *= -1           # timestamps running backwards now and then
    e["tsc"] = (10**9 + np.cumsum(step)).astype(np.uint64)
    return e


@pytest.mark.parametrize("seed,n,keys", [(1, 5000, 1), (2, 20000, 3), (3, 3000, 40), (4, 7, 2)])
def test_report_matches_reference_on_random_streams(rl, ref, seed, n, keys):
    rng = np.random.default_rng(seed)
    a, b = _reports(rl, ref, _ring(_random_stream(rng, n, keys)))
    assert a == b
    assert "Trace Latency Report" in a and a.count("\n") == 10


def test_report_matches_reference_on_pipeline_shaped_stream(rl, ref):
    """Windows of 32 descriptors per rollout: post, commit, device dequeue,
    completion posted, completion polled; rollout alloc, reward, trajectory."""
    ev = []
    t = 10**9
    rng = np.random.default_rng(7)
    for r in range(40):
        rid = r % 8
        ev.append((t, ALLOC, rid, 0))
        for w in range(0, 64, 32):
            for s in range(w, w + 32):
                t += 30
                ev.append((t, POSTED, rid, s))
                ev.append((t + 5, COMMITTED, rid, s))
            for s in range(w, w + 32):
                t += int(rng.integers(500, 3000))
                ev.append((t, CONSUMED, rid, s))
            for s in range(w, w + 32):
                t += int(rng.integers(100, 900))
                ev.append((t, POLLED, rid, s))
        t += 50
        ev.append((t, RPOSTED, rid, 0))
        ev.append((t + 3, RSCORED, rid, 0))
        ev.append((t + 9, TDONE, rid, 0))
        ev.append((t + 10, FREE, rid, 0))
    e = np.array(ev, dtype=ENTRY)
    a, b = _reports(rl, ref, _ring(e))
    assert a == b and "no samples" not in a


def test_report_matches_reference_empty_and_wrapped(rl, ref):
    a, b = _reports(rl, ref, _ring(np.zeros(0, ENTRY)), wall=0, prefix=None)
    assert a == b and a.count("no samples") == 8
    rng = np.random.default_rng(9)
    e = _random_stream(rng, 4096, 2)
    a, b = _reports(rl, ref, _ring(e, head=CAP + 12345))    # head past the capacity: all 2^20 entries read
    assert a == b and "(1048576 events" in a


def test_push_matches_reference_byte_for_byte(rl, ref):
    bufs = [np.zeros(RING, np.uint8) for _ in range(2)]
    for lib, buf in zip((_bind(rl.lib()), _bind(ref)), bufs):
        base = buf.ctypes.data
        r2 = np.random.default_rng(12)
        buf[CAP * 20:].view(np.uint64)[0] = CAP - 3     # wraps after 3 pushes
        for i in range(10):
            lib.trace_push_ts(base, int(r2.integers(0, 2**63)), int(r2.integers(0, 11)), i, 2 * i)
    assert np.array_equal(bufs[0], bufs[1])
    assert bufs[0][CAP * 20:].view(np.uint64)[0] == CAP + 7


def test_pair_stats_known_latencies(rl):
    L = rl.lib()
    L.trace_pair_stats.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(_Stats)]
    # 100 posts then 100 dequeues in the same order, latency 1000 + 10 i
    e = [(10**6 + i, POSTED, 5, i) for i in range(100)]
    e += [(10**6 + i + 1000 + 10 * i, CONSUMED, 5, i) for i in range(100)]
    e.sort()
    buf = _ring(np.array(e, dtype=ENTRY))
    s = _Stats()
    assert L.trace_pair_stats(buf.ctypes.data, POSTED, CONSUMED, C.byref(s)) == 0
    lat = 1000 + 10 * np.arange(100)
    assert (s.n, s.avg_ns, s.p50_ns, s.p90_ns, s.p99_ns) == (100, int(lat.sum() // 100), lat[50], lat[90], lat[99])
    # a key mismatch costs one pair; an end before its start is not counted
    e2 = [(10, POSTED, 1, 0), (20, CONSUMED, 2, 0), (30, POSTED, 1, 1), (40, CONSUMED, 1, 1),
          (60, POSTED, 1, 2), (50, CONSUMED, 1, 2)]
    buf = _ring(np.array(e2, dtype=ENTRY))
    assert L.trace_pair_stats(buf.ctypes.data, POSTED, CONSUMED, C.byref(s)) == 0
    assert (s.n, s.p50_ns) == (1, 10)


def test_clock_fit_rebase_and_merge(rl):
    L = rl.lib()
    L.trace_clock_fit.argtypes = [C.c_uint64, C.c_double, C.c_uint64, C.c_double, C.POINTER(_Map)]
    L.trace_rebase.argtypes = [C.c_void_p, C.POINTER(_Map)]
    L.trace_merge.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    L.trace_merge.restype = C.c_uint64
    m = _Map()
    # a device clock at 100 MHz running 20 ppm fast against the host
    t0, t1 = 5_000_000_000, 5_100_000_000
    h0 = 7.0e12
    h1 = h0 + (t1 - t0) * 10.0 / (1 + 20e-6)
    assert L.trace_clock_fit(t0, h0, t1, h1, C.byref(m)) == 0
    assert abs(m.ns_per_tick - 10.0 / (1 + 20e-6)) < 1e-9
    dev = _ring(np.array([(t0 + 100 * k, CONSUMED, 1, k) for k in range(5)], dtype=ENTRY))
    L.trace_rebase(dev.ctypes.data, C.byref(m))
    got = dev[:100].view(ENTRY)["tsc"]
    want = np.rint(h0 + 100 * np.arange(5) * m.ns_per_tick).astype(np.uint64)
    assert np.abs(got.astype(np.int64) - want.astype(np.int64)).max() <= 1
    assert L.trace_clock_fit(t0, h0, t0, h0, C.byref(m)) == 0 and m.ns_per_tick == 10.0
    host = _ring(np.array([(int(h0) - 1, POSTED, 1, k) for k in range(5)] + [(int(h0) + 10**6, POLLED, 1, 0)],
                          dtype=ENTRY))
    out = np.zeros(RING, np.uint8)
    srcs = (C.c_void_p * 2)(host.ctypes.data, dev.ctypes.data)
    assert L.trace_merge(out.ctypes.data, srcs, 2) == 11
    merged = out[:11 * 20].view(ENTRY)
    assert list(merged["type"]) == [POSTED] * 5 + [CONSUMED] * 5 + [POLLED]
    assert np.all(np.diff(merged["tsc"].astype(np.int64)) >= 0)
    assert out[CAP * 20:].view(np.uint64)[0] == 11
