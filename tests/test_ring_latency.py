"""The unloaded-latency drivers of ring_latency.h on the CPU: a Python
thread plays the persistent worker on every ring pair (pops a descriptor,
writes the two stamps, pushes the completion), the rings in ordinary host
memory (no device open). Checked: every sample taken, descriptors sent in
pair order with their tag, the stamps read back after the completion, the
host stamps ordered (submit < poll < next submit); a command ring that is
not empty and a completion that never comes stop the driver early."""
import ctypes as C
import threading

import numpy as np


def _u32(addr):
    return C.c_uint32.from_address(addr)


def _worker(rl, pairs, cmd, comp, stamps, kind, stop):
    """Consumes cmd[g] and produces comp[g] for every pair until stop is set."""
    L = rl.lib()
    tick = 1000
    while not stop.is_set():
        for g in range(pairs):
            head, tail = L.hw_ring_load_acquire(cmd[g]), L.hw_ring_load_acquire(cmd[g] + 64)
            if head == tail:
                continue
            tick += 1
            stamps[2 * g] = tick
            if kind == "hw":
                src = cmd[g] + 128 + (head & 0xFFFF) * 64
                body = C.string_at(src, 64)
                L.hw_ring_store_release(cmd[g], (head + 1) & 0xFFFFFFFF)
                ct = L.hw_ring_load_acquire(comp[g] + 64)
                C.memmove(comp[g] + 128 + (ct & 0xFFFF) * 64, body, 64)
            else:
                src = cmd[g] + 128 + (head & 4095) * 32
                seq = C.c_uint64.from_address(src).value
                L.hw_ring_store_release(cmd[g], (head + 1) & 0xFFFFFFFF)
                ct = L.hw_ring_load_acquire(comp[g] + 64)
                C.c_uint64.from_address(comp[g] + 256 + (ct & 4095) * 32).value = seq
            tick += 7
            stamps[2 * g + 1] = tick
            L.hw_ring_store_release(comp[g] + 64, (ct + 1) & 0xFFFFFFFF)


def _run(rl, kind, pairs, n):
    L = rl.lib()
    if kind == "hw":
        cmd = [L.hw_ring_create() for _ in range(pairs)]
        comp = [L.hw_ring_create() for _ in range(pairs)]
    else:
        cmd = [L.ring_create() for _ in range(pairs)]
        comp = [L.comp_ring_create() for _ in range(pairs)]
    tab = (C.c_void_p * (2 * pairs))(*(cmd + comp))
    stamps = np.zeros(2 * pairs, np.uint64)
    out = (rl.RingLockstepSample * n)()
    stop = threading.Event()
    th = threading.Thread(target=_worker, args=(rl, pairs, cmd, comp, stamps, kind, stop), daemon=True)
    th.start()
    try:
        base = C.addressof(tab)
        if kind == "hw":
            d = rl.HwDesc(opcode=1, seq_len=5, max_tokens=5)
            got = L.ring_lockstep_hw(base, base + 8 * pairs, pairs, C.byref(d), n, stamps.ctypes.data, 5 * 10**9, out)
        else:
            d = rl.Descriptor(num_kv_blocks=32)
            got = L.ring_lockstep_cmd(base, base + 8 * pairs, pairs, C.byref(d), 77, n, stamps.ctypes.data,
                                      5 * 10**9, out)
    finally:
        stop.set()
        th.join()
    for r in cmd + comp:
        (L.hw_ring_destroy if kind == "hw" else (L.ring_destroy if r in cmd else L.comp_ring_destroy))(r)
    return got, out


def test_lockstep_drivers_with_a_host_worker(rl):
    for kind in ("hw", "cmd"):
        n, pairs = 24, 3
        got, out = _run(rl, kind, pairs, n)
        assert got == n, kind
        cons = [s.consume_tick for s in out]
        comp = [s.complete_tick for s in out]
        # the worker's ticks: consume t, complete t + 7, the next consume t + 8
        assert all(b - a == 7 for a, b in zip(cons, comp)), kind
        assert all(c2 - c1 == 8 for c1, c2 in zip(cons, cons[1:])), kind
        for i, s in enumerate(out):
            assert s.submit_ns <= s.poll_ns, (kind, i)
            if i:
                assert out[i - 1].poll_ns <= s.submit_ns, (kind, i)


def test_lockstep_stops_on_busy_ring_and_timeout(rl):
    L = rl.lib()
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    tab = (C.c_void_p * 2)(cq, dq)
    stamps = np.zeros(2, np.uint64)
    out = (rl.RingLockstepSample * 4)()
    d = rl.HwDesc(opcode=1, seq_len=5, max_tokens=5)
    base = C.addressof(tab)
    # no worker: the first completion never arrives (1 ms timeout)
    assert L.ring_lockstep_hw(base, base + 8, 1, C.byref(d), 4, stamps.ctypes.data, 10**6, out) == 0
    # the command ring now holds that descriptor: not idle, nothing sent
    tail = L.hw_ring_load_acquire(cq + 64)
    assert L.ring_lockstep_hw(base, base + 8, 1, C.byref(d), 4, stamps.ctypes.data, 10**6, out) == 0
    assert L.hw_ring_load_acquire(cq + 64) == tail
    # NULL arguments take nothing
    assert L.ring_lockstep_hw(None, base + 8, 1, C.byref(d), 4, stamps.ctypes.data, 10**6, out) == 0
    L.hw_ring_destroy(cq)
    L.hw_ring_destroy(dq)
