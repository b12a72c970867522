"""The host rollout pipeline driving the persistent command-ring worker on
the GPU (rl_pipeline_cmd_run, the loop of bench/bench_pipeline.cu): 1,000
rollouts x 128 decode tokens, decode batches of 32 rollouts, decode_batch
windows of 32 descriptors, credits 256/128/128/1024.

Checked: the completions come back complete and in the order of the
descriptor stream the same driver posts to a host stand-in worker (whose
stream the CPU tests pin against a replay of the reference loop over the
reference's own pipeline functions); every descriptor has one KV token
(num_kv_blocks 1), so its attention output is row 0 of the block's V plane
exactly and the token is that row's lowest-index maximum, with cycles =
1 tile x 128 x 24; the pipeline ends empty.
"""
import ctypes as C

import numpy as np
import pytest

import helpers
import synth

pytestmark = pytest.mark.gpu

N, TOKENS, NBLK, IO = 1000, 128, 128, 4096


def _cfg(rl):
    return rl.CmdPipelineCfg(n_rollouts=N, tokens_per_rollout=TOKENS, batch_max=32, kv_blocks=NBLK,
                             max_decode_credits=256, max_reward_credits=128, max_trajectory_credits=128,
                             kv_block_limit=1024, seed_base=42, full_wait_ns=10**10, drain_wait_ns=10**10)


def _drive(rl, ring, comp, trace=None):
    L = rl.lib()
    pipe = np.zeros(rl.PIPELINE_BYTES, np.uint8)
    rew = np.zeros(rl.REWARD_RING_BYTES, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    L.reward_ring_init(rew.ctypes.data)
    st = rl.CmdPipelineStats()
    log = (rl.Completion * (N * TOKENS))()
    rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, ring, comp, rew.ctypes.data, C.byref(_cfg(rl)), C.byref(st),
                               C.addressof(log), N * TOKENS, trace)
    rows = np.frombuffer(log, dtype=np.dtype([("seq", "<u8"), ("tok", "<u4"), ("kv", "<u4"), ("cookie", "<u8"),
                                              ("cycles", "<u8")])).copy()
    return rc, st, rows, pipe


def test_pipeline_drives_the_gpu_worker(rl, gpu):
    L = rl.lib()
    sim = helpers.load_shared("tests/c/pipeline_sim.c")
    sim.sim_start.argtypes = [C.c_void_p, C.c_void_p]
    sim.sim_stop.restype = C.c_uint64
    ring, comp = L.ring_create(), L.comp_ring_create()
    assert sim.sim_start(C.c_void_p(ring), C.c_void_p(comp)) == 0
    try:
        rc, st_sim, want, _ = _drive(rl, ring, comp)
    finally:
        assert sim.sim_stop() == N * TOKENS
        L.ring_destroy(ring)
        L.comp_ring_destroy(comp)
    assert rc == 0

    rng = np.random.default_rng(91)
    arena16 = synth.f32_to_f16(rng.standard_normal(NBLK * 8192, dtype=np.float32))
    state = np.zeros(6, np.uint64)
    state[:4] = rng.integers(0, 2**63, 4, dtype=np.uint64)
    darena, dst = rl.DeviceBuffer.from_array(arena16), rl.DeviceBuffer.from_array(state)
    print(f"[pipeline] launching the command-ring worker; {N} rollouts x {TOKENS} tokens", flush=True)
    w = rl.CmdWorker(darena, IO, sample_state=dst)
    try:
        rc, st, got, pipe = _drive(rl, w.ring, w.comp)
    finally:
        wst = w.stop()
        w.close()
        darena.close()
        dst.close()
    print(f"[pipeline] {st.descriptors_consumed} completions in {st.wall_ns / 1e6:.1f} ms "
          f"({st.descriptors_consumed / (st.wall_ns * 1e-9):.0f} tokens/s)", flush=True)
    assert rc == 0
    assert (st.rollouts_completed, st.descriptors_posted, st.descriptors_consumed) == (N, N * TOKENS, N * TOKENS)
    assert st.pipeline_overflow == 0 and st.decode_batches == st_sim.decode_batches
    assert wst.tolist()[:2] == [N * TOKENS, N * TOKENS] and wst[3] == 0, wst
    assert np.array_equal(got["seq"], want["seq"]) and np.array_equal(got["cookie"], want["cookie"])
    assert np.array_equal(got["kv"], want["kv"])
    assert np.all(got["cycles"] == 128 * 24)
    v0 = synth.f16_to_f32(arena16.reshape(NBLK, 2, 32, 128)[:, 1, 0, :])      # V plane, token 0
    best = np.array([int(np.flatnonzero(r == r.max()).min()) for r in v0])
    assert np.array_equal(got["tok"], best[got["kv"]])
    snap = rl.PipelineSnapshot()
    L.pipeline_snapshot(pipe.ctypes.data, C.byref(snap))
    assert list(snap.queue_occupancy) == [0] * 6 and snap.credits.decode_used == 0


def _clock(rl):
    L = rl.lib()
    ticks, host, rtt = C.c_uint64(), C.c_double(), C.c_uint64()
    rl.check(L.rl_hip_trace_clock_sample(64, C.byref(ticks), C.byref(host), C.byref(rtt)),
             "rl_hip_trace_clock_sample")
    return ticks.value, host.value, rtt.value


def test_pipeline_traced_on_both_sides(rl, gpu):
    """The same run with tracing: host records from the driver, device
    records (s_memrealtime) from the worker, the device ring mapped onto the
    host clock through two ping-pong clock samples and merged. Every
    descriptor has post, commit, device dequeue, device completion and poll
    records under one (rid, step) key, in stream order on each side; on the
    host timeline the four stamps of a descriptor are ordered within the
    clock samples' uncertainty; the report pairs every descriptor."""
    L = rl.lib()
    rng = np.random.default_rng(92)
    arena16 = synth.f32_to_f16(rng.standard_normal(NBLK * 8192, dtype=np.float32))
    darena = rl.DeviceBuffer.from_array(arena16)
    host = np.zeros(rl.TRACE_RING_BYTES, np.uint8)
    L.trace_init(host.ctypes.data)
    dev_ring = L.rl_hip_host_alloc_coherent(rl.TRACE_RING_BYTES)
    assert dev_ring, rl._err()
    C.memset(dev_ring, 0, rl.TRACE_RING_BYTES)
    c0 = _clock(rl)
    print(f"[pipeline] clock sample: rtt {c0[2]} ns", flush=True)
    w = rl.CmdWorker(darena, IO, trace=dev_ring)
    try:
        rc, st, got, _ = _drive(rl, w.ring, w.comp, trace=host.ctypes.data)
    finally:
        wst = w.stop()
        w.close()
        darena.close()
    c1 = _clock(rl)
    assert rc == 0 and wst[1] == N * TOKENS
    m = rl.TraceClockMap()
    assert L.trace_clock_fit(c0[0], c0[1], c1[0], c1[1], C.byref(m)) == 0
    print(f"[pipeline] clock map: {m.ns_per_tick:.6f} ns/tick, rtt {c0[2]} / {c1[2]} ns", flush=True)
    assert abs(m.ns_per_tick - 10.0) < 0.01
    dbuf = np.frombuffer((C.c_uint8 * rl.TRACE_RING_BYTES).from_address(dev_ring), np.uint8)
    n_dev = int(dbuf[rl.TRACE_CAPACITY * 20:].view(np.uint64)[0])
    assert n_dev == 2 * N * TOKENS
    L.trace_rebase(dev_ring, C.byref(m))
    dev = dbuf[:n_dev * 20].view(rl.TRACE_ENTRY).copy()
    n_host = int(host[rl.TRACE_CAPACITY * 20:].view(np.uint64)[0])
    hst = host[:n_host * 20].view(rl.TRACE_ENTRY)
    T = rl.TRACE

    def of(e, name):
        return e[e["type"] == T[name]]
    post, commit, poll = of(hst, "DESC_POSTED"), of(hst, "DESC_COMMITTED"), of(hst, "COMPLETION_POLLED")
    deq, done = of(dev, "DESC_CONSUMED"), of(dev, "COMPLETION_POSTED")
    for x in (commit, poll, deq, done):
        assert len(x) == N * TOKENS
        assert np.array_equal(x["rollout_id"], post["rollout_id"]) and np.array_equal(x["seq"], post["seq"])
    assert np.array_equal(post["rollout_id"], got["seq"].astype(np.uint32))
    slack = (max(c0[2], c1[2]) + 1) // 2 + 1000
    t = [x["tsc"].astype(np.int64) for x in (commit, deq, done, poll)]
    for a, b in zip(t, t[1:]):
        assert np.all(b - a >= -slack), int((b - a).min())
    merged = np.zeros(rl.TRACE_RING_BYTES, np.uint8)
    srcs = (C.c_void_p * 2)(host.ctypes.data, dev_ring)
    assert L.trace_merge(merged.ctypes.data, srcs, 2) == n_host + n_dev
    s = rl.TracePairStats()
    lat = {}
    for a, b in (("DESC_POSTED", "DESC_COMMITTED"), ("DESC_POSTED", "DESC_CONSUMED"),
                 ("DESC_CONSUMED", "COMPLETION_POSTED"), ("DESC_POSTED", "COMPLETION_POLLED")):
        assert L.trace_pair_stats(merged.ctypes.data, T[a], T[b], C.byref(s)) == 0
        lat[f"{a}->{b}"] = (s.n, s.p50_ns, s.p99_ns)
    print(f"[pipeline] latency pairs (n, p50 ns, p99 ns): {lat}", flush=True)
    assert lat["DESC_POSTED->DESC_COMMITTED"][0] == N * TOKENS
    assert lat["DESC_POSTED->COMPLETION_POLLED"][0] == N * TOKENS
    assert lat["DESC_POSTED->DESC_CONSUMED"][0] >= 0.99 * N * TOKENS
    L.rl_hip_host_free(dev_ring)
