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


def _drive(rl, ring, comp):
    L = rl.lib()
    pipe = np.zeros(rl.PIPELINE_BYTES, np.uint8)
    rew = np.zeros(rl.REWARD_RING_BYTES, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    L.reward_ring_init(rew.ctypes.data)
    st = rl.CmdPipelineStats()
    log = (rl.Completion * (N * TOKENS))()
    rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, ring, comp, rew.ctypes.data, C.byref(_cfg(rl)), C.byref(st),
                               C.addressof(log), N * TOKENS)
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
