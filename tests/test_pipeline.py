"""The host rollout pipeline (include/rollout.h, include/pipeline.h,
include/reward.h's RewardRing) and its two drivers (include/pipeline_feed.h).
CPU only.

* Random operation traces through this runtime's pipeline and through the
  reference's own src/rollout.c + src/pipeline.c (compiled into oracle/_ref):
  return codes, popped ids, snapshots and the whole 493,376-byte
  RolloutPipeline image agree byte for byte.
* Past 2^32 operations a queue still works here; the reference's pop then
  reports an empty queue (its `tail >= head` test), which is pinned too.
* The command-ring driver against a replay of bench/bench_pipeline.cu's loop
  over the reference's own pipeline functions: the same descriptors, in the
  same order and windows, with a host thread standing in for the worker.
* The RequestRing feeder against a host model of the device scheduler
  (256 slots, requests taken only into a free slot, one token per step).
"""
import ctypes as C

import numpy as np
import pytest

import helpers

PIPE = 493376
SLAB = 99072
POLICY = 493344
MAXR = 8192
U32MAX = 0xFFFFFFFF


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def _bind(lib, rl):
    """The same signatures on either library."""
    vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
    sig = {"rollout_slab_init": (None, [vp]), "rollout_alloc": (i32, [vp, vp]), "rollout_free": (None, [vp, u32]),
           "rollout_get": (vp, [vp, u32]), "rollout_transition": (i32, [vp, i32, i32]),
           "pipeline_init": (i32, [vp]), "pipeline_push": (i32, [vp, i32, u32]), "pipeline_pop": (i32, [vp, i32, vp]),
           "pipeline_transition": (i32, [vp, u32, i32, i32]),
           "pipeline_credits_set": (None, [vp, u32, u32, u32, u32]), "pipeline_try_push": (i32, [vp, i32, u32]),
           "pipeline_release": (None, [vp, i32, u32]), "pipeline_set_schedule_policy": (i32, [vp, i32]),
           "pipeline_schedule": (i32, [vp, i32, vp]), "pipeline_occupancy": (u32, [vp, i32]),
           "pipeline_stage_available_credits": (u32, [vp, i32]),
           "pipeline_stage_target_batch": (u32, [vp, i32, u32]), "pipeline_snapshot": (None, [vp, vp])}
    out = {}
    for n, (res, args) in sig.items():
        f = getattr(lib, n)
        f.restype, f.argtypes = res, args
        out[n] = f
    return out


def _trace(mine, ref, seed, steps):
    imgs = [np.zeros(PIPE, np.uint8) for _ in range(2)]
    base = [int(i.ctypes.data) for i in imgs]
    impls = (mine, ref)
    for f, b in zip(impls, base):
        assert f["pipeline_init"](b) == 0
    rng = np.random.default_rng(seed)
    ops = ["alloc", "free", "get", "transition", "ptransition", "push", "pop", "try_push", "release", "credits",
           "policy", "poke_policy", "schedule", "occupancy", "available", "target", "snapshot"]
    weights = np.array([8, 4, 1, 6, 3, 8, 6, 10, 5, 1, 1, 1, 8, 2, 2, 2, 1], float)
    weights /= weights.sum()
    live = []
    for step in range(steps):
        op = ops[rng.choice(len(ops), p=weights)]
        q = int(rng.integers(0, 8))                    # 6 and 7 are out of range
        rid = int(rng.choice(live)) if live and rng.random() < 0.8 else int(rng.integers(0, MAXR + 4))
        st_from, st_to = int(rng.integers(0, 7)), int(rng.integers(0, 7))
        rel_n = int(rng.integers(0, 4)) if step % 2 else int(rng.integers(0, 2**32))
        cred = [int(x) for x in rng.integers(0, 6, 4)]
        pol = int(rng.integers(0, 3))
        tmax = int(rng.integers(0, 40))
        outs = []
        for f, b in zip(impls, base):
            o = np.zeros(21, np.uint32)
            po = o.ctypes.data
            if op == "alloc":
                r = f["rollout_alloc"](b + SLAB, po)
            elif op == "free":
                r = f["rollout_free"](b + SLAB, rid)
            elif op == "get":
                p = f["rollout_get"](b + SLAB, rid)
                r = -1 if p is None else p - b
            elif op == "transition":
                r = None if rid >= MAXR else f["rollout_transition"](b + SLAB + rid * 48, st_from, st_to)
            elif op == "ptransition":
                r = f["pipeline_transition"](b, rid, st_from, st_to)
            elif op == "push":
                r = f["pipeline_push"](b, q, rid)
            elif op == "pop":
                r = f["pipeline_pop"](b, q, po)
            elif op == "try_push":
                r = f["pipeline_try_push"](b, q, rid)
            elif op == "release":
                r = f["pipeline_release"](b, q, rel_n)
            elif op == "credits":
                r = f["pipeline_credits_set"](b, *cred)
            elif op == "policy":
                r = f["pipeline_set_schedule_policy"](b, pol)
            elif op == "poke_policy":      # test_smoke.c:265-272 writes the field directly
                C.c_int.from_address(b + POLICY).value = pol
                r = None
            elif op == "schedule":
                r = f["pipeline_schedule"](b, q, po)
            elif op == "occupancy":
                r = f["pipeline_occupancy"](b, q)
            elif op == "available":
                r = f["pipeline_stage_available_credits"](b, q)
            elif op == "target":
                r = f["pipeline_stage_target_batch"](b, q, tmax)
            else:
                r = f["pipeline_snapshot"](b, po)
            outs.append((r, o.tobytes()))
        assert outs[0] == outs[1], (step, op, q, rid, outs[0][0], outs[1][0])
        if op == "alloc" and outs[0][0] == 0:
            live.append(int(np.frombuffer(outs[0][1], np.uint32)[0]))
        if op == "free" and rid in live:
            live.remove(rid)
        if step == steps // 2:       # fill one queue to the brim once
            fills = []
            for f, b in zip(impls, base):
                k = 0
                while f["pipeline_push"](b, 4, k) == 0:
                    k += 1
                fills.append((k, f["pipeline_occupancy"](b, 4)))
            assert fills[0] == fills[1] and fills[0][1] == 4096, fills
        if step % 2000 == 0:
            assert np.array_equal(imgs[0], imgs[1]), step
    assert np.array_equal(imgs[0], imgs[1])
    return imgs[0]


def test_pipeline_trace_matches_reference(rl, ref):
    mine, theirs = _bind(rl.lib(), rl), _bind(ref, rl)
    img = _trace(mine, theirs, seed=11, steps=40_000)
    # the trace did reach full queues, credit refusals and allocations
    assert img[SLAB:SLAB + 48 * MAXR].any()


def test_pipeline_queue_wraps_past_2_32(rl, ref):
    """Indices start at 2^32 - 2: this runtime keeps FIFO order across the
    wrap; the reference's pop (src/pipeline.c:25-35, `t >= h`) reports the
    queue empty once head has wrapped, though its occupancy says 3."""
    results = {}
    for name, lib in (("mine", rl.lib()), ("ref", ref)):
        f = _bind(lib, rl)
        img = np.zeros(PIPE, np.uint8)
        b = img.ctypes.data
        f["pipeline_init"](b)
        q = 2                                           # Q_DECODE: its IdRing at 2 * 16,512
        head = b + q * 16512
        tail = head + 64 + 4
        C.c_uint32.from_address(head).value = 0xFFFFFFFE
        C.c_uint32.from_address(tail).value = 0xFFFFFFFE
        for i in range(3):
            assert f["pipeline_push"](b, q, 100 + i) == 0
        assert f["pipeline_occupancy"](b, q) == 3
        out = C.c_uint32()
        got = []
        for _ in range(4):
            got.append((f["pipeline_pop"](b, q, C.addressof(out)), out.value))
        results[name] = got
    assert [g for g in results["mine"]] == [(0, 100), (0, 101), (0, 102), (-1, 102)]
    # head wrapped to 1 while tail is 2^32 - 2: all 3 ids stranded
    assert results["ref"] == [(-1, 0)] * 4


# ---------------------------------------------------------------- command-ring driver
def _replay_bench_pipeline(ref, rl, n, tokens, batch_max, kv_blocks, credits):
    """bench/bench_pipeline.cu:271-311 and :348-383 replayed over the
    reference's own pipeline functions; returns the descriptor stream as rows
    (seq_id, kv_block_offset, output_token_offset, reward_cookie, batch_size,
    batch_index), the number of decode batches and the overflow / drop counts."""
    f = _bind(ref, rl)
    img = np.zeros(PIPE, np.uint8)
    b = img.ctypes.data
    f["pipeline_init"](b)
    f["pipeline_credits_set"](b, *credits)
    rows, batches = [], [0]
    counts = {"overflow": 0, "dropped": 0}
    out = C.c_uint32()

    def schedule_decode_batches(drain=False):
        want = min(f["pipeline_stage_target_batch"](b, 2, batch_max), 32)
        if want == 0 and drain:
            # the reference's final loop spins here forever (target_batch is
            # capped by the free credits, all held by queued rollouts); the
            # driver runs the queue in batches of min(batch_max, occupancy)
            want = min(batch_max, f["pipeline_occupancy"](b, 2))
        ids = []
        for _ in range(want):
            if f["pipeline_schedule"](b, 2, C.addressof(out)) != 0:
                break
            ids.append(out.value)
        if not ids:
            return 0
        batches[0] += 1
        for rid in ids:
            kv = rid % 128
            for t in range(0, tokens, 32):
                w = min(32, tokens - t)
                for i in range(w):
                    rows.append((rid, (kv + i) % kv_blocks, t + i, rid << 32 | (t + i), w, i))
                kv = (kv + w) % 128
            ro = b + SLAB + rid * 48
            assert f["rollout_transition"](ro, 2, 3) == 0
            f["pipeline_push"](b, 3, rid)
            assert f["rollout_transition"](ro, 3, 4) == 0
            f["pipeline_push"](b, 4, rid)
            assert f["rollout_transition"](ro, 4, 5) == 0
            f["pipeline_push"](b, 5, rid)
            f["rollout_free"](b + SLAB, rid)
        f["pipeline_release"](b, 2, len(ids))
        return len(ids)

    for r in range(n):
        rid = C.c_uint32()
        assert f["rollout_alloc"](b + SLAB, C.addressof(rid)) == 0
        ro = b + SLAB + rid.value * 48
        assert f["rollout_transition"](ro, 0, 1) == 0
        f["pipeline_push"](b, 1, rid.value)
        assert f["rollout_transition"](ro, 1, 2) == 0
        admitted = True
        while f["pipeline_try_push"](b, 2, rid.value) != 0:
            if schedule_decode_batches() == 0:
                # target_batch is capped by the free decode credits, so with every
                # credit taken nothing can be scheduled: the rollout is dropped
                counts["overflow"] += 1
                admitted = False
                break
        if not admitted:
            f["rollout_free"](b + SLAB, rid.value)
            counts["dropped"] += 1
            continue
        if (r + 1) % batch_max == 0:
            schedule_decode_batches()
    while f["pipeline_occupancy"](b, 2) > 0:
        assert schedule_decode_batches(drain=True) > 0
    return np.array(rows, dtype=np.uint64).reshape(-1, 6), batches[0], counts


def _run_cmd_driver(rl, sim, n, tokens, batch_max, kv_blocks, credits, trace=None):
    L = rl.lib()
    pipe = np.zeros(PIPE, np.uint8)
    rew = np.zeros(rl.REWARD_RING_BYTES, np.uint8)
    assert L.pipeline_init(pipe.ctypes.data) == 0
    L.reward_ring_init(rew.ctypes.data)
    cmd, comp = L.ring_create(), L.comp_ring_create()
    cfg = rl.CmdPipelineCfg(n_rollouts=n, tokens_per_rollout=tokens, batch_max=batch_max, kv_blocks=kv_blocks,
                            max_decode_credits=credits[0], max_reward_credits=credits[1],
                            max_trajectory_credits=credits[2], kv_block_limit=credits[3], seed_base=42,
                            full_wait_ns=10**9, drain_wait_ns=10**9)
    st = rl.CmdPipelineStats()
    log = (rl.Completion * (n * tokens))()
    assert sim.sim_start(C.c_void_p(cmd), C.c_void_p(comp)) == 0
    try:
        rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, cmd, comp, rew.ctypes.data, C.byref(cfg), C.byref(st),
                                   C.addressof(log), n * tokens, trace)
    finally:
        done = sim.sim_stop()
        L.ring_destroy(cmd)
        L.comp_ring_destroy(comp)
    return rc, st, log, done, pipe, rew


@pytest.fixture(scope="module")
def sim(rl):
    lib = helpers.load_shared("tests/c/pipeline_sim.c")
    lib.sim_start.argtypes = [C.c_void_p, C.c_void_p]
    lib.sim_stop.restype = C.c_uint64
    return lib


@pytest.mark.parametrize("n,tokens,batch_max,kv_blocks,credits", [
    (1000, 128, 32, 128, (256, 128, 128, 1024)),     # bench_pipeline's own settings
    (150, 40, 4, 128, (6, 2, 2, 16)),                # scarce credits: batches shrink, rollouts are dropped
    (90, 33, 8, 64, (9, 0, 0, 0)),                   # windows of 32 + 1 over a 64-block arena
    (64, 1, 32, 128, (0, 0, 0, 0)),                  # unlimited credits, one-token rollouts
])
def test_cmd_driver_matches_bench_pipeline_loop(rl, ref, sim, n, tokens, batch_max, kv_blocks, credits):
    want, n_batches, counts = _replay_bench_pipeline(ref, rl, n, tokens, batch_max, kv_blocks, credits)
    rc, st, log, done, pipe, rew = _run_cmd_driver(rl, sim, n, tokens, batch_max, kv_blocks, credits)
    ran = n - counts["dropped"]
    assert rc == 0 and done == ran * tokens == len(want)
    assert (st.rollouts_started, st.rollouts_completed, st.rollouts_dropped) == (n, ran, counts["dropped"])
    assert st.descriptors_posted == st.descriptors_consumed == ran * tokens
    assert st.decode_batches == n_batches and st.pipeline_overflow == counts["overflow"]
    assert st.reward_handoffs == min(ran, 1024) and st.decode_rollouts_scheduled == ran
    got = np.array([(c.seq_id, c.kv_block_offset, c.reward_cookie, c.cycles_taken) for c in log[:ran * tokens]],
                   dtype=np.uint64).reshape(-1, 4)
    assert np.array_equal(got[:, 0], want[:, 0])
    assert np.array_equal(got[:, 1], want[:, 1])
    assert np.array_equal(got[:, 2], want[:, 3])
    assert np.array_equal(got[:, 3], want[:, 4] | (want[:, 5] << np.uint64(16)))
    # the pipeline ends empty: every queue drained, every credit back, every slot free
    L = rl.lib()
    snap = rl.PipelineSnapshot()
    L.pipeline_snapshot(pipe.ctypes.data, C.byref(snap))
    assert list(snap.queue_occupancy) == [0] * 6
    assert (snap.credits.decode_used, snap.credits.reward_used, snap.credits.trajectory_used) == (0, 0, 0)
    assert np.all(pipe[SLAB + 48 * MAXR:SLAB + 48 * MAXR + 1024] == 0xFF)
    # the reward handoffs, in rollout order, with the reference's mock score
    rd = rl.RewardDesc()
    for i in range(min(ran, 1024)):
        assert L.reward_pop(rew.ctypes.data, C.byref(rd)) == 0
        assert (rd.token_count, rd.rollout_id) == (tokens, int(want[i * tokens, 0]))
        assert rd.reward == np.float32((tokens & 0xFF) / 255.0)


def test_cmd_driver_ring_never_drains(rl):
    """No consumer on the command ring: the first 4,096 descriptors (64
    rollouts of 64 tokens) fill it, then every window times out after
    full_wait_ns. Those rollouts are counted failed, freed and never handed to
    the reward ring; only the 64 fully posted ones complete, and the final
    drain gives up (rc -1) with the pipeline left empty."""
    L = rl.lib()
    n, tokens = 200, 64
    pipe = np.zeros(PIPE, np.uint8)
    rew = np.zeros(rl.REWARD_RING_BYTES, np.uint8)
    assert L.pipeline_init(pipe.ctypes.data) == 0
    L.reward_ring_init(rew.ctypes.data)
    cmd, comp = L.ring_create(), L.comp_ring_create()
    cfg = rl.CmdPipelineCfg(n_rollouts=n, tokens_per_rollout=tokens, batch_max=32, kv_blocks=128, seed_base=42,
                            full_wait_ns=10**6, drain_wait_ns=10**6)
    st = rl.CmdPipelineStats()
    try:
        rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, cmd, comp, rew.ctypes.data, C.byref(cfg), C.byref(st), None, 0,
                                   None)
    finally:
        L.ring_destroy(cmd)
        L.comp_ring_destroy(comp)
    assert rc == -1
    assert (st.descriptors_posted, st.descriptors_consumed) == (4096, 0)
    assert (st.rollouts_started, st.rollouts_completed, st.rollouts_failed, st.rollouts_dropped) == (n, 64, n - 64, 0)
    assert st.reward_handoffs == 64 and st.pipeline_overflow == n - 64
    rd = rl.RewardDesc()
    got = []
    while L.reward_pop(rew.ctypes.data, C.byref(rd)) == 0:
        got.append(rd.rollout_id)
    assert len(got) == 64
    snap = rl.PipelineSnapshot()
    L.pipeline_snapshot(pipe.ctypes.data, C.byref(snap))
    assert list(snap.queue_occupancy) == [0] * 6
    assert (snap.credits.decode_used, snap.credits.reward_used, snap.credits.trajectory_used) == (0, 0, 0)
    assert np.all(pipe[SLAB + 48 * MAXR:SLAB + 48 * MAXR + 1024] == 0xFF)


def test_cmd_driver_rejects_bad_config(rl):
    L = rl.lib()
    pipe = np.zeros(PIPE, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    st = rl.CmdPipelineStats()
    for bad in (dict(batch_max=0), dict(batch_max=33), dict(kv_blocks=0)):
        kw = dict(n_rollouts=1, tokens_per_rollout=1, batch_max=1, kv_blocks=1)
        kw.update(bad)
        cfg = rl.CmdPipelineCfg(**kw)
        assert L.rl_pipeline_cmd_run(pipe.ctypes.data, 1, 1, None, C.byref(cfg), C.byref(st), None, 0, None) == -1


# ---------------------------------------------------------------- RequestRing feeder
def _sched_model(rl, shim, req_ring, done_ring, slots, state, step_tokens=1):
    """One step of a host model of the device scheduler: requests are taken
    only into a free slot (lowest first), every active slot gains a token,
    finished slots push their done in slot order."""
    req = rl.RolloutRequest()
    for s in range(slots):
        if state["slot"][s] is None:
            if not shim.prod_req_ring_consume(req_ring, C.byref(req)):
                break
            if req.request_id == 2**64 - 1:
                state["end"] = True
                break
            state["slot"][s] = [req.request_id, 0, req.max_tokens, req.kv_blocks, req.rng_seed,
                                req.temperature, req.top_k, req.top_p]
            state["seen"].append((req.request_id, req.max_tokens, req.kv_blocks, req.rng_seed, req.temperature,
                                  req.top_k, round(req.top_p, 6)))
    for s in range(slots):
        a = state["slot"][s]
        if a is None:
            continue
        a[1] += step_tokens
        if a[1] >= a[2]:
            d = rl.RolloutDone(request_id=a[0], rollout_id=s, tokens_generated=a[2],
                               reward=np.float32((a[0] % 256) / 255.0), status=0)
            if shim.prod_done_ring_push(done_ring, C.byref(d)) == 0:
                state["slot"][s] = None


@pytest.fixture(scope="module")
def prod_shim(rl):
    lib = helpers.load_shared("tests/c/prod_shim.c")
    for n in ("prod_req_ring_consume", "prod_done_ring_push"):
        getattr(lib, n).argtypes = [C.c_void_p, C.c_void_p]
    return lib


@pytest.mark.parametrize("n_req,decode_credits,pump_every", [(512, 384, 7), (600, 0, 1), (300, 40, 3)])
def test_feeder_against_scheduler_model(rl, prod_shim, n_req, decode_credits, pump_every):
    L = rl.lib()
    pipe = np.zeros(PIPE, np.uint8)
    rew = np.zeros(rl.REWARD_RING_BYTES, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    L.pipeline_credits_set(pipe.ctypes.data, decode_credits, 8, 8, 0)
    L.reward_ring_init(rew.ctypes.data)
    req_ring, done_ring = L.req_ring_create(), L.done_ring_create()
    rmap = np.zeros(n_req, np.uint32)
    f = rl.PipelineFeeder()
    fp = rl.FeedParams(temperature=1.0, top_k=0, top_p=0.9, block_tokens=16)
    assert L.rl_feed_init(C.byref(f), pipe.ctypes.data, req_ring, done_ring, rew.ctypes.data, rmap.ctypes.data,
                          n_req, C.byref(fp)) == 0
    rng = np.random.default_rng(5)
    gen = rng.integers(1, 60, n_req)
    prompt = rng.integers(0, 1024, n_req)
    for r in range(n_req):
        assert L.rl_feed_register(C.byref(f), r, int(prompt[r]), int(gen[r]), 1000 + r) >= 0
    assert L.rl_feed_register(C.byref(f), 0, 1, 1, 1) == -1          # already registered
    assert L.rl_feed_register(C.byref(f), n_req, 1, 1, 1) == -1      # out of range
    state = {"slot": [None] * 256, "seen": [], "end": False}
    max_inflight, steps = 0, 0
    while f.stats.retired < n_req:
        if steps % pump_every == 0:
            L.rl_feed_pump(C.byref(f))
            if f.stats.sent == n_req:
                assert L.rl_feed_end(C.byref(f)) == 0
        inflight = f.stats.sent - f.stats.retired
        max_inflight = max(max_inflight, inflight)
        if decode_credits:
            assert f.stats.admitted - f.stats.retired <= decode_credits
        _sched_model(rl, prod_shim, req_ring, done_ring, 256, state)
        steps += 1
        assert steps < 20_000
    L.rl_feed_retire(C.byref(f))
    assert (f.stats.registered, f.stats.admitted, f.stats.sent, f.stats.retired) == (n_req,) * 4
    assert f.stats.bad_dones == 0 and f.stats.reward_handoffs + f.stats.reward_ring_full == n_req
    # requests went out FIFO in registration order with the rollout's fields
    want = [(r, int(gen[r]), int(-(-(prompt[r] + gen[r]) // 16)), 1000 + r, 1.0, 0, 0.9) for r in range(n_req)]
    assert state["seen"] == want
    _sched_model(rl, prod_shim, req_ring, done_ring, 256, state)
    assert state["end"]
    # every stage empty, every credit back, every slab slot free, the map cleared
    snap = rl.PipelineSnapshot()
    L.pipeline_snapshot(pipe.ctypes.data, C.byref(snap))
    assert list(snap.queue_occupancy) == [0] * 6
    assert (snap.credits.decode_used, snap.credits.reward_used, snap.credits.trajectory_used) == (0, 0, 0)
    assert np.all(pipe[SLAB + 48 * MAXR:SLAB + 48 * MAXR + 1024] == 0xFF)
    assert np.all(rmap == U32MAX)
    # the reward ring holds one RewardDesc per done: prompt length, tokens, reward
    rd = rl.RewardDesc()
    got = []
    while L.reward_pop(rew.ctypes.data, C.byref(rd)) == 0:
        got.append((rd.token_start, rd.token_count, rd.reward, rd.reward_model_id, rd.flags))
    want = sorted((int(prompt[r]), int(gen[r]), float(np.float32((r % 256) / 255.0)), 0, 0) for r in range(n_req))
    assert sorted(got) == want
    L.req_ring_destroy(req_ring)
    L.done_ring_destroy(done_ring)


def test_feeder_rejects_unknown_dones_and_bad_params(rl, prod_shim):
    L = rl.lib()
    pipe = np.zeros(PIPE, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    req_ring, done_ring = L.req_ring_create(), L.done_ring_create()
    rmap = np.zeros(4, np.uint32)
    f = rl.PipelineFeeder()
    for bad in (rl.FeedParams(block_tokens=0), rl.FeedParams(block_tokens=16, top_k=70000)):
        assert L.rl_feed_init(C.byref(f), pipe.ctypes.data, req_ring, done_ring, None, rmap.ctypes.data, 4,
                              C.byref(bad)) == -1
    fp = rl.FeedParams(temperature=0.7, top_k=50, top_p=1.0, block_tokens=16)
    assert L.rl_feed_init(C.byref(f), pipe.ctypes.data, req_ring, done_ring, None, rmap.ctypes.data, 4,
                          C.byref(fp)) == 0
    assert L.rl_feed_register(C.byref(f), 1, 17, 5, 9) >= 0
    for rid in (0, 1, 4, 2**40):      # 0: never registered, 1: still in PREFILL, 4 and 2^40: out of range
        d = rl.RolloutDone(request_id=rid, rollout_id=0, tokens_generated=1)
        assert prod_shim.prod_done_ring_push(done_ring, C.byref(d)) == 0
    assert L.rl_feed_retire(C.byref(f)) == 0 and f.stats.bad_dones == 4
    assert L.rl_feed_admit(C.byref(f), 10) == 1 and L.rl_feed_send(C.byref(f), 10) == 1
    req = rl.RolloutRequest()
    assert prod_shim.prod_req_ring_consume(req_ring, C.byref(req)) == 1
    assert (req.request_id, req.kv_blocks, req.max_tokens, req.top_k, req.rng_seed) == (1, 2, 5, 50, 9)  # 17 + 5 tokens
    d = rl.RolloutDone(request_id=1, rollout_id=3, tokens_generated=5, reward=0.5)
    assert prod_shim.prod_done_ring_push(done_ring, C.byref(d)) == 0
    assert L.rl_feed_retire(C.byref(f)) == 1 and rmap[1] == U32MAX
    assert L.rl_feed_end(C.byref(f)) == 0 and L.rl_feed_end(C.byref(f)) == 0
    assert L.rl_feed_send(C.byref(f), 10) == 0
    L.req_ring_destroy(req_ring)
    L.done_ring_destroy(done_ring)


def test_cmd_driver_host_trace(rl, sim):
    """The host-side trace records of a run: one of each rollout event per
    rollout, post / commit / poll per descriptor with its (rid, step) key, in
    an order the report pairs completely."""
    L = rl.lib()
    ring = np.zeros(rl.TRACE_RING_BYTES, np.uint8)
    L.trace_init(ring.ctypes.data)
    n, tokens = 200, 40
    rc, st, log, done, pipe, rew = _run_cmd_driver(rl, sim, n, tokens, 32, 128, (256, 128, 128, 1024),
                                                   trace=ring.ctypes.data)
    assert rc == 0
    cnt = int(ring[rl.TRACE_CAPACITY * 20:].view(np.uint64)[0])
    e = ring[:cnt * 20].view(rl.TRACE_ENTRY)
    T = rl.TRACE
    counts = {k: int((e["type"] == v).sum()) for k, v in T.items()}
    assert counts == {"ROLLOUT_ALLOC": n, "ROLLOUT_FREE": n, "DESC_POSTED": n * tokens,
                      "DESC_COMMITTED": n * tokens, "DESC_CONSUMED": 0, "COMPLETION_POSTED": 0,
                      "COMPLETION_POLLED": n * tokens, "DECODE_BATCH": st.decode_batches, "REWARD_POSTED": n,
                      "REWARD_SCORED": n, "TRAJECTORY_DONE": n}
    assert np.all(np.diff(e["tsc"].astype(np.int64)) >= 0)
    posted = e[e["type"] == T["DESC_POSTED"]]
    polled = e[e["type"] == T["COMPLETION_POLLED"]]
    assert np.array_equal(posted[["rollout_id", "seq"]], polled[["rollout_id", "seq"]])
    got = np.array([(c.seq_id, c.reward_cookie & 0xFFFFFFFF) for c in log[:n * tokens]], dtype=np.uint64)
    assert np.array_equal(got[:, 0], posted["rollout_id"]) and np.array_equal(got[:, 1], posted["seq"])
    s = rl.TracePairStats()
    for a, b, want in (("DESC_POSTED", "DESC_COMMITTED", n * tokens), ("DESC_POSTED", "COMPLETION_POLLED", n * tokens),
                       ("ROLLOUT_ALLOC", "REWARD_POSTED", n), ("ROLLOUT_ALLOC", "TRAJECTORY_DONE", n),
                       ("REWARD_POSTED", "REWARD_SCORED", n), ("REWARD_POSTED", "TRAJECTORY_DONE", n)):
        assert L.trace_pair_stats(ring.ctypes.data, T[a], T[b], C.byref(s)) == 0
        assert s.n == want, (a, b, s.n)
        assert s.p50_ns <= s.p90_ns <= s.p99_ns
