"""The device rollout scheduler (rl_hip_rollout_schedule) launch by launch
against a host model of its contract (include/rl_hip.h; the slot rules of
rollout_worker, cu/gpu_scheduler.cu:26-83, with requests taken only into a
free slot).

Model, per launch: commit the sampled token of every slot that took part in
the last step; retire slots with tokens_generated >= max_tokens in slot order,
each with the reward (count & 0xFF) / 255 where count is the host library's
reward_match_count over min(tokens_generated, gen_stride, target_len) tokens
against the group's target; consume requests in ring order into the free
slots, lowest first, stopping at the end marker (consumed, counters[2] = 1) or
a request id >= requests (consumed, status 2, nothing admitted after it);
write every slot's next-step arguments and copy the admitted slots' block-table
rows. A done ring without room for a launch's retirements stops the scheduler
with status 3 after max_spin polls.

Checked after every launch: the whole GpuRolloutState (slot records and
bitmap), counters, ring indexes, the RolloutDone records popped from the done
ring, the per-slot arguments, the block-table rows of every active slot, and
at the end the generated tokens and the rewards. The workloads stagger
max_tokens so that retirements and admissions of every size meet in one
launch, feed the request ring in bursts, and leave the done ring unpopped on
some steps.
"""
import ctypes as C

import numpy as np
import pytest

import grpo

pytestmark = pytest.mark.gpu

SLOTS = 256
U64 = 2**64 - 1
SLOT_DT = np.dtype({"names": ["active", "request_id", "tokens_generated", "max_tokens", "kv_blocks", "rng",
                              "temperature", "top_k", "top_p"],
                    "formats": ["<u4", "<u4", "<u4", "<u4", "<u4", ("<u8", 4), "<f4", "<u2", "<f4"],
                    "offsets": [0, 4, 8, 12, 16, 24, 56, 60, 64], "itemsize": 72})


class Model:
    def __init__(self, rl, requests, prompt, table, gen_stride, targets, group_size):
        self.L = rl.lib()
        self.requests, self.prompt, self.table = requests, prompt, table
        self.gen_stride, self.targets, self.group_size = gen_stride, targets, group_size
        self.slot = [None] * SLOTS          # [rid, t, max_tokens, kv_blocks, seed, temp, top_k, top_p]
        self.pos = np.full(SLOTS, 0xFFFFFFFF, np.uint32)
        self.counters = [0, 0, 0, 0]
        self.gen = np.zeros((requests, gen_stride), np.uint32)
        self.rewards = np.zeros(requests, np.float32)
        self.queue = []                     # requests in the ring, not yet consumed
        self.dtail = self.dhead = 0
        self.pending_dones = []             # pushed, not yet popped by the host

    def reward(self, rid, t):
        n = min(t, self.gen_stride, self.targets.shape[1])
        row = np.ascontiguousarray(self.gen[rid, :n])
        tgt = np.ascontiguousarray(self.targets[rid // self.group_size, :n])
        c = self.L.reward_match_count(row.ctypes.data, tgt.ctypes.data, n) if n else 0
        return np.float32(c & 0xFF) / np.float32(255.0)

    def launch(self, sampled):
        status0, ended = self.counters[3], self.counters[2]
        if sampled is not None:
            for s in range(SLOTS):
                a = self.slot[s]
                if a is not None and self.pos[s] != 0xFFFFFFFF:
                    if a[1] < self.gen_stride:
                        self.gen[a[0], a[1]] = sampled[s]
                    a[1] += 1
        retiring = [s for s in range(SLOTS) if status0 == 0 and self.slot[s] is not None
                    and self.slot[s][1] >= self.slot[s][2]]
        st = status0
        if retiring and 1024 - (self.dtail - self.dhead) < len(retiring):
            st = 3
        if retiring and st == 0:
            for s in retiring:
                rid, t = self.slot[s][0], self.slot[s][1]
                r = self.reward(rid, t)
                self.rewards[rid] = r
                self.pending_dones.append((rid, s, t, r))
                self.slot[s] = None
            self.dtail += len(retiring)
            self.counters[0] += len(retiring)
        if st == 0 and ended == 0:
            free = [s for s in range(SLOTS) if self.slot[s] is None]
            n_try = min(len(free), len(self.queue))
            adm = 0
            for i in range(n_try):
                q = self.queue.pop(0)
                if q.request_id == U64:
                    self.counters[2] = 1
                    break
                if (q.request_id & 0xFFFFFFFF) >= self.requests:
                    st = 2
                    break
                self.slot[free[adm]] = [q.request_id & 0xFFFFFFFF, 0, q.max_tokens, q.kv_blocks, q.rng_seed,
                                        np.float32(q.temperature), q.top_k, np.float32(q.top_p)]
                adm += 1
            self.counters[1] += adm
        self.counters[3] = st
        for s in range(SLOTS):
            a = self.slot[s]
            # a slot at max_tokens that could not retire is parked: no append position
            self.pos[s] = 0xFFFFFFFF if a is None or a[1] >= a[2] else self.prompt[a[0]] + a[1]

    def args(self):
        ctx = np.zeros(SLOTS, np.uint32)
        temp, topp = np.zeros(SLOTS, np.float32), np.ones(SLOTS, np.float32)
        topk, seed, step = np.zeros(SLOTS, np.uint32), np.zeros(SLOTS, np.uint64), np.zeros(SLOTS, np.uint64)
        for s, a in enumerate(self.slot):
            if a is not None and a[1] < a[2]:
                ctx[s] = self.prompt[a[0]] + a[1]
                temp[s], topk[s], topp[s], seed[s], step[s] = a[5], a[6], a[7], a[4], a[1]
        req = np.array([a[0] if a is not None and a[1] < a[2] else 0xFFFFFFFF for a in self.slot], np.uint32)
        return ctx, self.pos.copy(), temp, topk, topp, seed, step, req


def _run(rl, seed, requests, max_tok, feed, pop_every, max_spin=0, bad_at=None, steps=400, after_stop=0):
    L = rl.lib()
    rng = np.random.default_rng(seed)
    kvh, stride, gen_stride, target_len, gs = 2, 5, 32, 16, 4
    prompt = rng.integers(0, 900, requests).astype(np.uint32)
    table = rng.integers(0, 2**31, (requests, kvh, stride)).astype(np.uint32)
    targets = rng.integers(0, 3, (-(-requests // gs), target_len)).astype(np.uint32)
    ids = rng.permutation(requests)
    reqs = []
    for i, r in enumerate(ids):
        rid = int(r) if i != bad_at else requests + 7
        reqs.append(rl.RolloutRequest(request_id=rid, max_tokens=int(max_tok(rng)), kv_blocks=int(rng.integers(1, 9)),
                                      temperature=float(rng.choice([0.0, 0.7, 1.0])), top_k=int(rng.integers(0, 60)),
                                      top_p=float(rng.uniform(0.5, 1.0)), rng_seed=int(rng.integers(0, 2**63))))
    reqs.append(rl.RolloutRequest(request_id=U64))
    model = Model(rl, requests, prompt, table, gen_stride, targets, gs)

    dev = {k: rl.DeviceBuffer.from_array(v) for k, v in (("prompt", prompt), ("table", table), ("targets", targets))}
    for k, n in (("state", grpo.STATE_BYTES), ("counters", 16), ("gen", requests * gen_stride * 4),
                 ("rewards", requests * 4), ("stab", SLOTS * kvh * stride * 4), ("ctx", SLOTS * 4),
                 ("temp", SLOTS * 4), ("topk", SLOTS * 4), ("topp", SLOTS * 4), ("seed", SLOTS * 8),
                 ("step", SLOTS * 8), ("tok", SLOTS * 4), ("req", SLOTS * 4)):
        dev[k] = rl.DeviceBuffer(n, zero=True)
    dev["pos"] = rl.DeviceBuffer.from_array(np.full(SLOTS, 0xFFFFFFFF, np.uint32))
    rr, dr = L.req_ring_create(), L.done_ring_create()
    assert rr and dr
    a = rl.SchedArgs(req_ring=rr, done_ring=dr, state=dev["state"].ptr, requests=requests,
                     prompt_len=dev["prompt"].ptr, req_table=dev["table"].ptr, kv_heads=kvh, table_stride=stride,
                     gen_tokens=dev["gen"].ptr, gen_stride=gen_stride, targets=dev["targets"].ptr, group_size=gs,
                     target_len=target_len, rewards=dev["rewards"].ptr, slot_table=dev["stab"].ptr,
                     slot_ctx=dev["ctx"].ptr, slot_pos=dev["pos"].ptr, slot_temp=dev["temp"].ptr,
                     slot_topk=dev["topk"].ptr, slot_topp=dev["topp"].ptr, slot_seed=dev["seed"].ptr,
                     slot_step=dev["step"].ptr, sampled=None, counters=dev["counters"].ptr, max_spin=max_spin,
                     slot_request=dev["req"].ptr)
    fed = 0
    try:
        for step in range(steps):
            for _ in range(feed(step)):
                if fed < len(reqs) and grpo.req_ring_push(rr, reqs[fed]) == 0:
                    model.queue.append(reqs[fed])
                    fed += 1
            sampled = None
            if step > 0:
                sampled = rng.integers(0, 3, SLOTS).astype(np.uint32)
                dev["tok"].upload(sampled)
            a.sampled = dev["tok"].ptr if step > 0 else None
            assert L.rl_hip_rollout_schedule(C.byref(a)) == 0
            rl.sync()
            model.launch(sampled)

            ctx = f"seed {seed} launch {step}"
            assert dev["counters"].download(np.uint32, 4).tolist() == model.counters, ctx
            got = [dev[k].download(dt, SLOTS) for k, dt in (("ctx", np.uint32), ("pos", np.uint32),
                                                             ("temp", np.float32), ("topk", np.uint32),
                                                             ("topp", np.float32), ("seed", np.uint64),
                                                             ("step", np.uint64), ("req", np.uint32))]
            for name, g, w in zip(("ctx", "pos", "temp", "topk", "topp", "seed", "step", "request"), got,
                                  model.args()):
                np.testing.assert_array_equal(g, w, err_msg=f"{ctx}: slot_{name}")
            raw = dev["state"].download(np.uint8, grpo.STATE_BYTES)
            st = raw[:SLOTS * 72].view(SLOT_DT)
            bitmap = raw[SLOTS * 72:].view(np.uint64)
            want_bits = np.zeros(4, np.uint64)
            for s, m in enumerate(model.slot):
                if m is None:
                    assert st["active"][s] == 0, (ctx, s)
                    continue
                want_bits[s // 64] |= np.uint64(1 << (s % 64))
                assert st["active"][s] == 1 and st["request_id"][s] == m[0] and st["tokens_generated"][s] == m[1], (ctx, s)
                assert st["max_tokens"][s] == m[2] and st["kv_blocks"][s] == m[3], (ctx, s)
                sd = m[4]
                assert st["rng"][s].tolist() == [sd, sd ^ 0x9E3779B97F4A7C15, ((sd << 17) & U64) ^ 0x3C6EF372FE94F82A,
                                                 sd ^ U64], (ctx, s)
                assert st["temperature"][s] == m[5] and st["top_k"][s] == m[6] and st["top_p"][s] == m[7], (ctx, s)
            np.testing.assert_array_equal(bitmap, want_bits, err_msg=ctx)
            stab = dev["stab"].download(np.uint32, (SLOTS, kvh, stride))
            for s, m in enumerate(model.slot):
                if m is not None:
                    np.testing.assert_array_equal(stab[s], table[m[0]], err_msg=f"{ctx}: slot {s} table")
            assert L.hw_ring_load_acquire(dr + 64) == model.dtail, ctx
            if pop_every and step % pop_every == 0:
                while (d := grpo.done_ring_pop(dr)) is not None:
                    w = model.pending_dones.pop(0)
                    assert (d.request_id, d.rollout_id, d.tokens_generated, d.status) == (w[0], w[1], w[2], 0), ctx
                    assert np.float32(d.reward) == w[3], ctx
                    model.dhead += 1
            assert not model.pending_dones or not pop_every or step % pop_every != 0
            if model.counters[3] != 0:
                after_stop -= 1
                if after_stop < 0:
                    break
            elif model.counters[2] and all(m is None for m in model.slot):
                break
        np.testing.assert_array_equal(dev["gen"].download(np.uint32, (requests, gen_stride)), model.gen)
        np.testing.assert_array_equal(dev["rewards"].download(np.float32, requests), model.rewards)
        return model, step
    finally:
        L.req_ring_destroy(rr)
        L.done_ring_destroy(dr)
        for b in dev.values():
            b.close()


def test_staggered_lengths_bursty_feed(rl, gpu):
    """600 requests of 1..40 tokens, fed 120 at first and 37 every third
    launch; dones popped every second launch."""
    model, steps = _run(rl, 11, 600, lambda g: g.integers(1, 41), lambda t: 120 if t == 0 else (37 if t % 3 == 0 else 0),
                        pop_every=2)
    assert model.counters[:3] == [600, 600, 1] and model.counters[3] == 0
    print(f"[sched] staggered: {steps + 1} launches", flush=True)


def test_full_turnover_each_launch(rl, gpu):
    """Every slot retires and is refilled on every launch (1-token requests)."""
    model, steps = _run(rl, 12, 900, lambda g: 1, lambda t: 1000 if t == 0 else 0, pop_every=1)
    assert model.counters[:3] == [900, 900, 1] and model.counters[3] == 0


def test_bad_request_id_stops_admission(rl, gpu):
    model, steps = _run(rl, 13, 300, lambda g: g.integers(1, 9), lambda t: 400 if t == 0 else 0, pop_every=1,
                        bad_at=41)
    assert model.counters[3] == 2 and model.counters[1] == 41 and model.counters[2] == 0


def test_done_ring_full_stops_with_status_3(rl, gpu):
    """No done is ever popped: the fifth turnover of 256 slots finds no room
    and gives up after a short bounded wait. Four more launches after that:
    the slots at max_tokens stay parked (no context, no append position, no
    more tokens) instead of decoding past their blocks."""
    model, steps = _run(rl, 14, 1500, lambda g: 1, lambda t: 1000 if t == 0 else (600 if t == 3 else 0),
                        pop_every=0, max_spin=64, after_stop=4)
    assert model.counters[3] == 3 and model.counters[0] == 1024
    parked = [m for m in model.slot if m is not None]
    assert len(parked) == SLOTS and all(m[1] == m[2] for m in parked)
    assert (model.pos == 0xFFFFFFFF).all()


def test_launch_argument_checks(rl, gpu):
    """Refused on the host, nothing launched: a zero size, or 2^24 or more
    block-table entries per slot."""
    L = rl.lib()
    dev = rl.DeviceBuffer(1 << 16, zero=True)
    rr, dr = L.req_ring_create(), L.done_ring_create()
    try:
        ok = dict(req_ring=rr, done_ring=dr, state=dev.ptr, requests=4, prompt_len=dev.ptr, req_table=dev.ptr,
                  kv_heads=2, table_stride=5, gen_tokens=dev.ptr, gen_stride=8, targets=dev.ptr, group_size=2,
                  target_len=8, rewards=dev.ptr, slot_table=dev.ptr, slot_ctx=dev.ptr, slot_pos=dev.ptr,
                  slot_temp=dev.ptr, slot_topk=dev.ptr, slot_topp=dev.ptr, slot_seed=dev.ptr, slot_step=dev.ptr,
                  sampled=None, counters=dev.ptr)
        for bad in (dict(requests=0), dict(group_size=0), dict(gen_stride=0), dict(kv_heads=8, table_stride=1 << 21),
                    dict(kv_heads=1, table_stride=1 << 24), dict(counters=None)):
            a = rl.SchedArgs(**{**ok, **bad})
            assert L.rl_hip_rollout_schedule(C.byref(a)) == -1, bad
            assert b"rl_hip_rollout_schedule" in L.rl_hip_last_error(), bad
    finally:
        L.req_ring_destroy(rr)
        L.done_ring_destroy(dr)
        dev.close()
