"""The GRPO rollout loop on the device: request ring -> scheduler -> batched
decode steps -> done ring, then reward and group advantage.

512 requests in 64 groups of 8; each group shares a 512-token prefix (32 full
16-token blocks per kv head, the same physical blocks in every member's table,
registered as a kv_prefix with 8 branches) plus U[0, 512] private prompt
tokens; every request generates 256 tokens. Per step: GQA decode attention
(32 q / 8 kv heads, d128, bf16) over the 256 slots, logits = attn_out[4096] .
W (bf16 32,000 x 4096 ~N(0, 0.02^2)), top-p 0.9 sampling (temperature 1,
per-request Philox seed, step = index of the generated token), KV append.

Checked:
  * every request comes back once on the done ring with 256 tokens, status 0,
    and the reward of the reference rule on its generated tokens vs the
    group's seeded target (host reward_match_count); the device group
    advantage equals the host reward_group_advantage bit for bit;
  * scheduler state, counters and ring indices at the end (all slots free,
    513 requests consumed with the end marker, 512 dones);
  * at every step (every 8th step, and every step that admitted requests, in
    the pipeline-fed and copy-on-write variants): every row's token and
    logprob against the host sampler on the device logits (the "given
    identical logits" contract), so the rewards below, computed from the
    device's generated tokens, rest on checked tokens;
  * at three checkpoint steps: 16 attention rows within 1e-4 of fp64 over the
    arena as it stands, and 16 projection rows within the fp32 summation bound
    of an fp64 GEMM;
  * the whole arena at the end byte-equal to the oracle's appends replayed
    step by step (each step's append positions, the request each slot held,
    and that step's K/V pool rows), copy-on-write included;
  * kv_prefix refcounts: 9 while the 8 branches live, 1 after they are freed.
"""
import ctypes as C
import time

import numpy as np
import pytest

import grpo
import synth
from grpo import D, GEN, GROUPS, GS, HID, KVH, POOL, PREFIX, QH, REQ, SLOTS, TPB, VOCAB

pytestmark = pytest.mark.gpu

CHECK_STEPS = (0, 137, 306)


def _check_tokens(orc, olib, dev, t):
    """Every row's token and logprob of step t against the host sampler on the
    device logits (per-row temperature, top-k, top-p, seed and step)."""
    logits = dev["logits"].download(np.float32, (SLOTS, VOCAB))
    tok = dev["tok"].download(np.uint32, SLOTS)
    glp = dev["lp"].download(np.float32, SLOTS)
    want, wlp = orc.sample_rows_v(olib, logits, temperature=dev["temp"].download(np.float32, SLOTS),
                                  top_k=dev["topk"].download(np.uint32, SLOTS),
                                  top_p=dev["topp"].download(np.float32, SLOTS),
                                  seeds=dev["seed"].download(np.uint64, SLOTS),
                                  steps=dev["step"].download(np.uint64, SLOTS))
    bad = np.nonzero(tok != want)[0]
    assert len(bad) == 0, (t, bad[:8], tok[bad[:8]], want[bad[:8]])
    assert np.abs(glp - wlp).max() < 1e-4, t


class _Recorder:
    """on_check hook of RolloutLoop.run: after every step, the append positions
    and the slot -> request map that step used; tokens checked at every
    `every`-th step and every step that admitted requests, and the full check
    at `full_steps`."""

    def __init__(self, rl, orc, olib, cfg, loop, full_steps, pick=None, every=8):
        self.rl, self.orc, self.olib, self.cfg, self.loop = rl, orc, olib, cfg, loop
        self.full_steps, self.pick, self.every = full_steps, pick, every
        self.records, self.admitted, self.token_checks = [], 0, []

    def __call__(self, t):
        dev = self.loop.dev
        pos, sreq = dev["pos"].download(np.uint32, SLOTS), dev["sreq"].download(np.uint32, SLOTS)
        self.records.append((t, pos, sreq))
        adm = int(dev["counters"].download(np.uint32, 4)[1])
        if t in self.full_steps or adm != self.admitted or t % self.every == 0:
            _check_tokens(self.orc, self.olib, dev, t)
            self.token_checks.append(t)
        if t in self.full_steps:
            _check_step(self.rl, self.orc, self.olib, self.cfg, dev, t, self.pick(sreq) if self.pick else None)
        self.admitted = adm


def _replay_arena(olib, cfg, loop, records):
    """The arena after the oracle's appends of every recorded step (copy-on-write
    sources from the oracle's resolve of each slot's branch)."""
    arena = cfg["arena"].copy()
    stride, prefix = cfg["stride"], cfg["prefix"]
    block = 2 * TPB * D * 2
    cows = 0
    for t, pos, sreq in records:
        act = np.nonzero(pos != 0xFFFFFFFF)[0]
        if len(act) == 0:
            continue
        req = sreq[act]
        assert (req < REQ).all(), t
        p = np.ascontiguousarray(pos[act])
        tables = np.ascontiguousarray(cfg["table"][req])
        cow = np.full((len(act), KVH), -1, np.int32)
        for i in np.nonzero(p == prefix)[0]:   # the only position a copy-on-write source can have
            for h in range(KVH):
                cow[i, h] = olib.orc_kvb_cow_source(loop.ptab.ctypes.data, int(loop.branch[req[i]]), int(p[i]),
                                                    TPB, KVH, h)
            cows += int((cow[i] >= 0).all())
        kn = np.ascontiguousarray(cfg["kpool"][t % POOL][act])
        vn = np.ascontiguousarray(cfg["vpool"][t % POOL][act])
        olib.orc_kv_append(arena.ctypes.data, block, TPB, D * 2, tables.ctypes.data, stride, len(act), KVH,
                           p.ctypes.data, cow.ctypes.data, kn.ctypes.data, vn.ctypes.data)
    return arena, cows


def _check_step(rl, orc, olib, cfg, dev, t, pick=None):
    """Attention and projection of step t against the host (tokens: _check_tokens)."""
    logits = dev["logits"].download(np.float32, (SLOTS, VOCAB))
    ctx = dev["ctx"].download(np.uint32, SLOTS)
    active = np.nonzero(ctx)[0]
    assert len(active) > 0
    # attention of 16 active slots (spread over the batch) over the arena as the step saw it
    out32 = dev["out32"].download(np.float32, (SLOTS, QH, D))
    arena = dev["arena"].download(np.uint8, cfg["arena"].size)
    stab = dev["stab"].download(np.uint32, (SLOTS, KVH, cfg["stride"]))
    if pick is None or len(pick) == 0:
        pick = active[np.unique(np.linspace(0, len(active) - 1, 16).astype(np.int64))]
    wl = synth.DecodeWorkload(len(pick), QH, KVH, D, "bf16", TPB, ctx[pick].copy(), stab[pick].copy(), arena,
                              cfg["qpool"][t % POOL][pick].copy(), 0)
    ref = orc.attn_f64(olib, wl, 0)
    err = (np.abs(out32[pick] - ref).max(axis=-1) / np.abs(ref).max(axis=-1)).max()
    assert err < 1e-4, (t, err)
    # projection of 16 rows
    x = dev["out"].download(np.uint16, (SLOTS, HID))
    rows = active[np.unique(np.linspace(0, len(active) - 1, 16).astype(np.int64))]
    xf = synth.bf16_to_f32(x[rows]).astype(np.float64)
    wf = synth.bf16_to_f32(cfg["w"]).astype(np.float64)
    ref = xf @ wf.T
    bound = 2.0 * (HID - 1) * 2.0**-24 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(logits[rows] - ref) <= bound + 1e-30), t
    print(f"[rollout] step {t}: {len(active)} active slots, attention of {len(pick)} rows ({err:.1e}) and "
          f"projection of {len(rows)} rows match", flush=True)


def test_grpo_rollout_loop(rl, gpu, orc, olib):
    L = rl.lib()
    t0 = time.perf_counter()
    cfg = grpo.build_workload(404)
    print(f"[rollout] inputs built in {time.perf_counter() - t0:.1f}s (arena {cfg['arena'].nbytes / 1e9:.2f} GB)",
          flush=True)

    loop = grpo.RolloutLoop(cfg)
    dev = loop.dev
    # kv_prefix bookkeeping of the shared prompts (host, src/kv_prefix.c rules)
    ptab = loop.ptab.ctypes.data
    branch_ids = [int(b) for b in loop.branch]
    assert all(L.kv_prefix_get(ptab, g).contents.refcnt == GS + 1 for g in range(GROUPS))
    assert L.rl_hip_is_coherent_host(loop.rr) and L.rl_hip_is_coherent_host(loop.dr)
    loop.submit_requests()
    print("[rollout] running the loop", flush=True)
    rec = _Recorder(rl, orc, olib, cfg, loop, CHECK_STEPS, every=1)
    res = loop.run(check_steps=range(10**6), on_check=rec)
    dones = loop.dones
    assert rec.token_checks == list(range(res["steps"]))
    print(f"[rollout] tokens and logprobs checked at all {len(rec.token_checks)} steps", flush=True)
    want, cows = _replay_arena(olib, cfg, loop, rec.records)
    assert cows == 0                                      # a 512-token prefix fills whole blocks
    assert np.array_equal(dev["arena"].download(np.uint8, cfg["arena"].size), want)
    print(f"[rollout] arena equals the oracle's replay of {len(rec.records)} steps of appends", flush=True)
    print(f"[rollout] {res['steps']} steps in {res['wall_s']:.2f} s (synchronised after every step)", flush=True)

    counters = dev["counters"].download(np.uint32, 4)
    assert counters.tolist() == [REQ, REQ, 1, 0], counters
    assert len(dones) == REQ and sorted(d[0] for d in dones) == list(range(REQ))
    assert all(d[2] == GEN and d[4] == 0 and d[1] < SLOTS for d in dones)
    state = dev["state"].download(np.uint8, grpo.STATE_BYTES)
    assert not state[18432:].any()                        # bitmap
    assert not state.reshape(-1)[:256 * 72].reshape(256, 72)[:, :4].any()  # active flags

    # rewards: host rule on the device's generated tokens
    gen = dev["gen"].download(np.uint32, (REQ, GEN))
    rew_dev = dev["rewards"].download(np.float32, REQ)
    for rid, _, _, reward, _ in dones:
        tgt = np.ascontiguousarray(cfg["targets"][rid // GS])
        row = np.ascontiguousarray(gen[rid])
        c = L.reward_match_count(row.ctypes.data, tgt.ctypes.data, GEN)
        want = np.float32(c & 0xFF) / np.float32(255.0)
        assert np.float32(reward) == want and rew_dev[rid] == want, rid
    # group advantage on the device vs the host
    ntok = rl.DeviceBuffer.from_array(np.full(REQ, GEN, np.uint32))
    rew2, adv = rl.DeviceBuffer(REQ * 4, zero=True), rl.DeviceBuffer(REQ * 4, zero=True)
    ra = rl.RewardArgs(tokens=dev["gen"].ptr, n_tokens=ntok.ptr, targets=dev["targets"].ptr, rollouts=REQ,
                       group_size=GS, token_stride=GEN, target_stride=GEN, target_len=GEN, reward=rew2.ptr,
                       advantage=adv.ptr)
    rl.check(L.rl_hip_reward_advantage(C.byref(ra)), "rl_hip_reward_advantage")
    rl.sync()
    assert np.array_equal(rew2.download(np.float32, REQ), rew_dev)
    hadv = np.zeros(REQ, np.float32)
    assert L.reward_group_advantage(rew_dev.ctypes.data, GROUPS, GS, hadv.ctypes.data) == 0
    assert np.array_equal(adv.download(np.float32, REQ).view(np.uint32), hadv.view(np.uint32))
    hits = sum(int((gen[r] == cfg["targets"][r // GS]).sum()) for r in range(REQ))
    print(f"[rollout] {REQ} dones, {hits} target hits, mean reward {rew_dev.mean():.4f}", flush=True)

    rr, dr = loop.rr, loop.dr
    assert L.hw_ring_load_acquire(rr) == REQ + 1 and L.hw_ring_load_acquire(rr + 64) == REQ + 1
    assert L.hw_ring_load_acquire(dr) == REQ and L.hw_ring_load_acquire(dr + 64) == REQ
    for b in branch_ids:
        assert L.kv_branch_free(ptab, b) == 0
    assert all(L.kv_prefix_get(ptab, g).contents.refcnt == 1 for g in range(GROUPS))

    for b in (ntok, rew2, adv):
        b.close()
    loop.close()


def test_grpo_loop_fed_by_the_rollout_pipeline(rl, gpu, orc, olib):
    """The same loop with the request ring fed by the host rollout pipeline
    (pipeline_feed.h) under 384 decode credits: requests 0..383 go out at
    once, the rest as dones return credits. Every request finishes once with
    the reference rule's reward on its device tokens; the pipeline ends empty
    (queues, credits, slab, request map); the RewardRing holds one RewardDesc
    per done {prompt length, 256 tokens, reward}; at two checkpoint steps the
    tokens, attention and projection match the host as above."""
    L = rl.lib()
    cfg = grpo.build_workload(405)
    loop = grpo.RolloutLoop(cfg)
    dev = loop.dev
    loop.attach_pipeline(decode_credits=384)
    f = loop.feeder
    assert (f.stats.registered, f.stats.admitted, f.stats.sent) == (REQ, 384, 384)
    print("[rollout] running the pipeline-fed loop", flush=True)
    rec = _Recorder(rl, orc, olib, cfg, loop, (0, 300))
    res = loop.run(check_steps=range(10**6), on_check=rec)
    print(f"[rollout] pipeline-fed: {res['steps']} steps in {res['wall_s']:.2f} s; tokens checked at "
          f"{len(rec.token_checks)} steps", flush=True)
    want, _ = _replay_arena(olib, cfg, loop, rec.records)
    assert np.array_equal(dev["arena"].download(np.uint8, cfg["arena"].size), want)
    assert (f.stats.admitted, f.stats.sent, f.stats.retired, f.stats.reward_handoffs) == (REQ,) * 4
    assert f.stats.bad_dones == 0 and f.end_sent == 1
    assert dev["counters"].download(np.uint32, 4).tolist() == [REQ, REQ, 1, 0]
    dones = loop.dones
    assert sorted(d[0] for d in dones) == list(range(REQ)) and all(d[2] == GEN and d[4] == 0 for d in dones)
    gen = dev["gen"].download(np.uint32, (REQ, GEN))
    rew_dev = dev["rewards"].download(np.float32, REQ)
    for r, _, _, reward, _ in dones:
        tgt = np.ascontiguousarray(cfg["targets"][r // GS])
        row = np.ascontiguousarray(gen[r])
        want = np.float32(L.reward_match_count(row.ctypes.data, tgt.ctypes.data, GEN) & 0xFF) / np.float32(255.0)
        assert np.float32(reward) == want and rew_dev[r] == want, r
    snap = rl.PipelineSnapshot()
    L.pipeline_snapshot(loop.pipe.ctypes.data, C.byref(snap))
    assert list(snap.queue_occupancy) == [0] * 6 and snap.credits.decode_used == 0
    assert np.all(loop.pipe[rl.PIPELINE_SLAB_OFF + 48 * 8192:rl.PIPELINE_SLAB_OFF + 48 * 8192 + 1024] == 0xFF)
    assert np.all(loop.rid_map == 0xFFFFFFFF)
    assert L.hw_ring_load_acquire(loop.rr) == REQ + 1 and L.hw_ring_load_acquire(loop.dr) == REQ
    loop.close()


def test_grpo_loop_copy_on_write_prefix(rl, gpu, orc, olib):
    """The loop with a 520-token shared prefix: 32 full blocks per kv head are
    shared, and the 33rd holds 8 prefix tokens. Every second request has no
    private prompt tokens, so its first generated token lands in that block:
    before its first step rl_hip_kv_cow resolves the slot's branch on the
    device prefix table and copies the 8 prefix slots into the request's
    private block, which the step's attention then reads. Checked: 256
    copy-on-writes happen, the attention at step 0 of 16 such slots is within
    1e-4 of fp64 over the copied block, every token at admission steps and
    every 8th step, every request done once with the reference reward rule,
    and the final arena
    byte-equal to the oracle's replay of every step's copy-on-write and append."""
    L = rl.lib()
    cfg = grpo.build_workload(406, prefix=520, priv_zero_every=2)
    loop = grpo.RolloutLoop(cfg)
    dev = loop.dev
    assert loop.cow is not None
    loop.submit_requests()
    zero = set(int(r) for r in np.nonzero(cfg["priv"] == 0)[0])
    pick = lambda sreq: np.array([s for s in range(SLOTS) if int(sreq[s]) in zero][:16])
    rec = _Recorder(rl, orc, olib, cfg, loop, (0, 291), pick=pick)
    print("[rollout] running the copy-on-write loop (prefix 520)", flush=True)
    res = loop.run(check_steps=range(10**6), on_check=rec)
    print(f"[rollout] cow loop: {res['steps']} steps; tokens checked at {len(rec.token_checks)} steps", flush=True)
    assert dev["counters"].download(np.uint32, 4).tolist() == [REQ, REQ, 1, 0]
    dones = loop.dones
    assert sorted(d[0] for d in dones) == list(range(REQ)) and all(d[2] == GEN and d[4] == 0 for d in dones)
    gen = dev["gen"].download(np.uint32, (REQ, GEN))
    for rid, _, _, reward, _ in dones:
        tgt = np.ascontiguousarray(cfg["targets"][rid // GS])
        row = np.ascontiguousarray(gen[rid])
        want = np.float32(L.reward_match_count(row.ctypes.data, tgt.ctypes.data, GEN) & 0xFF) / np.float32(255.0)
        assert np.float32(reward) == want, rid
    want, cows = _replay_arena(olib, cfg, loop, rec.records)
    assert cows == len(zero) == REQ // 2, (cows, len(zero))
    assert np.array_equal(dev["arena"].download(np.uint8, cfg["arena"].size), want)
    print(f"[rollout] {cows} copy-on-writes; arena equals the oracle's replay", flush=True)
    loop.close()
