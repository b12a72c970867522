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
  * at three checkpoint steps: every row's token equals the host sampler's on
    the device logits (the "given identical logits" contract), attention rows
    within 1e-4 of fp64 over the arena as it stands, and projection rows within
    the fp32 summation bound of an fp64 GEMM;
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


def _check_step(rl, orc, olib, cfg, dev, t):
    """Tokens, attention and projection of step t against the host."""
    logits = dev["logits"].download(np.float32, (SLOTS, VOCAB))
    tok = dev["tok"].download(np.uint32, SLOTS)
    temp = dev["temp"].download(np.float32, SLOTS)
    topk = dev["topk"].download(np.uint32, SLOTS)
    topp = dev["topp"].download(np.float32, SLOTS)
    seed = dev["seed"].download(np.uint64, SLOTS)
    step = dev["step"].download(np.uint64, SLOTS)
    ctx = dev["ctx"].download(np.uint32, SLOTS)
    lp = C.c_double()
    active = np.nonzero(ctx)[0]
    assert len(active) > 0
    for r in range(SLOTS):
        greedy = int(not temp[r] > 0)
        want = olib.orc_sample_row(logits[r].ctypes.data, VOCAB, greedy, float(temp[r]), int(topk[r]),
                                   float(topp[r]), int(seed[r]), int(step[r]), r, C.byref(lp))
        assert tok[r] == want, (t, r, tok[r], want)
    # attention of two active slots over the arena as the step saw it
    out32 = dev["out32"].download(np.float32, (SLOTS, QH, D))
    arena = dev["arena"].download(np.uint8, cfg["arena"].size)
    stab = dev["stab"].download(np.uint32, (SLOTS, KVH, cfg["stride"]))
    pick = active[[0, len(active) // 2]]
    wl = synth.DecodeWorkload(len(pick), QH, KVH, D, "bf16", TPB, ctx[pick].copy(), stab[pick].copy(), arena,
                              cfg["qpool"][t % POOL][pick].copy(), 0)
    ref = orc.attn_f64(olib, wl, 0)
    err = (np.abs(out32[pick] - ref).max(axis=-1) / np.abs(ref).max(axis=-1)).max()
    assert err < 1e-4, (t, err)
    # projection of four rows
    x = dev["out"].download(np.uint16, (SLOTS, HID))
    rows = active[:4]
    xf = synth.bf16_to_f32(x[rows]).astype(np.float64)
    wf = synth.bf16_to_f32(cfg["w"]).astype(np.float64)
    ref = xf @ wf.T
    bound = 2.0 * (HID - 1) * 2.0**-24 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(logits[rows] - ref) <= bound + 1e-30), t
    print(f"[rollout] step {t}: {len(active)} active slots, tokens and attention ({err:.1e}) match", flush=True)


def test_grpo_rollout_loop(rl, gpu, orc, olib):
    L = rl.lib()
    t0 = time.perf_counter()
    cfg = grpo.build_workload(404)
    print(f"[rollout] inputs built in {time.perf_counter() - t0:.1f}s (arena {cfg['arena'].nbytes / 1e9:.2f} GB)",
          flush=True)

    # kv_prefix bookkeeping of the shared prompts (host, src/kv_prefix.c rules)
    ptab = (C.c_uint8 * grpo.PREFIX_TABLE_BYTES)()
    L.kv_prefix_table_init(ptab)
    pid, bid = C.c_uint32(), C.c_uint32()
    branch_ids = []
    for g in range(GROUPS):
        assert L.kv_prefix_register(ptab, int(cfg["prefix_blocks"][g, 0, 0]) * 8192, PREFIX, PREFIX // TPB,
                                    C.byref(pid)) == 0
        assert pid.value == g
        for m in range(GS):
            r = g * GS + m
            assert L.kv_branch_alloc(ptab, r, g, int(cfg["table"][r, 0, PREFIX // TPB]) * 8192,
                                     int(cfg["priv"][r]), int(cfg["n_blocks"][r]) - PREFIX // TPB, C.byref(bid)) == 0
            branch_ids.append(bid.value)
    assert all(L.kv_prefix_get(ptab, g).contents.refcnt == GS + 1 for g in range(GROUPS))

    loop = grpo.RolloutLoop(cfg)
    dev = loop.dev
    assert L.rl_hip_is_coherent_host(loop.rr) and L.rl_hip_is_coherent_host(loop.dr)
    loop.submit_requests()
    print("[rollout] running the loop", flush=True)
    res = loop.run(check_steps=CHECK_STEPS, on_check=lambda t: _check_step(rl, orc, olib, cfg, dev, t))
    dones = loop.dones
    print(f"[rollout] {res['steps']} steps in {res['wall_s']:.2f} s; steps 20-119 (256 active slots): "
          f"{res['window_us_per_step']:.0f} us/step, {SLOTS / res['window_us_per_step'] * 1e6:.0f} tokens/s",
          flush=True)

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
    res = loop.run(check_steps=(0, 300), on_check=lambda t: _check_step(rl, orc, olib, cfg, dev, t))
    print(f"[rollout] pipeline-fed: {res['steps']} steps in {res['wall_s']:.2f} s", flush=True)
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
