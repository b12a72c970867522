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

import synth

pytestmark = pytest.mark.gpu

GROUPS, GS = 64, 8
REQ = GROUPS * GS
PREFIX, PRIV_MAX, GEN = 512, 512, 256
QH, KVH, D, TPB = 32, 8, 128, 16
HID, VOCAB = QH * D, 32000
SLOTS = 256
POOL = 8
CHECK_STEPS = (0, 137, 306)


def req_ring_push(rl, ring, req):
    L = rl.lib()
    head, tail = L.hw_ring_load_acquire(ring), L.hw_ring_load_acquire(ring + 64)
    if (tail - head) & 0xFFFFFFFF >= 1024:
        return -1
    C.memmove(ring + 128 + (tail & 1023) * 34, C.byref(req), 34)
    L.hw_ring_store_release(ring + 64, (tail + 1) & 0xFFFFFFFF)
    return 0


def done_ring_pop(rl, ring):
    L = rl.lib()
    head = L.hw_ring_load_acquire(ring)
    if head == L.hw_ring_load_acquire(ring + 64):
        return None
    d = rl.RolloutDone.from_buffer_copy((C.c_char * 24).from_address(ring + 256 + (head & 1023) * 24))
    L.hw_ring_store_release(ring, (head + 1) & 0xFFFFFFFF)
    return d


def _build(seed):
    rng = np.random.default_rng(seed)
    priv = rng.integers(0, PRIV_MAX + 1, REQ)
    prompt = (PREFIX + priv).astype(np.uint32)
    n_prefix = PREFIX // TPB
    n_priv = -(-(priv + GEN + 1) // TPB)
    stride = n_prefix + -(-(PRIV_MAX + GEN + 1) // TPB)   # covers the largest context
    total = GROUPS * KVH * n_prefix + int(n_priv.sum()) * KVH
    perm = rng.permutation(total).astype(np.uint32)
    table = np.zeros((REQ, KVH, stride), np.uint32)
    k = 0
    prefix_blocks = np.zeros((GROUPS, KVH, n_prefix), np.uint32)
    for g in range(GROUPS):
        for h in range(KVH):
            prefix_blocks[g, h] = perm[k:k + n_prefix]
            k += n_prefix
    for r in range(REQ):
        for h in range(KVH):
            table[r, h, :n_prefix] = prefix_blocks[r // GS, h]
            m = int(n_priv[r])
            table[r, h, n_prefix:n_prefix + m] = perm[k:k + m]
            k += m
    arena = np.empty(total * 2 * TPB * D, np.uint16)
    synth._fill_normal(rng, arena.size, 1.0, "bf16", arena)
    w = synth.f32_to_bf16(rng.standard_normal((VOCAB, HID), dtype=np.float32) * np.float32(0.02))
    qpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, QH, D), dtype=np.float32))
    kpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, KVH, D), dtype=np.float32))
    vpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, KVH, D), dtype=np.float32))
    targets = rng.integers(0, VOCAB, (GROUPS, GEN), dtype=np.uint32)
    seeds = rng.integers(0, 2**63, REQ, dtype=np.uint64)
    return dict(prompt=prompt, table=table, stride=stride, arena=arena.view(np.uint8), w=w, qpool=qpool,
                kpool=kpool, vpool=vpool, targets=targets, seeds=seeds, prefix_blocks=prefix_blocks,
                priv=priv, n_blocks=n_prefix + n_priv)


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
    cfg = _build(404)
    print(f"[rollout] inputs built in {time.perf_counter() - t0:.1f}s (arena {cfg['arena'].nbytes / 1e9:.2f} GB)",
          flush=True)

    # kv_prefix bookkeeping of the shared prompts (host, src/kv_prefix.c rules)
    ptab = (C.c_uint8 * 606280)()
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

    dev = {}
    up = lambda k, a: dev.__setitem__(k, rl.DeviceBuffer.from_array(a))  # noqa: E731
    up("arena", cfg["arena"])
    up("w", cfg["w"])
    up("qpool", cfg["qpool"])
    up("kpool", cfg["kpool"])
    up("vpool", cfg["vpool"])
    up("prompt", cfg["prompt"])
    up("rtab", cfg["table"])
    up("targets", cfg["targets"])
    stride = cfg["stride"]
    zeros = lambda k, n: dev.__setitem__(k, rl.DeviceBuffer(n, zero=True))  # noqa: E731
    zeros("state", 18464)
    zeros("counters", 16)
    zeros("gen", REQ * GEN * 4)
    zeros("rewards", REQ * 4)
    zeros("stab", SLOTS * KVH * stride * 4)
    zeros("ctx", SLOTS * 4)
    up("pos", np.full(SLOTS, 0xFFFFFFFF, np.uint32))
    zeros("temp", SLOTS * 4)
    zeros("topk", SLOTS * 4)
    zeros("topp", SLOTS * 4)
    zeros("seed", SLOTS * 8)
    zeros("step", SLOTS * 8)
    zeros("out", SLOTS * HID * 2)
    zeros("out32", SLOTS * HID * 4)
    zeros("logits", SLOTS * VOCAB * 4)
    zeros("tok", SLOTS * 4)
    zeros("lp", SLOTS * 4)

    rr, dr = L.req_ring_create(), L.done_ring_create()
    assert L.rl_hip_is_coherent_host(rr) and L.rl_hip_is_coherent_host(dr)
    for r in range(REQ):
        req = rl.RolloutRequest(request_id=r, max_tokens=GEN, kv_blocks=int(cfg["n_blocks"][r]),
                                temperature=1.0, top_k=0, top_p=0.9, rng_seed=int(cfg["seeds"][r]))
        assert req_ring_push(rl, rr, req) == 0
    assert req_ring_push(rl, rr, rl.RolloutRequest(request_id=2**64 - 1)) == 0

    sched = rl.SchedArgs(req_ring=rr, done_ring=dr, state=dev["state"].ptr, requests=REQ,
                         prompt_len=dev["prompt"].ptr, req_table=dev["rtab"].ptr, kv_heads=KVH, table_stride=stride,
                         gen_tokens=dev["gen"].ptr, gen_stride=GEN, targets=dev["targets"].ptr, group_size=GS,
                         target_len=GEN, rewards=dev["rewards"].ptr, slot_table=dev["stab"].ptr,
                         slot_ctx=dev["ctx"].ptr, slot_pos=dev["pos"].ptr, slot_temp=dev["temp"].ptr,
                         slot_topk=dev["topk"].ptr, slot_topp=dev["topp"].ptr, slot_seed=dev["seed"].ptr,
                         slot_step=dev["step"].ptr, sampled=None, counters=dev["counters"].ptr)
    layout = rl.KvLayoutDesc.paged(TPB, D)
    max_ctx = PREFIX + PRIV_MAX + GEN + 1
    attn = rl.attn_args(dev["arena"], layout, dev["stab"], stride, SLOTS, QH, KVH, rl.DTYPE_BF16, dev["ctx"],
                        max_ctx, dev["qpool"], dev["out"], dev["out32"])
    attn_ws = rl.attn_workspace(attn)
    samp = rl.sample_args(dev["logits"], SLOTS, VOCAB, VOCAB, dev["tok"], dev["lp"])
    samp.temperature, samp.top_k, samp.top_p = dev["temp"].ptr, dev["topk"].ptr, dev["topp"].ptr
    samp.seed, samp.steps = dev["seed"].ptr, dev["step"].ptr
    samp_ws = rl.sample_workspace(samp)
    app = rl.AppendArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=layout,
                        block_table=dev["stab"].ptr, table_stride=stride, batch=SLOTS, kv_heads=KVH,
                        positions=dev["pos"].ptr, cow_src=None)
    q_row = SLOTS * QH * D * 2
    kv_row = SLOTS * KVH * D * 2

    dones = []
    t = 0
    timed = None
    print("[rollout] running the loop", flush=True)
    while len(dones) < REQ:
        assert t < 700, ("loop did not finish", len(dones), dev["counters"].download(np.uint32, 4))
        sched.sampled = dev["tok"].ptr if t > 0 else None
        rl.check(L.rl_hip_rollout_schedule(C.byref(sched)), "rl_hip_rollout_schedule")
        attn.q = dev["qpool"].ptr + (t % POOL) * q_row
        rl.attn_decode(attn)
        rl.logits_proj(dev["out"], dev["w"], dev["logits"], SLOTS, VOCAB, HID)
        rl.sample(samp)
        app.k_new = dev["kpool"].ptr + (t % POOL) * kv_row
        app.v_new = dev["vpool"].ptr + (t % POOL) * kv_row
        rl.kv_append(app)
        if t in CHECK_STEPS:
            rl.sync()
            _check_step(rl, orc, olib, cfg, dev, t)
        if t in (20, 120):             # a window without checkpoints or done polling
            rl.sync()
            if t == 20:
                timed = time.perf_counter()
            else:
                timed = (time.perf_counter() - timed) / 100
        t += 1
        if t % 32 == 0 and t not in range(20, 121):
            rl.sync()
            while (d := done_ring_pop(rl, dr)) is not None:
                dones.append((d.request_id, d.rollout_id, d.tokens_generated, d.reward, d.status))
            st = dev["counters"].download(np.uint32, 4)
            assert st[3] == 0, st
    # the commit of the last step and the final retirements happen in one more launch
    rl.check(L.rl_hip_rollout_schedule(C.byref(sched)), "rl_hip_rollout_schedule")
    rl.sync()
    while (d := done_ring_pop(rl, dr)) is not None:
        dones.append((d.request_id, d.rollout_id, d.tokens_generated, d.reward, d.status))
    print(f"[rollout] {t} steps; steps 20-119 (256 active slots): {timed * 1e6:.0f} us/step, "
          f"{SLOTS / timed:.0f} tokens/s", flush=True)

    counters = dev["counters"].download(np.uint32, 4)
    assert counters.tolist() == [REQ, REQ, 1, 0], counters
    assert len(dones) == REQ and sorted(d[0] for d in dones) == list(range(REQ))
    assert all(d[2] == GEN and d[4] == 0 and d[1] < SLOTS for d in dones)
    state = dev["state"].download(np.uint8, 18464)
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

    assert L.hw_ring_load_acquire(rr) == REQ + 1 and L.hw_ring_load_acquire(rr + 64) == REQ + 1
    assert L.hw_ring_load_acquire(dr) == REQ and L.hw_ring_load_acquire(dr + 64) == REQ
    for b in branch_ids:
        assert L.kv_branch_free(ptab, b) == 0
    assert all(L.kv_prefix_get(ptab, g).contents.refcnt == 1 for g in range(GROUPS))

    for b in list(dev.values()) + [attn_ws, samp_ws, ntok, rew2, adv]:
        b.close()
    L.req_ring_destroy(rr)
    L.done_ring_destroy(dr)
