"""The persistent worker on the hw_desc rings (plumbing decode, MHA d64 fp16).

One rollout, 8 heads x d64 fp16 K/V ~N(0, 0.5^2) in 16-token blocks, KV
length 256 at the start. 100 decode steps go through infer_submit_decode
(seq_len 256 + i, max_tokens 257 + i) into the command ring, the gfx950 worker
runs each one (attention, greedy token over 32,000 fp32 logits ~N(0, 2^2),
KV append) and publishes the descriptor on the completion ring.

Checked against the CPU path on the same inputs:
  * completion descriptors and final ring indices byte-identical to
    hw_worker_sim_run fed the same submissions (reference
    src/hw_worker_sim.c:23-59);
  * tokens bit-exact (lowest-index argmax), logprobs within 1e-4 of fp64;
  * every step's attention within 1e-4 row-normalised of the fp64 oracle over
    the arena as it stands after the earlier appends;
  * the arena after 100 appends byte-identical to the host-side appends.
"""
import ctypes as C
import time

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

STEPS = 100
CTX0 = 256
VOCAB = 32000


def _alloc_coherent(rl, n):
    p = rl.lib().rl_hip_host_alloc_coherent(n)
    assert p, rl._err()
    C.memset(p, 0, n)
    return p


def _sim_completions(rl, submitted):
    """hw_worker_sim_run over the same submissions, then STOP."""
    L = rl.lib()
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    stop = C.c_uint32(0)
    try:
        for d in submitted:
            assert rl.hw_ring_push(cq, d) == 0
        assert rl.hw_ring_push(cq, rl.HwDesc(opcode=255)) == 0
        sim = rl.HwWorkerSim(cmdq=cq, doneq=dq, stop=C.addressof(stop))
        L.hw_worker_sim_run(C.byref(sim))
        out = []
        while (d := rl.hw_ring_pop(dq)) is not None:
            out.append(bytes(d))
        return out, rl.hw_ring_indices(cq), rl.hw_ring_indices(dq), (sim.decoded_tokens, sim.completions)
    finally:
        L.hw_ring_destroy(cq)
        L.hw_ring_destroy(dq)


def _append_host(w, pos, k, v):
    """Writes token `pos` of every kv head of rollout 0 into the host arena."""
    tc, d = w.token_count, w.head_dim
    rb = 2 * d
    for h in range(w.kv_heads):
        blk = int(w.table[0, h, pos // tc])
        base = blk * w.block_bytes + (pos % tc) * rb
        w.arena[base:base + rb] = k[h].view(np.uint8)
        w.arena[base + tc * rb:base + tc * rb + rb] = v[h].view(np.uint8)


def test_plumbing_decode_through_rings(rl, gpu, orc, olib):
    L = rl.lib()
    rng = np.random.default_rng(1001)
    w = synth.make_decode(1000, 1, 8, 8, 64, CTX0, CTX0, dtype="fp16", kv_std=0.5,
                          reserve_tokens=CTX0 + STEPS + 1)
    host_arena0 = w.arena.copy()
    q_all = synth.f32_to_f16(rng.standard_normal((STEPS, 8, 64), dtype=np.float32))
    k_all = synth.f32_to_f16(rng.standard_normal((STEPS, 8, 64), dtype=np.float32) * np.float32(0.5))
    v_all = synth.f32_to_f16(rng.standard_normal((STEPS, 8, 64), dtype=np.float32) * np.float32(0.5))
    logits = (rng.standard_normal((STEPS, VOCAB), dtype=np.float32) * np.float32(2.0))

    layout = rl.KvLayoutDesc.paged(16, 64)
    bufs = {n: rl.DeviceBuffer.from_array(a) for n, a in
            (("arena", w.arena), ("table", w.table), ("q", q_all), ("k", k_all), ("v", v_all),
             ("logits", logits))}
    attn_out = rl.DeviceBuffer(STEPS * 8 * 64 * 4, zero=True)
    tok = rl.DeviceBuffer(STEPS * 4, zero=True)
    lp = rl.DeviceBuffer(STEPS * 4, zero=True)
    stats = rl.DeviceBuffer(4 * 8, zero=True)
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    assert L.rl_hip_is_coherent_host(cq) and L.rl_hip_is_coherent_host(dq)
    rings = _alloc_coherent(rl, 16)
    C.cast(rings, C.POINTER(C.c_void_p))[0] = cq
    C.cast(rings, C.POINTER(C.c_void_p))[1] = dq
    stop = _alloc_coherent(rl, 64)
    doorbell = _alloc_coherent(rl, 64)

    a = rl.HwWorkerArgs(cmdq=rings, doneq=rings + 8, groups=1, stop=stop, max_idle_polls=1 << 22,
                        arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes, layout=layout,
                        block_table=bufs["table"].ptr, table_stride=w.table_stride, rollouts=1, q_heads=8,
                        kv_heads=8, dtype=rl.DTYPE_FP16, scale=0.0, max_steps=STEPS, q=bufs["q"].ptr,
                        k_new=bufs["k"].ptr, v_new=bufs["v"].ptr, logits=bufs["logits"].ptr, vocab=VOCAB,
                        attn_out=attn_out.ptr, token_out=tok.ptr, logprob_out=lp.ptr, stats=stats.ptr)
    ws = rl.hw_worker_workspace(a)
    ctx = rl.InferHwCtx(cmdq=cq, doneq=dq, doorbell=doorbell, gpu_group_id=7, kv_arena_id=42)
    submitted, got = [], []
    print("[worker] launching persistent worker, 1 group", flush=True)
    rl.hw_worker_launch(a)
    try:
        t0 = time.perf_counter()
        for i in range(STEPS):
            assert L.infer_submit_decode(C.byref(ctx), 0, 0x1000 * i, 0x40 * i, 0, CTX0 + i, CTX0 + i + 1) == 0
        deadline = time.perf_counter() + 60.0
        while len(got) < STEPS and time.perf_counter() < deadline:
            d = rl.hw_ring_pop(dq)
            if d is None:
                time.sleep(1e-4)
                continue
            got.append(bytes(d))
        elapsed = time.perf_counter() - t0
        assert rl.hw_ring_push(cq, rl.HwDesc(opcode=255)) == 0
        print(f"[worker] {len(got)} completions in {elapsed * 1e3:.1f} ms "
              f"({len(got) / max(elapsed, 1e-9):.0f} steps/s submitted back-to-back)", flush=True)
    finally:
        # every exit path ends the worker before synchronising
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rl.sync()
    st = stats.download(np.uint64, 4)
    assert len(got) == STEPS, (len(got), st)
    assert st.tolist() == [STEPS, STEPS, STEPS, 0], st

    # the submitted descriptors, as the CPU simulator sees them
    cq2 = L.hw_ring_create()
    try:
        ctx2 = rl.InferHwCtx(cmdq=cq2, doneq=dq, doorbell=doorbell, gpu_group_id=7, kv_arena_id=42)
        for i in range(STEPS):
            assert L.infer_submit_decode(C.byref(ctx2), 0, 0x1000 * i, 0x40 * i, 0, CTX0 + i, CTX0 + i + 1) == 0
            submitted.append(rl.hw_ring_pop(cq2))
    finally:
        L.hw_ring_destroy(cq2)
    sim_out, sim_cq, sim_dq, sim_counts = _sim_completions(rl, submitted)
    assert got == sim_out
    assert rl.hw_ring_indices(cq) == sim_cq == (STEPS + 1, STEPS + 1)
    assert rl.hw_ring_indices(dq) == sim_dq == (STEPS, STEPS)
    assert sim_counts == (STEPS, STEPS)

    # tokens and logprobs
    gt = tok.download(np.uint32, STEPS)
    glp = lp.download(np.float32, STEPS)
    ot, olp = orc.sample_rows(olib, logits, True, 1.0, 0, 1.0, 0, 0)
    assert np.array_equal(gt, ot)
    assert np.array_equal(gt, np.argmax(logits, axis=1).astype(np.uint32))
    assert np.abs(glp - olp).max() < 1e-4

    # attention of every step over the arena as the earlier appends left it
    gout = attn_out.download(np.float32, (STEPS, 8, 64))
    w.arena[:] = host_arena0
    worst = 0.0
    for i in range(STEPS):
        w.ctx = np.array([CTX0 + i], dtype=np.uint32)
        w.q = q_all[i].reshape(1, 8, 64)
        ref = orc.attn_f64(olib, w, 1)[0]
        err = (np.abs(gout[i] - ref).max(axis=-1) / np.abs(ref).max(axis=-1)).max()
        worst = max(worst, float(err))
        _append_host(w, CTX0 + i, k_all[i], v_all[i])
    assert worst < 1e-4, worst
    assert np.array_equal(bufs["arena"].download(np.uint8, w.arena.size), w.arena)

    for b in list(bufs.values()) + [attn_out, tok, lp, stats, ws]:
        b.close()
    L.hw_ring_destroy(cq)
    L.hw_ring_destroy(dq)
    for p in (rings, stop, doorbell):
        L.rl_hip_host_free(p)


def test_worker_exits_on_idle_limit(rl, gpu):
    """No submissions and no stop: the worker gives up after max_idle_polls
    empty polls and reports status 1 (the host never has to rescue it)."""
    L = rl.lib()
    w = synth.make_decode(7, 1, 8, 8, 64, 16, 16, dtype="fp16")
    layout = rl.KvLayoutDesc.paged(16, 64)
    arena, table = rl.DeviceBuffer.from_array(w.arena), rl.DeviceBuffer.from_array(w.table)
    scratch = rl.DeviceBuffer(1 << 20, zero=True)
    stats = rl.DeviceBuffer(4 * 8, zero=True)
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    rings = _alloc_coherent(rl, 16)
    C.cast(rings, C.POINTER(C.c_void_p))[0] = cq
    C.cast(rings, C.POINTER(C.c_void_p))[1] = dq
    stop = _alloc_coherent(rl, 64)
    a = rl.HwWorkerArgs(cmdq=rings, doneq=rings + 8, groups=1, stop=stop, max_idle_polls=2000,
                        arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=layout, block_table=table.ptr,
                        table_stride=w.table_stride, rollouts=1, q_heads=8, kv_heads=8, dtype=rl.DTYPE_FP16,
                        max_steps=1, q=scratch.ptr, k_new=scratch.ptr, v_new=scratch.ptr, logits=scratch.ptr,
                        vocab=16, attn_out=scratch.ptr, token_out=scratch.ptr, logprob_out=scratch.ptr,
                        stats=stats.ptr)
    ws = rl.hw_worker_workspace(a)
    print("[worker] launching an idle worker (max_idle_polls 2000)", flush=True)
    rl.hw_worker_launch(a)
    rl.sync()  # returns once the worker gave up on its own
    st = stats.download(np.uint64, 4)
    assert st.tolist() == [0, 0, 0, 1], st
    for b in (arena, table, scratch, stats, ws):
        b.close()
    L.hw_ring_destroy(cq)
    L.hw_ring_destroy(dq)
    L.rl_hip_host_free(rings)
    L.rl_hip_host_free(stop)


def _pairs_run(rl, gpu, orc, olib, *, seed, S, q_heads, kv_heads, head_dim, dtype, tc, ctx_lo, ctx_hi, kv_std,
               vocab=VOCAB):
    """One persistent worker per compute unit (256 on MI355X), each the single
    consumer / producer of its own ring pair and its own rollout, rollout g
    starting at KV length ctx_g ~ U[ctx_lo, ctx_hi]: S decode steps per pair
    through infer_submit_decode (seq_len ctx_g + i, max_tokens ctx_g + i + 1),
    submitted while the workers poll. Per pair: the completions and ring
    indices byte-identical to hw_worker_sim_run fed the same submissions, and
    the counters; over all pairs: tokens bit-exact, logprobs within 1e-4,
    every step's attention within 1e-4 of fp64 over the arena as the earlier
    appends left it, and the final arena byte-identical to the host appends."""
    L = rl.lib()
    G = int(gpu.cu_count)
    code = rl.DTYPE_BF16 if dtype == "bf16" else rl.DTYPE_FP16
    rng = np.random.default_rng(seed + 1)
    ctx0 = np.random.default_rng(seed + 2).integers(ctx_lo, ctx_hi + 1, size=G).astype(np.uint32)
    # every row owns blocks for ctx0 + S + 1 tokens: the S appended slots are in its table
    w = synth.make_decode(seed, G, q_heads, kv_heads, head_dim, 0, 0, dtype=dtype, kv_std=kv_std, token_count=tc,
                          ctx=ctx0 + S)
    host_arena0 = w.arena.copy()
    q_all = synth.to_scalar16(rng.standard_normal((G, S, q_heads, head_dim), dtype=np.float32), dtype)
    k_all = synth.to_scalar16(rng.standard_normal((G, S, kv_heads, head_dim), dtype=np.float32)
                              * np.float32(kv_std), dtype)
    v_all = synth.to_scalar16(rng.standard_normal((G, S, kv_heads, head_dim), dtype=np.float32)
                              * np.float32(kv_std), dtype)
    logits = rng.standard_normal((G, S, vocab), dtype=np.float32) * np.float32(2.0)
    layout = rl.KvLayoutDesc.paged(tc, head_dim)
    bufs = {n: rl.DeviceBuffer.from_array(a) for n, a in
            (("arena", w.arena), ("table", w.table), ("q", q_all), ("k", k_all), ("v", v_all), ("logits", logits))}
    attn_out = rl.DeviceBuffer(G * S * q_heads * head_dim * 4, zero=True)
    tok = rl.DeviceBuffer(G * S * 4, zero=True)
    lp = rl.DeviceBuffer(G * S * 4, zero=True)
    stats = rl.DeviceBuffer(G * 4 * 8, zero=True)
    cqs = [L.hw_ring_create() for _ in range(G)]
    dqs = [L.hw_ring_create() for _ in range(G)]
    assert all(cqs) and all(dqs)
    rings = _alloc_coherent(rl, 16 * G)
    for g in range(G):
        C.cast(rings, C.POINTER(C.c_void_p))[g] = cqs[g]
        C.cast(rings, C.POINTER(C.c_void_p))[G + g] = dqs[g]
    stop = _alloc_coherent(rl, 64)
    doorbells = _alloc_coherent(rl, 64 * G)
    a = rl.HwWorkerArgs(cmdq=rings, doneq=rings + 8 * G, groups=G, stop=stop, max_idle_polls=1 << 22,
                        arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes, layout=layout,
                        block_table=bufs["table"].ptr, table_stride=w.table_stride, rollouts=G, q_heads=q_heads,
                        kv_heads=kv_heads, dtype=code, scale=0.0, max_steps=S, q=bufs["q"].ptr,
                        k_new=bufs["k"].ptr, v_new=bufs["v"].ptr, logits=bufs["logits"].ptr, vocab=vocab,
                        attn_out=attn_out.ptr, token_out=tok.ptr, logprob_out=lp.ptr, stats=stats.ptr)
    ws = rl.hw_worker_workspace(a)
    ctxs = [rl.InferHwCtx(cmdq=cqs[g], doneq=dqs[g], doorbell=doorbells + 64 * g, gpu_group_id=g, kv_arena_id=42)
            for g in range(G)]

    def submit(c, g, i):
        return L.infer_submit_decode(C.byref(c), g, 0x1000 * i, 0x40 * i, 0, int(ctx0[g]) + i, int(ctx0[g]) + i + 1)

    got = [[] for _ in range(G)]
    print(f"[worker] launching {G} persistent workers, one per compute unit: {q_heads}/{kv_heads} heads, "
          f"d{head_dim} {dtype}, {tc}-token blocks, ctx U[{ctx_lo}, {ctx_hi}], {S} steps each", flush=True)
    rl.hw_worker_launch(a)
    try:
        t0 = time.perf_counter()
        for i in range(S):
            for g in range(G):
                assert submit(ctxs[g], g, i) == 0
        deadline = time.perf_counter() + 60.0
        n = 0
        while n < G * S and time.perf_counter() < deadline:
            for g in range(G):
                while (d := rl.hw_ring_pop(dqs[g])) is not None:
                    got[g].append(bytes(d))
                    n += 1
        elapsed = time.perf_counter() - t0
        for g in range(G):
            assert rl.hw_ring_push(cqs[g], rl.HwDesc(opcode=255)) == 0
        print(f"[worker] {n} completions from {G} pairs in {elapsed * 1e3:.1f} ms", flush=True)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rl.sync()
    st = stats.download(np.uint64, (G, 4))
    assert all(len(x) == S for x in got), [len(x) for x in got]
    assert (st == np.array([S, S, S, 0], np.uint64)).all(), st

    # every pair against the CPU simulator fed the same submissions
    for g in range(G):
        cq2 = L.hw_ring_create()
        sub = []
        try:
            c2 = rl.InferHwCtx(cmdq=cq2, doneq=dqs[g], doorbell=doorbells + 64 * g, gpu_group_id=g, kv_arena_id=42)
            for i in range(S):
                assert submit(c2, g, i) == 0
                sub.append(rl.hw_ring_pop(cq2))
        finally:
            L.hw_ring_destroy(cq2)
        sim_out, sim_cq, sim_dq, sim_counts = _sim_completions(rl, sub)
        assert got[g] == sim_out, g
        assert rl.hw_ring_indices(cqs[g]) == sim_cq == (S + 1, S + 1), g
        assert rl.hw_ring_indices(dqs[g]) == sim_dq == (S, S), g
        assert sim_counts == (S, S)

    gt = tok.download(np.uint32, (G, S))
    glp = lp.download(np.float32, (G, S))
    ot, olp = orc.sample_rows(olib, logits.reshape(G * S, vocab), True, 1.0, 0, 1.0, 0, 0)
    assert np.array_equal(gt.ravel(), ot)
    assert np.abs(glp.ravel() - olp).max() < 1e-4

    gout = attn_out.download(np.float32, (G, S, q_heads, head_dim))
    w.arena[:] = host_arena0
    worst = 0.0
    rb = 2 * head_dim
    for i in range(S):
        w.ctx = ctx0 + np.uint32(i)
        w.q = np.ascontiguousarray(q_all[:, i])
        ref = orc.attn_f64(olib, w, code)
        worst = max(worst, float((np.abs(gout[:, i] - ref).max(axis=-1) / np.abs(ref).max(axis=-1)).max()))
        for g in range(G):
            pos = int(ctx0[g]) + i
            for h in range(kv_heads):
                blk = int(w.table[g, h, pos // tc])
                base = blk * w.block_bytes + (pos % tc) * rb
                w.arena[base:base + rb] = k_all[g, i, h].view(np.uint8)
                w.arena[base + tc * rb:base + tc * rb + rb] = v_all[g, i, h].view(np.uint8)
    assert worst < 1e-4, worst
    assert np.array_equal(bufs["arena"].download(np.uint8, w.arena.size), w.arena)

    for b in list(bufs.values()) + [attn_out, tok, lp, stats, ws]:
        b.close()
    for q in cqs + dqs:
        L.hw_ring_destroy(q)
    for p in (rings, stop, doorbells):
        L.rl_hip_host_free(p)


def test_plumbing_one_worker_per_cu(rl, gpu, orc, olib):
    """The plumbing rollout shape (MHA 8 x d64 fp16, KV length 256) on one
    worker per compute unit, 8 steps per pair."""
    _pairs_run(rl, gpu, orc, olib, seed=1002, S=8, q_heads=8, kv_heads=8, head_dim=64, dtype="fp16", tc=16,
               ctx_lo=CTX0, ctx_hi=CTX0, kv_std=0.5)


# The worker's other instantiations at one worker per compute unit:
#  - the batched-decode rollout shape: GQA 32/8 (group 4), d128 bf16, ctx U[512, 4096], 16-token blocks;
#  - group 8 at d128 (GQA 64/8, the long-context head shape): four waves with up to four tile stages;
#  - 32-token blocks (GQA 16/8 d64 fp16, group 2) and a d128 fp16 MHA case.
@pytest.mark.parametrize("shape", [
    dict(seed=2101, S=4, q_heads=32, kv_heads=8, head_dim=128, dtype="bf16", tc=16, ctx_lo=512, ctx_hi=4096, kv_std=1.0),
    dict(seed=2102, S=4, q_heads=64, kv_heads=8, head_dim=128, dtype="bf16", tc=16, ctx_lo=512, ctx_hi=2048,
         kv_std=1.0),
    dict(seed=2103, S=6, q_heads=16, kv_heads=8, head_dim=64, dtype="fp16", tc=32, ctx_lo=100, ctx_hi=900, kv_std=0.5),
    dict(seed=2104, S=4, q_heads=8, kv_heads=8, head_dim=128, dtype="fp16", tc=32, ctx_lo=31, ctx_hi=700, kv_std=0.5),
], ids=["gqa4_d128_bf16_tc16", "gqa8_d128_bf16_tc16", "gqa2_d64_fp16_tc32", "mha_d128_fp16_tc32"])
def test_worker_shapes_one_per_cu(rl, gpu, orc, olib, shape):
    _pairs_run(rl, gpu, orc, olib, **shape)


def test_worker_stamps_lockstep(rl, gpu):
    """Four workers with stamps set, 64 descriptors one at a time through
    ring_lockstep_hw (seq_len = max_tokens: no decode step, the completion is
    the descriptor unchanged): every sample arrives with its tag, each
    worker's consume stamp precedes its completion stamp, the stamps of
    successive samples ascend on the device's common clock, and the workers
    end on the stop flag (status 0) with 16 completions each."""
    L = rl.lib()
    pairs, n = 4, 64
    w = synth.make_decode(7, 1, 8, 8, 64, 16, 16, dtype="fp16")
    layout = rl.KvLayoutDesc.paged(16, 64)
    arena, table = rl.DeviceBuffer.from_array(w.arena), rl.DeviceBuffer.from_array(w.table)
    scratch = rl.DeviceBuffer(1 << 20, zero=True)
    stats = rl.DeviceBuffer(pairs * 32, zero=True)
    cqs = [L.hw_ring_create() for _ in range(pairs)]
    dqs = [L.hw_ring_create() for _ in range(pairs)]
    rings = _alloc_coherent(rl, 16 * pairs)
    for g in range(pairs):
        C.cast(rings, C.POINTER(C.c_void_p))[g] = cqs[g]
        C.cast(rings, C.POINTER(C.c_void_p))[pairs + g] = dqs[g]
    stop, stamps = _alloc_coherent(rl, 64), _alloc_coherent(rl, 16 * pairs)
    a = rl.HwWorkerArgs(cmdq=rings, doneq=rings + 8 * pairs, groups=pairs, stop=stop, max_idle_polls=1 << 24,
                        arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=layout, block_table=table.ptr,
                        table_stride=w.table_stride, rollouts=1, q_heads=8, kv_heads=8, dtype=rl.DTYPE_FP16,
                        max_steps=1, q=scratch.ptr, k_new=scratch.ptr, v_new=scratch.ptr, logits=scratch.ptr,
                        vocab=16, attn_out=scratch.ptr, token_out=scratch.ptr, logprob_out=scratch.ptr,
                        stats=stats.ptr, stamps=stamps)
    ws = rl.hw_worker_workspace(a)
    out = (rl.RingLockstepSample * n)()
    d = rl.HwDesc(opcode=1, rollout_id=0, seq_len=16, max_tokens=16)
    print(f"[worker] {pairs} workers with stamps, {n} lock-step descriptors", flush=True)
    rl.hw_worker_launch(a)
    try:
        got = L.ring_lockstep_hw(rings, rings + 8 * pairs, pairs, C.byref(d), n, stamps, 10**10, out)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rl.sync()
    st = stats.download(np.uint64, (pairs, 4))
    assert got == n
    assert (st[:, 1] == n // pairs).all() and (st[:, 3] == 0).all(), st
    for i, s in enumerate(out):
        assert s.consume_tick <= s.complete_tick and s.submit_ns < s.poll_ns, i
        if i:
            assert out[i - 1].complete_tick <= s.consume_tick, i
    for b in (arena, table, scratch, stats, ws):
        b.close()
    for r in cqs + dqs:
        L.hw_ring_destroy(r)
    for p in (rings, stop, stamps):
        L.rl_hip_host_free(p)
