"""The batched decode step driven through the hw_desc rings
(rl_hip_ring_step_enqueue): descriptors in through infer_submit_decode, one
decode step over all compute units per batch, completions out on the done
ring, checked against the CPU path.

1. The benchmark's shape: 64 rollouts, GQA 32/8, d128, bf16, ctx U[512,
   4096], sampling of 128,256 logits (T 0.8, top-k 50, top-p 0.9, Philox key
   = the rollout's seed, counter = seq_len), one token per descriptor,
   submitted in a shuffled rollout order. Completions byte-identical to
   hw_worker_sim_run fed the same submissions; every row's attention bit-equal
   to rl_hip_decode_sample_step launched on the same rows (the same fused
   launch: the split depends only on the contexts and the sampled rows'
   shape) and within 1e-4 of fp64;
   tokens bit-exact and logprobs within 1e-4 against the oracle; the arena
   after the step byte-equal to the oracle's append.
2. The control rule over many steps with 8 rows for 13 descriptors:
   multi-token descriptors (DONE at max_tokens, NEEDS_REWARD at a multiple of
   32), a passthrough (seq_len == max_tokens), a dropped non-DECODE opcode,
   rows refilled as they free, then STOP. Each rollout's completion equals the
   simulator's; for every step, every row that decoded (by the recorded row
   map) is checked against the oracle with the rollout's context at that
   step, and the final arena against the oracle's replay of every append.
3. The exit paths of admission, each a bounded wait: an idle limit (status
   1), a rollout id past the table (2), the host's stop flag (4), and a full
   completion ring (3), where the finished descriptor stays in its row and a
   later call pushes it once the host has made room."""
import ctypes as C

import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu

QH, KVH, D, TPB = 32, 8, 128, 16


def _sim(rl, submitted):
    """hw_worker_sim_run over the submissions, then STOP: completions in order."""
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
        return out, (sim.decoded_tokens, sim.completions)
    finally:
        L.hw_ring_destroy(cq)
        L.hw_ring_destroy(dq)


def _as_submitted(rl, calls):
    """The descriptors infer_submit_decode writes for (rollout, seq, max) calls."""
    L = rl.lib()
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    bell = (C.c_uint32 * 16)()
    ctx = rl.InferHwCtx(cmdq=cq, doneq=dq, doorbell=C.addressof(bell), gpu_group_id=0, kv_arena_id=0)
    out = []
    try:
        for r, s, m in calls:
            assert L.infer_submit_decode(C.byref(ctx), r, 0, 0, 0, s, m) == 0
            out.append(rl.hw_ring_pop(cq))
    finally:
        L.hw_ring_destroy(cq)
        L.hw_ring_destroy(dq)
    return out


def _launched_fused(rl, w, logits, max_ctx):
    """rl_hip_decode_sample_step (no append) on a gathered batch with the
    step's logits shape: the attention outputs (bf16 bits, fp32)."""
    layout = rl.KvLayoutDesc.paged(w.token_count, w.head_dim)
    n = w.batch * w.q_heads * w.head_dim
    bufs = [rl.DeviceBuffer.from_array(x) for x in (w.arena, w.table, w.ctx, w.q, logits)]
    out, out32 = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4)
    tok, lp = rl.DeviceBuffer(w.batch * 4), rl.DeviceBuffer(w.batch * 4)
    a = rl.attn_args(bufs[0], layout, bufs[1], w.table_stride, w.batch, w.q_heads, w.kv_heads, rl.DTYPE_BF16,
                     bufs[2], max_ctx, bufs[3], out, out32)
    rows, V = logits.shape
    s = rl.sample_args(bufs[4], rows, V, V, tok, lp, temperature=0.8, top_k=50, top_p=0.9)
    ws = rl.decode_sample_step_workspace(a, s)
    rl.decode_sample_step(a, None, s, ws)
    rl.sync()
    sh = (w.batch, w.q_heads, w.head_dim)
    res = out.download(np.uint16, sh), out32.download(np.float32, sh)
    for b in bufs + [out, out32, tok, lp, ws]:
        b.close()
    return res


def test_ring_step_batch64(rl, gpu, orc, olib):
    import ringstep

    B, V = 64, 128256
    rng = np.random.default_rng(5150)
    w = synth.make_decode(5151, B, QH, KVH, D, 512, 4096, max_ctx=4096)
    arena = rl.Arena(w.arena.nbytes, w.block_bytes)
    n_blocks = w.arena.nbytes // w.block_bytes
    assert np.array_equal(arena.acquire_n(n_blocks), np.arange(n_blocks))
    arena.upload(w.arena)
    seeds = rng.integers(0, 2**63, B, dtype=np.uint64)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, 4096, B, V, output_slots=2,
                               temperature=0.8, top_k=50, top_p=0.9, seeds=seeds)
    perm = rng.permutation(B)                          # row i decodes rollout perm[i]
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    logits = synth.make_logits(5152, B, V, spikes=5)
    run.set_inputs(0, q, kn, vn, logits)
    calls = [(int(r), int(w.ctx[r]), int(w.ctx[r]) + 1) for r in perm]
    for r, s, m in calls:
        run.submit_decode(r, s, m)
    run.push(rl.HwDesc(opcode=255))
    print("[ring] enqueueing two ring steps (64 descriptors, then STOP)", flush=True)
    run.enqueue(2)
    rl.sync()
    got = run.completions()
    sim, counts = _sim(rl, _as_submitted(rl, calls))
    assert got == sim and counts == (B, B)
    assert run.stats() == [B, B, 1, 4]
    o = run.outputs(0)
    assert np.array_equal(o["rows"], perm.astype(np.uint32))

    # the launched path on the same rows: bit-equal attention
    ref_arena = w.arena.copy()
    wb = synth.DecodeWorkload(B, QH, KVH, D, "bf16", TPB, w.ctx[perm].copy(), np.ascontiguousarray(w.table[perm]),
                              w.arena, q, 0)
    o16, o32 = _launched_fused(rl, wb, logits, 4096)
    assert np.array_equal(o["out"], o16) and np.array_equal(o["out32"], o32)
    gh.check_attn(o["out"], o["out32"], orc.attn_f64(olib, wb, 0), "bf16")
    # tokens and logprobs
    lp = C.c_double()
    for i in range(B):
        r = int(perm[i])
        want = olib.orc_sample_row(logits[i].ctypes.data, V, 0, 0.8, 50, 0.9, int(seeds[r]), int(w.ctx[r]), r,
                                   C.byref(lp))
        assert o["tok"][i] == want, (i, o["tok"][i], want)
        assert abs(o["lp"][i] - lp.value) < 1e-4, i
    # the arena: one appended token per (rollout, kv head) at position seq_len
    olib.orc_kv_append(ref_arena.ctypes.data, w.block_bytes, TPB, D * 2, wb.table.ctypes.data, w.table_stride, B, KVH,
                       wb.ctx.ctypes.data, None, kn.ctypes.data, vn.ctypes.data)
    assert np.array_equal(arena.download(np.uint8, arena.nbytes), ref_arena)
    run.close()
    arena.close()


def test_ring_step_control_rule_over_steps(rl, gpu, orc, olib):
    import ringstep

    B, R, V, STEPS = 8, 13, 1024, 12
    rng = np.random.default_rng(6160)
    seq0 = rng.integers(20, 300, R).astype(np.int64)
    seq0[1] = 30
    w = synth.make_decode(6161, R, QH, KVH, D, 0, 0, ctx=seq0.astype(np.uint32), reserve_tokens=int(seq0.max()) + 16)
    arena = rl.DeviceBuffer.from_array(w.arena)
    seeds = rng.integers(0, 2**63, R, dtype=np.uint64)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(seq0.max()) + 16, B, V,
                               input_slots=STEPS, output_slots=STEPS, temperature=1.0, top_k=20, top_p=0.8,
                               seeds=seeds)
    q = synth.f32_to_bf16(rng.standard_normal((STEPS, B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((STEPS, B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((STEPS, B, KVH, D), dtype=np.float32))
    logits = rng.standard_normal((STEPS, B, V), dtype=np.float32)
    for s in range(STEPS):
        run.set_inputs(s, q[s], kn[s], vn[s], logits[s])
    # rollout 0: 3 tokens; 1: NEEDS_REWARD at 32 after 2; 2: passthrough; then a
    # dropped REWARD descriptor; the rest 1-4 tokens each
    max_tok = seq0 + rng.integers(1, 5, R)
    max_tok[0], max_tok[1], max_tok[2] = seq0[0] + 3, 40, seq0[2]
    order = [0, 1, 2, None] + list(range(3, R))
    calls = []
    for r in order:
        if r is None:
            run.push(rl.HwDesc(opcode=2, rollout_id=99))
            continue
        run.submit_decode(r, int(seq0[r]), int(max_tok[r]))
        calls.append((r, int(seq0[r]), int(max_tok[r])))
    run.push(rl.HwDesc(opcode=255))
    print(f"[ring] enqueueing {STEPS} ring steps over {B} rows", flush=True)
    run.enqueue(STEPS)
    rl.sync()
    got = run.completions()
    sim, (sim_dec, sim_comp) = _sim(rl, _as_submitted(rl, calls))
    by_rollout = {rl.HwDesc.from_buffer_copy(b).rollout_id: b for b in got}
    assert len(got) == len(sim) == R and by_rollout == {rl.HwDesc.from_buffer_copy(b).rollout_id: b for b in sim}
    st = run.stats()
    assert st[0] == sim_dec and st[1] == sim_comp and st[3] == 4, (st, sim_dec, sim_comp)

    # every decoded row of every step against the oracle, replaying the appends
    cur = seq0.copy()
    host = w.arena.copy()
    lp = C.c_double()
    decoded = 0
    for s in range(STEPS):
        o = run.outputs(s)
        rows = [i for i in range(B) if o["rows"][i] != 0xFFFFFFFF]
        if not rows:
            continue
        rs = [int(o["rows"][i]) for i in rows]
        ctx = cur[rs].astype(np.uint32)
        wb = synth.DecodeWorkload(len(rows), QH, KVH, D, "bf16", TPB, ctx, np.ascontiguousarray(w.table[rs]), host,
                                  np.ascontiguousarray(q[s][rows]), 0)
        gh.check_attn(o["out"][rows], o["out32"][rows], orc.attn_f64(olib, wb, 0), "bf16")
        for j, i in enumerate(rows):
            want = olib.orc_sample_row(logits[s][i].ctypes.data, V, 0, 1.0, 20, 0.8, int(seeds[rs[j]]), int(ctx[j]),
                                       rs[j], C.byref(lp))
            assert o["tok"][i] == want, (s, i)
            assert abs(o["lp"][i] - lp.value) < 1e-4, (s, i)
        k_rows, v_rows = np.ascontiguousarray(kn[s][rows]), np.ascontiguousarray(vn[s][rows])  # alive across the call
        olib.orc_kv_append(host.ctypes.data, w.block_bytes, TPB, D * 2, wb.table.ctypes.data, w.table_stride,
                           len(rows), KVH, ctx.ctypes.data, None, k_rows.ctypes.data, v_rows.ctypes.data)
        cur[rs] += 1
        decoded += len(rows)
    assert decoded == sim_dec
    for r in range(R):
        d = rl.HwDesc.from_buffer_copy(by_rollout[r])
        assert cur[r] == d.seq_len, r
    assert np.array_equal(arena.download(np.uint8, arena.nbytes), host)
    run.close()
    arena.close()


def test_ring_step_draw_follows_rollout(rl, gpu, orc, olib):
    """The Philox counter of a decoded token is (seq_len, rollout): the same
    descriptors submitted in two different orders land in different batch
    rows, and every rollout still draws the same token. All rows see the same
    logits, so only the draw could tell the rows apart."""
    import ringstep

    B, V = 16, 4096
    rng = np.random.default_rng(7170)
    w = synth.make_decode(7171, B, QH, KVH, D, 40, 300)
    seeds = rng.integers(0, 2**63, B, dtype=np.uint64)
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    logits = np.repeat(rng.standard_normal((1, V), dtype=np.float32) * np.float32(0.5), B, axis=0)
    tok_of = []
    for order in (np.arange(B), rng.permutation(B)):
        arena = rl.DeviceBuffer.from_array(w.arena)
        run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()) + 1, B, V,
                                   output_slots=2, temperature=1.0, top_k=200, top_p=0.95, seeds=seeds)
        run.set_inputs(0, q, kn, vn, logits)
        for r in order:
            run.submit_decode(int(r), int(w.ctx[r]), int(w.ctx[r]) + 1)
        run.push(rl.HwDesc(opcode=255))
        print(f"[ring] one step, rollouts admitted in order {order.tolist()}", flush=True)
        run.enqueue(2)
        rl.sync()
        o = run.outputs(0)
        assert np.array_equal(o["rows"], order.astype(np.uint32))
        t = np.zeros(B, dtype=np.uint32)
        t[o["rows"]] = o["tok"]
        tok_of.append(t)
        run.close()
        arena.close()
    assert np.array_equal(tok_of[0], tok_of[1])
    lp = C.c_double()
    want = [olib.orc_sample_row(logits[0].ctypes.data, V, 0, 1.0, 200, 0.95, int(seeds[r]), int(w.ctx[r]), r,
                                C.byref(lp)) for r in range(B)]
    assert tok_of[0].tolist() == want
    assert len(set(want)) > 1  # the rollouts' draws differ, so a row-keyed draw would show


def test_ring_step_exit_paths(rl, gpu):
    """Each end of admission is a bounded wait that leaves its status: no
    descriptor within max_idle_polls (1), a rollout id past the block table
    (2, nothing decoded), the host's stop flag (4), and a completion ring the
    host keeps full (3): the finished descriptor then stays in its row, and
    the next call pushes it, unchanged, once the host has made room."""
    import ringstep

    B, V = 4, 4096
    rng = np.random.default_rng(7180)
    w = synth.make_decode(7181, B, QH, KVH, D, 40, 300)
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    logits = rng.standard_normal((B, V), dtype=np.float32)

    def run_of(arena):
        r = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()) + 1, B, V,
                                 greedy=True, max_idle_polls=2000)
        r.set_inputs(0, q, kn, vn, logits)
        return r

    arena = rl.DeviceBuffer.from_array(w.arena)
    for case in ("idle", "bad_id", "stop"):
        run = run_of(arena)
        if case == "bad_id":
            run.submit_decode(B + 3, 10, 11)
        if case == "stop":
            run.stop()
        print(f"[ring] exit path: {case}", flush=True)
        run.enqueue(1)
        rl.sync()
        st = run.stats()
        assert st == [0, 0, 0, {"idle": 1, "bad_id": 2, "stop": 4}[case]], (case, st)
        assert run.completions() == []
        run.close()

    # a full completion ring: the host fills it with 65,536 entries of its own
    run = run_of(arena)
    L = rl.lib()
    filler = rl.HwDesc(opcode=7)
    for _ in range(65536):
        assert rl.hw_ring_push(run.dq, filler) == 0
    r0 = 1
    run.submit_decode(r0, int(w.ctx[r0]), int(w.ctx[r0]) + 1)
    print("[ring] exit path: completion ring full", flush=True)
    run.enqueue(1)
    rl.sync()
    assert run.stats() == [1, 0, 1, 3]
    assert L.hw_ring_load_acquire(run.dq + 64) == 65536   # nothing pushed
    got = run.completions()                                # the host drains its entries
    assert len(got) == 65536 and all(g == bytes(filler) for g in got)
    run.enqueue(1)                                         # admission stays closed; the row is pushed
    rl.sync()
    got = run.completions()
    assert len(got) == 1
    d = rl.HwDesc.from_buffer_copy(got[0])
    assert (d.rollout_id, d.seq_len, d.max_tokens) == (r0, int(w.ctx[r0]) + 1, int(w.ctx[r0]) + 1)
    assert d.flags & 2 and d.opcode == 1                   # DONE (rule of src/hw_worker_sim.c:23-59)
    st = run.stats()
    assert st[0] == 1 and st[1] == 1 and st[3] == 3, st
    run.close()
    arena.close()
