"""The self-scheduled ring loop (rl_hip_ring_loop_launch): the ring-driven
batched decode step as one persistent launch, held to the launched pipeline
(rl_hip_ring_step_enqueue), which the ring-step tests pin to the oracle and
to hw_worker_sim_run. Each case runs the same submissions through both on
copies of the same arena and compares what the host can see: completions,
stats, per-step rows, tokens and logprobs (bits) and the final arena are
equal; the attention, which the loop splits over the compute units left
beside its turn and merges (a different split from the launched step's, so
other fp32 roundings), is checked against the oracle's fp64 in both runs,
every decoded row of every step.

1. The control rule over many steps (8 rows, 13 descriptors of 1-8 tokens,
   NEEDS_REWARD at 32, a passthrough, a dropped opcode, STOP): the loop
   ends by itself once admission has ended and every row is free, and the
   launched run's later steps decoded nothing; every decoded row of every
   step against the oracle with the rollout's context at that step. At the
   headline shape and at four more (GQA 1, 2, 4; d64 and d128; fp16 and
   bf16; 16- and 32-token blocks); loops and launched steps alternating
   on one run; and with greedy sampling (tokens the
   first index of each row's maximum, logprobs the fp64 log-softmax).
2. The benchmark's shape (64 rollouts, GQA 32/8, d128, ctx U[512, 4096],
   128,256 logits): max_steps 1, then a second loop that finds only STOP,
   against two launched steps. The control rule at 1,024 rows, the most a
   step takes, with more descriptors than rows.
3. Exit paths: idle limit, bad rollout id, the host's stop flag (zero steps
   run, status 1 / 2 / 4) and a full completion ring (status 3; the finished
   descriptor stays in its row until a later loop pushes it). A lock-step
   host: it submits a batch only after it has seen the previous batch's
   completions, which the loop makes visible before it waits for the host.
4. Arguments the loop does not take: max_steps 0, fewer than three output
   slots (a step's split rows are merged while the next two steps run, so
   three consecutive steps need their own slots) and a GQA group of 8 at d128
   (outside the fused kernel) return errors before any launch."""
import ctypes as C

import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu

QH, KVH, D, TPB = 32, 8, 128, 16


def _outputs(run, steps):
    return [run.outputs(s) for s in range(steps)]


def _same_outputs(a, b, what):
    for k in ("rows", "tok"):
        assert np.array_equal(a[k], b[k]), (what, k)
    assert np.array_equal(a["lp"].view(np.uint32), b["lp"].view(np.uint32)), (what, "lp")


def _control_rule_case(rl, driver, shape=(QH, KVH, D, "bf16", TPB), B=8, R=13, V=1024, STEPS=40, seed=6160,
                       greedy=False):
    """The submissions of the ring-step control-rule test (at the given
    q_heads, kv_heads, head_dim, dtype and block size) on a fresh arena, run
    by driver(run, STEPS); returns what the host sees."""
    import ringstep

    qh, kvh, d, dtype, tc = shape
    code = rl.DTYPE_BF16 if dtype == "bf16" else rl.DTYPE_FP16
    rng = np.random.default_rng(seed)
    seq0 = rng.integers(20, 300, R).astype(np.int64)
    seq0[1] = 30
    w = synth.make_decode(seed + 1, R, qh, kvh, d, 0, 0, dtype=dtype, token_count=tc, ctx=seq0.astype(np.uint32),
                          reserve_tokens=int(seq0.max()) + 16)
    arena = rl.DeviceBuffer.from_array(w.arena)
    seeds = rng.integers(0, 2**63, R, dtype=np.uint64)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(tc, d), w.table, qh, int(seq0.max()) + 16, B, V,
                               input_slots=STEPS, output_slots=STEPS, dtype=code, greedy=greedy, temperature=1.0,
                               top_k=20, top_p=0.8, seeds=seeds)
    q = synth.to_scalar16(rng.standard_normal((STEPS, B, qh, d), dtype=np.float32), dtype)
    kn = synth.to_scalar16(rng.standard_normal((STEPS, B, kvh, d), dtype=np.float32), dtype)
    vn = synth.to_scalar16(rng.standard_normal((STEPS, B, kvh, d), dtype=np.float32), dtype)
    logits = rng.standard_normal((STEPS, B, V), dtype=np.float32)
    for s in range(STEPS):
        run.set_inputs(s, q[s], kn[s], vn[s], logits[s])
    max_tok = seq0 + rng.integers(1, 9, R)
    max_tok[0], max_tok[1], max_tok[2] = seq0[0] + 3, 40, seq0[2]
    for r in [0, 1, 2, None] + list(range(3, R)):
        if r is None:
            run.push(rl.HwDesc(opcode=2, rollout_id=99))
        else:
            run.submit_decode(r, int(seq0[r]), int(max_tok[r]))
    run.push(rl.HwDesc(opcode=255))
    ran = driver(run, STEPS)
    rl.sync()
    res = {"ran": ran, "completions": run.completions(), "stats": run.stats(), "out": _outputs(run, STEPS),
           "arena": arena.download(np.uint8, arena.nbytes), "w": w, "seq0": seq0, "q": q, "kn": kn, "vn": vn,
           "logits": logits}
    run.close()
    arena.close()
    return res


def _enqueue(run, steps):
    run.enqueue(steps)
    return steps


def _loop_against_launched(rl, orc, olib, shape=(QH, KVH, D, "bf16", TPB), B=8, R=13, STEPS=40, seed=6160,
                           greedy=False, driver=None):
    """The control-rule submissions through STEPS launched steps and through
    one loop of up to STEPS steps: the loop ends by itself, and everything but
    the attention's fp32 rounding is the launched run's; both runs' attention,
    step by step, against the oracle's fp64 with the appends replayed."""
    qh, kvh, d, dtype, tc = shape
    print(f"[loop] control rule {qh}/{kvh} d{d} {dtype} tc{tc}: {STEPS} launched steps", flush=True)
    want = _control_rule_case(rl, _enqueue, shape, B, R, STEPS=STEPS, seed=seed, greedy=greedy)
    print(f"[loop] control rule {qh}/{kvh} d{d} {dtype} tc{tc}: one loop of up to {STEPS} steps", flush=True)
    got = _control_rule_case(rl, driver or (lambda run, steps: run.loop(steps)), shape, B, R, STEPS=STEPS,
                             seed=seed, greedy=greedy)
    n = got["ran"]
    assert 0 < n < STEPS, n
    assert got["completions"] == want["completions"] and len(got["completions"]) == R
    assert got["stats"] == want["stats"] and got["stats"][3] == 4, (got["stats"], want["stats"])
    for s in range(n):
        _same_outputs(got["out"][s], want["out"][s], s)
    # the launched run's later steps decoded nothing
    assert any((want["out"][n - 1]["rows"] != 0xFFFFFFFF))
    for s in range(n, STEPS):
        assert (want["out"][s]["rows"] == 0xFFFFFFFF).all(), s
    assert np.array_equal(got["arena"], want["arena"])
    for res in (got, want):
        _attn_against_fp64(orc, olib, res, shape, B, n)
    return got


def _attn_against_fp64(orc, olib, res, shape, B, n):
    """Every decoded row of steps 0 .. n - 1 of a run against the oracle's fp64
    attention over the arena as it stood at that step (the earlier steps'
    appends replayed by the oracle), and the final arena against the replay."""
    qh, kvh, d, dtype, tc = shape
    w, q, kn, vn = res["w"], res["q"], res["kn"], res["vn"]
    cur, host = res["seq0"].copy(), w.arena.copy()
    for s in range(n):
        o = res["out"][s]
        rows = [i for i in range(B) if o["rows"][i] != 0xFFFFFFFF]
        if not rows:
            continue
        rs = [int(o["rows"][i]) for i in rows]
        ctx = cur[rs].astype(np.uint32)
        wb = synth.DecodeWorkload(len(rows), qh, kvh, d, dtype, tc, ctx, np.ascontiguousarray(w.table[rs]), host,
                                  np.ascontiguousarray(q[s][rows]), 0)
        gh.check_attn(o["out"][rows], o["out32"][rows], orc.attn_f64(olib, wb, 0 if dtype == "bf16" else 1), dtype)
        k_rows, v_rows = np.ascontiguousarray(kn[s][rows]), np.ascontiguousarray(vn[s][rows])
        olib.orc_kv_append(host.ctypes.data, w.block_bytes, tc, d * 2, wb.table.ctypes.data, w.table_stride,
                           len(rows), kvh, ctx.ctypes.data, None, k_rows.ctypes.data, v_rows.ctypes.data)
        cur[rs] += 1
    assert np.array_equal(res["arena"], host)


def test_ring_loop_equals_enqueue_control_rule(rl, gpu, orc, olib):
    _loop_against_launched(rl, orc, olib)


@pytest.mark.parametrize("shape", [(16, 8, 64, "fp16", 32), (8, 8, 128, "fp16", 32), (16, 8, 128, "bf16", 16),
                                   (8, 2, 64, "bf16", 16)],
                         ids=["gqa2_d64_fp16_tc32", "mha_d128_fp16_tc32", "gqa2_d128_bf16", "gqa4_d64_bf16_kv2"])
def test_ring_loop_shapes(rl, gpu, orc, olib, shape):
    """The control rule through the loop on the other shapes the fused kernel
    takes: GQA groups 1, 2 and 4, head_dim 64 and 128, fp16 and bf16, 16- and
    32-token blocks (a loop kernel instantiation each)."""
    _loop_against_launched(rl, orc, olib, shape, STEPS=32, seed=6170 + shape[0] + shape[1] + shape[2])


def test_ring_loop_continues_launched_steps(rl, gpu, orc, olib):
    """Calls that share one run's workspace and rings: a loop of 4 steps,
    3 launched steps, then a loop to the end. Each call starts at the step
    after the last one run and publishes its own last step, so the whole
    equals one launched run."""
    def mixed(run, steps):
        a = run.loop(4)
        assert a == 4, a
        run.enqueue(3)
        return 7 + run.loop(steps - 7)

    _loop_against_launched(rl, orc, olib, STEPS=40, seed=6200, driver=mixed)


def test_ring_loop_greedy(rl, gpu, orc, olib):
    """The control rule with greedy sampling (the sampling function's argmax
    path): the loop against the launched run, and every decoded row's token
    the lowest index of its row's maximum (numpy's argmax), its logprob the
    fp64 log-softmax of that maximum within 1e-4."""
    got = _loop_against_launched(rl, orc, olib, STEPS=32, seed=6180, greedy=True)
    checked = 0
    for s in range(got["ran"]):
        o, x = got["out"][s], got["logits"][s].astype(np.float64)
        for i in np.nonzero(o["rows"] != 0xFFFFFFFF)[0]:
            row = x[i]
            assert o["tok"][i] == np.argmax(row), (s, i)
            m = row.max()
            want_lp = -np.log(np.exp(row - m).sum())
            assert abs(float(o["lp"][i]) - want_lp) < 1e-4, (s, i, o["lp"][i], want_lp)
            checked += 1
    assert checked > 0


def _batch64(rl, driver):
    import ringstep

    B, V = 64, 128256
    rng = np.random.default_rng(5150)
    w = synth.make_decode(5151, B, QH, KVH, D, 512, 4096, max_ctx=4096)
    arena = rl.DeviceBuffer.from_array(w.arena)
    seeds = rng.integers(0, 2**63, B, dtype=np.uint64)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, 4096, B, V, output_slots=3,
                               temperature=0.8, top_k=50, top_p=0.9, seeds=seeds)
    perm = rng.permutation(B)
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    run.set_inputs(0, q, kn, vn, synth.make_logits(5152, B, V, spikes=5))
    for r in perm:
        run.submit_decode(int(r), int(w.ctx[r]), int(w.ctx[r]) + 1)
    run.push(rl.HwDesc(opcode=255))
    ran = driver(run)
    rl.sync()
    res = {"ran": ran, "completions": run.completions(), "stats": run.stats(), "out": run.outputs(0),
           "arena": arena.download(np.uint8, arena.nbytes),
           "wb": synth.DecodeWorkload(B, QH, KVH, D, "bf16", TPB, w.ctx[perm].copy(),
                                      np.ascontiguousarray(w.table[perm]), w.arena, q, 0)}
    run.close()
    arena.close()
    return res


def test_ring_loop_batch64(rl, gpu, orc, olib):
    print("[loop] batch 64: two launched steps", flush=True)
    want = _batch64(rl, lambda run: _enqueue(run, 2))
    print("[loop] batch 64: loop of 1 step, then a loop that finds STOP", flush=True)
    got = _batch64(rl, lambda run: (run.loop(1), run.loop(4)))
    assert got["ran"] == (1, 0)
    assert got["completions"] == want["completions"] and len(got["completions"]) == 64
    assert got["stats"] == want["stats"] == [64, 64, 1, 4]
    _same_outputs(got["out"], want["out"], "step 0")
    assert np.array_equal(got["arena"], want["arena"])
    gh.check_attn(got["out"]["out"], got["out"]["out32"], orc.attn_f64(olib, got["wb"], 0), "bf16")


def test_ring_loop_max_batch(rl, gpu, orc, olib):
    """The control rule at the most rows a step takes: 1,024 rows and 1,100
    descriptors (GQA 16/4 d64 bf16), so the last 76 wait for rows that free
    up; the launched pipeline and the loop against each other and the
    loop's attention against fp64 at every step."""
    _loop_against_launched(rl, orc, olib, (16, 4, 64, "bf16", 16), B=1024, R=1100, STEPS=24, seed=6190)


def test_ring_loop_exit_paths(rl, gpu):
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
                                 output_slots=3, greedy=True, max_idle_polls=2000)
        r.set_inputs(0, q, kn, vn, logits)
        return r

    arena = rl.DeviceBuffer.from_array(w.arena)
    for case in ("idle", "bad_id", "stop"):
        run = run_of(arena)
        if case == "bad_id":
            run.submit_decode(B + 3, 10, 11)
        if case == "stop":
            run.stop()
        print(f"[loop] exit path: {case}", flush=True)
        assert run.loop(3) == 0
        st = run.stats()
        assert st == [0, 0, 0, {"idle": 1, "bad_id": 2, "stop": 4}[case]], (case, st)
        assert run.completions() == []
        run.close()

    run = run_of(arena)
    L = rl.lib()
    filler = rl.HwDesc(opcode=7)
    for _ in range(65536):
        assert rl.hw_ring_push(run.dq, filler) == 0
    r0 = 1
    run.submit_decode(r0, int(w.ctx[r0]), int(w.ctx[r0]) + 1)
    print("[loop] exit path: completion ring full", flush=True)
    assert run.loop(1) == 1
    assert run.stats() == [1, 0, 1, 3]
    assert L.hw_ring_load_acquire(run.dq + 64) == 65536
    got = run.completions()
    assert len(got) == 65536 and all(g == bytes(filler) for g in got)
    # the row stays held (a finished descriptor with no room), so the loop
    # does not end early: its last turn pushes the row
    assert run.loop(1) == 1
    got = run.completions()
    assert len(got) == 1
    d = rl.HwDesc.from_buffer_copy(got[0])
    assert (d.rollout_id, d.seq_len, d.max_tokens) == (r0, int(w.ctx[r0]) + 1, int(w.ctx[r0]) + 1)
    assert d.flags & 2 and d.opcode == 1
    st = run.stats()
    assert st[0] == 1 and st[1] == 1 and st[3] == 3, st
    assert run.loop(2) == 0                                # nothing held, admission closed
    run.close()
    arena.close()


def test_ring_loop_lock_step_host(rl, gpu, orc, olib):
    """A host that submits its next batch only after it has seen the previous
    batch's completions, while the loop runs: 8 one-token descriptors, no
    STOP; every row finishes and the ring is empty, so the turn waits for the
    host - after making those completions visible (the step's merges are done
    early for it). A host thread pops the 8 completions during that wait, then
    submits 8 more and STOP, which the same launch decodes. Both batches'
    completions follow the control rule and every decoded row matches the
    oracle's tokens."""
    import threading
    import ringstep

    B, V = 8, 4096
    rng = np.random.default_rng(7290)
    w = synth.make_decode(7291, 2 * B, QH, KVH, D, 40, 300)
    arena = rl.DeviceBuffer.from_array(w.arena)
    seeds = rng.integers(0, 2**63, 2 * B, dtype=np.uint64)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()) + 1, B, V,
                               output_slots=8, temperature=1.0, top_k=50, top_p=0.9, seeds=seeds)
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    logits = rng.standard_normal((B, V), dtype=np.float32)
    run.set_inputs(0, q, kn, vn, logits)
    for r in range(B):
        run.submit_decode(r, int(w.ctx[r]), int(w.ctx[r]) + 1)
    seen, errs = [], []

    def host():
        try:
            import time
            t_end = time.monotonic() + 20
            while len(seen) < B and time.monotonic() < t_end:
                seen.extend(run.completions())
            if len(seen) != B:
                errs.append(f"first batch: {len(seen)} completions")
                return
            for r in range(B, 2 * B):
                run.submit_decode(r, int(w.ctx[r]), int(w.ctx[r]) + 1)
            run.push(rl.HwDesc(opcode=255))
        except Exception as e:  # reported by the main thread
            errs.append(repr(e))

    th = threading.Thread(target=host)
    print("[loop] lock-step host: 8 descriptors, then 8 more after their completions", flush=True)
    run.loop_launch(8)
    th.start()
    ran = run.loop_done()
    th.join(timeout=30)
    assert not errs, errs
    # the second batch may be admitted over several turns, as the host's
    # pushes arrive
    assert 2 <= ran <= 8, ran
    got = seen + run.completions()
    assert len(got) == 2 * B
    by = {rl.HwDesc.from_buffer_copy(g).rollout_id: rl.HwDesc.from_buffer_copy(g) for g in got}
    assert sorted(by) == list(range(2 * B))
    for r, d in by.items():
        assert (d.seq_len, d.max_tokens) == (int(w.ctx[r]) + 1, int(w.ctx[r]) + 1) and d.flags & 2, r
    assert run.stats() == [2 * B, 2 * B, ran, 4]
    lp = C.c_double()
    decoded = []
    for s in range(ran):
        o = run.outputs(s)
        for i in range(B):
            r = int(o["rows"][i])
            if r == 0xFFFFFFFF:
                continue
            decoded.append(r)
            want = olib.orc_sample_row(logits[i].ctypes.data, V, 0, 1.0, 50, 0.9, int(seeds[r]), int(w.ctx[r]), r,
                                       C.byref(lp))
            assert o["tok"][i] == want, (s, i)
    assert sorted(decoded) == list(range(2 * B))
    assert sorted(run.outputs(0)["rows"].tolist()) == list(range(B))
    run.close()
    arena.close()


def test_ring_loop_rejects(rl, gpu):
    import ringstep

    B, V = 4, 1024
    w = synth.make_decode(7191, B, 64, KVH, D, 40, 100)
    arena = rl.DeviceBuffer.from_array(w.arena)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, 64, int(w.ctx.max()), B, V,
                               greedy=True)
    with pytest.raises(rl.RlrtError, match="fused kernel"):
        run.loop(1)
    run.close()
    w = synth.make_decode(7192, B, QH, KVH, D, 40, 100)
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()), B, V,
                               greedy=True)
    with pytest.raises(rl.RlrtError, match="output_slots"):
        run.loop(1)
    run.close()
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()), B, V,
                               output_slots=2, greedy=True)
    with pytest.raises(rl.RlrtError, match="output_slots"):
        run.loop(1)
    run.close()
    run = ringstep.RingStepRun(arena, rl.KvLayoutDesc.paged(TPB, D), w.table, QH, int(w.ctx.max()), B, V,
                               output_slots=3, greedy=True)
    with pytest.raises(rl.RlrtError, match="max_steps"):
        run.loop(0)
    run.close()
    arena.close()
