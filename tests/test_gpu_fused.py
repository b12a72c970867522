"""The decode step of one micro-batch fused with the sampling of another
(rl_hip_decode_sample_step) against the oracle.

Checked on every shape:
  * attention: fp32 output within 1e-4 of fp64 (row-normalised), the stored
    bf16/fp16 output the round-to-nearest-even of it; rows with ctx beyond
    max_ctx NaN, rows without context zero;
  * the arena after the step byte-equal to the oracle's append of every
    row's K/V token (copy-on-write rows included);
  * tokens bit-exact and logprobs within 1e-4 against the oracle sampler on
    the same logits and per-row parameters;
  * a second call on the same workspace gives the same bits (the pieces are
    cut at tile positions that depend only on the contexts).
Shapes whose tiles do not fit the fused kernel run rl_hip_decode_step then
rl_hip_sample: there the results equal those two calls bit for bit. Without an append (append NULL) the arena is unchanged.
"""
import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu


def _run(rl, w, max_ctx, pos, cow, kn, vn, logits, repeats=2, append=True, **samp):
    """Uploads the decode workload and the logits, runs the fused step
    `repeats` times on one workspace (re-uploading the arena each time; with
    append False the step has no KV append), and returns a list of (out16,
    out32, arena, tok, lp) per call."""
    B, QH, D = w.batch, w.q_heads, w.head_dim
    layout = rl.KvLayoutDesc.paged(w.token_count, D)
    code = rl.DTYPE_BF16 if w.dtype == "bf16" else rl.DTYPE_FP16
    rows, V = logits.shape
    bufs = {k: rl.DeviceBuffer.from_array(v) for k, v in
            (("arena", w.arena), ("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", pos), ("kn", kn),
             ("vn", vn), ("logits", logits))}
    if cow is not None:
        bufs["cow"] = rl.DeviceBuffer.from_array(cow)
    arrays = {}
    for k in ("temperature", "top_k", "top_p", "seed", "steps"):
        if k in samp and isinstance(samp[k], np.ndarray):
            arrays[k] = rl.DeviceBuffer.from_array(samp.pop(k))
    n = B * QH * D
    out, out32 = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4)
    tok, lp = rl.DeviceBuffer(rows * 4), rl.DeviceBuffer(rows * 4)
    a = rl.attn_args(bufs["arena"], layout, bufs["table"], w.table_stride, B, QH, w.kv_heads, code, bufs["ctx"],
                     max_ctx, bufs["q"], out, out32)
    ap = rl.AppendArgs(arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes, layout=layout,
                       block_table=bufs["table"].ptr, table_stride=w.table_stride, batch=B, kv_heads=w.kv_heads,
                       positions=bufs["pos"].ptr, cow_src=bufs["cow"].ptr if cow is not None else None,
                       k_new=bufs["kn"].ptr, v_new=bufs["vn"].ptr)
    s = rl.sample_args(bufs["logits"], rows, V, V, tok, lp, **{k: v for k, v in samp.items()
                                                               if k in ("greedy", "temperature", "top_k", "top_p",
                                                                        "seed", "step")})
    s.temperature = arrays["temperature"].ptr if "temperature" in arrays else None
    s.top_k = arrays["top_k"].ptr if "top_k" in arrays else None
    s.top_p = arrays["top_p"].ptr if "top_p" in arrays else None
    s.seed = arrays["seed"].ptr if "seed" in arrays else None
    s.steps = arrays["steps"].ptr if "steps" in arrays else None
    ws = rl.decode_sample_step_workspace(a, s)
    res = []
    for i in range(repeats):
        if i:
            bufs["arena"].upload(w.arena)
        print(f"[fused] call {i}: batch {B}, {QH}/{w.kv_heads} heads d{D} {w.dtype}, sampling {rows} x {V}",
              flush=True)
        rl.decode_sample_step(a, ap if append else None, s, ws)
        rl.sync()
        res.append((out.download(np.uint16, (B, QH, D)), out32.download(np.float32, (B, QH, D)),
                    bufs["arena"].download(np.uint8, w.arena.size), tok.download(np.uint32, rows),
                    lp.download(np.float32, rows)))
    for b in list(bufs.values()) + list(arrays.values()) + [out, out32, tok, lp, ws]:
        b.close()
    return res


def _check(orc, olib, w, max_ctx, pos, cow, kn, vn, logits, res, want_tok, want_lp):
    code = 0 if w.dtype == "bf16" else 1
    o16, o32, arena, tok, lp = res[0]
    for r in res[1:]:
        for x, y in zip(res[0], r):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
    ok = w.ctx <= max_ctx
    if (~ok).any():
        assert np.isnan(o32[~ok]).all()
    if ok.any():
        wv = synth.DecodeWorkload(int(ok.sum()), w.q_heads, w.kv_heads, w.head_dim, w.dtype, w.token_count,
                                  w.ctx[ok].copy(), np.ascontiguousarray(w.table[ok]), w.arena,
                                  np.ascontiguousarray(w.q[ok]), 0)
        ref = orc.attn_f64(olib, wv, code)
        empty = wv.ctx == 0
        assert not o32[ok][empty].any()
        if (~empty).any():
            gh.check_attn(o16[ok][~empty], o32[ok][~empty], ref[~empty], w.dtype)
    want_arena = w.arena.copy()
    if pos is not None:  # None: a step without append
        olib.orc_kv_append(want_arena.ctypes.data, w.block_bytes, w.token_count, w.head_dim * 2,
                           w.table.ctypes.data, w.table_stride, w.batch, w.kv_heads, pos.ctypes.data,
                           cow.ctypes.data if cow is not None else None, kn.ctypes.data, vn.ctypes.data)
    assert np.array_equal(arena, want_arena)
    bad = np.nonzero(tok != want_tok)[0]
    assert len(bad) == 0, (bad[:8], tok[bad[:8]], want_tok[bad[:8]])
    assert np.abs(lp - want_lp).max() < 1e-4


def _kv_rows(rng, w):
    """The step's new K and V rows, N(0, 1) in the workload's 16-bit format
    (finite: a later step's attention reads them), as bytes."""
    shape = (w.batch, w.kv_heads, w.head_dim)
    kn = synth.to_scalar16(rng.standard_normal(shape, dtype=np.float32), w.dtype).view(np.uint8)
    vn = synth.to_scalar16(rng.standard_normal(shape, dtype=np.float32), w.dtype).view(np.uint8)
    return kn, vn


def test_fused_step_batch64(rl, gpu, orc, olib):
    """The batched-decode shape (64 rollouts, GQA 32/8, d128 bf16, ctx
    U[512, 4096], permuted 16-token blocks) with 64 rows x 128,256 of
    sampling (T 0.8, top-k 50, top-p 0.9, per-row seeds, 5 spikes per row)."""
    B, V = 64, 128256
    w = synth.make_decode(8101, B, 32, 8, 128, 512, 4096, max_ctx=4096)
    rng = np.random.default_rng(8102)
    pos = w.ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = synth.make_logits(8103, B, V, spikes=5)
    seeds = rng.integers(0, 2**63, B, dtype=np.uint64)
    res = _run(rl, w, 4096, pos, None, kn, vn, logits, temperature=0.8, top_k=50, top_p=0.9, seed=seeds, step=7)
    want, wlp = orc.sample_rows_v(olib, logits, seeds=seeds, temperature_all=0.8, top_k_all=50, top_p_all=0.9,
                                  step_all=7)
    _check(orc, olib, w, 4096, pos, None, kn, vn, logits, res, want, wlp)


def test_fused_step_max_batch(rl, gpu, orc, olib):
    """1,024 rollouts, the most the fused kernel takes (its tile prefix and
    the loop's staged contexts are sized for it): GQA 16/4 d64 bf16, ctx
    U[0, 600] (a few rows without context), every row appending; 1,024 rows
    x 4,096 of sampling (T 0.9, top-k 40, top-p 0.9, per-row seeds), sixteen
    rows per sampling workgroup."""
    B, V = 1024, 4096
    w = synth.make_decode(8106, B, 16, 4, 64, 0, 600)
    rng = np.random.default_rng(8107)
    pos = w.ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    seeds = rng.integers(0, 2**63, B, dtype=np.uint64)
    res = _run(rl, w, int(w.ctx.max()), pos, None, kn, vn, logits, temperature=0.9, top_k=40, top_p=0.9,
               seed=seeds.copy(), step=3)
    want, wlp = orc.sample_rows_v(olib, logits, seeds=seeds, temperature_all=0.9, top_k_all=40, top_p_all=0.9,
                                  step_all=3)
    _check(orc, olib, w, int(w.ctx.max()), pos, None, kn, vn, logits, res, want, wlp)


def test_fused_step_ragged_edges(rl, gpu, orc, olib):
    """Contexts 0, 1, 15, 16, 17 tokens, one beyond max_ctx (NaN rows), long
    ones; GQA 16/8 d64 fp16 in 32-token blocks; copy-on-write on a third of
    the rows; 3 greedy rows of 32,000 (fewer rows than the sampling
    workgroups)."""
    ctx = np.array([0, 1, 15, 16, 17, 700, 5000, 33, 2048, 1, 64, 0], np.uint32)
    B, max_ctx = len(ctx), 2048
    w = synth.make_decode(8111, B, 16, 8, 64, 0, 0, dtype="fp16", token_count=32, ctx=ctx, max_ctx=5000,
                          spare_blocks=24, kv_std=0.5)
    rng = np.random.default_rng(8112)
    pos = np.minimum(ctx, 4000).astype(np.uint32)
    n_used = w.arena.size // w.block_bytes - 24
    cow = np.full((B, 8), -1, np.int32)
    cow[::3] = n_used + rng.integers(0, 24, (len(cow[::3]), 8))
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((3, 32000), dtype=np.float32)
    res = _run(rl, w, max_ctx, pos, cow, kn, vn, logits, greedy=True)
    want, wlp = orc.sample_rows(olib, logits, True, 1.0, 0, 1.0, 0, 0)
    _check(orc, olib, w, max_ctx, pos, cow, kn, vn, logits, res, want, wlp)


def test_fused_step_many_rows_mixed(rl, gpu, orc, olib):
    """200 rows of 50,000 logits (several rows per sampling workgroup) with
    per-row temperature (a quarter greedy), top-k (0 = whole-vocabulary
    nucleus, or up to 256), top-p, seed and step; 40 rollouts of GQA 32/8
    d128 bf16, ctx U[1, 3000]."""
    R, V = 200, 50000
    w = synth.make_decode(8121, 40, 32, 8, 128, 1, 3000)
    rng = np.random.default_rng(8122)
    pos = w.ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((R, V), dtype=np.float32) * np.float32(1.5)
    temp = np.where(rng.random(R) < 0.25, 0.0, rng.uniform(0.5, 1.5, R)).astype(np.float32)
    topk = rng.choice([0, 1, 20, 50, 256], R).astype(np.uint32)
    topp = rng.choice([1.0, 0.95, 0.7, 0.2], R).astype(np.float32)
    seeds = rng.integers(0, 2**63, R, dtype=np.uint64)
    steps = rng.integers(0, 10**6, R, dtype=np.uint64)
    res = _run(rl, w, int(w.ctx.max()), pos, None, kn, vn, logits, temperature=temp.copy(), top_k=topk.copy(),
               top_p=topp.copy(), seed=seeds.copy(), steps=steps.copy())
    want, wlp = orc.sample_rows_v(olib, logits, temperature=temp, top_k=topk, top_p=topp, seeds=seeds, steps=steps)
    _check(orc, olib, w, int(w.ctx.max()), pos, None, kn, vn, logits, res, want, wlp)


def test_fused_step_no_context(rl, gpu, orc, olib):
    """Every rollout at context 0: no tiles at all, zero outputs, the appends
    and the sampling still done."""
    ctx = np.zeros(16, np.uint32)
    w = synth.make_decode(8131, 16, 32, 8, 128, 0, 0, ctx=ctx, max_ctx=64)
    rng = np.random.default_rng(8132)
    pos = ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((16, 4096), dtype=np.float32)
    res = _run(rl, w, 64, pos, None, kn, vn, logits, temperature=1.0, top_k=40, top_p=0.9, seed=5, step=1)
    want, wlp = orc.sample_rows(olib, logits, False, 1.0, 40, 0.9, 5, 1)
    _check(orc, olib, w, 64, pos, None, kn, vn, logits, res, want, wlp)


def test_fused_step_outside_the_kernel_equals_two_calls(rl, gpu, orc, olib):
    """GQA 64/8 at d128 does not fit the fused kernel's LDS: the entry point
    runs rl_hip_decode_step then rl_hip_sample, and the results equal those
    two calls bit for bit."""
    B, V = 8, 20000
    w = synth.make_decode(8141, B, 64, 8, 128, 100, 2000)
    rng = np.random.default_rng(8142)
    pos = w.ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((B, V), dtype=np.float32)
    res = _run(rl, w, int(w.ctx.max()), pos, None, kn, vn, logits, repeats=1, temperature=0.9, top_k=30, top_p=0.8,
               seed=3, step=2)
    want, wlp = orc.sample_rows(olib, logits, False, 0.9, 30, 0.8, 3, 2)
    _check(orc, olib, w, int(w.ctx.max()), pos, None, kn, vn, logits, res, want, wlp)
    # the two calls themselves
    o16, o32 = gh.run_attn(rl, w)
    assert np.array_equal(res[0][0], o16) and np.array_equal(res[0][1], o32)
    lg, tok, lp = rl.DeviceBuffer.from_array(logits), rl.DeviceBuffer(B * 4), rl.DeviceBuffer(B * 4)
    s = rl.sample_args(lg, B, V, V, tok, lp, temperature=0.9, top_k=30, top_p=0.8, seed=3, step=2)
    sws = rl.sample_workspace(s)
    rl.sample(s)
    rl.sync()
    assert np.array_equal(tok.download(np.uint32, B), res[0][3])
    assert np.array_equal(lp.download(np.float32, B), res[0][4])
    for b in (lg, tok, lp, sws):
        b.close()


class _Batch:
    """One micro-batch's device buffers: arena, table, ctx, q, outputs, the
    append's positions and K/V rows."""

    def __init__(self, rl, w, max_ctx, pos, kn, vn):
        self.rl, self.w = rl, w
        self.n = w.batch * w.q_heads * w.head_dim
        self.buf = {k: rl.DeviceBuffer.from_array(v) for k, v in
                    (("arena", w.arena), ("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", pos), ("kn", kn),
                     ("vn", vn))}
        self.out, self.out32 = rl.DeviceBuffer(self.n * 2), rl.DeviceBuffer(self.n * 4)
        layout = rl.KvLayoutDesc.paged(w.token_count, w.head_dim)
        code = rl.DTYPE_BF16 if w.dtype == "bf16" else rl.DTYPE_FP16
        b = self.buf
        self.attn = rl.attn_args(b["arena"], layout, b["table"], w.table_stride, w.batch, w.q_heads, w.kv_heads, code,
                                 b["ctx"], max_ctx, b["q"], self.out, self.out32)
        self.app = rl.AppendArgs(arena_base=b["arena"].ptr, arena_bytes=b["arena"].nbytes, layout=layout,
                                 block_table=b["table"].ptr, table_stride=w.table_stride, batch=w.batch,
                                 kv_heads=w.kv_heads, positions=b["pos"].ptr, cow_src=None, k_new=b["kn"].ptr,
                                 v_new=b["vn"].ptr)

    def outputs(self):
        w = self.w
        sh = (w.batch, w.q_heads, w.head_dim)
        return self.out.download(np.uint16, sh), self.out32.download(np.float32, sh)

    def close(self):
        for x in list(self.buf.values()) + [self.out, self.out32]:
            x.close()


def test_fused_pipeline_two_microbatches(rl, gpu, orc, olib):
    """Three pipelined steps over micro-batches A, B, A (the second A step at
    context + 1, so it reads the token the first one appended) and a flush.
    Every micro-batch's attention is within 1e-4 of fp64; the first step's
    (nothing to merge before it, so the same split) equals
    rl_hip_decode_sample_step's bit for bit, which pins the wave-level merge
    to the merge kernel's arithmetic; the arenas equal the oracle's appends;
    every step's tokens equal the oracle's."""
    QH, KVH, D, V = 32, 8, 128, 32000
    rng = np.random.default_rng(8151)
    # A: 64 rollouts of up to 1,200 tokens, so that no row spans more than 16
    # pieces (the merge kernel's register path, which the bit check compares)
    wa = synth.make_decode(8152, 64, QH, KVH, D, 300, 1200, reserve_tokens=1300)
    wb = synth.make_decode(8153, 40, QH, KVH, D, 1, 1200, max_ctx=1300)
    mc = 1300
    pa1, pb = wa.ctx.copy(), wb.ctx.copy()
    ka1, va1 = _kv_rows(rng, wa)
    ka2, va2 = _kv_rows(rng, wa)
    kb, vb = _kv_rows(rng, wb)
    qa2 = synth.f32_to_bf16(rng.standard_normal(wa.q.shape, dtype=np.float32))
    lg = [rng.standard_normal((64, V), dtype=np.float32) for _ in range(3)]
    seeds = rng.integers(0, 2**63, 64, dtype=np.uint64)

    A1 = _Batch(rl, wa, mc, pa1, ka1, va1)
    B = _Batch(rl, wb, mc, pb, kb, vb)
    # A's second step shares A's arena and table: its own ctx (+1), q, positions, rows, outputs
    A2 = _Batch(rl, synth.DecodeWorkload(wa.batch, QH, KVH, D, "bf16", 16, wa.ctx + np.uint32(1), wa.table,
                                         wa.arena, qa2, 0), mc, pa1 + np.uint32(1), ka2, va2)
    for k in ("arena", "table"):
        A2.buf[k].close()
        A2.buf[k] = A1.buf[k]
    A2.attn.arena_base, A2.attn.block_table = A1.attn.arena_base, A1.attn.block_table
    A2.app.arena_base, A2.app.block_table = A1.app.arena_base, A1.app.block_table
    seed_buf = rl.DeviceBuffer.from_array(seeds)
    lgb = [rl.DeviceBuffer.from_array(x) for x in lg]
    tok = [rl.DeviceBuffer(64 * 4) for _ in range(3)]
    lp = [rl.DeviceBuffer(64 * 4) for _ in range(3)]
    samp = [rl.sample_args(lgb[i], 64, V, V, tok[i], lp[i], temperature=0.9, top_k=64, top_p=0.9, seeds=seed_buf,
                           step=i) for i in range(3)]
    # one workspace per micro-batch, both of the larger size (the call takes one size for both)
    n_ws = max(rl.decode_sample_step_workspace_bytes(bt.attn, samp[0]) for bt in (A1, B))
    ws = [rl.DeviceBuffer(n_ws) for _ in range(2)]
    print("[fused] pipeline: A, B, A, flush", flush=True)
    rl.decode_pipeline_step(A1.attn, samp[0], ws[0])
    rl.decode_pipeline_step(B.attn, samp[1], ws[1], A1.attn, A1.app, ws[0])
    rl.decode_pipeline_step(A2.attn, samp[2], ws[0], B.attn, B.app, ws[1])
    rl.decode_pipeline_flush(A2.attn, A2.app, ws[0])
    rl.sync()
    outs = {name: bt.outputs() for name, bt in (("A1", A1), ("B", B), ("A2", A2))}
    arena_a = A1.buf["arena"].download(np.uint8, wa.arena.size)
    arena_b = B.buf["arena"].download(np.uint8, wb.arena.size)
    toks = [(t.download(np.uint32, 64), l.download(np.float32, 64)) for t, l in zip(tok, lp)]

    # the first step's attention through rl_hip_decode_sample_step, bit for bit
    res = _run(rl, wa, mc, pa1, None, ka1, va1, lg[0], repeats=1, temperature=0.9, top_k=64, top_p=0.9,
               seed=seeds.copy(), step=0)
    assert np.array_equal(res[0][0], outs["A1"][0]) and np.array_equal(res[0][1], outs["A1"][1])
    for name, w in (("A1", wa), ("B", wb)):
        gh.check_attn(outs[name][0], outs[name][1], orc.attn_f64(olib, w, 0), "bf16")
    # A's second step read the token A's first step appended
    arena_a1 = wa.arena.copy()
    olib.orc_kv_append(arena_a1.ctypes.data, wa.block_bytes, 16, D * 2, wa.table.ctypes.data, wa.table_stride,
                       wa.batch, KVH, pa1.ctypes.data, None, ka1.ctypes.data, va1.ctypes.data)
    w2 = synth.DecodeWorkload(wa.batch, QH, KVH, D, "bf16", 16, wa.ctx + np.uint32(1), wa.table, arena_a1, qa2, 0)
    gh.check_attn(outs["A2"][0], outs["A2"][1], orc.attn_f64(olib, w2, 0), "bf16")
    pa2 = pa1 + np.uint32(1)
    olib.orc_kv_append(arena_a1.ctypes.data, wa.block_bytes, 16, D * 2, wa.table.ctypes.data, wa.table_stride,
                       wa.batch, KVH, pa2.ctypes.data, None, ka2.ctypes.data, va2.ctypes.data)
    assert np.array_equal(arena_a, arena_a1)
    arena_b1 = wb.arena.copy()
    olib.orc_kv_append(arena_b1.ctypes.data, wb.block_bytes, 16, D * 2, wb.table.ctypes.data, wb.table_stride,
                       wb.batch, KVH, pb.ctypes.data, None, kb.ctypes.data, vb.ctypes.data)
    assert np.array_equal(arena_b, arena_b1)
    for i in range(3):
        want, wlp = orc.sample_rows(olib, lg[i], False, 0.9, 64, 0.9, seeds, i)
        assert np.array_equal(toks[i][0], want), i
        assert np.abs(toks[i][1] - wlp).max() < 1e-4, i
    for x in lgb + tok + lp + ws + [seed_buf]:
        x.close()
    A2.buf.pop("arena"), A2.buf.pop("table")
    for bt in (A1, B, A2):
        bt.close()


def _next_step(rl, first, w, mc, q2, pos2, k2, v2):
    """The micro-batch's next step: the first step's arena and table, ctx + 1,
    its own queries, positions, K/V rows and outputs."""
    w2 = synth.DecodeWorkload(w.batch, w.q_heads, w.kv_heads, w.head_dim, w.dtype, w.token_count,
                              w.ctx + np.uint32(1), w.table, w.arena, q2, 0)
    nxt = _Batch(rl, w2, mc, pos2, k2, v2)
    for k in ("arena", "table"):
        nxt.buf[k].close()
        nxt.buf[k] = first.buf[k]
    nxt.attn.arena_base, nxt.attn.block_table = first.attn.arena_base, first.attn.block_table
    nxt.app.arena_base, nxt.app.block_table = first.app.arena_base, first.app.block_table
    return nxt


def _lanes_case(rl, orc, olib, QH, KVH, D, dtype, tc, sizes, ctx_hi, seed, V=32000):
    """Four micro-batches (batches `sizes`, ctx U[1 or 300, ctx_hi]) for two
    steps each on the two lanes (step t: micro-batch t % 4 on lane t % 2,
    merging step t - 2; the last two flushed, then joined), against the same
    calls on the library stream bit for bit, fp64, the oracle's appends and
    the oracle's tokens."""
    code = rl.DTYPE_BF16 if dtype == "bf16" else rl.DTYPE_FP16
    ocode = 0 if dtype == "bf16" else 1
    mc = ctx_hi + 100
    rng = np.random.default_rng(seed)
    ws_ = [synth.make_decode(seed + 1 + m, n, QH, KVH, D, 1 if m % 2 else min(300, ctx_hi), ctx_hi, dtype=dtype,
                             token_count=tc, reserve_tokens=mc) for m, n in enumerate(sizes)]
    pos1 = [w.ctx.copy() for w in ws_]
    rows1 = [_kv_rows(rng, w) for w in ws_]
    rows2 = [_kv_rows(rng, w) for w in ws_]
    q2 = [synth.to_scalar16(rng.standard_normal(w.q.shape, dtype=np.float32), dtype) for w in ws_]
    lg = [rng.standard_normal((64, V), dtype=np.float32) for _ in range(8)]
    seeds = rng.integers(0, 2**63, 64, dtype=np.uint64)
    seed_buf = rl.DeviceBuffer.from_array(seeds)
    lgb = [rl.DeviceBuffer.from_array(x) for x in lg]

    def run(on_lanes):
        first = [_Batch(rl, w, mc, p, k, v) for w, p, (k, v) in zip(ws_, pos1, rows1)]
        second = [_next_step(rl, f, w, mc, q, p + np.uint32(1), k, v)
                  for f, w, q, p, (k, v) in zip(first, ws_, q2, pos1, rows2)]
        steps = first + second                      # step t runs micro-batch t % 4
        tok = [rl.DeviceBuffer(64 * 4) for _ in range(8)]
        lp = [rl.DeviceBuffer(64 * 4) for _ in range(8)]
        samp = [rl.sample_args(lgb[t], 64, V, V, tok[t], lp[t], temperature=0.9, top_k=64, top_p=0.9,
                               seeds=seed_buf, step=t) for t in range(8)]
        n_ws = max(rl.decode_sample_step_workspace_bytes(bt.attn, samp[0]) for bt in first)
        ws = [rl.DeviceBuffer(n_ws) for _ in range(4)]
        print(f"[fused] four micro-batches {sizes} ({QH}/{KVH} d{D} {dtype} tc{tc}), two steps each, "
              f"{'on the lanes' if on_lanes else 'one stream'}", flush=True)
        if on_lanes:
            rl.lanes_fork()
        for t in range(8):
            prev = (steps[t - 2].attn, steps[t - 2].app, ws[(t - 2) % 4]) if t >= 2 else (None, None, None)
            if on_lanes:
                rl.decode_lane_step(t % 2, steps[t].attn, samp[t], ws[t % 4], *prev)
            else:
                rl.decode_pipeline_step(steps[t].attn, samp[t], ws[t % 4], *prev)
        for t in (6, 7):
            if on_lanes:
                rl.decode_lane_flush(t % 2, steps[t].attn, steps[t].app, ws[t % 4])
            else:
                rl.decode_pipeline_flush(steps[t].attn, steps[t].app, ws[t % 4])
        if on_lanes:
            rl.lanes_join()
        rl.sync()
        res = {"out": [bt.outputs() for bt in steps],
               "arena": [f.buf["arena"].download(np.uint8, w.arena.size) for f, w in zip(first, ws_)],
               "tok": [(t.download(np.uint32, 64), l.download(np.float32, 64)) for t, l in zip(tok, lp)]}
        for x in tok + lp + ws:
            x.close()
        for bt in second:
            bt.buf.pop("arena"), bt.buf.pop("table")
        for bt in first + second:
            bt.close()
        return res

    lanes, one = run(True), run(False)
    for t in range(8):
        assert np.array_equal(lanes["out"][t][0], one["out"][t][0]), t
        assert np.array_equal(lanes["out"][t][1], one["out"][t][1]), t
        assert np.array_equal(lanes["tok"][t][0], one["tok"][t][0]), t
        assert np.array_equal(lanes["tok"][t][1], one["tok"][t][1]), t
    rb = D * 2
    for m, w in enumerate(ws_):
        assert np.array_equal(lanes["arena"][m], one["arena"][m]), m
        gh.check_attn(lanes["out"][m][0], lanes["out"][m][1], orc.attn_f64(olib, w, ocode), dtype)
        arena1 = w.arena.copy()
        k1, v1 = rows1[m]
        olib.orc_kv_append(arena1.ctypes.data, w.block_bytes, tc, rb, w.table.ctypes.data, w.table_stride,
                           w.batch, KVH, pos1[m].ctypes.data, None, k1.ctypes.data, v1.ctypes.data)
        w2 = synth.DecodeWorkload(w.batch, QH, KVH, D, dtype, tc, w.ctx + np.uint32(1), w.table, arena1, q2[m], 0)
        gh.check_attn(lanes["out"][4 + m][0], lanes["out"][4 + m][1], orc.attn_f64(olib, w2, ocode), dtype)
        k2, v2 = rows2[m]
        p2 = pos1[m] + np.uint32(1)
        olib.orc_kv_append(arena1.ctypes.data, w.block_bytes, tc, rb, w.table.ctypes.data, w.table_stride,
                           w.batch, KVH, p2.ctypes.data, None, k2.ctypes.data, v2.ctypes.data)
        assert np.array_equal(lanes["arena"][m], arena1), m
    for t in range(8):
        want, wlp = orc.sample_rows(olib, lg[t], False, 0.9, 64, 0.9, seeds, t)
        assert np.array_equal(lanes["tok"][t][0], want), t
        assert np.abs(lanes["tok"][t][1] - wlp).max() < 1e-4, t
    for x in lgb + [seed_buf]:
        x.close()


def test_fused_lanes_four_microbatches(rl, gpu, orc, olib):
    """Four micro-batches of the benchmark's shape (64, 48, 64 and 33
    rollouts of GQA 32/8, d128, bf16, 16-token blocks) on the two lanes
    against the same calls on one stream: outputs, arenas and tokens bit for
    bit (the lanes change where steps run, not what they compute), every
    attention within 1e-4 of fp64, the arenas equal to the oracle's two
    appends, every step's tokens equal to the oracle's."""
    _lanes_case(rl, orc, olib, 32, 8, 128, "bf16", 16, (64, 48, 64, 33), 1200, 9161)


@pytest.mark.parametrize("shape", [(16, 8, 64, "fp16", 32), (8, 8, 128, "fp16", 32), (16, 8, 128, "bf16", 16),
                                   (8, 2, 64, "bf16", 16)],
                         ids=["gqa2_d64_fp16_tc32", "mha_d128_fp16_tc32", "gqa2_d128_bf16", "gqa4_d64_bf16_kv2"])
def test_fused_lanes_shapes(rl, gpu, orc, olib, shape):
    """The lanes case on the other shapes the fused kernel takes: GQA groups
    1, 2 and 4, head_dim 64 and 128, fp16 and bf16, 16- and 32-token blocks."""
    QH, KVH, D, dtype, tc = shape
    _lanes_case(rl, orc, olib, QH, KVH, D, dtype, tc, (24, 17, 24, 9), 700, 9300 + QH * 10 + KVH + D)


def test_fused_step_without_append(rl, gpu, orc, olib):
    """append NULL: the fused kernel (GQA 32/8) and the two-call path (GQA
    64/8, 8 rollouts of up to 3,000 tokens with greedy over 8 x 128,256, the
    long-context step's sampler) leave the arena untouched, the attention is
    within 1e-4 of fp64, a second call on the same workspace gives the same
    bits and the tokens equal the oracle's; on the two-call path everything
    equals rl_hip_attn_decode and rl_hip_sample bit for bit."""
    rng = np.random.default_rng(8171)
    w = synth.make_decode(8172, 48, 32, 8, 128, 1, 2500)
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((48, 32000), dtype=np.float32)
    res = _run(rl, w, int(w.ctx.max()), w.ctx.copy(), None, kn, vn, logits, append=False, temperature=0.7, top_k=40,
               top_p=0.95, seed=11, step=5)
    want, wlp = orc.sample_rows(olib, logits, False, 0.7, 40, 0.95, 11, 5)
    _check(orc, olib, w, int(w.ctx.max()), None, None, kn, vn, logits, res, want, wlp)

    V = 128256
    w8 = synth.make_decode(8173, 8, 64, 8, 128, 1000, 3000)
    kn8, vn8 = _kv_rows(rng, w8)
    lg8 = rng.standard_normal((8, V), dtype=np.float32)
    res8 = _run(rl, w8, int(w8.ctx.max()), w8.ctx.copy(), None, kn8, vn8, lg8, append=False, greedy=True)
    want8, wlp8 = orc.sample_rows(olib, lg8, True, 1.0, 0, 1.0, 0, 0)
    _check(orc, olib, w8, int(w8.ctx.max()), None, None, kn8, vn8, lg8, res8, want8, wlp8)
    o16, o32 = gh.run_attn(rl, w8)
    assert np.array_equal(res8[0][0], o16) and np.array_equal(res8[0][1], o32)
    lg, tok, lp = rl.DeviceBuffer.from_array(lg8), rl.DeviceBuffer(8 * 4), rl.DeviceBuffer(8 * 4)
    s = rl.sample_args(lg, 8, V, V, tok, lp, greedy=True)
    sws = rl.sample_workspace(s)
    rl.sample(s)
    rl.sync()
    assert np.array_equal(tok.download(np.uint32, 8), res8[0][3])
    assert np.array_equal(lp.download(np.float32, 8), res8[0][4])
    for b in (lg, tok, lp, sws):
        b.close()


def test_fused_pipeline_long_rows(rl, gpu, orc, olib):
    """Few rollouts with long contexts: 2 rollouts of ~4,000 tokens (16 rows
    of ~250 tiles over 2,048 pieces, so every row is split over ~128 pieces,
    more than one wave's 64 lanes) then 3 rollouts of ~3,000, pipelined and
    flushed. The sampling waves' merge of the first step takes its partials
    64 at a time: both steps' attention within 1e-4 of fp64, the arenas equal
    the oracle's appends and the tokens the oracle's."""
    QH, KVH, D, V = 32, 8, 128, 32000
    rng = np.random.default_rng(8191)
    wa = synth.make_decode(8192, 2, QH, KVH, D, 3900, 4100, reserve_tokens=4200)
    wb = synth.make_decode(8193, 3, QH, KVH, D, 2900, 3100, reserve_tokens=4200)
    mc = 4200
    pa, pb = wa.ctx.copy(), wb.ctx.copy()
    ka, va = _kv_rows(rng, wa)
    kb, vb = _kv_rows(rng, wb)
    A, Bt = _Batch(rl, wa, mc, pa, ka, va), _Batch(rl, wb, mc, pb, kb, vb)
    lg = [rng.standard_normal((64, V), dtype=np.float32) for _ in range(2)]
    seeds = rng.integers(0, 2**63, 64, dtype=np.uint64)
    seed_buf = rl.DeviceBuffer.from_array(seeds)
    lgb = [rl.DeviceBuffer.from_array(x) for x in lg]
    tok = [rl.DeviceBuffer(64 * 4) for _ in range(2)]
    lp = [rl.DeviceBuffer(64 * 4) for _ in range(2)]
    samp = [rl.sample_args(lgb[i], 64, V, V, tok[i], lp[i], temperature=0.9, top_k=64, top_p=0.9, seeds=seed_buf,
                           step=i) for i in range(2)]
    n_ws = max(rl.decode_sample_step_workspace_bytes(bt.attn, samp[0]) for bt in (A, Bt))
    ws = [rl.DeviceBuffer(n_ws) for _ in range(2)]
    print("[fused] pipeline over long rows: A (2 x ~4,000), B (3 x ~3,000), flush", flush=True)
    rl.decode_pipeline_step(A.attn, samp[0], ws[0])
    rl.decode_pipeline_step(Bt.attn, samp[1], ws[1], A.attn, A.app, ws[0])
    rl.decode_pipeline_flush(Bt.attn, Bt.app, ws[1])
    rl.sync()
    for name, bt, w in (("A", A, wa), ("B", Bt, wb)):
        o16, o32 = bt.outputs()
        gh.check_attn(o16, o32, orc.attn_f64(olib, w, 0), "bf16")
    for bt, w, pos, k, v in ((A, wa, pa, ka, va), (Bt, wb, pb, kb, vb)):
        want = w.arena.copy()
        olib.orc_kv_append(want.ctypes.data, w.block_bytes, 16, D * 2, w.table.ctypes.data, w.table_stride,
                           w.batch, KVH, pos.ctypes.data, None, k.ctypes.data, v.ctypes.data)
        assert np.array_equal(bt.buf["arena"].download(np.uint8, w.arena.size), want)
    for i in range(2):
        want, wlp = orc.sample_rows(olib, lg[i], False, 0.9, 64, 0.9, seeds, i)
        assert np.array_equal(tok[i].download(np.uint32, 64), want), i
        assert np.abs(lp[i].download(np.float32, 64) - wlp).max() < 1e-4, i
    for x in lgb + tok + lp + ws + [seed_buf]:
        x.close()
    A.close()
    Bt.close()


def test_fused_greedy_rides_in_the_attention(rl, gpu, orc, olib):
    """GQA 64/8 (outside the fused kernel) with the KV append and greedy over
    12 rows of 50,000 logits: the sampler's slices run as workgroups after
    the attention's and its row merges in the attention merge's grid (three
    rows per extra workgroup row). Attention, arena, tokens and logprobs
    equal rl_hip_decode_step then rl_hip_sample bit for bit (attention within
    1e-4 of fp64, the arena equal to the oracle's append, tokens equal to the
    oracle's), on two calls in a row."""
    B, V, R = 8, 50000, 12
    w = synth.make_decode(8201, B, 64, 8, 128, 100, 2000)
    rng = np.random.default_rng(8202)
    pos = w.ctx.copy()
    kn, vn = _kv_rows(rng, w)
    logits = rng.standard_normal((R, V), dtype=np.float32)
    logits[3, [5, 17, 49999]] = np.float32(9.0)          # a tie: lowest index
    logits[7, :40000] = -np.inf                           # -inf over the first slices
    res = _run(rl, w, int(w.ctx.max()), pos, None, kn, vn, logits, repeats=2, greedy=True)
    want, wlp = orc.sample_rows(olib, logits, True, 1.0, 0, 1.0, 0, 0)
    _check(orc, olib, w, int(w.ctx.max()), pos, None, kn, vn, logits, res, want, wlp)
    assert res[0][3][3] == 5 and res[0][3][7] >= 40000
    o16, o32 = gh.run_attn(rl, w)
    assert np.array_equal(res[0][0], o16) and np.array_equal(res[0][1], o32)
    lg, tok, lp = rl.DeviceBuffer.from_array(logits), rl.DeviceBuffer(R * 4), rl.DeviceBuffer(R * 4)
    s = rl.sample_args(lg, R, V, V, tok, lp, greedy=True)
    sws = rl.sample_workspace(s)
    rl.sample(s)
    rl.sync()
    assert np.array_equal(tok.download(np.uint32, R), res[0][3])
    assert np.array_equal(lp.download(np.float32, R).view(np.uint32), res[0][4].view(np.uint32))
    for b in (lg, tok, lp, sws):
        b.close()
