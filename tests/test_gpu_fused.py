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
rl_hip_sample: there the results equal those two calls bit for bit.
"""
import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu


def _run(rl, w, max_ctx, pos, cow, kn, vn, logits, repeats=2, **samp):
    """Uploads the decode workload and the logits, runs the fused step
    `repeats` times on one workspace (re-uploading the arena each time), and
    returns a list of (out16, out32, arena, tok, lp) per call."""
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
        rl.decode_sample_step(a, ap, s, ws)
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
    olib.orc_kv_append(want_arena.ctypes.data, w.block_bytes, w.token_count, w.head_dim * 2, w.table.ctypes.data,
                       w.table_stride, w.batch, w.kv_heads, pos.ctypes.data,
                       cow.ctypes.data if cow is not None else None, kn.ctypes.data, vn.ctypes.data)
    assert np.array_equal(arena, want_arena)
    bad = np.nonzero(tok != want_tok)[0]
    assert len(bad) == 0, (bad[:8], tok[bad[:8]], want_tok[bad[:8]])
    assert np.abs(lp - want_lp).max() < 1e-4


def _kv_rows(rng, w):
    kn = rng.integers(0, 256, (w.batch, w.kv_heads, w.head_dim * 2), dtype=np.uint8)
    vn = rng.integers(0, 256, (w.batch, w.kv_heads, w.head_dim * 2), dtype=np.uint8)
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
