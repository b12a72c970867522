"""Paged GQA decode attention on the GPU vs the fp64 oracle.

Tolerance: attention outputs within 2e-3 relative (bf16 in, fp32
accumulate), measured row-normalised (max_d |delta| / max_d |ref| per rollout
and head) on the fp32-accumulated result, which is held to 1e-4. The stored
bf16/fp16 output must be bit-equal to the round-to-nearest-even of that fp32
value; its own rounding (up to 2^-8 relative for bf16) is the format's, not
the kernel's.
"""
import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu


def _case(rl, orc, olib, w, **kw):
    print(f"[attn] B={w.batch} qh={w.q_heads} kvh={w.kv_heads} d={w.head_dim} {w.dtype} "
          f"tpb={w.token_count} ctx={w.ctx.min()}..{w.ctx.max()} {kw}", flush=True)
    out16, out32 = gh.run_attn(rl, w, **kw)
    ref = orc.attn_f64(olib, w, 0 if w.dtype == "bf16" else 1)
    return gh.check_attn(out16, out32, ref, w.dtype)


def test_gqa_batch64_ragged_512_4096(rl, gpu, orc, olib):
    """The batched GQA decode workload: 64 rollouts, 32 q / 8 kv heads, d128,
    bf16 K/V ~N(0,1), ragged ctx U[512, 4096], permuted 16-token blocks."""
    w = synth.make_decode(2, 64, 32, 8, 128, 512, 4096, dtype="bf16", max_ctx=4096)
    _case(rl, orc, olib, w, max_ctx=4096)


def test_long_context_split_kv(rl, gpu, orc, olib):
    """Batch 8, ctx 32,768, 64 q / 8 kv heads (GQA group 8), d128: split-KV
    with the fp32 log-sum-exp merge."""
    w = synth.make_decode(5, 8, 64, 8, 128, 32768, 32768, dtype="bf16")
    _case(rl, orc, olib, w)


def test_mha_fp16_d64_plumbing_shape(rl, gpu, orc, olib):
    """One rollout, MHA 8 heads, d64, fp16 K/V ~N(0, 0.5^2), ctx 256..356."""
    for ctx in (256, 300, 356):
        w = synth.make_decode(1 + ctx, 1, 8, 8, 64, ctx, ctx, dtype="fp16", kv_std=0.5)
        _case(rl, orc, olib, w)


@pytest.mark.parametrize("qh,kvh,d,dt,tpb", [(8, 8, 128, "bf16", 16), (16, 8, 128, "fp16", 16),
                                            (32, 8, 128, "bf16", 32), (64, 8, 64, "bf16", 16),
                                            (4, 1, 64, "fp16", 32), (8, 1, 128, "bf16", 16),
                                            (2, 2, 64, "bf16", 16)])
def test_shapes_and_edges(rl, gpu, orc, olib, qh, kvh, d, dt, tpb):
    # contexts straddling tile (16) and block (16/32) boundaries; the wave
    # counts put row starts and ends at every position of a wave's range:
    # one wave streaming every row, odd splits, more waves than tiles
    ctx = np.array([1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 513], dtype=np.uint32)
    w = synth.make_decode(7, len(ctx), qh, kvh, d, 0, 0, dtype=dt, token_count=tpb, ctx=ctx)
    for waves in (0, 1, 7, 61, 5000):
        _case(rl, orc, olib, w, grid_waves=waves)


def test_long_rows_in_few_waves(rl, gpu, orc, olib):
    """Rows of up to 512 tiles streamed by 1-3 waves: block-table windows of
    128 entries are reloaded inside a row, rows continue across waves."""
    ctx = np.array([8192, 3000, 17, 4100], dtype=np.uint32)
    w = synth.make_decode(11, len(ctx), 16, 4, 128, 0, 0, dtype="bf16", ctx=ctx)
    for waves in (1, 2, 3):
        _case(rl, orc, olib, w, grid_waves=waves)


def test_row_split_over_hundreds_of_waves(rl, gpu, orc, olib):
    """One 16,384-token row per kv head shared by 300 / 700 waves: partial
    counts below and above the merge's 256-entry LDS stage."""
    ctx = np.array([16384], dtype=np.uint32)
    w = synth.make_decode(12, 1, 8, 2, 128, 0, 0, dtype="bf16", ctx=ctx)
    for waves in (300, 700):
        _case(rl, orc, olib, w, grid_waves=waves)


def test_empty_context_gives_zeros(rl, gpu, orc, olib):
    ctx = np.array([0, 40, 0, 1], dtype=np.uint32)
    w = synth.make_decode(8, 4, 8, 2, 128, 0, 0, dtype="bf16", ctx=ctx)
    out16, out32 = gh.run_attn(rl, w)
    assert np.all(out32[[0, 2]] == 0) and np.all(out16[[0, 2]] == 0)
    ref = orc.attn_f64(olib, w, 0)
    gh.check_attn(out16[[1, 3]], out32[[1, 3]], ref[[1, 3]], "bf16")


def test_fixed128_reference_vector(rl, gpu, orc, olib):
    """test/test_bench.cu:91-155 closed-form vector (fp16, one head, d128, 17
    tokens in a 32-token block): |gpu - host| < 1e-4 and the lowest-index
    argmax token agree."""
    d = np.arange(128)
    q = ((d % 17) - 8) / 8.0
    t = np.arange(32)[:, None]
    K = ((((t + 1) * ((d % 13) + 1)) % 23) - 11) / 32.0
    V = ((((t + 3) * ((d % 11) + 5)) % 29) - 14) / 29.0
    q16, K16, V16 = (synth.f32_to_f16(a.astype(np.float32)) for a in (q, K, V))
    w = synth.DecodeWorkload(1, 1, 1, 128, "fp16", 32, np.array([17], np.uint32), np.zeros((1, 1, 1), np.uint32),
                             np.concatenate([K16.ravel(), V16.ravel()]).view(np.uint8), q16.reshape(1, 1, 128), 0)
    out16, out32 = gh.run_attn(rl, w)
    ref = orc.attn_f64(olib, w, 1)
    assert np.abs(out32[0, 0] - ref[0, 0]).max() < 1e-4
    assert int(np.argmax(out32[0, 0])) == int(np.argmax(ref[0, 0]))


def test_repeated_split_launches_are_identical(rl, gpu, orc, olib):
    """Back-to-back launches (partials and prefix rewritten each time) give
    bit-identical results."""
    w = synth.make_decode(9, 4, 32, 8, 128, 1500, 3000, dtype="bf16")
    res = gh.run_attn(rl, w, grid_waves=37, repeats=3)
    for o16, o32 in res[1:]:
        assert np.array_equal(o16, res[0][0]) and np.array_equal(o32, res[0][1])
    gh.check_attn(res[0][0], res[0][1], orc.attn_f64(olib, w, 0), "bf16")


def test_guards_poison_instead_of_faulting(rl, gpu, orc, olib):
    """ctx beyond max_ctx, or a block id past the arena, yields NaN outputs for
    that rollout only (the bad block is never read)."""
    w = synth.make_decode(10, 3, 8, 2, 128, 100, 100, dtype="bf16")
    w.ctx[1] = 130                                  # > max_ctx passed below
    w.table[2, 1, 3] = 10_000_000                   # far outside the arena (kv head 1 = q heads 4..7)
    out16, out32 = gh.run_attn(rl, w, max_ctx=100)
    assert np.isnan(out32[1]).all() and np.isnan(out32[2, 4:8]).all()
    assert np.isfinite(out32[0]).all() and np.isfinite(out32[2, :4]).all()
