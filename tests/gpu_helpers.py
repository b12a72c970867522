"""Drives the gfx950 kernels through the C ABI for the parity tests."""
import numpy as np

import synth


def run_attn(rl, w, grid_waves=0, max_ctx=None, repeats=1, arena_bytes=None):
    """Uploads a DecodeWorkload, runs rl_hip_attn_decode, returns (out16, out_f32)."""
    layout = rl.KvLayoutDesc.paged(w.token_count, w.head_dim)
    arena = rl.DeviceBuffer.from_array(w.arena)
    table = rl.DeviceBuffer.from_array(w.table)
    ctx = rl.DeviceBuffer.from_array(w.ctx)
    q = rl.DeviceBuffer.from_array(w.q)
    n = w.batch * w.q_heads * w.head_dim
    out = rl.DeviceBuffer(n * 2)
    out32 = rl.DeviceBuffer(n * 4)
    mc = w.max_ctx if max_ctx is None else max_ctx
    args = rl.attn_args(arena, layout, table, w.table_stride, w.batch, w.q_heads, w.kv_heads,
                        rl.DTYPE_BF16 if w.dtype == "bf16" else rl.DTYPE_FP16, ctx, max(mc, 1), q, out, out32,
                        grid_waves=grid_waves)
    if arena_bytes is not None:
        args.arena_bytes = arena_bytes
    ws = rl.attn_workspace(args)
    results = []
    for _ in range(repeats):
        rl.attn_decode(args)
        rl.sync()
        results.append((out.download(np.uint16, (w.batch, w.q_heads, w.head_dim)),
                        out32.download(np.float32, (w.batch, w.q_heads, w.head_dim))))
    for b in (arena, table, ctx, q, out, out32, ws):
        b.close()
    return results if repeats > 1 else results[0]


def rownorm_err(got, ref):
    """max_d |got - ref| / max_d |ref| per (rollout, head); 0-rows compare absolutely."""
    num = np.abs(got.astype(np.float64) - ref).max(axis=-1)
    den = np.abs(ref).max(axis=-1)
    return np.where(den > 0, num / np.maximum(den, 1e-300), num)


def check_attn(out16, out32, ref, dtype):
    """The fp32-accumulated result is within 1e-4 of fp64 (row-normalised),
    i.e. well inside the 2e-3 relative budget; the stored 2-byte output is
    exactly the round-to-nearest-even of that fp32 value, so its distance to
    fp64 is bounded by the format's own half-ulp: 2^-8 relative for bf16
    (8 significant bits), 2^-11 for fp16, plus the fp32 error."""
    assert np.isfinite(out32).all()
    e32 = rownorm_err(out32, ref).max()
    assert e32 < 1e-4, e32
    assert np.array_equal(out16, synth.to_scalar16(out32, dtype))
    half_ulp = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    e16 = rownorm_err(synth.from_scalar16(out16, dtype), ref).max()
    assert e16 <= half_ulp + 1e-4, e16
    return e32, e16
