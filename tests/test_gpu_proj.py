"""Logits projection on MFMA vs an fp64 GEMM of the same bf16 operands.

logits = X[rows, hidden] . W[vocab, hidden]^T, X ~N(0,1), W ~N(0, 0.02^2)
(the rollout-loop shape is 512 x 4096 -> 32,000). The products of bf16 values
are exact in fp32, so the only error is fp32 summation: any summation order
keeps |got - exact| <= (hidden - 1) * 2^-24 * sum_k |x_k w_k| (first order);
the test allows twice that. A transposed operand, a wrong row or a dropped
K step breaks the bound by orders of magnitude.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _case(rl, rows, vocab, hidden, seed, check_rows=None, check_cols=None, repeats=1):
    print(f"[proj] rows={rows} vocab={vocab} hidden={hidden}", flush=True)
    rng = np.random.default_rng(seed)
    x = synth.f32_to_bf16(rng.standard_normal((rows, hidden), dtype=np.float32))
    w = synth.f32_to_bf16(rng.standard_normal((vocab, hidden), dtype=np.float32) * np.float32(0.02))
    dx, dw = rl.DeviceBuffer.from_array(x), rl.DeviceBuffer.from_array(w)
    out = rl.DeviceBuffer(rows * vocab * 4)
    timer = rl.Timer()
    rl.logits_proj(dx, dw, out, rows, vocab, hidden)
    rl.sync()
    timer.begin()
    for _ in range(repeats):
        rl.logits_proj(dx, dw, out, rows, vocab, hidden)
    ms = timer.end() / repeats
    got = out.download(np.float32, (rows, vocab))
    xr = np.arange(rows) if check_rows is None else check_rows
    vc = np.arange(vocab) if check_cols is None else check_cols
    xf = synth.bf16_to_f32(x).astype(np.float64)
    wf = synth.bf16_to_f32(w).astype(np.float64)
    ref = xf[xr] @ wf[vc].T
    mag = np.abs(xf[xr]) @ np.abs(wf[vc]).T
    err = np.abs(got[np.ix_(xr, vc)] - ref)
    bound = 2.0 * (hidden - 1) * 2.0**-24 * mag
    assert np.all(err <= bound + 1e-30), float((err / np.maximum(bound, 1e-30)).max())
    print(f"[proj] max err {err.max():.3e}, worst err/bound {(err / np.maximum(bound, 1e-30)).max():.3f}, "
          f"{ms * 1e3:.1f} us, {2.0 * rows * vocab * hidden / (ms * 1e-3) / 1e12:.1f} TFLOP/s", flush=True)
    for b in (dx, dw, out):
        b.close()


# up to 256 rows the 256 x 128 tile, above it the 256 x 256 tile (three M
# tiles and a partial N tile at 700 x 777)
@pytest.mark.parametrize("rows,vocab,hidden", [(1, 129, 64), (130, 1000, 128), (64, 32000, 256),
                                               (256, 130, 192), (200, 4000, 128), (257, 300, 4096),
                                               (700, 777, 192)])
def test_projection_shapes(rl, gpu, rows, vocab, hidden):
    _case(rl, rows, vocab, hidden, seed=rows + vocab + hidden)


def test_projection_loop_shape(rl, gpu):
    """256 x 4096 -> 32,000 (the rollout loop's 256 slots, the tile whose
    waves split the X and W copies): every column of 24 rows, every row of
    64 columns."""
    rng = np.random.default_rng(6)
    rows = np.sort(rng.choice(256, 24, replace=False))
    _case(rl, 256, 32000, 4096, seed=8, check_rows=rows, repeats=5)
    cols = np.sort(rng.choice(32000, 64, replace=False))
    _case(rl, 256, 32000, 4096, seed=8, check_cols=cols)


def test_projection_rollout_shape(rl, gpu):
    """512 x 4096 -> 32,000: every column of 24 rows, every row of 64 columns."""
    rng = np.random.default_rng(5)
    rows = np.sort(rng.choice(512, 24, replace=False))
    _case(rl, 512, 32000, 4096, seed=4, check_rows=rows, repeats=5)
    cols = np.sort(rng.choice(32000, 64, replace=False))
    _case(rl, 512, 32000, 4096, seed=4, check_cols=cols)


@pytest.mark.parametrize("rows,vocab,hidden,pad_x,pad_w,pad_o", [(130, 1000, 128, 8, 24, 3), (300, 517, 192, 64, 8, 1)])
def test_projection_padded_strides(rl, gpu, rows, vocab, hidden, pad_x, pad_w, pad_o):
    """Row strides past the data (x, w padded by multiples of 8 elements, the
    logits by any count): the padding is never read as data, the logits'
    padding is never written, and the result meets the same bound as the
    contiguous case. Both tiles (up to and above 256 rows)."""
    import ctypes as C
    print(f"[proj] padded strides rows={rows} vocab={vocab} hidden={hidden}", flush=True)
    rng = np.random.default_rng(rows + pad_w)
    xs, ws, los = hidden + pad_x, hidden + pad_w, vocab + pad_o
    x = np.full((rows, xs), synth.f32_to_bf16(np.float32([1e4]))[0], dtype=np.uint16)
    w = np.full((vocab, ws), synth.f32_to_bf16(np.float32([-1e4]))[0], dtype=np.uint16)
    x[:, :hidden] = synth.f32_to_bf16(rng.standard_normal((rows, hidden), dtype=np.float32))
    w[:, :hidden] = synth.f32_to_bf16(rng.standard_normal((vocab, hidden), dtype=np.float32) * np.float32(0.02))
    sentinel = np.float32(-12345.5)
    dx, dw = rl.DeviceBuffer.from_array(x), rl.DeviceBuffer.from_array(w)
    out = rl.DeviceBuffer.from_array(np.full((rows, los), sentinel, np.float32))
    a = rl.ProjArgs(x=dx.ptr, w=dw.ptr, logits=out.ptr, rows=rows, vocab=vocab, hidden=hidden, x_stride=xs,
                    w_stride=ws, logits_stride=los)
    rl.check(rl.lib().rl_hip_logits_proj(C.byref(a)), "rl_hip_logits_proj")
    rl.sync()
    got = out.download(np.float32, (rows, los))
    assert (got[:, vocab:] == sentinel).all()
    xf = synth.bf16_to_f32(x[:, :hidden]).astype(np.float64)
    wf = synth.bf16_to_f32(w[:, :hidden]).astype(np.float64)
    ref = xf @ wf.T
    bound = 2.0 * (hidden - 1) * 2.0**-24 * (np.abs(xf) @ np.abs(wf).T)
    err = np.abs(got[:, :vocab] - ref)
    assert np.all(err <= bound + 1e-30), float((err / np.maximum(bound, 1e-30)).max())
    for b in (dx, dw, out):
        b.close()
