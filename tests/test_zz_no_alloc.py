"""rl_hip_decode_step_noalloc (the fused decode step on the library's fixed
scratch array) against rl_hip_decode_step (caller workspace): outputs, fp32
outputs and the appended arena bit-identical, over two calls in a row with the
second smaller, so stale scratch contents from the first would show."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

QH, KVH, D, TPB = 32, 8, 128, 16


def _case(synth, seed, batch, lo, hi, cow_every):
    w = synth.make_decode(seed, batch, QH, KVH, D, lo, hi, spare_blocks=32)
    rng = np.random.default_rng(seed + 1)
    n_used = w.arena.size // w.block_bytes - 32
    cow = np.full((batch, KVH), -1, np.int32)
    cow[::cow_every] = n_used + rng.integers(0, 32, (len(cow[::cow_every]), KVH))
    kn = rng.integers(0, 256, (batch, KVH, D * 2), dtype=np.uint8)
    vn = rng.integers(0, 256, (batch, KVH, D * 2), dtype=np.uint8)
    return w, w.ctx.copy(), cow, kn, vn


class _Step:
    """Device copies of one case and the argument structs of its decode step."""

    def __init__(self, rl, case, with_workspace):
        w, pos, cow, kn, vn = case
        self.w = w
        self.bufs = {k: rl.DeviceBuffer.from_array(v) for k, v in
                     (("arena", w.arena), ("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", pos),
                      ("cow", cow), ("kn", kn), ("vn", vn))}
        n = w.batch * QH * D
        self.out, self.out32 = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4)
        layout = rl.KvLayoutDesc.paged(TPB, D)
        b = self.bufs
        self.a = rl.attn_args(b["arena"], layout, b["table"], w.table_stride, w.batch, QH, KVH, rl.DTYPE_BF16,
                              b["ctx"], w.max_ctx, b["q"], self.out, self.out32)
        self.ws = rl.attn_workspace(self.a) if with_workspace else None
        self.ap = rl.AppendArgs(arena_base=b["arena"].ptr, arena_bytes=b["arena"].nbytes, layout=layout,
                                block_table=b["table"].ptr, table_stride=w.table_stride, batch=w.batch,
                                kv_heads=KVH, positions=b["pos"].ptr, cow_src=b["cow"].ptr, k_new=b["kn"].ptr,
                                v_new=b["vn"].ptr)

    def results(self, rl):
        w = self.w
        n = w.batch * QH * D
        return (self.out.download(np.uint16, n), self.out32.download(np.float32, (w.batch, QH, D)),
                self.bufs["arena"].download(np.uint8, w.arena.size))

    def close(self):
        for b in list(self.bufs.values()) + [self.out, self.out32] + ([self.ws] if self.ws else []):
            b.close()


def test_noalloc_step_equals_decode_step_twice(rl, gpu, orc, olib):
    import gpu_helpers as gh
    import synth

    cases = [_case(synth, 71, 48, 300, 3000, 3), _case(synth, 72, 10, 20, 700, 2)]
    # the existing entry point, each case with its own workspace
    want = []
    for c in cases:
        s = _Step(rl, c, True)
        rl.decode_step(s.a, s.ap)
        rl.sync()
        want.append(s.results(rl))
        s.close()
    # the no-alloc entry point: two calls in a row on the shared scratch, the second smaller
    steps = [_Step(rl, c, False) for c in cases]
    for s in steps:
        assert s.a.workspace is None
        rl.decode_step_noalloc(s.a, s.ap)
    rl.sync()
    for i, (s, c, ref) in enumerate(zip(steps, cases, want)):
        got = s.results(rl)
        assert np.array_equal(got[0], ref[0]), f"call {i}: bf16 outputs differ"
        assert np.array_equal(got[1], ref[1]), f"call {i}: fp32 outputs differ"
        assert np.array_equal(got[2], ref[2]), f"call {i}: arenas differ"
        w, pos, cow, kn, vn = c
        gh.check_attn(got[0].reshape(w.batch, QH, D), got[1], orc.attn_f64(olib, w, 0), "bf16")
        s.close()


def test_noalloc_step_refuses_more_than_its_scratch(rl, gpu):
    """A step whose workspace exceeds the scratch is refused before any launch.
    Every buffer is sized for the whole call, all contexts are 0 and every
    append position lies past the table, so even a launch would stay in bounds."""
    B = 4096
    layout = rl.KvLayoutDesc.paged(TPB, D)
    arena = rl.DeviceBuffer(layout.block_bytes, zero=True)
    table = rl.DeviceBuffer(B * KVH * 4, zero=True)
    ctx = rl.DeviceBuffer(B * 4, zero=True)
    q = rl.DeviceBuffer(B * QH * D * 2, zero=True)
    out = rl.DeviceBuffer(B * QH * D * 2)
    pos = rl.DeviceBuffer.from_array(np.full(B, 1 << 20, np.uint32))
    kv = rl.DeviceBuffer(B * KVH * D * 2, zero=True)
    a = rl.attn_args(arena, layout, table, 1, B, QH, KVH, rl.DTYPE_BF16, ctx, 16, q, out)
    need = rl.lib().rl_hip_attn_decode_workspace(rl.C.byref(a))
    assert need > rl.DECODE_STEP_NOALLOC_SCRATCH_BYTES
    ap = rl.AppendArgs(arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=layout, block_table=table.ptr,
                       table_stride=1, batch=B, kv_heads=KVH, positions=pos.ptr, cow_src=None, k_new=kv.ptr,
                       v_new=kv.ptr)
    with pytest.raises(rl.RlrtError, match="above the"):
        rl.decode_step_noalloc(a, ap)
    rl.sync()
    for b in (arena, table, ctx, q, out, pos, kv):
        b.close()
