"""KV append with copy-on-write on the GPU vs the oracle (bit-exact arena)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,tpb", [(128, 16), (64, 16), (128, 32)])
def test_append_with_cow(rl, gpu, olib, d, tpb):
    rng = np.random.default_rng(d + tpb)
    B, H, stride = 64, 8, 8
    row = d * 2
    block = 2 * tpb * row
    nblocks = B * H * stride + 64
    arena = rng.integers(0, 256, nblocks * block, dtype=np.uint8)
    table = rng.permutation(B * H * stride).astype(np.uint32).reshape(B, H, stride)
    pos = rng.integers(0, stride * tpb, B).astype(np.uint32)
    cow = np.full((B, H), -1, dtype=np.int32)
    shared = B * H * stride + rng.integers(0, 64, (B, H))
    cow[::3] = shared[::3]                                  # a third of the rollouts copy-on-write
    kn = rng.integers(0, 256, (B, H, row), dtype=np.uint8)
    vn = rng.integers(0, 256, (B, H, row), dtype=np.uint8)
    ref = arena.copy()
    olib.orc_kv_append(ref.ctypes.data, block, tpb, row, table.ctypes.data, stride, B, H, pos.ctypes.data,
                       cow.ctypes.data, kn.ctypes.data, vn.ctypes.data)
    bufs = [rl.DeviceBuffer.from_array(a) for a in (arena, table, pos, cow, kn, vn)]
    a = rl.AppendArgs()
    a.arena_base, a.arena_bytes, a.layout = bufs[0].ptr, bufs[0].nbytes, rl.KvLayoutDesc.paged(tpb, d)
    a.block_table, a.table_stride, a.batch, a.kv_heads = bufs[1].ptr, stride, B, H
    a.positions, a.cow_src, a.k_new, a.v_new = bufs[2].ptr, bufs[3].ptr, bufs[4].ptr, bufs[5].ptr
    rl.kv_append(a)
    rl.sync()
    got = bufs[0].download(np.uint8, arena.shape)
    assert np.array_equal(got, ref)
    for b in bufs:
        b.close()


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_decode_step_equals_attention_then_append(rl, gpu, orc, olib, dtype):
    """rl_hip_decode_step (the append inside the attention's merge kernel)
    gives the same bytes as rl_hip_attn_decode followed by rl_hip_kv_append:
    outputs, fp32 outputs and the whole arena, with copy-on-write for a third
    of the rows; the attention matches fp64 over the arena as it was before
    the append, and the arena matches the oracle's append."""
    import gpu_helpers as gh
    import synth

    B, QH, KVH, D, TPB = 24, 32, 8, 128, 16
    w = synth.make_decode(31, B, QH, KVH, D, 200, 1500, dtype=dtype, spare_blocks=40)
    rng = np.random.default_rng(32)
    pos = w.ctx.copy()                                        # the slot right after each context
    n_used = w.arena.size // w.block_bytes - 40
    cow = np.full((B, KVH), -1, np.int32)
    cow[::3] = n_used + rng.integers(0, 40, (len(cow[::3]), KVH))
    kn = rng.integers(0, 256, (B, KVH, D * 2), dtype=np.uint8)
    vn = rng.integers(0, 256, (B, KVH, D * 2), dtype=np.uint8)
    layout = rl.KvLayoutDesc.paged(TPB, D)
    n = B * QH * D
    res = []
    for fused in (False, True):
        bufs = {k: rl.DeviceBuffer.from_array(v) for k, v in
                (("arena", w.arena), ("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", pos), ("cow", cow),
                 ("kn", kn), ("vn", vn))}
        out, out32 = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4)
        a = rl.attn_args(bufs["arena"], layout, bufs["table"], w.table_stride, B, QH, KVH,
                         rl.DTYPE_BF16 if dtype == "bf16" else rl.DTYPE_FP16, bufs["ctx"], w.max_ctx, bufs["q"],
                         out, out32)
        ws = rl.attn_workspace(a)
        ap = rl.AppendArgs(arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes, layout=layout,
                           block_table=bufs["table"].ptr, table_stride=w.table_stride, batch=B, kv_heads=KVH,
                           positions=bufs["pos"].ptr, cow_src=bufs["cow"].ptr, k_new=bufs["kn"].ptr,
                           v_new=bufs["vn"].ptr)
        if fused:
            rl.decode_step(a, ap)
        else:
            rl.attn_decode(a)
            rl.kv_append(ap)
        rl.sync()
        res.append((out.download(np.uint16, n), out32.download(np.float32, (B, QH, D)),
                    bufs["arena"].download(np.uint8, w.arena.size)))
        for b in list(bufs.values()) + [out, out32, ws]:
            b.close()
    (o16a, o32a, ara), (o16b, o32b, arb) = res
    assert np.array_equal(o16a, o16b) and np.array_equal(o32a, o32b)
    assert np.array_equal(ara, arb)
    ref_arena = w.arena.copy()
    olib.orc_kv_append(ref_arena.ctypes.data, w.block_bytes, TPB, D * 2, w.table.ctypes.data, w.table_stride, B, KVH,
                       pos.ctypes.data, cow.ctypes.data, kn.ctypes.data, vn.ctypes.data)
    assert np.array_equal(arb, ref_arena)
    gh.check_attn(o16b.reshape(B, QH, D), o32b, orc.attn_f64(olib, w, 0 if dtype == "bf16" else 1), dtype)
