"""The KV arena (arena.h, reference src/arena.c:7-58) on the GPU path:
rl_hip_open, then arena_init places `base` in HBM (zero-filled), block ids
come from arena_acquire (lowest clear bit first), and the fused decode step
reads and appends through arena.base.

The batched GQA shape of the benchmark (64 rollouts, 32 q / 8 kv heads, d128,
bf16, ctx U[512, 4096]): every (rollout, kv head, block) takes an id from
arena_acquire, and the ids are dealt to the block tables in a seeded random
order. Checked: the ids are 0, 1, 2, ... in acquisition order; spare blocks
read back as zeros; the attention within 1e-4 of fp64 and the stored bf16 its
rounding; the arena after the step byte-equal to the oracle's append. Then
eight rollouts release their blocks, a new batch acquires them again (the
same lowest ids come back) with fresh contents, and a second step over the
reused blocks is checked the same way."""
import numpy as np
import pytest

import gpu_helpers as gh
import synth

pytestmark = pytest.mark.gpu

B, QH, KVH, D, TPB = 64, 32, 8, 128, 16
SPARE = 64


def _step(rl, orc, olib, arena, w, pos, kn, vn):
    layout = rl.KvLayoutDesc.paged(TPB, D)
    dev = {k: rl.DeviceBuffer.from_array(v) for k, v in
           (("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", pos), ("kn", kn), ("vn", vn))}
    n = w.batch * QH * D
    out, out32 = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4)
    a = rl.attn_args(arena, layout, dev["table"], w.table_stride, w.batch, QH, KVH, rl.DTYPE_BF16, dev["ctx"],
                     w.max_ctx, dev["q"], out, out32)
    ws = rl.attn_workspace(a)
    ap = rl.AppendArgs(arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=layout, block_table=dev["table"].ptr,
                       table_stride=w.table_stride, batch=w.batch, kv_heads=KVH, positions=dev["pos"].ptr,
                       cow_src=None, k_new=dev["kn"].ptr, v_new=dev["vn"].ptr)
    rl.decode_step(a, ap)
    rl.sync()
    o16, o32 = out.download(np.uint16, (w.batch, QH, D)), out32.download(np.float32, (w.batch, QH, D))
    gh.check_attn(o16, o32, orc.attn_f64(olib, w, 0), "bf16")
    for b in list(dev.values()) + [out, out32, ws]:
        b.close()


def _fill(rng, n_blocks):
    a = np.empty(n_blocks * 2 * TPB * D, np.uint16)
    synth._fill_normal(rng, a.size, 1.0, "bf16", a)
    return a.view(np.uint8)


def test_decode_step_over_kvarena(rl, gpu, orc, olib):
    L = rl.lib()
    rng = np.random.default_rng(2024)
    block = 2 * TPB * D * 2
    ctx = rng.integers(512, 4097, B).astype(np.uint32)
    nblk = -(-(ctx.astype(np.int64) + 1) // TPB)              # room for the appended token
    stride = int(nblk.max())
    n = int(nblk.sum()) * KVH
    arena = rl.Arena((n + SPARE) * block, block)
    assert L.arena_is_device(arena.struct.ctypes.data) == 1
    ids = arena.acquire_n(n)
    assert np.array_equal(ids, np.arange(n))                   # lowest clear bit first
    deal = ids[rng.permutation(n)]
    table = np.zeros((B, KVH, stride), np.uint32)
    k = 0
    for b in range(B):
        for g in range(KVH):
            m = int(nblk[b])
            table[b, g, :m] = deal[k:k + m]
            k += m
    image = _fill(rng, n)
    arena.upload(image)
    assert not arena.download(np.uint8, SPARE * block, offset=n * block).any()   # arena_init zero-filled
    q = synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32))
    w = synth.DecodeWorkload(B, QH, KVH, D, "bf16", TPB, ctx, table, image, q, 0)
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32))
    _step(rl, orc, olib, arena, w, ctx.copy(), kn, vn)
    want = np.concatenate([image, np.zeros(SPARE * block, np.uint8)])
    olib.orc_kv_append(want.ctypes.data, block, TPB, D * 2, table.ctypes.data, stride, B, KVH, ctx.ctypes.data,
                       None, kn.ctypes.data, vn.ctypes.data)
    assert np.array_equal(arena.download(np.uint8, arena.nbytes), want)

    # rollouts 8..15 finish: their blocks go back to the bitmap, and the next
    # acquisitions return exactly those ids, lowest first
    freed = np.sort(np.concatenate([table[b, g, :int(nblk[b])] for b in range(8, 16)
                                    for g in range(KVH)]).astype(np.int64))
    for i in freed[::-1]:
        arena.release(int(i))
    again = arena.acquire_n(len(freed))
    assert np.array_equal(again, freed)
    assert arena.acquire() == n                                # then the first never-used block
    # a new batch of 8 rollouts on the reused blocks, fresh contents
    ctx2 = rng.integers(512, 4097, 8).astype(np.uint32)
    nb2 = -(-(ctx2.astype(np.int64) + 1) // TPB)
    assert int(nb2.sum()) * KVH <= len(again)
    table2 = np.zeros((8, KVH, stride), np.uint32)
    deal2 = again[rng.permutation(len(again))]
    k = 0
    host = arena.download(np.uint8, arena.nbytes)
    fresh = _fill(rng, len(again)).reshape(len(again), block)
    for i, blk in enumerate(again):
        host[blk * block:(blk + 1) * block] = fresh[i]
    for i, blk in enumerate(again):
        arena.upload(fresh[i], offset=int(blk) * block)
    for b in range(8):
        for g in range(KVH):
            m = int(nb2[b])
            table2[b, g, :m] = deal2[k:k + m]
            k += m
    q2 = synth.f32_to_bf16(rng.standard_normal((8, QH, D), dtype=np.float32))
    w2 = synth.DecodeWorkload(8, QH, KVH, D, "bf16", TPB, ctx2, table2, host, q2, 0)
    kn2 = synth.f32_to_bf16(rng.standard_normal((8, KVH, D), dtype=np.float32))
    vn2 = synth.f32_to_bf16(rng.standard_normal((8, KVH, D), dtype=np.float32))
    _step(rl, orc, olib, arena, w2, ctx2.copy(), kn2, vn2)
    olib.orc_kv_append(host.ctypes.data, block, TPB, D * 2, table2.ctypes.data, stride, 8, KVH, ctx2.ctypes.data,
                       None, kn2.ctypes.data, vn2.ctypes.data)
    assert np.array_equal(arena.download(np.uint8, arena.nbytes), host)
    arena.close()
    assert arena.ptr is None
