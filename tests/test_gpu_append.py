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
