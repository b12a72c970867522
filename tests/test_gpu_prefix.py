"""The prefix table on the device: kv_branch_resolve (cu/kv_prefix.cu:4-23)
over the byte-compatible KVPrefixTable image against the oracle, and the
copy-on-write of a prefix's partly filled block before the step's attention
reads it (rl_hip_kv_cow, then rl_hip_decode_step through one table)."""
import ctypes as C

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

TABLE_BYTES = 606280
MAX_BRANCHES = 16384


def _random_table(L, rng):
    """A table built by the library's host rules (src/kv_prefix.c) with live,
    released and out-of-range prefixes, live and freed branches."""
    t = np.zeros(TABLE_BYTES, np.uint8)
    L.kv_prefix_table_init(t.ctypes.data)
    pid, bid = C.c_uint32(), C.c_uint32()
    prefixes = []
    for _ in range(300):
        assert L.kv_prefix_register(t.ctypes.data, int(rng.integers(0, 2**40)), int(rng.integers(1, 4000)),
                                    int(rng.integers(1, 900)), C.byref(pid)) == 0
        prefixes.append(pid.value)
    branches = []
    for _ in range(9000):
        p = int(rng.choice(prefixes)) if rng.random() < 0.9 else int(rng.integers(512, 2**32))
        assert L.kv_branch_alloc(t.ctypes.data, int(rng.integers(0, 2**32)), p, int(rng.integers(-2**40, 2**40)),
                                 int(rng.integers(0, 999)), int(rng.integers(0, 99)), C.byref(bid)) == 0
        branches.append(bid.value)
    for b in rng.choice(branches, 2500, replace=False):
        assert L.kv_branch_free(t.ctypes.data, int(b)) == 0
    for p in rng.choice(prefixes, 120, replace=False):   # drop every reference of some prefixes
        while L.kv_prefix_release(t.ctypes.data, int(p)) == 0:
            pass
    return t


def test_branch_resolve_matches_oracle(rl, gpu, olib):
    L = rl.lib()
    rng = np.random.default_rng(77)
    for trial in range(3):
        t = _random_table(L, rng)
        ids = np.concatenate([np.arange(MAX_BRANCHES + 40, dtype=np.uint32),
                              rng.integers(0, 2**32, 1000, dtype=np.uint32)])
        dt, di, do = (rl.DeviceBuffer.from_array(t), rl.DeviceBuffer.from_array(ids),
                      rl.DeviceBuffer(ids.size * 8, zero=True))
        rl.check(L.rl_hip_kv_branch_resolve(dt.ptr, di.ptr, do.ptr, ids.size), "rl_hip_kv_branch_resolve")
        rl.sync()
        got = do.download(np.int64, ids.size)
        want = np.array([olib.orc_kvb_resolve(t.ctypes.data, int(i)) for i in ids], np.int64)
        assert np.array_equal(got, want), trial
        # the device rule differs from the host total_offset exactly where a
        # branch names a prefix whose refcount fell to 0
        host = np.array([L.kv_branch_total_offset(t.ctypes.data, int(i)) for i in ids[:MAX_BRANCHES]], np.int64)
        diff = np.nonzero(host != got[:MAX_BRANCHES])[0]
        assert len(diff) > 0
        for i in diff:
            pid = L.kv_branch_get(t.ctypes.data, int(i)).contents.prefix_id
            assert pid < 512 and L.kv_prefix_get(t.ctypes.data, pid).contents.refcnt == 0
        for b in (dt, di, do):
            b.close()


def test_cow_before_attention_then_decode_step(rl, gpu, orc, olib):
    """16 rows, each with its own prefix (GQA 32/8, d128, bf16): rows 0-11 at
    their first own token of a prefix ending inside a block (copy-on-write),
    row 12 one token later (no copy), row 13 on a prefix ending on a block
    boundary, row 14 on a released prefix, row 15 on a branch with an
    out-of-range prefix id. Step 1: rl_hip_kv_cow, then rl_hip_decode_step
    through one table mapping the private blocks; the attention equals fp64
    over the arena with the copies made, the arena equals the oracle's
    copy-on-write plus append. Step 2 attends one token further over the same
    table and matches fp64 too."""
    L = rl.lib()
    rng = np.random.default_rng(91)
    B, QH, KVH, D, TPB = 16, 32, 8, 128, 16
    lens = rng.integers(17, 700, B).astype(np.int64)
    lens[lens % TPB == 0] += 3
    lens[13] = 640                                           # ends on a block boundary
    per_head = -(-lens // TPB)
    nblk = int(per_head.sum()) * KVH + B * KVH * 2 + 8
    stride = int(per_head.max()) + 2
    n_prefix_blocks = int(per_head.sum()) * KVH
    arena = np.empty(nblk * 2 * TPB * D, np.uint16)
    synth._fill_normal(rng, arena.size, 1.0, "bf16", arena)
    arena = arena.view(np.uint8)
    t = np.zeros(TABLE_BYTES, np.uint8)
    L.kv_prefix_table_init(t.ctypes.data)
    table = np.zeros((B, KVH, stride), np.uint32)
    pos = np.zeros(B, np.uint32)
    branch = np.zeros(B, np.uint32)
    # prefix ranges must be contiguous: take them from the front of the block space
    nxt = 0
    private = list((n_prefix_blocks + rng.permutation(nblk - n_prefix_blocks)).astype(np.uint32))
    pid, bid = C.c_uint32(), C.c_uint32()
    for b in range(B):
        base = nxt
        nxt += int(per_head[b]) * KVH
        assert L.kv_prefix_register(t.ctypes.data, base, int(lens[b]), int(per_head[b]) * KVH, C.byref(pid)) == 0
        n_sh = int(lens[b]) // TPB
        for h in range(KVH):
            table[b, h, :n_sh] = base + h * per_head[b] + np.arange(n_sh)
            table[b, h, n_sh] = private.pop()
            table[b, h, n_sh + 1] = private.pop()
        prefix_id = pid.value if b != 15 else 700
        assert L.kv_branch_alloc(t.ctypes.data, b, prefix_id, 5, 0, 1, C.byref(bid)) == 0
        branch[b] = bid.value
        pos[b] = lens[b] + (1 if b == 12 else 0)
    while L.kv_prefix_release(t.ctypes.data, 14) == 0:
        pass
    ctx = pos.copy()
    # the appended rows are attended by step 2: finite bf16 values, not random bytes
    kn = [synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32)).view(np.uint8) for _ in range(2)]
    vn = [synth.f32_to_bf16(rng.standard_normal((B, KVH, D), dtype=np.float32)).view(np.uint8) for _ in range(2)]
    q = [synth.f32_to_bf16(rng.standard_normal((B, QH, D), dtype=np.float32)) for _ in range(2)]

    # oracle: copy-on-write sources, then the appends of both steps
    cow = np.array([[olib.orc_kvb_cow_source(t.ctypes.data, int(branch[b]), int(pos[b]), TPB, KVH, h)
                     for h in range(KVH)] for b in range(B)], np.int32)
    assert (cow[:12] >= 0).all() and (cow[12:] < 0).all()
    block = 2 * TPB * D * 2
    ref1 = arena.copy()
    olib.orc_kv_append(ref1.ctypes.data, block, TPB, D * 2, table.ctypes.data, stride, B, KVH, pos.ctypes.data,
                       cow.ctypes.data, kn[0].ctypes.data, vn[0].ctypes.data)
    pos2 = pos + 1
    ref2 = ref1.copy()
    none = np.full((B, KVH), -1, np.int32)
    olib.orc_kv_append(ref2.ctypes.data, block, TPB, D * 2, table.ctypes.data, stride, B, KVH, pos2.ctypes.data,
                       none.ctypes.data, kn[1].ctypes.data, vn[1].ctypes.data)

    dev = {k: rl.DeviceBuffer.from_array(v) for k, v in
           (("arena", arena), ("table", table), ("ptab", t), ("branch", branch), ("pos", pos), ("ctx", ctx),
            ("q0", q[0]), ("q1", q[1]), ("k0", kn[0]), ("v0", vn[0]), ("k1", kn[1]), ("v1", vn[1]))}
    dev["status"] = rl.DeviceBuffer(B * KVH * 4, zero=True)
    layout = rl.KvLayoutDesc.paged(TPB, D)
    out, out32 = rl.DeviceBuffer(B * QH * D * 2), rl.DeviceBuffer(B * QH * D * 4)
    cw = rl.CowArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=layout,
                    prefixes=dev["ptab"].ptr, row_key=dev["branch"].ptr, branch_of_key=None, keys=0,
                    block_table=dev["table"].ptr, table_stride=stride, batch=B, kv_heads=KVH, positions=dev["pos"].ptr,
                    row_status=dev["status"].ptr)
    a = rl.attn_args(dev["arena"], layout, dev["table"], stride, B, QH, KVH, rl.DTYPE_BF16, dev["ctx"],
                     int(pos2.max()), dev["q0"], out, out32)
    ws = rl.attn_workspace(a)
    ap = rl.AppendArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=layout,
                       block_table=dev["table"].ptr, table_stride=stride, batch=B, kv_heads=KVH,
                       positions=dev["pos"].ptr, cow_src=None, k_new=dev["k0"].ptr, v_new=dev["v0"].ptr)
    import gpu_helpers as gh
    for step in range(2):
        rl.kv_cow(cw)
        rl.decode_step(a, ap)
        rl.sync()
        got = dev["arena"].download(np.uint8, arena.size)
        assert np.array_equal(got, ref1 if step == 0 else ref2), step
        status = dev["status"].download(np.uint32, (B, KVH))
        want = np.full((B, KVH), rl.COW_NONE, np.uint32)
        if step == 0:
            want[:12] = rl.COW_COPIED                          # rows 12-15: no copy due (see above)
        assert np.array_equal(status, want), (step, status)
        w = synth.DecodeWorkload(B, QH, KVH, D, "bf16", TPB, ctx + step, table, got, q[step], 0)
        gh.check_attn(out.download(np.uint16, (B, QH, D)), out32.download(np.float32, (B, QH, D)),
                      orc.attn_f64(olib, w, 0), "bf16")
        # step 2: one token further, same table; no row is at its first own token any more
        dev["pos"].upload(pos2)
        dev["ctx"].upload(ctx + 1)
        a.q, ap.k_new, ap.v_new = dev["q1"].ptr, dev["k1"].ptr, dev["v1"].ptr
    for b in list(dev.values()) + [out, out32, ws]:
        b.close()


def test_cow_reports_shared_and_out_of_range(rl, gpu):
    """Four rows on four prefixes of 20 tokens (2 KV heads, d64, 16-token
    blocks: slot 4 of block 1 is each branch's first own token): row 0 maps a
    private block (copied), row 1 maps the prefix's own block 1 (RL_COW_SHARED,
    nothing copied), row 2 maps a block id past the arena (RL_COW_OUT_OF_RANGE,
    nothing written), row 3 is one token past its first own token (no copy due).
    The arena changes only in row 0's private blocks, by the 4 filled slots of
    each plane of the prefix block."""
    L = rl.lib()
    rng = np.random.default_rng(93)
    B, KVH, D, TPB, P = 4, 2, 64, 16, 20
    per_head = 2
    n_prefix_blocks = B * KVH * per_head
    nblk = n_prefix_blocks + B * KVH * 2
    block = 2 * TPB * D * 2
    arena = rng.integers(0, 256, nblk * block, dtype=np.uint8)
    t = np.zeros(TABLE_BYTES, np.uint8)
    L.kv_prefix_table_init(t.ctypes.data)
    table = np.zeros((B, KVH, 3), np.uint32)
    branch = np.zeros(B, np.uint32)
    pid, bid = C.c_uint32(), C.c_uint32()
    for b in range(B):
        base = b * KVH * per_head
        assert L.kv_prefix_register(t.ctypes.data, base, P, KVH * per_head, C.byref(pid)) == 0
        assert L.kv_branch_alloc(t.ctypes.data, b, pid.value, 5, 0, 1, C.byref(bid)) == 0
        branch[b] = bid.value
        for h in range(KVH):
            table[b, h, 0] = base + h * per_head
            table[b, h, 1] = n_prefix_blocks + b * KVH + h        # private
            table[b, h, 2] = n_prefix_blocks + B * KVH + b * KVH + h
    table[1, :, 1] = [1 * KVH * per_head + h * per_head + 1 for h in range(KVH)]   # the prefix block itself
    table[2, :, 1] = nblk + 5                                                        # past the arena
    pos = np.array([P, P, P, P + 1], np.uint32)
    dev = {k: rl.DeviceBuffer.from_array(v) for k, v in
           (("arena", arena), ("table", table), ("ptab", t), ("branch", branch), ("pos", pos))}
    status = rl.DeviceBuffer(B * KVH * 4, zero=True)
    cw = rl.CowArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=rl.KvLayoutDesc.paged(TPB, D),
                    prefixes=dev["ptab"].ptr, row_key=dev["branch"].ptr, branch_of_key=None, keys=0,
                    block_table=dev["table"].ptr, table_stride=3, batch=B, kv_heads=KVH, positions=dev["pos"].ptr,
                    row_status=status.ptr)
    print("[prefix] copy-on-write with a shared and an out-of-range entry", flush=True)
    rl.kv_cow(cw)
    rl.sync()
    st = status.download(np.uint32, (B, KVH))
    assert st.tolist() == [[rl.COW_COPIED] * KVH, [rl.COW_SHARED] * KVH, [rl.COW_OUT_OF_RANGE] * KVH,
                           [rl.COW_NONE] * KVH], st
    got = dev["arena"].download(np.uint8, arena.size)
    want = arena.copy().reshape(nblk, block)
    filled = (P % TPB) * D * 2
    for h in range(KVH):
        src = want[0 * KVH * per_head + h * per_head + 1]
        dst = want[table[0, h, 1]]
        dst[:filled] = src[:filled]                                    # K plane
        dst[TPB * D * 2:TPB * D * 2 + filled] = src[TPB * D * 2:TPB * D * 2 + filled]   # V plane
    assert np.array_equal(got, want.reshape(-1))
    for b in list(dev.values()) + [status]:
        b.close()
