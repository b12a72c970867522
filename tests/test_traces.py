"""Random operation traces replayed through three implementations of the
integer host path: the runtime (librlrt_amd.so + its header-inline ring
functions), the oracle's byte-image restatement, and the reference's own C
sources compiled into oracle/_ref (where they build). Return codes, popped
items and the final memory images must agree bit for bit. CPU only."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import helpers

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def prod_shim(rl):
    return helpers.load_shared("tests/c/prod_shim.c")


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def _img(n):
    return np.zeros(n, dtype=np.uint8)


def _setup(lib, name, res, args):
    f = getattr(lib, name)
    f.restype, f.argtypes = res, args
    return f


def test_hw_ring_trace(prod_shim, olib, orc, ref):
    vp = C.c_void_p
    impls = []
    for lib, pre in ((prod_shim, "prod_"), (ref, "ref_")):
        push = _setup(lib, pre + "hw_ring_push", C.c_int, [vp, vp])
        pop = _setup(lib, pre + "hw_ring_pop", C.c_int, [vp, vp])
        impls.append((push, pop))
    impls.append((olib.orc_hw_ring_push, olib.orc_hw_ring_pop))
    rings = [_img(4194432) for _ in impls]
    rng = np.random.default_rng(1)
    # long enough to wrap the 65,536-slot ring and hit full/empty
    depth = 0
    for step in range(200_000):
        if depth >= 65536 or (depth > 0 and rng.random() < 0.45):
            outs = []
            for (push, pop), ring in zip(impls, rings):
                o = np.zeros(64, dtype=np.uint8)
                outs.append((pop(ring.ctypes.data, o.ctypes.data), o.tobytes()))
            assert outs[0] == outs[1] == outs[2], step
            depth -= outs[0][0] == 0
        else:
            d = rng.integers(0, 256, 64, dtype=np.uint8)
            rcs = [push(ring.ctypes.data, d.ctypes.data) for (push, pop), ring in zip(impls, rings)]
            assert rcs[0] == rcs[1] == rcs[2], step
            depth += rcs[0] == 0
        if step == 100_000:  # fill to the brim once
            while depth < 65537:
                d = rng.integers(0, 256, 64, dtype=np.uint8)
                rcs = [push(ring.ctypes.data, d.ctypes.data) for (push, pop), ring in zip(impls, rings)]
                assert rcs[0] == rcs[1] == rcs[2]
                if rcs[0] != 0:
                    break
                depth += 1
    assert np.array_equal(rings[0], rings[1]) and np.array_equal(rings[0], rings[2])


def _generic_ring_trace(kind, prod_shim, olib, orc, ref, steps=30_000, seed=2):
    vp, u32 = C.c_void_p, C.c_uint32
    shape = {"cmd": orc.CMD_RING, "comp": orc.COMP_RING, "req": orc.REQ_RING, "done": orc.DONE_RING}[kind]
    size = {"cmd": 131200, "comp": 131328, "req": 34944, "done": 24832}[kind]
    rings = [_img(size) for _ in range(3)]
    rng = np.random.default_rng(seed)
    names = {"cmd": ("ring_acquire", "ring_consume"), "req": ("req_ring_acquire", "req_ring_consume"),
             "comp": ("comp_ring_push", "comp_ring_poll"), "done": ("done_ring_push", "done_ring_pop")}[kind]
    libs = [(prod_shim, "prod_"), (ref, "ref_")]
    if kind in ("cmd", "req"):
        acq = [_setup(l, p + names[0], u32, [vp, u32] if kind == "cmd" else [vp]) for l, p in libs]
        com = [_setup(l, p + ("ring_commit" if kind == "cmd" else "req_ring_commit"), None,
                      [vp, u32] if kind == "cmd" else [vp]) for l, p in libs]
        con = [_setup(l, p + names[1], C.c_int, [vp, vp]) for l, p in libs]
        for step in range(steps):
            if rng.random() < 0.5:
                n = int(rng.integers(1, 40)) if kind == "cmd" else 1
                pos = [a(r.ctypes.data, n) if kind == "cmd" else a(r.ctypes.data) for a, r in zip(acq, rings[:2])]
                pos.append(olib.orc_ring_acquire(rings[2].ctypes.data, C.byref(shape), n))
                assert pos[0] == pos[1] == pos[2], step
                if pos[0] != 0xFFFFFFFF:
                    items = rng.integers(0, 256, n * shape.slot_size, dtype=np.uint8)
                    for r in rings:
                        for i in range(n):
                            off = shape.slot_off + ((pos[0] + i) % shape.n_slots) * shape.slot_size
                            r[off:off + shape.slot_size] = items[i * shape.slot_size:(i + 1) * shape.slot_size]
                    for c_, r in zip(com, rings[:2]):
                        c_(r.ctypes.data, n) if kind == "cmd" else c_(r.ctypes.data)
                    olib.orc_ring_commit(rings[2].ctypes.data, n)
            else:
                outs = []
                for c_, r in zip(con, rings[:2]):
                    o = np.zeros(shape.slot_size, dtype=np.uint8)
                    outs.append((c_(r.ctypes.data, o.ctypes.data), o.tobytes()))
                o = np.zeros(shape.slot_size, dtype=np.uint8)
                outs.append((olib.orc_ring_consume(rings[2].ctypes.data, C.byref(shape), o.ctypes.data), o.tobytes()))
                assert outs[0] == outs[1] == outs[2], step
    else:
        push = [_setup(l, p + names[0], C.c_int, [vp, vp]) for l, p in libs]
        pop = [_setup(l, p + names[1], C.c_int, [vp, vp]) for l, p in libs]
        for step in range(steps):
            if rng.random() < 0.55:
                it = rng.integers(0, 256, shape.slot_size, dtype=np.uint8)
                rcs = [f(r.ctypes.data, it.ctypes.data) for f, r in zip(push, rings[:2])]
                rcs.append(olib.orc_ring_push_or_overflow(rings[2].ctypes.data, C.byref(shape), it.ctypes.data))
                assert rcs[0] == rcs[1] == rcs[2], step
            else:
                outs = []
                for f, r in zip(pop, rings[:2]):
                    o = np.zeros(shape.slot_size, dtype=np.uint8)
                    outs.append((f(r.ctypes.data, o.ctypes.data), o.tobytes()))
                o = np.zeros(shape.slot_size, dtype=np.uint8)
                outs.append((olib.orc_ring_consume(rings[2].ctypes.data, C.byref(shape), o.ctypes.data), o.tobytes()))
                assert outs[0] == outs[1] == outs[2], step
    assert np.array_equal(rings[0], rings[1]) and np.array_equal(rings[0], rings[2])


@pytest.mark.parametrize("kind", ["cmd", "comp", "req", "done"])
def test_v02_v03_ring_traces(kind, prod_shim, olib, orc, ref):
    _generic_ring_trace(kind, prod_shim, olib, orc, ref)


def test_decode_batch_submit_trace(rl, prod_shim, olib, orc, ref):
    vp = C.c_void_p
    ref_submit = _setup(ref, "decode_batch_submit", C.c_int, [vp, vp])
    ref_consume = _setup(ref, "ref_ring_consume", C.c_int, [vp, vp])
    prod_consume = _setup(prod_shim, "prod_ring_consume", C.c_int, [vp, vp])
    rings = [_img(131200) for _ in range(3)]
    rng = np.random.default_rng(3)
    for step in range(3000):
        if rng.random() < 0.5:
            n = int(rng.integers(0, 34))
            descs = rng.integers(0, 256, (max(n, 1), 32), dtype=np.uint8)
            batch = rl.DecodeDispatchBatch()
            batch.count = min(n, 32)
            C.memmove(C.addressof(batch.descs), descs.ctypes.data, min(n, 32) * 32)
            rc0 = rl.lib().decode_batch_submit(rings[0].ctypes.data, C.byref(batch))
            rc1 = ref_submit(rings[1].ctypes.data, C.addressof(batch))
            rc2 = olib.orc_decode_batch_submit(rings[2].ctypes.data, descs.ctypes.data, min(n, 32))
            assert rc0 == rc1 == rc2, step
        else:
            for _ in range(int(rng.integers(1, 40))):
                o0, o1, o2 = (np.zeros(32, dtype=np.uint8) for _ in range(3))
                c0 = prod_consume(rings[0].ctypes.data, o0.ctypes.data)
                c1 = ref_consume(rings[1].ctypes.data, o1.ctypes.data)
                c2 = olib.orc_ring_consume(rings[2].ctypes.data, C.byref(orc.CMD_RING), o2.ctypes.data)
                assert c0 == c1 == c2 and o0.tobytes() == o1.tobytes() == o2.tobytes()
    assert np.array_equal(rings[0], rings[1]) and np.array_equal(rings[0], rings[2])


def test_submit_and_worker_sim_trace(rl, olib, ref):
    """infer_submit_decode -> cmdq -> hw_worker_sim -> doneq, 3 ways."""
    vp, u32, u64 = C.c_void_p, C.c_uint32, C.c_uint64
    ref_submit = _setup(ref, "infer_submit_decode", C.c_int, [vp, u32, u64, u64, u32, u32, u32])
    ref_run = _setup(ref, "hw_worker_sim_run", None, [vp])
    ref_push = _setup(ref, "ref_hw_ring_push", C.c_int, [vp, vp])
    rng = np.random.default_rng(4)
    imgs = {k: [_img(4194432) for _ in range(3)] for k in ("cmd", "done")}
    doorbells = [np.zeros(1, dtype=np.uint32) for _ in range(3)]
    n = 5000
    for i in range(n):
        rid, kv, dl = int(rng.integers(0, 2**32)), int(rng.integers(0, 2**40)), int(rng.integers(0, 2**40))
        prefix = int(rng.integers(0, 3))
        seq = int(rng.integers(0, 300))
        mx = seq + int(rng.integers(-2, 80))
        mx = max(mx, 0)
        for k in range(2):
            ctx = rl.InferHwCtx(imgs["cmd"][k].ctypes.data, imgs["done"][k].ctypes.data,
                                doorbells[k].ctypes.data, 7, 42)
            f = rl.lib().infer_submit_decode if k == 0 else ref_submit
            rc = f(C.byref(ctx), rid, kv, dl, prefix, seq, mx) if k == 0 else f(C.addressof(ctx), rid, kv, dl,
                                                                                  prefix, seq, mx)
            assert rc == 0
        db = olib.orc_submit_decode(imgs["cmd"][2].ctypes.data, 7, 42, rid, kv, dl, prefix, seq, mx)
        assert db == doorbells[0][0] == doorbells[1][0]
        if rng.random() < 0.05:  # a non-DECODE opcode the worker must drop
            junk = np.zeros(64, dtype=np.uint8)
            junk[0] = 3
            for k in range(3):
                ref_push(imgs["cmd"][k].ctypes.data, junk.ctypes.data)
    stop_desc = np.zeros(64, dtype=np.uint8)
    stop_desc[0] = 255
    for k in range(3):
        ref_push(imgs["cmd"][k].ctypes.data, stop_desc.ctypes.data)
    assert np.array_equal(imgs["cmd"][0], imgs["cmd"][1]) and np.array_equal(imgs["cmd"][0], imgs["cmd"][2])
    stop = np.zeros(1, dtype=np.uint32)
    ws = []
    for k in range(2):
        w = rl.HwWorkerSim(imgs["cmd"][k].ctypes.data, imgs["done"][k].ctypes.data, stop.ctypes.data, 0, 0)
        (rl.lib().hw_worker_sim_run(C.byref(w)) if k == 0 else ref_run(C.addressof(w)))
        ws.append((w.decoded_tokens, w.completions))
    dec = C.c_uint64(0)
    stopped = C.c_int(0)
    comp = olib.orc_worker_sim_drain(imgs["cmd"][2].ctypes.data, imgs["done"][2].ctypes.data, C.byref(dec),
                                     C.byref(stopped))
    assert stopped.value == 1
    assert ws[0] == ws[1] == (dec.value, comp)
    for k in ("cmd", "done"):
        assert np.array_equal(imgs[k][0], imgs[k][1]) and np.array_equal(imgs[k][0], imgs[k][2])


def test_arena_trace(rl, olib, ref):
    vp = C.c_void_p
    ref_init = _setup(ref, "arena_init", None, [vp, C.c_size_t, C.c_size_t])
    ref_acq = _setup(ref, "arena_acquire", C.c_int64, [vp])
    ref_rel = _setup(ref, "arena_release", None, [vp, C.c_int64])
    ref_destroy = _setup(ref, "arena_destroy", None, [vp])
    a0, a1 = _img(131096), _img(131096)
    rl.lib().arena_init(a0.ctypes.data, 1 << 20, 8192)
    ref_init(a1.ctypes.data, 1 << 20, 8192)
    bm = np.zeros(16384, dtype=np.uint64)
    rng = np.random.default_rng(5)
    live = []
    for step in range(20000):
        if live and rng.random() < 0.4:
            idx = live.pop(int(rng.integers(0, len(live))))
            rl.lib().arena_release(a0.ctypes.data, idx)
            ref_rel(a1.ctypes.data, idx)
            olib.orc_arena_release(bm.ctypes.data, idx)
        else:
            r = (rl.lib().arena_acquire(a0.ctypes.data), ref_acq(a1.ctypes.data), olib.orc_arena_acquire(bm.ctypes.data))
            assert r[0] == r[1] == r[2], step
            live.append(r[0])
    assert np.array_equal(a0[24:], a1[24:]) and np.array_equal(a0[24:].view(np.uint64), bm)
    rl.lib().arena_destroy(a0.ctypes.data)
    ref_destroy(a1.ctypes.data)


def test_kv_prefix_trace(rl, olib):
    """Runtime vs oracle (the reference kv_prefix.c does not compile as shipped:
    its header's size asserts are wrong)."""
    t0 = _img(606280)
    t1 = _img(606280)
    L = rl.lib()
    L.kv_prefix_table_init(t0.ctypes.data)
    olib.orc_kvp_init(t1.ctypes.data)
    assert np.array_equal(t0, t1)
    rng = np.random.default_rng(6)
    for step in range(40000):
        op = rng.integers(0, 6)
        if op == 0:
            off, ln, nb = int(rng.integers(-5, 2**40)), int(rng.integers(0, 4096)), int(rng.integers(0, 300))
            i0, i1 = C.c_uint32(0), C.c_uint32(0)
            r = (L.kv_prefix_register(t0.ctypes.data, off, ln, nb, C.byref(i0)),
                 olib.orc_kvp_register(t1.ctypes.data, off, ln, nb, C.byref(i1)))
            assert r[0] == r[1] and i0.value == i1.value
        elif op == 1:
            pid = int(rng.integers(0, 520))
            assert L.kv_prefix_acquire(t0.ctypes.data, pid) == olib.orc_kvp_acquire(t1.ctypes.data, pid)
        elif op == 2:
            pid = int(rng.integers(0, 520))
            assert L.kv_prefix_release(t0.ctypes.data, pid) == olib.orc_kvp_release(t1.ctypes.data, pid)
        elif op == 3:
            args = (int(rng.integers(0, 2**32)), int(rng.integers(0, 520)), int(rng.integers(-3, 2**40)),
                    int(rng.integers(0, 999)), int(rng.integers(0, 99)))
            i0, i1 = C.c_uint32(0), C.c_uint32(0)
            r = (L.kv_branch_alloc(t0.ctypes.data, *args, C.byref(i0)),
                 olib.orc_kvb_alloc(t1.ctypes.data, *args, C.byref(i1)))
            assert r[0] == r[1] and i0.value == i1.value
        elif op == 4:
            bid = int(rng.integers(0, 16400))
            assert L.kv_branch_free(t0.ctypes.data, bid) == olib.orc_kvb_free(t1.ctypes.data, bid)
        else:
            bid = int(rng.integers(0, 16400))
            assert L.kv_branch_total_offset(t0.ctypes.data, bid) == olib.orc_kvb_total_offset(t1.ctypes.data, bid)
        if step % 5000 == 0:
            assert np.array_equal(t0, t1), step
    assert np.array_equal(t0, t1)


def test_kv_layout_fixed128_known_answers(prod_shim, orc):
    """The fixed128 block math: the runtime's header against the values the
    reference's layout bench prints (bench/bench_kv_layout.cu:20-22: block[3]
    = 49,152, K token 7 = 1,792, V token 7 = 9,984) and the descriptor of
    kv_layout_desc_fixed128, then against the reference's own header
    compiled into oracle/_ref over every block and token index used."""
    import rlrt

    u32 = C.c_uint32
    fns = {}
    libs = [(prod_shim, "prod_")]
    r = orc.load_ref()
    if r is not None:
        libs.append((r, "ref_"))
    for lib, pre in libs:
        fns[pre] = [_setup(lib, pre + n, u32, [u32]) for n in
                    ("kv_layout_block_offset_bytes", "kv_layout_k_offset_bytes", "kv_layout_v_offset_bytes")]
        d = rlrt.KvLayoutDesc()
        _setup(lib, pre + "kv_layout_desc_fixed128", None, [C.c_void_p])(C.addressof(d))
        assert (d.token_count, d.head_dim, d.scalar_bytes, d.vec_bytes, d.k_stride_bytes, d.v_stride_bytes,
                d.block_bytes, d.alignment) == (32, 128, 2, 16, 256, 256, 16384, 128), pre
        blk, k, v = fns[pre]
        assert (blk(3), k(7), v(7)) == (49152, 1792, 9984), pre
    if r is None:
        pytest.skip("oracle/_ref not built: known answers checked, reference header not compared")
    for i in range(4096):
        assert [f(i) for f in fns["prod_"]] == [f(i) for f in fns["ref_"]], i
