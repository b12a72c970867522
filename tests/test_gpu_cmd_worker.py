"""The persistent worker on the v0.2 command / completion rings.

Descriptors go in through decode_batch windows (the reference's
decode_batch_push / decode_batch_submit, src/decode_batch.c:3-51) and single
ring pushes; the gfx950 worker runs the fixed128 decode step of each and
pushes the completions. Checked against the host:
  * completions in descriptor order with seq_id, kv_block_offset and
    reward_cookie passed through and cycles_taken = ceil(seq_len / 16) *
    128 * 24 (cu/attention_decode.cu:196-201), seq_len = num_kv_blocks
    clamped to [1, 32];
  * every output row within 1e-4 of fp64 attention over the block (the
    reference test's bound, test/test_bench.cu:716-717) and the token the
    lowest index of that row's maximum (bit-exact given the GPU's row);
  * the closed-form vector of test/test_bench.cu:91-155 through the ring;
  * synthesized queries (no q buffer) from seq_id, cookie and the sample
    state, equal to the oracle's restatement;
  * a block past the arena gives NaN and token 0; the sentinel is consumed
    without a completion; ring indices and the worker's counters at the end.
"""
import ctypes as C
import time

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

BLOCK = 16384
COMP_SLOTS = 4096


def _coherent(rl, n):
    p = rl.lib().rl_hip_host_alloc_coherent(n)
    assert p, rl._err()
    C.memset(p, 0, n)
    return p


def _comp_pop_all(rl, cr):
    """Consumer side of completion.h's ring (head @0, tail @64, slots @256)."""
    L = rl.lib()
    out = []
    while True:
        head, tail = L.hw_ring_load_acquire(cr), L.hw_ring_load_acquire(cr + 64)
        if head == tail:
            return out
        raw = (C.c_char * 32).from_address(cr + 256 + (head % COMP_SLOTS) * 32)
        out.append(rl.Completion.from_buffer_copy(raw))
        L.hw_ring_store_release(cr, (head + 1) & 0xFFFFFFFF)


def _ref_row(arena16, blk, seq, q):
    kv = synth.f16_to_f32(arena16[blk * BLOCK // 2:(blk + 1) * BLOCK // 2]).astype(np.float64).reshape(2, 32, 128)
    s = kv[0, :seq] @ q.astype(np.float64) / np.sqrt(128.0)
    p = np.exp(s - s.max())
    return (p @ kv[1, :seq]) / p.sum()


def _run(rl, descs_windows, arena, q_buf, io_slots, sample_state=None, expect=None):
    L = rl.lib()
    ring, cr = L.ring_create(), L.comp_ring_create()
    assert L.rl_hip_is_coherent_host(ring) and L.rl_hip_is_coherent_host(cr)
    pairs = _coherent(rl, 16)
    C.cast(pairs, C.POINTER(C.c_void_p))[0] = ring
    C.cast(pairs, C.POINTER(C.c_void_p))[1] = cr
    stop = _coherent(rl, 64)
    darena = rl.DeviceBuffer.from_array(arena)
    dq = rl.DeviceBuffer.from_array(q_buf) if q_buf is not None else None
    do = rl.DeviceBuffer(max(io_slots, 1) * 128 * 4, zero=True)
    dst = rl.DeviceBuffer.from_array(sample_state) if sample_state is not None else None
    stats = rl.DeviceBuffer(32, zero=True)
    a = rl.CmdWorkerArgs(rings=pairs, comp_rings=pairs + 8, groups=1, stop=stop, max_idle_polls=1 << 22,
                         arena_base=darena.ptr, arena_bytes=darena.nbytes,
                         sample_state=dst.ptr if dst is not None else None,
                         q_buffer=dq.ptr if dq is not None else None, o_buffer=do.ptr, io_slots=io_slots,
                         stats=stats.ptr)
    n_desc = sum(len(w) for w in descs_windows)
    got = []
    print(f"[cmd] launching the v0.2 worker: {n_desc} descriptors in {len(descs_windows)} windows", flush=True)
    rl.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
    try:
        batch = rl.DecodeDispatchBatch()
        for win in descs_windows:
            L.decode_batch_reset(C.byref(batch))
            for d in win:
                assert L.decode_batch_push(C.byref(batch), C.byref(d)) == 0
            assert L.decode_batch_submit(ring, C.byref(batch)) == 0
        # the sentinel, pushed on its own
        sent = rl.Descriptor(seq_id=2**64 - 1)
        L.decode_batch_reset(C.byref(batch))
        assert L.decode_batch_push(C.byref(batch), C.byref(sent)) == 0
        assert L.decode_batch_submit(ring, C.byref(batch)) == 0
        deadline = time.perf_counter() + 60
        while len(got) < n_desc and time.perf_counter() < deadline:
            got += _comp_pop_all(rl, cr)
            time.sleep(1e-4)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1   # every exit path ends the worker before the sync
        rl.sync()
    st = stats.download(np.uint64, 4)
    o = do.download(np.float32, (max(io_slots, 1), 128))
    heads = (L.hw_ring_load_acquire(ring), L.hw_ring_load_acquire(ring + 64), L.hw_ring_load_acquire(cr),
             L.hw_ring_load_acquire(cr + 64))
    for b in [darena, do, stats] + [x for x in (dq, dst) if x is not None]:
        b.close()
    L.ring_destroy(ring)
    L.comp_ring_destroy(cr)
    L.rl_hip_host_free(pairs)
    L.rl_hip_host_free(stop)
    return got, st, o, heads


def _check(descs, got, o, io_slots, arena16, qvec):
    assert len(got) == len(descs)
    for d, c in zip(descs, got):
        seq = 1 if d.num_kv_blocks == 0 else min(int(d.num_kv_blocks), 32)
        assert (c.seq_id, c.kv_block_offset, c.reward_cookie) == (d.seq_id, d.kv_block_offset, d.reward_cookie)
        assert c.cycles_taken == -(-seq // 16) * 128 * 24
        slot = d.output_token_offset & (io_slots - 1)
        row = o[slot]
        ref = _ref_row(arena16, d.kv_block_offset, seq, qvec(d, slot))
        assert np.abs(row - ref).max() < 1e-4, (d.seq_id, np.abs(row - ref).max())
        assert c.token_id == int(np.flatnonzero(row == row.max()).min())


def test_windows_through_the_rings(rl, gpu):
    rng = np.random.default_rng(61)
    nblk, io = 48, 64
    arena16 = synth.f32_to_f16(rng.standard_normal(nblk * BLOCK // 2, dtype=np.float32))
    qf = synth.f32_to_f16(rng.standard_normal((io, 128), dtype=np.float32))
    lens = [0, 1, 5, 16, 17, 31, 32, 40, 300]
    windows, k = [], 0
    for size in (1, 7, 32, 3, 32, 16, 1):      # decode_batch windows of up to 32
        win = []
        for _ in range(size):
            win.append(rl.Descriptor(seq_id=1000 + k, kv_block_offset=int(rng.integers(0, nblk)),
                                     num_kv_blocks=lens[k % len(lens)], output_token_offset=k,
                                     reward_cookie=int(rng.integers(0, 2**63))))
            k += 1
        windows.append(win)
    # io_slots = 64 and 92 descriptors: slots are reused, so check window by window
    got, st, o, heads = [], None, None, None
    for wi in range(0, len(windows), 2):
        part = windows[wi:wi + 2]
        g, st, o, heads = _run(rl, part, arena16.view(np.uint8), qf, io)
        descs = [d for w in part for d in w]
        _check(descs, g, o, io, arena16, lambda d, slot: synth.f16_to_f32(qf[slot]))
        n = len(descs)
        assert st.tolist()[0:2] == [n, n] and st[3] == 0, st
        assert heads == (n + 1, n + 1, n, n)
        got += g


def test_closed_form_vector_and_bad_block(rl, gpu):
    """test/test_bench.cu:91-155 (17 tokens) in block 1, and a block index past
    the arena (NaN output, token 0), through one window."""
    d = np.arange(128)
    q = ((d % 17) - 8) / 8.0
    t = np.arange(32)[:, None]
    K = ((((t + 1) * ((d % 13) + 1)) % 23) - 11) / 32.0
    V = ((((t + 3) * ((d % 11) + 5)) % 29) - 14) / 29.0
    arena16 = np.zeros(3 * BLOCK // 2, np.uint16)
    arena16[BLOCK // 2:2 * BLOCK // 2] = np.concatenate([synth.f32_to_f16(K.astype(np.float32)).ravel(),
                                                         synth.f32_to_f16(V.astype(np.float32)).ravel()])
    qf = np.zeros((2, 128), np.uint16)
    qf[0] = synth.f32_to_f16(q.astype(np.float32))
    descs = [rl.Descriptor(seq_id=7, kv_block_offset=1, num_kv_blocks=17, output_token_offset=0, reward_cookie=5),
             rl.Descriptor(seq_id=8, kv_block_offset=3, num_kv_blocks=4, output_token_offset=1, reward_cookie=6)]
    got, st, o, heads = _run(rl, [descs], arena16.view(np.uint8), qf, 2)
    ref = _ref_row(arena16, 1, 17, synth.f16_to_f32(qf[0]))
    assert np.abs(o[0] - ref).max() < 1e-4
    assert got[0].token_id == int(np.argmax(ref)) and got[0].cycles_taken == 2 * 128 * 24
    assert np.isnan(o[1]).all() and got[1].token_id == 0
    assert heads == (3, 3, 2, 2)


def test_synthesized_queries(rl, gpu, olib):
    """No q buffer: the query comes from seq_id, reward_cookie and the sample
    state's rng words, as the oracle restates it."""
    rng = np.random.default_rng(62)
    nblk = 8
    arena16 = synth.f32_to_f16(rng.standard_normal(nblk * BLOCK // 2, dtype=np.float32))
    state = np.zeros(6, np.uint64)                    # SampleState: rng_state[4], then the sampling fields
    state[:4] = rng.integers(0, 2**63, 4, dtype=np.uint64)
    descs = [rl.Descriptor(seq_id=int(rng.integers(0, 2**40)), kv_block_offset=i % nblk, num_kv_blocks=9 + i,
                           output_token_offset=i, reward_cookie=int(rng.integers(0, 2**63))) for i in range(12)]
    got, st, o, heads = _run(rl, [descs], arena16.view(np.uint8), None, 16, sample_state=state)

    def qvec(d, slot):
        return np.array([olib.orc_synth_query(d.seq_id, d.reward_cookie, state.ctypes.data, i) for i in range(128)],
                        dtype=np.float32)
    _check(descs, got, o, 16, arena16, qvec)


def test_one_worker_per_cu(rl, gpu):
    """One persistent worker per compute unit, each the only consumer and
    producer of its own CommandRing / CompletionRing pair: two decode_batch
    windows (16 and 9 descriptors) per pair, output slots disjoint across
    pairs. Per pair: completions in order and every row against fp64 as
    above, ring indices and counters."""
    L = rl.lib()
    G = int(gpu.cu_count)
    rng = np.random.default_rng(63)
    nblk = 64
    per = 32
    io = 1 << int(np.ceil(np.log2(G * per)))
    arena16 = synth.f32_to_f16(rng.standard_normal(nblk * BLOCK // 2, dtype=np.float32))
    qf = synth.f32_to_f16(rng.standard_normal((io, 128), dtype=np.float32))
    lens = [0, 1, 5, 16, 17, 31, 32, 40]
    windows = []
    for g in range(G):
        ws_ = []
        k = 0
        for size in (16, 9):
            win = []
            for _ in range(size):
                win.append(rl.Descriptor(seq_id=(g << 20) + k, kv_block_offset=int(rng.integers(0, nblk)),
                                         num_kv_blocks=lens[int(rng.integers(0, len(lens)))],
                                         output_token_offset=g * per + k, reward_cookie=int(rng.integers(0, 2**63))))
                k += 1
            ws_.append(win)
        windows.append(ws_)
    rings = [L.ring_create() for _ in range(G)]
    comps = [L.comp_ring_create() for _ in range(G)]
    assert all(rings) and all(comps)
    pairs = _coherent(rl, 16 * G)
    for g in range(G):
        C.cast(pairs, C.POINTER(C.c_void_p))[g] = rings[g]
        C.cast(pairs, C.POINTER(C.c_void_p))[G + g] = comps[g]
    stop = _coherent(rl, 64)
    darena = rl.DeviceBuffer.from_array(arena16.view(np.uint8))
    dq = rl.DeviceBuffer.from_array(qf)
    do = rl.DeviceBuffer(io * 128 * 4, zero=True)
    stats = rl.DeviceBuffer(32 * G, zero=True)
    a = rl.CmdWorkerArgs(rings=pairs, comp_rings=pairs + 8 * G, groups=G, stop=stop, max_idle_polls=1 << 22,
                         arena_base=darena.ptr, arena_bytes=darena.nbytes, sample_state=None, q_buffer=dq.ptr,
                         o_buffer=do.ptr, io_slots=io, stats=stats.ptr)
    got = [[] for _ in range(G)]
    print(f"[cmd] launching {G} command-ring workers, one per compute unit", flush=True)
    rl.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
    try:
        batch = rl.DecodeDispatchBatch()
        for wi in range(2):
            for g in range(G):
                L.decode_batch_reset(C.byref(batch))
                for d in windows[g][wi]:
                    assert L.decode_batch_push(C.byref(batch), C.byref(d)) == 0
                assert L.decode_batch_submit(rings[g], C.byref(batch)) == 0
        deadline = time.perf_counter() + 60
        n = 0
        while n < G * 25 and time.perf_counter() < deadline:
            for g in range(G):
                c = _comp_pop_all(rl, comps[g])
                got[g] += c
                n += len(c)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rl.sync()
    st = stats.download(np.uint64, (G, 4))
    o = do.download(np.float32, (io, 128))
    for g in range(G):
        descs = windows[g][0] + windows[g][1]
        _check(descs, got[g], o, io, arena16, lambda d, slot: synth.f16_to_f32(qf[slot]))
        assert st[g, 0] == 25 and st[g, 1] == 25 and st[g, 3] == 0, (g, st[g])
        assert (L.hw_ring_load_acquire(rings[g]), L.hw_ring_load_acquire(rings[g] + 64),
                L.hw_ring_load_acquire(comps[g]), L.hw_ring_load_acquire(comps[g] + 64)) == (25, 25, 25, 25), g
    for b in (darena, dq, do, stats):
        b.close()
    for r, c in zip(rings, comps):
        L.ring_destroy(r)
        L.comp_ring_destroy(c)
    L.rl_hip_host_free(pairs)
    L.rl_hip_host_free(stop)


def test_launch_refuses_more_workers_than_resident(rl, gpu):
    """Workers beyond what the device holds at once would leave their ring
    pairs unserved: the launch is refused on the host, nothing runs. (A
    1,024-thread worker takes 16 of a compute unit's 32 wave slots, so twice
    the compute units plus one exceeds the device whatever the LDS use.)"""
    L = rl.lib()
    dev = rl.DeviceBuffer(1 << 16, zero=True)
    a = rl.CmdWorkerArgs(rings=dev.ptr, comp_rings=dev.ptr, groups=2 * int(gpu.cu_count) + 1, stop=dev.ptr,
                         max_idle_polls=16, arena_base=dev.ptr, arena_bytes=dev.nbytes, sample_state=None,
                         q_buffer=None, o_buffer=dev.ptr, io_slots=1, stats=dev.ptr)
    assert L.rl_hip_cmd_worker_launch(C.byref(a)) == -1
    assert b"exceed" in L.rl_hip_last_error()
    a.groups = 0
    assert L.rl_hip_cmd_worker_launch(C.byref(a)) == -1
    dev.close()


def test_stamps_lockstep(rl, gpu):
    """Four workers with stamps set, 64 descriptors one at a time through
    ring_lockstep_cmd: every completion carries its seq_id, each worker's
    consume stamp precedes its completion stamp, successive samples' stamps
    ascend on the device's common clock, the outputs are the fixed128 step's
    (checked against fp64 like the other cases), and the workers end on the
    stop flag with 16 descriptors each."""
    L = rl.lib()
    pairs, n, io = 4, 64, 64
    rng = np.random.default_rng(4401)
    arena16 = synth.f32_to_f16(rng.standard_normal(4 * BLOCK // 2, dtype=np.float32))
    q = synth.f32_to_f16(rng.standard_normal((io, 128), dtype=np.float32))
    darena, dq = rl.DeviceBuffer.from_array(arena16.view(np.uint8)), rl.DeviceBuffer.from_array(q)
    do = rl.DeviceBuffer(io * 128 * 4, zero=True)
    stats = rl.DeviceBuffer(pairs * 32, zero=True)
    rs = [L.ring_create() for _ in range(pairs)]
    crs = [L.comp_ring_create() for _ in range(pairs)]
    tab = _coherent(rl, 16 * pairs)
    for g in range(pairs):
        C.cast(tab, C.POINTER(C.c_void_p))[g] = rs[g]
        C.cast(tab, C.POINTER(C.c_void_p))[pairs + g] = crs[g]
    stop, stamps = _coherent(rl, 64), _coherent(rl, 16 * pairs)
    a = rl.CmdWorkerArgs(rings=tab, comp_rings=tab + 8 * pairs, groups=pairs, stop=stop, max_idle_polls=1 << 24,
                         arena_base=darena.ptr, arena_bytes=darena.nbytes, sample_state=None, q_buffer=dq.ptr,
                         o_buffer=do.ptr, io_slots=io, stats=stats.ptr, stamps=stamps)
    out = (rl.RingLockstepSample * n)()
    d = rl.Descriptor(kv_block_offset=2, num_kv_blocks=32, output_token_offset=5, reward_cookie=9)
    print(f"[cmd] {pairs} workers with stamps, {n} lock-step descriptors", flush=True)
    rl.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
    try:
        got = L.ring_lockstep_cmd(tab, tab + 8 * pairs, pairs, C.byref(d), 1000, n, stamps, 10**10, out)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rl.sync()
    st = stats.download(np.uint64, (pairs, 4))
    o = do.download(np.float32, (io, 128))
    assert got == n
    assert (st[:, 0] == n // pairs).all() and (st[:, 3] == 0).all(), st
    for i, s in enumerate(out):
        assert s.consume_tick <= s.complete_tick and s.submit_ns < s.poll_ns, i
        if i:
            assert out[i - 1].complete_tick <= s.consume_tick, i
    # every descriptor wrote slot 5 from block 2 and q slot 5
    want = _ref_row(arena16, 2, 32, synth.f16_to_f32(q[5]))
    assert np.abs(o[5] - want).max() < 1e-4
    for b in (darena, dq, do, stats):
        b.close()
    for r in rs:
        L.ring_destroy(r)
    for r in crs:
        L.comp_ring_destroy(r)
    for p in (tab, stop, stamps):
        L.rl_hip_host_free(p)
