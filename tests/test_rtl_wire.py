"""The descriptor / completion contract toward the RTL queue ports
(include/rtl_wire.h). CPU only.

Pinned independently of the C shifts:
* the word images equal the SystemVerilog packed-struct rule (first declared
  field in the most significant bits, rtl/desc_pkg.sv:8-27), restated here as
  an integer concatenation of the fields and cut into 32-bit words, word i =
  bits [32i + 31 : 32i] (verilator/rtl_bridge.cpp:114-146);
* the completions of the RTL testbench's own three cases
  (rtl/tb_rl_runtime_top.sv:81-147: rollout 7, seq 0, max 10 -> DONE at 10;
  rollout 9, seq 0, max 40 -> REWARD_NEEDED at 32; rollout 11, seq 8, max 12
  -> DONE at 12) and the bridge test's vectors ((0, 64) -> REWARD_NEEDED at
  32, (7, 32) -> DONE at 32), produced by this library's C worker model
  (hw_worker_sim_run, the C fast path) and packed, decode to exactly what the
  RTL testbench expects.
The reference bridge itself needs Verilator-generated headers and is not
built here.
"""
import ctypes as C

import numpy as np
import pytest

DESC_FIELDS = [("opcode", 8), ("flags", 8), ("rollout_id", 16), ("kv_arena_id", 16), ("prefix_id", 16),
               ("kv_offset", 32), ("delta_offset", 32), ("seq_len", 16), ("max_tokens", 16),
               ("reward_model_id", 16), ("reserved0", 16)]
COMP_FIELDS = [("rollout_id", 16), ("status", 8), ("final_seq_len", 16), ("reward_id", 16)]


def _concat(fields, values):
    """SystemVerilog packed struct: the first field ends up in the top bits."""
    v = 0
    for name, width in fields:
        x = values[name]
        assert 0 <= x < (1 << width)
        v = (v << width) | x
    return v


def _words(v, n):
    return [(v >> (32 * i)) & 0xFFFFFFFF for i in range(n)]


def _pack(rl, d):
    w = (C.c_uint32 * 6)()
    rc = rl.lib().rtl_desc_pack(C.byref(d), w)
    return rc, list(w)


def _desc(rl, **kw):
    d = rl.HwDesc()
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_desc_words_follow_the_packed_struct_rule(rl):
    vals = dict(opcode=1, flags=0x05, rollout_id=0xBEEF, kv_arena_id=0x1234, prefix_id=0x0042,
                kv_offset=0xDEADBEEF, delta_offset=0x01020304, seq_len=355, max_tokens=356,
                reward_model_id=0x0A0B, reserved0=7)
    rc, w = _pack(rl, _desc(rl, **vals))
    assert rc == 0
    assert w == _words(_concat(DESC_FIELDS, vals), 6)
    # the bridge's own image of a decode of rollout 3 (opcode in the top byte of word 5)
    rc, w = _pack(rl, _desc(rl, opcode=1, rollout_id=3, seq_len=31, max_tokens=96, reward_model_id=2))
    assert rc == 0 and w[5] == 0x01000003 and w[1] == (31 << 16) | 96 and w[0] == 2 << 16


def test_desc_round_trip_random(rl):
    L = rl.lib()
    rng = np.random.default_rng(5)
    for _ in range(2000):
        vals = {name: int(rng.integers(0, 1 << width)) for name, width in DESC_FIELDS}
        vals["opcode"] = int(rng.choice([1, 2, 255]))
        d = _desc(rl, **vals, user_data=int(rng.integers(0, 2**63)), checksum_or_cookie=12345)
        rc, w = _pack(rl, d)
        assert rc == 0 and w == _words(_concat(DESC_FIELDS, vals), 6)
        back = rl.HwDesc()
        assert L.rtl_desc_unpack((C.c_uint32 * 6)(*w), C.byref(back)) == 0
        for name, _ in DESC_FIELDS:
            assert getattr(back, name) == vals[name], name
        assert back.user_data == 0 and back.checksum_or_cookie == 0   # software metadata does not cross


@pytest.mark.parametrize("field,value", [("flags", 0x100), ("rollout_id", 1 << 16), ("kv_arena_id", 1 << 16),
                                         ("prefix_id", 1 << 16), ("seq_len", 1 << 16), ("max_tokens", 1 << 16),
                                         ("reward_model_id", 1 << 16), ("reserved0", 1 << 16),
                                         ("kv_offset", 1 << 32), ("delta_offset", 1 << 32)])
def test_desc_pack_refuses_what_does_not_fit(rl, field, value):
    d = _desc(rl, opcode=1, **{field: value})
    w = (C.c_uint32 * 6)(*([0xA5A5A5A5] * 6))
    assert rl.lib().rtl_desc_pack(C.byref(d), w) == -1
    assert list(w) == [0xA5A5A5A5] * 6          # nothing written
    ok = _desc(rl, opcode=1, **{field: value - 1})
    assert _pack(rl, ok)[0] == 0


def test_opcode_namespace(rl):
    L = rl.lib()
    assert _pack(rl, _desc(rl, opcode=3))[0] == -1      # PREFILL: no RTL value
    assert _pack(rl, _desc(rl, opcode=0))[0] == -1
    assert _pack(rl, _desc(rl, opcode=7))[0] == -1
    for op, ok in ((0, False), (1, True), (2, True), (3, False), (255, True), (254, False)):
        w = (C.c_uint32 * 6)(0, 0, 0, 0, 0, op << 24)
        assert (L.rtl_desc_unpack(w, C.byref(rl.HwDesc())) == 0) == ok, op
    assert L.rtl_desc_pack(None, (C.c_uint32 * 6)()) == -1
    assert L.rtl_desc_unpack(None, C.byref(rl.HwDesc())) == -1


def _run_c_worker(rl, descs):
    """The C fast path: the descriptors, then STOP, through hw_worker_sim_run."""
    L = rl.lib()
    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    stop = C.c_uint32(0)
    try:
        for d in descs:
            assert rl.hw_ring_push(cq, d) == 0
        assert rl.hw_ring_push(cq, rl.HwDesc(opcode=255)) == 0
        sim = rl.HwWorkerSim(cmdq=cq, doneq=dq, stop=C.addressof(stop))
        L.hw_worker_sim_run(C.byref(sim))
        out = []
        while (d := rl.hw_ring_pop(dq)) is not None:
            out.append(d)
        return out
    finally:
        L.hw_ring_destroy(cq)
        L.hw_ring_destroy(dq)


def _comp_fields(rl, d):
    L = rl.lib()
    w = (C.c_uint32 * 2)()
    assert L.rtl_comp_pack(C.byref(d), w) == 0
    f = [C.c_uint32() for _ in range(4)]
    assert L.rtl_comp_unpack(w, *[C.byref(x) for x in f]) == 0
    vals = dict(zip(("rollout_id", "status", "final_seq_len", "reward_id"), (x.value for x in f)))
    assert list(w) == _words(_concat(COMP_FIELDS, vals), 2)
    return vals


# (rollout, seq_len, max_tokens, reward_model) -> (status, final_seq_len) the RTL reports
RTL_CASES = [((7, 0, 10, 3), (1, 10)), ((9, 0, 40, 5), (2, 32)), ((11, 8, 12, 1), (1, 12)),
             ((4, 0, 64, 2), (2, 32)), ((5, 7, 32, 6), (1, 32))]


def test_completions_of_the_c_worker_match_the_rtl_testbench(rl):
    descs = [_desc(rl, opcode=1, rollout_id=r, seq_len=s, max_tokens=m, reward_model_id=rm)
             for (r, s, m, rm), _ in RTL_CASES]
    # the descriptors cross to the RTL port and back unchanged
    for d in descs:
        rc, w = _pack(rl, d)
        back = rl.HwDesc()
        assert rc == 0 and rl.lib().rtl_desc_unpack((C.c_uint32 * 6)(*w), C.byref(back)) == 0
        assert bytes(back) == bytes(d)
    done = _run_c_worker(rl, descs)
    assert len(done) == len(RTL_CASES)
    for d, ((r, _, _, rm), (status, final)) in zip(done, RTL_CASES):
        assert _comp_fields(rl, d) == dict(rollout_id=r, status=status, final_seq_len=final, reward_id=rm)


def test_completion_edges(rl):
    L = rl.lib()
    w = (C.c_uint32 * 2)()
    # a decode returned with neither flag (it arrived with seq_len >= max_tokens) has no status
    assert L.rtl_comp_pack(C.byref(_desc(rl, opcode=1, seq_len=9, max_tokens=9)), w) == -1
    # DONE wins over a reward flag left from an earlier round
    both = _desc(rl, opcode=1, flags=3, rollout_id=2, seq_len=64, max_tokens=64, reward_model_id=1)
    assert _comp_fields(rl, both)["status"] == 1
    assert _comp_fields(rl, _desc(rl, opcode=255, rollout_id=3))["status"] == 255
    assert L.rtl_comp_pack(C.byref(_desc(rl, opcode=1, flags=2, rollout_id=1 << 16)), w) == -1
    f = [C.c_uint32() for _ in range(4)]
    assert L.rtl_comp_unpack((C.c_uint32 * 2)(0, 1 << 24), *[C.byref(x) for x in f]) == -1   # bits above 55
    assert L.rtl_comp_unpack((C.c_uint32 * 2)(0, 3), *[C.byref(x) for x in f]) == -1         # status 3
