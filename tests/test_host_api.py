"""The reference's CPU test scenarios (test/test_hw_ring.c, test/test_smoke.c,
test/test_bench.cu CPU parts) run in C against the runtime's headers and
library, plus ctypes-level checks of the exported entry points."""
import ctypes as C
import subprocess

import numpy as np

import helpers


def test_reference_cpu_scenarios_in_c(rl):
    exe = helpers.build("tests/c/test_host_api.c", link_runtime=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout


def test_worker_rule_known_answers(rl):
    """hw_worker_sim rule vs the RTL/Verilator known answers that agree with
    the C simulator (rtl/rollout_worker_fsm.sv:63-78, verilator/test_rtl_bridge.cpp)."""
    cases = [((0, 10), (10, 2)), ((0, 64), (32, 1)), ((8, 12), (12, 2)), ((0, 40), (32, 1)), ((7, 32), (32, 2)),
             ((31, 96), (32, 1)), ((255, 257), (256, 1)), ((256, 257), (257, 2))]
    for (seq, mx), (seq_out, flags) in cases:
        d = rl.HwDesc(opcode=1, seq_len=seq, max_tokens=mx)
        n = rl.lib().hw_worker_apply_decode_rule(C.byref(d))
        assert (d.seq_len, d.flags) == (seq_out, flags), (seq, mx)
        assert n == seq_out - seq
    # seq >= max on entry: unchanged, no flag (src/hw_worker_sim.c:39)
    d = rl.HwDesc(opcode=1, seq_len=9, max_tokens=9)
    assert rl.lib().hw_worker_apply_decode_rule(C.byref(d)) == 0 and d.flags == 0 and d.seq_len == 9


def test_reward_and_advantage(rl, olib):
    toks = np.array([1, 2, 3, 4, 5], dtype=np.uint32)
    tgt = np.array([1, 0, 3, 0, 5], dtype=np.uint32)
    assert rl.lib().reward_match_count(toks.ctypes.data, tgt.ctypes.data, 5) == 3
    r = np.array([0.0, 1 / 255, 2 / 255, 3 / 255, 0.5, 0.5, 0.5, 0.5], dtype=np.float32)
    adv = np.zeros(8, dtype=np.float32)
    assert rl.lib().reward_group_advantage(r.ctypes.data, 2, 4, adv.ctypes.data) == 0
    g0 = r[:4].astype(np.float64)
    np.testing.assert_allclose(adv[:4], (g0 - g0.mean()) / g0.std(), rtol=1e-6)
    assert np.all(adv[4:] == 0.0)  # std 0 -> 0
    ref = np.zeros(8, dtype=np.float32)
    olib.orc_group_advantage(r.ctypes.data, 2, 4, ref.ctypes.data)
    assert np.array_equal(adv, ref)
