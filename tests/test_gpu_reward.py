"""Reward rule and group advantage on the device vs the oracle and the host C
(reward.h).

count = matches against the group's target at the same positions, reward =
(count & 0xFF) / 255.0f (src/reward.c:36-41), advantage = (r - mean) / std
with the population std in double, 0 when std is 0: floats bit-identical to
the oracle's orc_match_count / orc_reward_score / orc_group_advantage and to
the runtime's host reward_match_count / reward_group_advantage.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _oracle(olib, tokens, n_tok, targets, gs, tlen):
    R = tokens.shape[0]
    rew = np.zeros(R, np.float32)
    for r in range(R):
        n = min(int(n_tok[r]), tlen, tokens.shape[1])
        t = np.ascontiguousarray(tokens[r])
        g = np.ascontiguousarray(targets[r // gs])
        rew[r] = olib.orc_reward_score(olib.orc_match_count(t.ctypes.data, g.ctypes.data, n))
    adv = np.zeros(R, np.float32)
    olib.orc_group_advantage(rew.ctypes.data, R // gs, gs, adv.ctypes.data)
    return rew, adv


def _host(rl, tokens, n_tok, targets, gs, tlen):
    L = rl.lib()
    R = tokens.shape[0]
    rew = np.zeros(R, np.float32)
    for r in range(R):
        n = min(int(n_tok[r]), tlen, tokens.shape[1])
        t = np.ascontiguousarray(tokens[r])
        g = np.ascontiguousarray(targets[r // gs])
        c = L.reward_match_count(t.ctypes.data, g.ctypes.data, n)
        rew[r] = np.float32(c & 0xFF) / np.float32(255.0)
    adv = np.zeros(R, np.float32)
    assert L.reward_group_advantage(rew.ctypes.data, R // gs, gs, adv.ctypes.data) == 0
    return rew, adv


@pytest.mark.parametrize("groups,gs,T,match", [(64, 8, 256, 0.3), (3, 5, 1000, 0.9), (2, 8, 40, 0.0),
                                               (4, 1, 17, 0.5)])
def test_reward_advantage_matches_oracle_and_host(rl, gpu, olib, groups, gs, T, match):
    rng = np.random.default_rng(groups * 100 + gs)
    R = groups * gs
    targets = rng.integers(0, 32000, (groups, T), dtype=np.uint32)
    tokens = rng.integers(0, 32000, (R, T), dtype=np.uint32)
    hit = rng.random((R, T)) < match
    tokens[hit] = np.repeat(targets, gs, axis=0)[hit]
    n_tok = rng.integers(0, T + 20, R).astype(np.uint32)  # some beyond the target length
    if groups > 2:
        tokens[gs:2 * gs] = targets[1]                         # one group of equal rewards: std 0
        n_tok[gs:2 * gs] = T
    d = {k: rl.DeviceBuffer.from_array(v) for k, v in (("tok", tokens), ("n", n_tok), ("tgt", targets))}
    rew, adv = rl.DeviceBuffer(R * 4, zero=True), rl.DeviceBuffer(R * 4, zero=True)
    descs = rl.DeviceBuffer(R * 24, zero=True)
    a = rl.RewardArgs(tokens=d["tok"].ptr, n_tokens=d["n"].ptr, targets=d["tgt"].ptr, rollouts=R, group_size=gs,
                      token_stride=T, target_stride=T, target_len=T, descs=descs.ptr, reward=rew.ptr,
                      advantage=adv.ptr)
    rl.check(rl.lib().rl_hip_reward_advantage(C.byref(a)), "rl_hip_reward_advantage")
    rl.sync()
    hr, ha = _host(rl, tokens, n_tok, targets, gs, T)
    orr, ora = _oracle(olib, tokens, n_tok, targets, gs, T)
    gr, ga = rew.download(np.float32, R), adv.download(np.float32, R)
    assert np.array_equal(gr.view(np.uint32), orr.view(np.uint32))
    assert np.array_equal(ga.view(np.uint32), ora.view(np.uint32))
    assert np.array_equal(gr.view(np.uint32), hr.view(np.uint32))
    assert np.array_equal(ga.view(np.uint32), ha.view(np.uint32))
    dd = descs.download(np.uint32, (R, 6))
    assert np.array_equal(dd[:, 0], np.arange(R)) and np.array_equal(dd[:, 4].view(np.float32), hr)
    if groups > 2:
        assert np.all(ga[gs:2 * gs] == 0)
    for b in list(d.values()) + [rew, adv, descs]:
        b.close()


def test_reward_distinct_strides_largest_group(rl, gpu, olib):
    """Token rows of 300, target rows of 260 holding 256 target tokens, groups
    of 64 (the largest): counts stop at min(n_tokens, target_len,
    token_stride), with n_tokens past both; bit-identical to the oracle."""
    groups, gs, TS, GS_, TL = 2, 64, 300, 260, 256
    rng = np.random.default_rng(64)
    R = groups * gs
    targets = rng.integers(0, 32000, (groups, GS_), dtype=np.uint32)
    tokens = rng.integers(0, 32000, (R, TS), dtype=np.uint32)
    full = np.zeros((R, TS), np.uint32)
    full[:, :GS_] = np.repeat(targets, gs, axis=0)
    hit = rng.random((R, TS)) < 0.7
    tokens[hit] = full[hit]
    tokens[:, TL:GS_] = full[:, TL:GS_]                       # matches past target_len never count
    n_tok = rng.integers(200, 330, R).astype(np.uint32)
    d = {k: rl.DeviceBuffer.from_array(v) for k, v in (("tok", tokens), ("n", n_tok), ("tgt", targets))}
    rew, adv = rl.DeviceBuffer(R * 4, zero=True), rl.DeviceBuffer(R * 4, zero=True)
    a = rl.RewardArgs(tokens=d["tok"].ptr, n_tokens=d["n"].ptr, targets=d["tgt"].ptr, rollouts=R, group_size=gs,
                      token_stride=TS, target_stride=GS_, target_len=TL, descs=None, reward=rew.ptr,
                      advantage=adv.ptr)
    rl.check(rl.lib().rl_hip_reward_advantage(C.byref(a)), "rl_hip_reward_advantage")
    rl.sync()
    orr = np.zeros(R, np.float32)
    for r in range(R):
        n = min(int(n_tok[r]), TL, TS)
        t = np.ascontiguousarray(tokens[r])
        g = np.ascontiguousarray(targets[r // gs])
        orr[r] = olib.orc_reward_score(olib.orc_match_count(t.ctypes.data, g.ctypes.data, n))
    ora = np.zeros(R, np.float32)
    olib.orc_group_advantage(orr.ctypes.data, groups, gs, ora.ctypes.data)
    assert np.array_equal(rew.download(np.float32, R).view(np.uint32), orr.view(np.uint32))
    assert np.array_equal(adv.download(np.float32, R).view(np.uint32), ora.view(np.uint32))
    for b in list(d.values()) + [rew, adv]:
        b.close()


def test_reward_argument_checks(rl, gpu):
    """Refused before any launch: target_len past target_stride, groups of 0
    or more than 64, rollouts not a multiple of the group size."""
    buf = rl.DeviceBuffer(4096, zero=True)
    base = dict(tokens=buf.ptr, n_tokens=buf.ptr, targets=buf.ptr, rollouts=8, group_size=4, token_stride=8,
                target_stride=8, target_len=8, descs=None, reward=buf.ptr, advantage=buf.ptr)
    for bad in ({"target_len": 9}, {"group_size": 0}, {"group_size": 65, "rollouts": 130}, {"rollouts": 6}):
        a = rl.RewardArgs(**{**base, **bad})
        assert rl.lib().rl_hip_reward_advantage(C.byref(a)) != 0, bad
    buf.close()
