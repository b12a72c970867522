"""Pins the oracle (and the shared sampling-math specification) against what
fixes the answer independently: published known-answer vectors, libm, exact
integer arithmetic, the reference's closed-form decode vector, textbook
softmax attention in numpy, and a brute-force restatement of the sampling
specification in plain Python. CPU only."""
import ctypes as C
import json
import math
import os

import numpy as np
import pytest

import helpers

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def sm():
    lib = helpers.load_shared("tests/c/sample_math_probe.c", link_runtime=False)
    u32, u64, f = C.c_uint32, C.c_uint64, C.c_float
    for name, res, args in [("probe_philox", None, [C.c_void_p] * 3), ("probe_draw64", u64, [u64, u64, u32]),
                            ("probe_mulhi", u64, [u64, u64]), ("probe_expf_cw", f, [f]), ("probe_weight", u32, [f]),
                            ("probe_key", u32, [f]), ("probe_key_float", f, [u32]), ("probe_topp", u64, [f, u64]),
                            ("probe_expf_many", None, [C.c_void_p, C.c_void_p, u32]),
                            ("probe_weight_pair_many", None, [C.c_void_p, C.c_void_p, C.c_void_p, u32]),
                            ("probe_weight_f_many", None, [C.c_void_p] * 4 + [u32])]:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


# ------------------------------------------------------------------ Philox
def test_philox_known_answers(sm, olib):
    kat = json.load(open(os.path.join(GOLD, "philox_kat.json")))
    for v in kat:
        ctr = np.array(v["ctr"], dtype=np.uint32)
        key = np.array(v["key"], dtype=np.uint32)
        for fn in (sm.probe_philox, olib.orc_philox4x32_10):
            out = np.zeros(4, dtype=np.uint32)
            fn(ctr.ctypes.data, key.ctypes.data, out.ctypes.data)
            assert out.tolist() == v["out"]


def _py_philox(ctr, key):
    c, k = list(ctr), list(key)
    M = 0xFFFFFFFF
    for r in range(10):
        if r:
            k = [(k[0] + 0x9E3779B9) & M, (k[1] + 0xBB67AE85) & M]
        a, b = 0xD2511F53 * c[0], 0xCD9E8D57 * c[2]
        c = [(b >> 32) ^ c[1] ^ k[0], b & M, (a >> 32) ^ c[3] ^ k[1], a & M]
    return c


def test_philox_product_vs_oracle_random(sm, olib):
    rng = np.random.default_rng(11)
    for _ in range(2000):
        ctr = rng.integers(0, 2**32, 4, dtype=np.uint64).astype(np.uint32)
        key = rng.integers(0, 2**32, 2, dtype=np.uint64).astype(np.uint32)
        a, b = np.zeros(4, np.uint32), np.zeros(4, np.uint32)
        sm.probe_philox(ctr.ctypes.data, key.ctypes.data, a.ctypes.data)
        olib.orc_philox4x32_10(ctr.ctypes.data, key.ctypes.data, b.ctypes.data)
        assert a.tolist() == b.tolist()
    assert a.tolist() == _py_philox(ctr.tolist(), key.tolist())


def test_draw64_layout(sm):
    seed, step, row = 0x0123456789ABCDEF, 0xFEDCBA9876543210, 77
    o = _py_philox([step & 0xFFFFFFFF, step >> 32, row, 0], [seed & 0xFFFFFFFF, seed >> 32])
    assert sm.probe_draw64(seed, step, row) == o[0] | (o[1] << 32)


def test_mulhi_exact(sm):
    rng = np.random.default_rng(12)
    vals = [0, 1, 2**32 - 1, 2**32, 2**63, 2**64 - 1] + [int(x) for x in rng.integers(0, 2**63, 200)]
    for a in vals:
        for b in vals[:40]:
            assert sm.probe_mulhi(a, b) == (a * b) >> 64


# ------------------------------------------------------------------ exp / weights / keys
def test_expf_cw_against_libm(sm):
    x = np.concatenate([np.linspace(-87.0, 0.0, 2_000_001, dtype=np.float32),
                        -np.geomspace(1e-30, 87, 200_001).astype(np.float32), np.float32([0.0, -0.0])])
    y = np.zeros_like(x)
    sm.probe_expf_many(x.ctypes.data, y.ctypes.data, x.size)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(y.astype(np.float64) - ref) / ref
    assert rel.max() < 4e-7, rel.max()              # ~3 ulp
    assert sm.probe_expf_cw(0.0) == 1.0
    assert sm.probe_expf_cw(-math.inf) == 0.0 and sm.probe_expf_cw(float("nan")) == 0.0
    assert sm.probe_expf_cw(-100.0) == 0.0


def test_weights(sm):
    assert sm.probe_weight(0.0) == 1 << 24
    assert sm.probe_weight(-math.inf) == 0
    d = np.linspace(-20, 0, 200001, dtype=np.float32)
    w = np.array([sm.probe_weight(float(v)) for v in d[::100]], dtype=np.int64)
    assert np.all(np.diff(w) >= 0)                  # monotone
    exact = np.floor(np.exp(d[::100].astype(np.float64)) * 2**24)
    assert np.max(np.abs(w - exact)) <= 8           # a few units of 2^-24


def test_branch_free_weight_equals_weight(sm):
    """rl_sample_weight_nb (the kernels' per-element form) equals
    rl_sample_weight bit for bit on non-positive floats: a stride-997 sweep of
    all 2^31 bit patterns with the sign bit set (through -inf and the NaNs), a
    stride-211 sweep of [-18, -0] (the 2^-24 cut-off of the weights sits at
    -16.6), and every float in [-87.5, -86.5] around the -87 clamp."""
    neg0, m18 = 0x80000000, int(np.float32(-18.0).view(np.uint32))
    lo87, hi87 = int(np.float32(-86.5).view(np.uint32)), int(np.float32(-87.5).view(np.uint32))
    pats = np.arange(neg0, 0x100000000, 997, dtype=np.uint64).astype(np.uint32)
    dense = np.concatenate([np.arange(neg0, m18 + 1, 211, dtype=np.uint64),
                            np.arange(lo87, hi87 + 1, dtype=np.uint64)]).astype(np.uint32)
    for u in (pats, dense):
        d = np.concatenate([u.view(np.float32), np.float32([0.0, -0.0, -np.inf, np.nan])])
        a = np.zeros(d.size, np.uint32)
        b = np.zeros(d.size, np.uint32)
        sm.probe_weight_pair_many(d.ctypes.data, a.ctypes.data, b.ctypes.data, d.size)
        assert np.array_equal(a, b), d[np.nonzero(a != b)[0][:5]]


def test_weight_with_float_equals_weight(sm):
    """rl_sample_weight_f (the row kernel's form: one scaling by 2^(n+24),
    no final select) equals rl_sample_weight bit for bit on the same sweeps
    as above, and its float is e^d 2^24 to within 2 ulp in double for
    d in [-87, 0] (the row kernel sums it for the log-sum-exp)."""
    neg0, m18 = 0x80000000, int(np.float32(-18.0).view(np.uint32))
    lo87, hi87 = int(np.float32(-86.5).view(np.uint32)), int(np.float32(-87.5).view(np.uint32))
    pats = np.arange(neg0, 0x100000000, 997, dtype=np.uint64).astype(np.uint32)
    dense = np.concatenate([np.arange(neg0, m18 + 1, 211, dtype=np.uint64),
                            np.arange(lo87, hi87 + 1, dtype=np.uint64)]).astype(np.uint32)
    for u in (pats, dense):
        d = np.concatenate([u.view(np.float32), np.float32([0.0, -0.0, -np.inf, np.nan])])
        a = np.zeros(d.size, np.uint32)
        b = np.zeros(d.size, np.uint32)
        f = np.zeros(d.size, np.float32)
        sm.probe_weight_f_many(d.ctypes.data, a.ctypes.data, b.ctypes.data, f.ctypes.data, d.size)
        assert np.array_equal(a, b), d[np.nonzero(a != b)[0][:5]]
        sel = (d >= -87.0) & (d <= 0.0)
        want = np.exp(d[sel].astype(np.float64)) * 2.0**24
        rel = np.abs(f[sel].astype(np.float64) - want) / want
        assert rel.max() < 2.0**-22, rel.max()
    assert sm.probe_weight(-87.0) == 0  # (the clamp itself weighs 0)


def test_float_key_orders_like_floats(sm):
    rng = np.random.default_rng(13)
    x = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10,
                        np.float32([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38])])
    k = np.array([sm.probe_key(float(v)) for v in x], dtype=np.uint64)
    for i in range(0, len(x), 7):
        for j in range(0, len(x), 11):
            assert (k[i] < k[j]) == (x[i] < x[j]) and (k[i] == k[j]) == (x[i] == x[j])
    for v in x:
        if v != 0:
            assert sm.probe_key_float(sm.probe_key(float(v))) == v


def test_topp_threshold(sm):
    assert sm.probe_topp(0.9, 100) == 90
    assert sm.probe_topp(0.5, 3) == 2
    w = 50 * (1 << 24)
    assert sm.probe_topp(np.float32(0.9), w) == math.ceil(float(np.float32(0.9)) * w)


# ------------------------------------------------------------------ attention
def _textbook_attention(q, K, V, scale):
    s = (K @ q) * scale
    p = np.exp(s - s.max())
    return (p[:, None] * V).sum(0) / p.sum()


def _fixed128_vector():
    """test/test_bench.cu:91-107 closed form, 17 tokens in a 32-token fp16 block."""
    d = np.arange(128)
    q = ((d % 17) - 8) / 8.0
    t = np.arange(32)[:, None]
    K = ((((t + 1) * ((d % 13) + 1)) % 23) - 11) / 32.0
    V = ((((t + 3) * ((d % 11) + 5)) % 29) - 14) / 29.0
    return q, K, V


def test_attention_oracle_fixed128_closed_form(orc, olib, rl):
    import synth
    q, K, V = _fixed128_vector()
    q16, K16, V16 = (synth.f32_to_f16(a.astype(np.float32)) for a in (q, K, V))
    w = synth.DecodeWorkload(1, 1, 1, 128, "fp16", 32, np.array([17], np.uint32), np.zeros((1, 1, 1), np.uint32),
                             np.concatenate([K16.ravel(), V16.ravel()]).view(np.uint8), q16.reshape(1, 1, 128), 0)
    ref = _textbook_attention(synth.f16_to_f32(q16).astype(np.float64), synth.f16_to_f32(K16)[:17].astype(np.float64),
                              synth.f16_to_f32(V16)[:17].astype(np.float64), 1 / np.sqrt(128))
    o64 = orc.attn_f64(olib, w, 1)[0, 0]
    o32 = orc.attn_f32(olib, w, 1)[0, 0]
    np.testing.assert_allclose(o64, ref, rtol=0, atol=1e-12)
    assert np.max(np.abs(o32 - ref)) < 1e-4         # the reference test's bound (test_bench.cu:716-717)
    assert int(np.argmax(o64)) == int(np.argmax(ref))  # lowest-index argmax token


def test_synth_query_known_values(olib):
    """decode_synth_query_component (cu/attention_decode.cu:16-28), values
    worked out by hand: with seq_id = cookie = 0 the seed of component idx is
    (idx + 1) * 0x9e3779b97f4a7c15 mod 2^64; idx 0: 0x9e3779b97f4a7c15, folded
    0x7f4a7c15 ^ 0x9e3779b9 = 0xe17d05ac, low byte 0xac = 172 -> 45/127;
    idx 1: 0x3c6ef372fe94f82a, folded 0xc2fa0b58, 0x58 = 88 -> -39/127. A
    sample state xors rng_state[idx & 3] into the seed: rng_state[0] = 1 turns
    idx 0's low byte into 0xad -> 46/127, and rng_state[1] = 0x100 leaves
    idx 1's low byte alone (-39/127)."""
    f = np.float32
    assert olib.orc_synth_query(0, 0, None, 0) == f(45) / f(127)
    assert olib.orc_synth_query(0, 0, None, 1) == f(-39) / f(127)
    st = np.array([1, 0x100, 0, 0], dtype=np.uint64)
    assert olib.orc_synth_query(0, 0, st.ctypes.data, 0) == f(46) / f(127)
    assert olib.orc_synth_query(0, 0, st.ctypes.data, 1) == f(-39) / f(127)
    # seq_id and cookie enter the seed symmetrically
    assert olib.orc_synth_query(5, 9, None, 7) == olib.orc_synth_query(9, 5, None, 7)


def _numpy_paged(w):
    import synth
    f = synth.bf16_to_f32 if w.dtype == "bf16" else synth.f16_to_f32
    arena = f(w.arena.view(np.uint16)).astype(np.float64).reshape(-1, 2, w.token_count, w.head_dim)
    q = f(w.q).astype(np.float64)
    G = w.q_heads // w.kv_heads
    out = np.zeros((w.batch, w.q_heads, w.head_dim))
    for b in range(w.batch):
        n = int(w.ctx[b])
        for g in range(w.kv_heads):
            blocks = w.table[b, g, : -(-n // w.token_count)]
            K = arena[blocks, 0].reshape(-1, w.head_dim)[:n]
            V = arena[blocks, 1].reshape(-1, w.head_dim)[:n]
            for i in range(G):
                if n:
                    out[b, g * G + i] = _textbook_attention(q[b, g * G + i], K, V, 1 / np.sqrt(w.head_dim))
    return out


@pytest.mark.parametrize("cfg", [(3, 8, 2, 128, "bf16", 1, 300), (2, 8, 8, 64, "fp16", 1, 100),
                                 (2, 16, 2, 128, "bf16", 1, 70), (4, 4, 4, 64, "bf16", 0, 40)])
def test_attention_oracle_vs_numpy(orc, olib, rl, cfg):
    import synth
    B, QH, KVH, D, dt, lo, hi = cfg
    w = synth.make_decode(21, B, QH, KVH, D, lo, hi, dtype=dt)
    if lo == 0:
        w.ctx[0] = 0
    ref = _numpy_paged(w)
    code = 0 if dt == "bf16" else 1
    np.testing.assert_allclose(orc.attn_f64(olib, w, code), ref, rtol=0, atol=1e-12)
    assert np.max(np.abs(orc.attn_f32(olib, w, code) - ref)) < 2e-5


def test_attention_oracle_invariants(orc, olib, rl):
    """Closed forms: identical V rows -> that row; a single token -> V[0];
    shift-invariance of softmax (adding the same q.k to every token)."""
    import synth
    w = synth.make_decode(22, 2, 4, 1, 64, 50, 80, dtype="bf16")
    a = w.arena.view(np.uint16).reshape(-1, 2, 16, 64)
    a[:, 1] = a[0, 1, 0]                           # all V rows equal
    out = orc.attn_f64(olib, w, 0)
    np.testing.assert_allclose(out, np.broadcast_to(synth.bf16_to_f32(a[0, 1, 0]), out.shape), atol=1e-12)
    w2 = synth.make_decode(23, 2, 4, 2, 64, 1, 1, dtype="bf16")
    out2 = orc.attn_f64(olib, w2, 0)
    a2 = w2.arena.view(np.uint16).reshape(-1, 2, 16, 64)
    for b in range(2):
        for h in range(4):
            blk = w2.table[b, h // 2, 0]
            np.testing.assert_allclose(out2[b, h], synth.bf16_to_f32(a2[blk, 1, 0]), atol=1e-12)


# ------------------------------------------------------------------ sampling
def _py_sample(l, greedy, T, k, p, seed, step, row, weight):
    """Plain-Python restatement of the sampling specification in sample.h."""
    V = len(l)
    if greedy or not T > 0:
        tok = max(range(V), key=lambda i: (l[i], -i))
        m = max(l)
        return tok, l[tok] - (m + math.log(sum(math.exp(v - m) for v in l)))
    inv = np.float32(1.0) / np.float32(T)
    x = [float(np.float32(v) * inv) for v in l]
    m = max(x)
    keff = min(k, 256) if 0 < k < V else 0
    cut = sorted(x, reverse=True)[keff - 1] if keff else -math.inf
    kept = sorted([i for i in range(V) if x[i] >= cut and x[i] != -math.inf], key=lambda i: (-x[i], i))
    w = {i: weight(float(np.float32(x[i]) - np.float32(m))) for i in kept}
    wk = sum(w.values())
    P = kept
    if 0 < p < 1:
        thr = math.ceil(float(np.float32(p)) * wk)
        c = 0
        for j, i in enumerate(kept):
            c += w[i]
            if c >= thr:
                P = kept[: j + 1]
                break
    wp = sum(w[i] for i in P)
    o = _py_philox([step & 0xFFFFFFFF, step >> 32, row, 0], [seed & 0xFFFFFFFF, seed >> 32])
    u = ((o[0] | (o[1] << 32)) * wp) >> 64
    c, tok = 0, min(P)
    for i in sorted(P):
        c += w[i]
        if c > u:
            tok = i
            break
    mm = max(x)
    return tok, x[tok] - (mm + math.log(sum(math.exp(v - mm) for v in x)))


def test_sampling_oracle_vs_python_bruteforce(sm, orc, olib):
    rng = np.random.default_rng(31)
    weight = sm.probe_weight
    for trial in range(300):
        V = int(rng.integers(2, 160))
        l = (rng.standard_normal(V) * rng.choice([0.3, 1, 3])).astype(np.float32)
        if trial % 5 == 0:                          # ties, including at the top-k cutoff
            l = np.round(l).astype(np.float32)
        T = float(rng.choice([0.0, 0.5, 0.8, 1.0, 1.7]))
        k = int(rng.choice([0, 1, 3, 10, 50, V - 1, V]))
        p = float(rng.choice([1.0, 0.9, 0.5, 0.05]))
        seed, step, row = int(rng.integers(0, 2**63)), int(rng.integers(0, 2**40)), int(rng.integers(0, 300))
        lp = C.c_double()
        tok = olib.orc_sample_row(l.ctypes.data, V, 0, T, k, p, seed, step, row, C.byref(lp))
        ptok, plp = _py_sample(l.tolist(), False, T, k, p, seed, step, row, weight)
        assert tok == ptok, (trial, V, T, k, p)
        assert abs(lp.value - plp) < 1e-9


def test_sampling_greedy_lowest_index_tie(olib):
    l = np.array([0, 3, 1, 3, 3, -1], dtype=np.float32)
    lp = C.c_double()
    assert olib.orc_sample_row(l.ctypes.data, 6, 1, 1.0, 0, 1.0, 0, 0, 0, C.byref(lp)) == 1
    assert abs(lp.value - (3 - np.log(np.exp(l.astype(np.float64)).sum()))) < 1e-12


def test_sampling_oracle_distribution(olib):
    """Frequencies over many Philox steps match the truncated softmax."""
    l = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 3.0], dtype=np.float32)
    counts = np.zeros(6)
    n = 20000
    lp = C.c_double()
    for s in range(n):
        counts[olib.orc_sample_row(l.ctypes.data, 6, 0, 1.0, 3, 1.0, 99, s, 0, C.byref(lp))] += 1
    top = [5, 0, 1]
    pr = np.exp(l[top] - l[top].max())
    pr /= pr.sum()
    assert counts[[2, 3, 4]].sum() == 0
    np.testing.assert_allclose(counts[top] / n, pr, atol=0.015)
    # top-p 0.5 over these: keeps {5} (p=0.665 > 0.5) only
    for s in range(200):
        assert olib.orc_sample_row(l.ctypes.data, 6, 0, 1.0, 3, 0.5, 99, s, 0, C.byref(lp)) == 5


# ------------------------------------------------------------------ KV append
def test_kv_append_oracle(olib):
    tc, rb, stride = 16, 256, 4
    arena = np.zeros(8 * 2 * tc * rb, dtype=np.uint8)
    src = np.arange(2 * tc * rb, dtype=np.uint32).astype(np.uint8)
    arena[3 * 2 * tc * rb:4 * 2 * tc * rb] = src          # shared block 3
    table = np.array([[5, 6, 0, 0]], dtype=np.uint32)
    pos = np.array([16 + 5], dtype=np.uint32)              # block 1 (phys 6), slot 5
    cow = np.array([3], dtype=np.int32)
    kn = np.full(rb, 0xAA, np.uint8)
    vn = np.full(rb, 0xBB, np.uint8)
    olib.orc_kv_append(arena.ctypes.data, 2 * tc * rb, tc, rb, table.ctypes.data, stride, 1, 1, pos.ctypes.data,
                       cow.ctypes.data, kn.ctypes.data, vn.ctypes.data)
    blk = arena[6 * 2 * tc * rb:7 * 2 * tc * rb].reshape(2, tc, rb)
    s = src.reshape(2, tc, rb)
    assert np.array_equal(blk[:, :5], s[:, :5])            # copied slots
    assert np.all(blk[0, 5] == 0xAA) and np.all(blk[1, 5] == 0xBB)
    assert np.all(blk[:, 6:] == 0)


def test_sampling_all_masked_row(olib):
    """Every logit -inf: the kept set is empty and the token is 0 (specified),
    whatever the nucleus; the logprob is NaN."""
    x = np.full(300, -np.inf, dtype=np.float32)
    lp = C.c_double()
    for k, p in ((0, 1.0), (0, 0.9), (3, 0.3), (50, 1.0)):
        assert olib.orc_sample_row(x.ctypes.data, 300, 0, 0.7, k, p, 9, 2, 2, C.byref(lp)) == 0
        assert math.isnan(lp.value)


def test_branch_resolve_oracle_known_cases(olib):
    """The device resolve rule (cu/kv_prefix.cu:4-15) on hand-built tables:
    a live prefix gives its offset; a released prefix (refcount 0) gives the
    branch's delta, where the host total_offset gives the -1 that release
    stored; a prefix id past 512 gives the delta; a branch id past 16,384
    gives -1. The copy-on-write source follows the head-major prefix layout."""
    t = np.zeros(606280, np.uint8)
    olib.orc_kvp_init(t.ctypes.data)
    pid, bid = C.c_uint32(), C.c_uint32()
    assert olib.orc_kvp_register(t.ctypes.data, 4096, 520, 8 * 33, C.byref(pid)) == 0 and pid.value == 0
    assert olib.orc_kvb_alloc(t.ctypes.data, 7, 0, 90000, 3, 1, C.byref(bid)) == 0 and bid.value == 0
    assert olib.orc_kvb_resolve(t.ctypes.data, 0) == 4096
    assert olib.orc_kvb_total_offset(t.ctypes.data, 0) == 4096
    # token_len 520 = 32 full blocks + 8 slots: block 32 of head h is 4096 + 33 h + 32
    assert olib.orc_kvb_cow_source(t.ctypes.data, 0, 520, 16, 8, 0) == 4096 + 32
    assert olib.orc_kvb_cow_source(t.ctypes.data, 0, 520, 16, 8, 5) == 4096 + 5 * 33 + 32
    assert olib.orc_kvb_cow_source(t.ctypes.data, 0, 521, 16, 8, 5) == -1      # not the first own token
    assert olib.orc_kvb_cow_source(t.ctypes.data, 0, 520, 8, 8, 0) == -1       # 520 = 65 whole 8-token blocks
    # a branch whose prefix id is out of range: the delta
    assert olib.orc_kvb_alloc(t.ctypes.data, 8, 600, 123456, 3, 1, C.byref(bid)) == 0 and bid.value == 1
    assert olib.orc_kvb_resolve(t.ctypes.data, 1) == 123456
    assert olib.orc_kvb_cow_source(t.ctypes.data, 1, 520, 16, 8, 0) == -1
    # release the prefix to refcount 0 (branch 0 holds one reference, register the other)
    assert olib.orc_kvp_release(t.ctypes.data, 0) == 0 and olib.orc_kvp_release(t.ctypes.data, 0) == 0
    assert olib.orc_kvb_total_offset(t.ctypes.data, 0) == -1
    assert olib.orc_kvb_resolve(t.ctypes.data, 0) == 90000
    assert olib.orc_kvb_cow_source(t.ctypes.data, 0, 520, 16, 8, 0) == -1
    assert olib.orc_kvb_resolve(t.ctypes.data, 16384) == -1


def test_plumbing_cpu_path_equals_sequential_oracle(orc, olib):
    """The CPU baseline of the plumbing decode (hw_worker_sim loop on a pthread
    with a real step per token) computes what the oracle computes step by
    step: greedy tokens equal argmax, each step's fp32 attention equals
    orc_attn_decode_f32 over the arena as the earlier appends left it, and the
    final arena equals the sequential appends."""
    import synth

    n, ctx0, V = 6, 40, 512
    steps = 2 * n
    rng = np.random.default_rng(9)
    w = synth.make_decode(8, 1, 8, 8, 64, ctx0, ctx0, dtype="fp16", kv_std=0.5, reserve_tokens=ctx0 + steps + 1)
    q = synth.f32_to_f16(rng.standard_normal((steps, 8, 64), dtype=np.float32))
    kn = synth.f32_to_f16(rng.standard_normal((steps, 8, 64), dtype=np.float32))
    vn = synth.f32_to_f16(rng.standard_normal((steps, 8, 64), dtype=np.float32))
    logits = rng.standard_normal((steps, V), dtype=np.float32)
    arena = w.arena.copy()
    out = np.zeros((steps, 8, 64), np.float32)
    tok = np.zeros(steps, np.uint32)
    p = orc.OrcPlumbing(arena=arena.ctypes.data, block_bytes=w.block_bytes, token_count=16, head_dim=64, dtype=1,
                        table=w.table.ctypes.data, table_stride=w.table_stride, q_heads=8, kv_heads=8,
                        scale=1.0 / 8.0, q=q.ctypes.data, k_new=kn.ctypes.data, v_new=vn.ctypes.data,
                        logits=logits.ctypes.data, vocab=V, steps=steps, attn_out=out.ctypes.data,
                        tokens=tok.ctypes.data)
    pipe = C.c_double()
    lat = np.zeros(n, np.float64)
    assert olib.orc_plumbing_run(C.byref(p), ctx0, n, C.byref(pipe), lat.ctypes.data) == 0
    assert pipe.value > 0 and (lat > 0).all()
    assert np.array_equal(tok, np.argmax(logits, axis=1).astype(np.uint32))
    host = w.arena.copy()
    for k in range(steps):
        wk = synth.DecodeWorkload(1, 8, 8, 64, "fp16", 16, np.array([ctx0 + k], np.uint32), w.table, host,
                                  q[k].reshape(1, 8, 64), 0)
        assert np.array_equal(out[k], orc.attn_f32(olib, wk, 1)[0]), k
        pos = np.array([ctx0 + k], np.uint32)
        k_row, v_row = np.ascontiguousarray(kn[k]), np.ascontiguousarray(vn[k])
        olib.orc_kv_append(host.ctypes.data, w.block_bytes, 16, 128, w.table.ctypes.data, w.table_stride, 1, 8,
                           pos.ctypes.data, None, k_row.ctypes.data, v_row.ctypes.data)
    assert np.array_equal(arena, host)


def test_decode_workload_spare_blocks_owned_by_no_row():
    """The synthetic decode workload's spare blocks (the copy-on-write sources
    of the append tests) are the arena's last ids and no row's table holds
    them; every owned block belongs to exactly one (rollout, kv head, block)."""
    import synth

    for spare in (0, 8, 40):
        w = synth.make_decode(31, 24, 32, 8, 128, 200, 1500, spare_blocks=spare)
        total = w.arena.size // w.block_bytes
        nblk = -(-(w.ctx.astype(np.int64) + 1) // w.token_count)
        owned = np.concatenate([w.table[b, g, :nblk[b]] for b in range(w.batch) for g in range(w.table.shape[1])])
        assert len(np.unique(owned)) == len(owned)
        assert owned.max() < total - spare
        assert total - spare == len(owned)


def test_sample_rows_v_matches_per_row_calls(olib):
    """orc_sample_rows_v (per-row parameters, OpenMP over rows) returns what
    orc_sample_row returns row by row with the same parameters, draw ids
    included."""
    import orc
    rng = np.random.default_rng(91)
    rows, V = 24, 3000
    x = rng.standard_normal((rows, V), dtype=np.float32)
    temp = np.where(rng.random(rows) < 0.25, 0.0, rng.uniform(0.5, 1.5, rows)).astype(np.float32)
    topk = rng.choice([0, 5, 50, 300], rows).astype(np.uint32)
    topp = rng.choice([1.0, 0.9, 0.5], rows).astype(np.float32)
    seeds = rng.integers(0, 2**63, rows, dtype=np.uint64)
    steps = rng.integers(0, 1000, rows, dtype=np.uint64)
    ids = rng.integers(0, 1 << 20, rows).astype(np.uint32)
    tok, lp = orc.sample_rows_v(olib, x, temperature=temp, top_k=topk, top_p=topp, seeds=seeds, steps=steps,
                                draw_ids=ids)
    one = C.c_double()
    for r in range(rows):
        want = olib.orc_sample_row(x[r].ctypes.data, V, int(not temp[r] > 0), float(temp[r]), int(topk[r]),
                                   float(topp[r]), int(seeds[r]), int(steps[r]), int(ids[r]), C.byref(one))
        assert tok[r] == want and lp[r] == one.value, r
    # scalar parameters and the row index as the draw id
    tok2, _ = orc.sample_rows_v(olib, x, seeds=seeds, temperature_all=1.0, top_k_all=50, top_p_all=0.9, step_all=7)
    want2, _ = orc.sample_rows(olib, x, False, 1.0, 50, 0.9, seeds, 7)
    assert np.array_equal(tok2, want2)
