"""ctypes binding of the oracle (oracle/liboracle.so) and of the reference C
sources compiled into oracle/_ref/libgbref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, to check results or as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libgbref.so")


class OrcAttn(C.Structure):
    _fields_ = [("arena", C.c_void_p), ("block_bytes", C.c_uint64), ("token_count", C.c_uint32),
                ("head_dim", C.c_uint32), ("dtype", C.c_uint32), ("table", C.c_void_p),
                ("table_stride", C.c_uint32), ("batch", C.c_uint32), ("q_heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("ctx", C.c_void_p), ("q", C.c_void_p), ("scale", C.c_double)]


class OrcPlumbing(C.Structure):
    _fields_ = [("arena", C.c_void_p), ("block_bytes", C.c_uint64), ("token_count", C.c_uint32),
                ("head_dim", C.c_uint32), ("dtype", C.c_uint32), ("table", C.c_void_p),
                ("table_stride", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("scale", C.c_double), ("q", C.c_void_p), ("k_new", C.c_void_p), ("v_new", C.c_void_p),
                ("logits", C.c_void_p), ("vocab", C.c_uint32), ("steps", C.c_uint32), ("attn_out", C.c_void_p),
                ("tokens", C.c_void_p)]


class RingShape(C.Structure):
    _fields_ = [("slot_size", C.c_uint32), ("n_slots", C.c_uint32), ("slot_off", C.c_uint32),
                ("overflow_off", C.c_int32)]


CMD_RING = RingShape(32, 4096, 128, -1)
COMP_RING = RingShape(32, 4096, 256, 128)
REQ_RING = RingShape(34, 1024, 128, -1)
DONE_RING = RingShape(24, 1024, 256, 128)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def load_oracle() -> C.CDLL:
    if not os.path.exists(ORACLE_PATH):
        raise FileNotFoundError(f"{ORACLE_PATH} not built (make -C oracle)")
    o = C.CDLL(ORACLE_PATH)
    vp, u32, u64, i64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int64, C.c_int
    sigs = {
        "orc_hw_ring_push": (i32, [vp, vp]), "orc_hw_ring_pop": (i32, [vp, vp]),
        "orc_synth_query": (C.c_float, [u64, u64, vp, u32]),
        "orc_submit_decode": (i64, [vp, u32, u32, u32, u64, u64, u32, u32, u32]),
        "orc_worker_sim_drain": (u64, [vp, vp, C.POINTER(u64), C.POINTER(i32)]),
        "orc_ring_acquire": (u32, [vp, C.POINTER(RingShape), u32]),
        "orc_ring_commit": (None, [vp, u32]),
        "orc_ring_consume": (i32, [vp, C.POINTER(RingShape), vp]),
        "orc_ring_push_or_overflow": (i32, [vp, C.POINTER(RingShape), vp]),
        "orc_decode_batch_submit": (i32, [vp, vp, u32]),
        "orc_arena_acquire": (i64, [vp]), "orc_arena_release": (None, [vp, i64]),
        "orc_kvp_init": (None, [vp]),
        "orc_kvp_register": (i32, [vp, i64, u32, u32, C.POINTER(u32)]),
        "orc_kvp_acquire": (i32, [vp, u32]), "orc_kvp_release": (i32, [vp, u32]),
        "orc_kvb_alloc": (i32, [vp, u32, u32, i64, u32, u32, C.POINTER(u32)]),
        "orc_kvb_free": (i32, [vp, u32]), "orc_kvb_total_offset": (i64, [vp, u32]),
        "orc_kvb_resolve": (i64, [vp, u32]), "orc_kvb_cow_source": (i64, [vp, u32, u32, u32, u32, u32]),
        "orc_reward_score": (C.c_float, [u32]), "orc_match_count": (u32, [vp, vp, u32]),
        "orc_group_advantage": (None, [vp, u32, u32, vp]),
        "orc_philox4x32_10": (None, [vp, vp, vp]),
        "orc_attn_decode_f64": (None, [C.POINTER(OrcAttn), vp]),
        "orc_attn_decode_f32": (None, [C.POINTER(OrcAttn), vp]),
        "orc_sample_row": (u32, [vp, u32, i32, C.c_float, u32, C.c_float, u64, u64, u32, C.POINTER(C.c_double)]),
        "orc_sample_rows": (None, [vp, u32, u32, u32, i32, C.c_float, u32, C.c_float, vp, u64, vp, vp]),
        "orc_sample_rows_v": (None, [vp, u32, u32, u32, vp, vp, vp, vp, vp, vp, C.c_float, u32, C.c_float, u64, vp,
                                     vp]),
        "orc_kv_append": (None, [vp, u64, u32, u32, vp, u32, u32, u32, vp, vp, vp, vp]),
        "orc_num_threads": (i32, []), "orc_set_num_threads": (None, [i32]),
        "orc_plumbing_run": (i32, [C.POINTER(OrcPlumbing), u32, u32, C.POINTER(C.c_double), vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(o, name)
        fn.restype, fn.argtypes = res, args
    return o


def load_ref() -> C.CDLL | None:
    """The reference's own C sources (oracle/_ref), or None when not built."""
    if not os.path.exists(REF_PATH):
        return None
    return C.CDLL(REF_PATH)


# ---------------------------------------------------------------- wrappers
def attn_struct(w, dtype_code: int, scale: float | None = None) -> OrcAttn:
    a = OrcAttn()
    a.arena, a.block_bytes, a.token_count = _p(w.arena), w.block_bytes, w.token_count
    a.head_dim, a.dtype = w.head_dim, dtype_code
    a.table, a.table_stride = _p(w.table), w.table_stride
    a.batch, a.q_heads, a.kv_heads = w.batch, w.q_heads, w.kv_heads
    a.ctx, a.q = _p(w.ctx), _p(w.q)
    a.scale = float(scale) if scale is not None else 1.0 / np.sqrt(w.head_dim)
    return a


def attn_f64(o: C.CDLL, w, dtype_code: int, scale: float | None = None) -> np.ndarray:
    out = np.zeros((w.batch, w.q_heads, w.head_dim), dtype=np.float64)
    a = attn_struct(w, dtype_code, scale)
    o.orc_attn_decode_f64(C.byref(a), _p(out))
    return out


def attn_f32(o: C.CDLL, w, dtype_code: int, scale: float | None = None) -> np.ndarray:
    out = np.zeros((w.batch, w.q_heads, w.head_dim), dtype=np.float32)
    a = attn_struct(w, dtype_code, scale)
    o.orc_attn_decode_f32(C.byref(a), _p(out))
    return out


def sample_rows(o: C.CDLL, logits: np.ndarray, greedy: bool, temperature: float, top_k: int, top_p: float,
                seeds, step: int, vocab: int | None = None):
    """seeds: one per row (array) or a scalar for every row."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, stride = logits.shape
    vocab = stride if vocab is None else vocab
    seeds = np.ascontiguousarray(np.broadcast_to(np.asarray(seeds, dtype=np.uint64), (rows,)))
    tok = np.zeros(rows, dtype=np.uint32)
    lp = np.zeros(rows, dtype=np.float64)
    o.orc_sample_rows(_p(logits), rows, vocab, stride, int(greedy), temperature, top_k, top_p, _p(seeds), step,
                      _p(tok), _p(lp))
    return tok, lp


def sample_rows_v(o: C.CDLL, logits: np.ndarray, temperature=None, top_k=None, top_p=None, seeds=None, steps=None,
                  draw_ids=None, temperature_all: float = 1.0, top_k_all: int = 0, top_p_all: float = 1.0,
                  step_all: int = 0):
    """Per-row parameters (arrays of `rows` entries, or None for the scalar)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, stride = logits.shape

    def arr(a, dt):
        return None if a is None else np.ascontiguousarray(a, dtype=dt)
    t, k, p = arr(temperature, np.float32), arr(top_k, np.uint32), arr(top_p, np.float32)
    s, st, di = arr(seeds, np.uint64), arr(steps, np.uint64), arr(draw_ids, np.uint32)
    tok = np.zeros(rows, dtype=np.uint32)
    lp = np.zeros(rows, dtype=np.float64)
    ptr = lambda a: None if a is None else _p(a)  # noqa: E731
    o.orc_sample_rows_v(_p(logits), rows, stride, stride, ptr(t), ptr(k), ptr(p), ptr(s), ptr(st), ptr(di),
                        temperature_all, top_k_all, top_p_all, step_all, _p(tok), _p(lp))
    return tok, lp
