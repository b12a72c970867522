"""Seeded synthetic inputs for the decode workloads (numpy, host side).

One generator per workload shape; every tensor is drawn from
numpy.random.default_rng(seed) and rounded to bf16 (round-to-nearest-even)
or fp16, then uploaded as-is. The arena is laid out as the runtime's paged
KV arena: blocks of `token_count` tokens of one KV head, K plane then V
plane; each (rollout, KV head) owns ceil((ctx + 1) / token_count) blocks (one
slot is kept free for the next appended token), placed at a seeded random
permutation of the physical block ids.
"""
from __future__ import annotations

import dataclasses

import numpy as np


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_scalar16(x: np.ndarray, dtype: str) -> np.ndarray:
    return f32_to_bf16(x) if dtype == "bf16" else f32_to_f16(x)


def from_scalar16(h: np.ndarray, dtype: str) -> np.ndarray:
    return bf16_to_f32(h) if dtype == "bf16" else f16_to_f32(h)


@dataclasses.dataclass
class DecodeWorkload:
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: str                 # "bf16" | "fp16"
    token_count: int           # tokens per arena block
    ctx: np.ndarray            # [batch] uint32
    table: np.ndarray          # [batch, kv_heads, table_stride] uint32
    arena: np.ndarray          # [n_blocks * block_bytes] uint8
    q: np.ndarray              # [batch, q_heads, head_dim] uint16
    seed: int

    @property
    def block_bytes(self) -> int:
        return 2 * self.token_count * self.head_dim * 2

    @property
    def table_stride(self) -> int:
        return self.table.shape[2]

    @property
    def max_ctx(self) -> int:
        return int(self.ctx.max()) if self.ctx.size else 0

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes one decode step reads."""
        return int(self.ctx.astype(np.int64).sum()) * self.kv_heads * self.head_dim * 2 * 2


def _fill_normal(rng: np.random.Generator, n: int, std: float, dtype: str, out: np.ndarray,
                 chunk: int = 1 << 22) -> None:
    """out[:n] = round16(N(0, std^2)), in chunks with reused scratch buffers."""
    f = np.empty(min(chunk, max(n, 1)), dtype=np.float32)
    r = np.empty_like(f, dtype=np.uint32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        fv, rv = f[:m], r[:m]
        rng.standard_normal(out=fv, dtype=np.float32)
        if std != 1.0:
            fv *= np.float32(std)
        if dtype == "bf16":
            u = fv.view(np.uint32)
            np.right_shift(u, np.uint32(16), out=rv)
            rv &= np.uint32(1)
            rv += np.uint32(0x7FFF)
            u += rv
            u >>= np.uint32(16)
            np.copyto(out[s:s + m], u, casting="unsafe")
        else:
            out[s:s + m] = fv.astype(np.float16).view(np.uint16)


def make_decode(seed: int, batch: int, q_heads: int, kv_heads: int, head_dim: int, ctx_lo: int, ctx_hi: int,
                dtype: str = "bf16", kv_std: float = 1.0, token_count: int = 16, max_ctx: int | None = None,
                ctx: np.ndarray | None = None, spare_blocks: int = 0,
                reserve_tokens: int = 0) -> DecodeWorkload:
    """Ragged contexts uniform in [ctx_lo, ctx_hi] (or given), permuted blocks;
    every row owns blocks for max(ctx + 1, reserve_tokens) tokens. The
    spare_blocks spare blocks are the last ids of the arena, owned by no row
    (copy-on-write sources read while rows append)."""
    rng = np.random.default_rng(seed)
    if ctx is None:
        ctx = rng.integers(ctx_lo, ctx_hi + 1, size=batch, dtype=np.int64)
    ctx = np.asarray(ctx, dtype=np.uint32)
    cap = int(max_ctx if max_ctx is not None else (ctx.max() if batch else 0))
    cap = max(cap, reserve_tokens - 1)
    stride = max(1, -(-(cap + 1) // token_count))
    nblk = -(-np.maximum(ctx.astype(np.int64) + 1, reserve_tokens) // token_count)  # blocks per (b, g)
    owned = int(nblk.sum()) * kv_heads
    total = owned + spare_blocks
    perm = rng.permutation(total if spare_blocks == 0 else owned).astype(np.uint32)
    table = np.zeros((batch, kv_heads, stride), dtype=np.uint32)
    k = 0
    for b in range(batch):
        for g in range(kv_heads):
            n = int(nblk[b])
            table[b, g, :n] = perm[k:k + n]
            k += n
    block_elems = 2 * token_count * head_dim
    arena = np.empty(total * block_elems, dtype=np.uint16)
    _fill_normal(rng, arena.size, kv_std, dtype, arena)
    q = np.empty(batch * q_heads * head_dim, dtype=np.uint16)
    _fill_normal(rng, q.size, 1.0, dtype, q)
    return DecodeWorkload(batch, q_heads, kv_heads, head_dim, dtype, token_count, ctx, table,
                          arena.view(np.uint8), q.reshape(batch, q_heads, head_dim), seed)


def make_logits(seed: int, rows: int, vocab: int, std: float = 1.0, spikes: int = 0,
                spike_value: float = 8.0) -> np.ndarray:
    """fp32 logits ~N(0, std^2); `spikes` seeded tokens per row SET to spike_value."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(std)
    for r in range(rows):
        if spikes:
            idx = rng.choice(vocab, size=spikes, replace=False)
            x[r, idx] = np.float32(spike_value)
    return x
