/*
 * kv_layout.h - KV block layout descriptor.
 *
 * KvLayoutDesc is byte-compatible with the reference (include/kv_layout.h:
 * 26-35: eight u32 fields). One block holds `token_count` tokens of ONE KV
 * head: the K plane ([token_count][head_dim] scalars, row stride
 * k_stride_bytes) followed by the V plane at byte offset
 * token_count * k_stride_bytes ([token_count][head_dim], stride
 * v_stride_bytes).
 *
 * kv_layout_desc_fixed128() keeps the reference's fixed128 constants
 * (32 tokens x 128 dims x 2 B, 16 KiB blocks). The paged configurations of
 * this runtime use kv_layout_desc_paged(16, head_dim, scalar_bytes): e.g.
 * {16, 128, 2, 16, 256, 256, 8192, 128} for bf16 d128 and
 * {16, 64, 2, 16, 128, 128, 4096, 128} for fp16 d64.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define KV_LAYOUT_HEAD_DIM 128U
#define KV_LAYOUT_TOKENS_PER_BLOCK 32U
#define KV_LAYOUT_SCALAR_BYTES 2U
#define KV_LAYOUT_VEC_BYTES 16U
#define KV_LAYOUT_ALIGNMENT 128U

#define KV_LAYOUT_K_BYTES (KV_LAYOUT_TOKENS_PER_BLOCK * KV_LAYOUT_HEAD_DIM * KV_LAYOUT_SCALAR_BYTES)
#define KV_LAYOUT_V_BYTES KV_LAYOUT_K_BYTES
#define KV_LAYOUT_BLOCK_BYTES (KV_LAYOUT_K_BYTES + KV_LAYOUT_V_BYTES)

/* Tokens per block of the paged arena used by every decode configuration. */
#define KV_PAGED_TOKENS_PER_BLOCK 16U

typedef struct {
    uint32_t token_count;
    uint32_t head_dim;
    uint32_t scalar_bytes;
    uint32_t vec_bytes;
    uint32_t k_stride_bytes;
    uint32_t v_stride_bytes;
    uint32_t block_bytes;
    uint32_t alignment;
} KvLayoutDesc;

RL_STATIC_ASSERT(sizeof(KvLayoutDesc) == 32, "KvLayoutDesc size");
RL_STATIC_ASSERT((KV_LAYOUT_HEAD_DIM * KV_LAYOUT_SCALAR_BYTES) % KV_LAYOUT_VEC_BYTES == 0,
                 "head dimension must support 16-byte vector loads");
RL_STATIC_ASSERT(KV_LAYOUT_BLOCK_BYTES % KV_LAYOUT_ALIGNMENT == 0, "KV block alignment");

static inline KvLayoutDesc
kv_layout_desc_paged(uint32_t token_count, uint32_t head_dim, uint32_t scalar_bytes)
{
    KvLayoutDesc d;
    d.token_count = token_count;
    d.head_dim = head_dim;
    d.scalar_bytes = scalar_bytes;
    d.vec_bytes = KV_LAYOUT_VEC_BYTES;
    d.k_stride_bytes = head_dim * scalar_bytes;
    d.v_stride_bytes = head_dim * scalar_bytes;
    d.block_bytes = 2u * token_count * head_dim * scalar_bytes;
    d.alignment = KV_LAYOUT_ALIGNMENT;
    return d;
}

static inline KvLayoutDesc
kv_layout_desc_fixed128(void)
{
    return kv_layout_desc_paged(KV_LAYOUT_TOKENS_PER_BLOCK, KV_LAYOUT_HEAD_DIM,
                                KV_LAYOUT_SCALAR_BYTES);
}

static inline uint32_t
kv_layout_block_offset_bytes(uint32_t block_idx)
{
    return block_idx * KV_LAYOUT_BLOCK_BYTES;
}

static inline uint32_t
kv_layout_k_offset_bytes(uint32_t token_idx)
{
    return token_idx * (KV_LAYOUT_HEAD_DIM * KV_LAYOUT_SCALAR_BYTES);
}

static inline uint32_t
kv_layout_v_plane_base_bytes(void)
{
    return KV_LAYOUT_K_BYTES;
}

static inline uint32_t
kv_layout_v_offset_bytes(uint32_t token_idx)
{
    return kv_layout_v_plane_base_bytes() + kv_layout_k_offset_bytes(token_idx);
}

/* 0 when the layout is one the gfx950 decode kernels accept: 16- or
 * 32-token blocks of one KV head, head_dim 64 or 128, 2-byte scalars,
 * contiguous rows, V plane right after the K plane. -1 otherwise. */
static inline int
kv_layout_check_paged(const KvLayoutDesc *d)
{
    if (!d)
        return -1;
    if (d->token_count != 16u && d->token_count != 32u)
        return -1;
    if (d->head_dim != 64u && d->head_dim != 128u)
        return -1;
    if (d->scalar_bytes != 2u)
        return -1;
    if (d->k_stride_bytes != d->head_dim * 2u || d->v_stride_bytes != d->head_dim * 2u)
        return -1;
    if (d->block_bytes != 2u * d->token_count * d->k_stride_bytes)
        return -1;
    return 0;
}
