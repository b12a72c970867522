// kv_append_core.h - the device side of the one-token KV append with
// copy-on-write of a partially filled shared block, shared by the standalone
// append kernel and the attention merge kernel of a fused decode step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_layout.h"
#include "rl_dev_common.h"
#include "rl_hip.h"

namespace {

struct AppendParams {
    uint8_t *arena;         // NULL: no append
    uint64_t block_bytes;
    uint64_t arena_blocks;
    uint32_t token_count;   // tokens per block
    uint32_t row_bytes;     // K (and V) bytes per token
    const uint32_t *table;
    uint32_t table_stride;
    const uint32_t *row_map;  // [batch]: the table row (rollout) of batch row b, or NULL: b itself
    uint32_t kv_heads;
    const uint32_t *positions;
    const int32_t *cow_src;
    const uint8_t *k_new;
    const uint8_t *v_new;
};

inline AppendParams append_params(const rl_kv_append_args_t *a)
{
    AppendParams p;
    p.arena = (uint8_t *)a->arena_base;
    p.block_bytes = a->layout.block_bytes;
    p.arena_blocks = a->arena_bytes / a->layout.block_bytes;
    p.token_count = a->layout.token_count;
    p.row_bytes = a->layout.k_stride_bytes;
    p.table = a->block_table;
    p.table_stride = a->table_stride;
    p.row_map = nullptr;
    p.kv_heads = a->kv_heads;
    p.positions = a->positions;
    p.cow_src = a->cow_src;
    p.k_new = (const uint8_t *)a->k_new;
    p.v_new = (const uint8_t *)a->v_new;
    return p;
}

// Appends the new K and V rows of (rollout b, kv head g) at slot
// positions[b] of its block, after copying the filled slots of the shared
// source block when cow_src names one. Threads tid, tid + nthr, ... of the
// caller share the 16-byte copies.
__device__ __forceinline__ void append_row(const AppendParams &p, uint32_t b, uint32_t g, uint32_t tid,
                                           uint32_t nthr)
{
    const uint32_t row_id = b * p.kv_heads + g;
    const uint32_t pos = p.positions[b];
    const uint32_t slot = pos % p.token_count;
    if (pos / p.token_count >= p.table_stride)
        return;  // position outside the rollout's table row: nothing written
    const uint32_t trow = (p.row_map ? p.row_map[b] : b) * p.kv_heads + g;
    const uint32_t blk = p.table[(size_t)trow * p.table_stride + pos / p.token_count];
    if (blk >= p.arena_blocks)
        return;
    uint8_t *dst = p.arena + (uint64_t)blk * p.block_bytes;
    const uint32_t v_plane = p.token_count * p.row_bytes;
    const uint32_t chunks = p.row_bytes / 16;  // 16-byte chunks per row

    if (p.cow_src) {
        const int32_t src_blk = p.cow_src[row_id];
        if (src_blk >= 0 && (uint64_t)src_blk < p.arena_blocks && slot > 0) {
            const uint8_t *src = p.arena + (uint64_t)(uint32_t)src_blk * p.block_bytes;
            const uint32_t n = slot * chunks;  // chunks of the filled rows of one plane
            for (uint32_t i = tid; i < 2 * n; i += nthr) {
                const uint32_t plane = i / n, c = i % n;
                const uint32_t off = plane * v_plane + c * 16;
                *(rl_u32x4 *)(dst + off) = *(const rl_u32x4 *)(src + off);
            }
        }
    }
    const uint8_t *kn = p.k_new + (size_t)row_id * p.row_bytes;
    const uint8_t *vn = p.v_new + (size_t)row_id * p.row_bytes;
    for (uint32_t i = tid; i < 2 * chunks; i += nthr) {
        const uint32_t plane = i / chunks, c = i % chunks;
        const uint8_t *s = (plane ? vn : kn) + c * 16;
        *(rl_u32x4 *)(dst + plane * v_plane + slot * p.row_bytes + c * 16) = *(const rl_u32x4 *)s;
    }
}

// Host-side checks of an append's arguments (0 or -1 with the error set).
inline int append_validate(const rl_kv_append_args_t *a, const char *who)
{
    if (!a || !a->arena_base || !a->block_table || !a->positions || !a->k_new || !a->v_new) {
        rl_set_error("%s: NULL append argument", who);
        return -1;
    }
    if (kv_layout_check_paged(&a->layout) != 0) {
        rl_set_error("%s: unsupported KV layout", who);
        return -1;
    }
    if (a->batch == 0 || a->kv_heads == 0 || a->batch > 65535 || a->kv_heads > 65535) {
        rl_set_error("%s: batch %u kv_heads %u out of range", who, a->batch, a->kv_heads);
        return -1;
    }
    return 0;
}

}  // namespace
