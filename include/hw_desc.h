/*
 * hw_desc.h - 64-byte hardware submission descriptor.
 *
 * Byte-compatible with the reference descriptor (include/hw_desc.h:5-35):
 * same opcodes, flag bits, field order, packing and 64-byte alignment.
 * One descriptor is one cache line of fine-grained coherent host memory
 * that the persistent gfx950 worker reads with a single 64-byte load.
 */
#pragma once

#include <stdint.h>
#include "rl_abi.h"

#define DESC_OP_DECODE  1U
#define DESC_OP_REWARD  2U
#define DESC_OP_PREFILL 3U
#define DESC_OP_STOP    255U

#define DESC_FLAG_NEEDS_REWARD (1u << 0)
#define DESC_FLAG_DONE         (1u << 1)
#define DESC_FLAG_COW_PREFIX   (1u << 2)

typedef struct __attribute__((packed, aligned(64))) {
    uint16_t opcode;
    uint16_t flags;
    uint32_t rollout_id;

    uint32_t kv_arena_id;
    uint32_t prefix_id;

    uint64_t kv_offset;
    uint64_t delta_offset;

    uint32_t seq_len;
    uint32_t max_tokens;

    uint32_t reward_model_id;
    uint32_t reserved0; /* gpu_group_id stamped by infer_submit_decode */

    uint64_t user_data;
    uint64_t checksum_or_cookie;
} hw_desc_t;

RL_STATIC_ASSERT(sizeof(hw_desc_t) == 64, "hw_desc_t must be one cache line");
RL_STATIC_ASSERT(RL_OFFSETOF(hw_desc_t, kv_offset) == 16, "hw_desc_t.kv_offset");
RL_STATIC_ASSERT(RL_OFFSETOF(hw_desc_t, seq_len) == 32, "hw_desc_t.seq_len");
RL_STATIC_ASSERT(RL_OFFSETOF(hw_desc_t, reserved0) == 44, "hw_desc_t.reserved0");
RL_STATIC_ASSERT(RL_OFFSETOF(hw_desc_t, checksum_or_cookie) == 56, "hw_desc_t.cookie");
