/*
 * infer_submit.h - host C submit API for one decode step.
 *
 * Replaces the reference interface include/infer_submit.h:7-21 with the
 * same context struct (32 bytes: cmdq, doneq, doorbell, gpu_group_id,
 * kv_arena_id) and the same function signature and return convention
 * (0 on success; -1 on NULL ctx/cmdq/doorbell or a full command ring).
 *
 * Field mapping written into the descriptor (src/infer_submit.c:17-30):
 * opcode DECODE; flags COW_PREFIX iff prefix_id != 0; kv_arena_id from ctx;
 * reserved0 = gpu_group_id; reward_model_id 0; user_data = rollout_id;
 * checksum_or_cookie = kv_offset ^ delta_offset ^ (rollout_id << 32).
 * After the push the new tail is written to the doorbell behind a store fence.
 */
#pragma once

#include <stdint.h>
#include "hw_ring.h"
#include "mmio.h"

typedef struct {
    hw_ring_t *cmdq;
    hw_ring_t *doneq;
    volatile uint32_t *doorbell;
    uint32_t gpu_group_id;
    uint32_t kv_arena_id;
} infer_hw_ctx_t;

RL_STATIC_ASSERT(sizeof(infer_hw_ctx_t) == 32, "infer_hw_ctx_t size");

RL_EXTERN_C_BEGIN

int infer_submit_decode(infer_hw_ctx_t *ctx,
                        uint32_t rollout_id,
                        uint64_t kv_offset,
                        uint64_t delta_offset,
                        uint32_t prefix_id,
                        uint32_t seq_len,
                        uint32_t max_tokens);

RL_EXTERN_C_END
