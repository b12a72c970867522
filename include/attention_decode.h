/*
 * attention_decode.h - decode-attention step types.
 *
 * DecodeStepArgs / DecodeStepResult / DecodeMicrokernelConfig keep the
 * reference layouts (include/attention_decode.h:23-67; 40 / 24 / 20 B).
 * attention_decode_config_fixed128() is exported with the reference's
 * values (head_dim 128, 32 tokens per block, 16-token tiles, 3 stages,
 * 3 x 16 KiB staging). The gfx950 paged GQA kernels that replace the
 * reference microkernel are reached through rl_hip_attn_decode (rl_hip.h).
 *
 * Result bookkeeping (cu/attention_decode.cu:196-203): bytes_touched =
 * seq * head_dim * 2 * 2, tile_count = ceil(seq / 16), cycle_estimate =
 * tiles * head_dim * 24.
 */
#pragma once

#include <stdint.h>
#include "descriptor.h"
#include "kv_layout.h"

#define DECODE_FIXED_HEAD_DIM KV_LAYOUT_HEAD_DIM
#define DECODE_TILE_TOKENS 16U
#define DECODE_PREFETCH_STAGES 3U
#define DECODE_WARPS_PER_BLOCK 1U

typedef enum {
    DECODE_PATH_STUB = 0,
    DECODE_PATH_FIXED128 = 1
} DecodePathKind;

typedef struct {
    const void *q_ptr;
    void *o_ptr;
    uint32_t seq_len;
    uint32_t head_dim;
    uint32_t kv_block_base_idx;
    uint32_t kv_block_count;
    uint32_t output_token_offset;
} DecodeStepArgs;

typedef struct {
    uint32_t path_kind;
    uint32_t token_id;
    uint32_t bytes_touched;
    uint32_t tile_count;
    uint64_t cycle_estimate;
} DecodeStepResult;

typedef struct {
    uint32_t head_dim;
    uint32_t tokens_per_block;
    uint32_t tile_tokens;
    uint32_t prefetch_stages;
    uint32_t shared_bytes;
} DecodeMicrokernelConfig;

RL_STATIC_ASSERT(sizeof(DecodeStepArgs) == 40, "DecodeStepArgs size");
RL_STATIC_ASSERT(sizeof(DecodeStepResult) == 24, "DecodeStepResult size");

RL_EXTERN_C_BEGIN

DecodeMicrokernelConfig attention_decode_config_fixed128(void);

/* Bookkeeping half of the reference step result for `seq_len` tokens
 * (clamped to [1, 32] as the reference does); token_id is left 0. */
DecodeStepResult attention_decode_result_fixed128(uint32_t seq_len);

RL_EXTERN_C_END
