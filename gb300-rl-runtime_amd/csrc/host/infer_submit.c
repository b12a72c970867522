/*
 * infer_submit.c - one DECODE descriptor into the command ring, then the
 * doorbell (reference src/infer_submit.c:3-37; same field mapping, same
 * return convention).
 */
#include "infer_submit.h"

int
infer_submit_decode(infer_hw_ctx_t *ctx, uint32_t rollout_id, uint64_t kv_offset,
                    uint64_t delta_offset, uint32_t prefix_id, uint32_t seq_len,
                    uint32_t max_tokens)
{
    if (ctx == NULL || ctx->cmdq == NULL || ctx->doorbell == NULL)
        return -1;

    const hw_desc_t desc = {
        .opcode = (uint16_t)DESC_OP_DECODE,
        .flags = (uint16_t)(prefix_id != 0u ? DESC_FLAG_COW_PREFIX : 0u),
        .rollout_id = rollout_id,
        .kv_arena_id = ctx->kv_arena_id,
        .prefix_id = prefix_id,
        .kv_offset = kv_offset,
        .delta_offset = delta_offset,
        .seq_len = seq_len,
        .max_tokens = max_tokens,
        .reward_model_id = 0u,
        .reserved0 = ctx->gpu_group_id,
        .user_data = rollout_id,
        .checksum_or_cookie = kv_offset ^ delta_offset ^ ((uint64_t)rollout_id << 32),
    };

    if (hw_ring_push(ctx->cmdq, &desc) != 0)
        return -1;
    mmio_write32(ctx->doorbell, hw_ring_load_acquire(&ctx->cmdq->tail));
    return 0;
}
