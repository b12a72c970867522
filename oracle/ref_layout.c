/*
 * ref_layout.c - prints sizeof/offsetof of the reference ABI structs as JSON,
 * compiled against the reference headers (oracle/_ref/ref_layout). The output
 * is committed as tests/golden/abi_layout_ref.json.
 */
#include <stddef.h>
#include <stdio.h>

#include "arena.h"
#include "completion.h"
#include "decode_batch.h"
#include "descriptor.h"
#include "hw_desc.h"
#include "hw_ring.h"
#include "hw_worker_sim.h"
#include "infer_submit.h"
#include "kv_layout.h"
#include "pipeline.h"
#include "request.h"
#include "reward.h"
#include "ring.h"
#include "rollout.h"
#include "trace.h"

static int first = 1;
#define S(T) emit(#T, "sizeof", sizeof(T))
#define O(T, f) emit(#T, #f, offsetof(T, f))

static void
emit(const char *t, const char *f, size_t v)
{
    printf("%s\n  \"%s.%s\": %zu", first ? "{" : ",", t, f, v);
    first = 0;
}

int
main(void)
{
    S(hw_desc_t); O(hw_desc_t, opcode); O(hw_desc_t, flags); O(hw_desc_t, rollout_id);
    O(hw_desc_t, kv_arena_id); O(hw_desc_t, prefix_id); O(hw_desc_t, kv_offset); O(hw_desc_t, delta_offset);
    O(hw_desc_t, seq_len); O(hw_desc_t, max_tokens); O(hw_desc_t, reward_model_id); O(hw_desc_t, reserved0);
    O(hw_desc_t, user_data); O(hw_desc_t, checksum_or_cookie);
    S(hw_ring_t); O(hw_ring_t, head); O(hw_ring_t, tail); O(hw_ring_t, desc);
    S(infer_hw_ctx_t); O(infer_hw_ctx_t, cmdq); O(infer_hw_ctx_t, doneq); O(infer_hw_ctx_t, doorbell);
    O(infer_hw_ctx_t, gpu_group_id); O(infer_hw_ctx_t, kv_arena_id);
    S(hw_worker_sim_t); O(hw_worker_sim_t, stop); O(hw_worker_sim_t, decoded_tokens); O(hw_worker_sim_t, completions);
    S(Descriptor); O(Descriptor, seq_id); O(Descriptor, kv_block_offset); O(Descriptor, num_kv_blocks);
    O(Descriptor, attention_flags); O(Descriptor, pad); O(Descriptor, output_token_offset);
    O(Descriptor, reward_cookie); O(Descriptor, batch_size); O(Descriptor, batch_index);
    S(CommandRing); O(CommandRing, cons); O(CommandRing, prod); O(CommandRing, slots);
    S(Completion); O(Completion, seq_id); O(Completion, token_id); O(Completion, kv_block_offset);
    O(Completion, reward_cookie); O(Completion, cycles_taken);
    S(CompletionRing); O(CompletionRing, cons); O(CompletionRing, prod); O(CompletionRing, overflow);
    O(CompletionRing, slots);
    S(DecodeDispatchBatch); O(DecodeDispatchBatch, descs); S(DecodeBatchContract);
    S(RolloutRequest); O(RolloutRequest, request_id); O(RolloutRequest, max_tokens); O(RolloutRequest, kv_blocks);
    O(RolloutRequest, temperature); O(RolloutRequest, top_k); O(RolloutRequest, top_p); O(RolloutRequest, rng_seed);
    S(RolloutDone); O(RolloutDone, request_id); O(RolloutDone, rollout_id); O(RolloutDone, tokens_generated);
    O(RolloutDone, reward); O(RolloutDone, status);
    S(RequestRing); O(RequestRing, prod); O(RequestRing, slots);
    S(DoneRing); O(DoneRing, prod); O(DoneRing, overflow); O(DoneRing, slots);
    S(GpuRolloutSlot); O(GpuRolloutSlot, rng_state); O(GpuRolloutSlot, temperature); O(GpuRolloutSlot, top_k);
    O(GpuRolloutSlot, top_p);
    S(GpuRolloutState); O(GpuRolloutState, bitmap);
    S(KVArena); O(KVArena, base); O(KVArena, capacity); O(KVArena, block_size); O(KVArena, bitmap);
    S(KvLayoutDesc); O(KvLayoutDesc, block_bytes); O(KvLayoutDesc, alignment);
    S(RewardDesc); O(RewardDesc, reward); O(RewardDesc, flags);
    S(rollout_t); O(rollout_t, state); O(rollout_t, kv_arena_id); O(rollout_t, kv_block_idx);
    O(rollout_t, seq_len); O(rollout_t, max_tokens); O(rollout_t, reward_id); O(rollout_t, flags);
    O(rollout_t, rng_seed); O(rollout_t, pad);
    S(rollout_slab_t); O(rollout_slab_t, free_bitmap);
    S(IdRingIndex); O(IdRingIndex, tail); S(IdRing); O(IdRing, cons); O(IdRing, slots);
    S(PipelineCredits); O(PipelineCredits, decode_used); O(PipelineCredits, kv_blocks_used);
    S(RolloutPipeline); O(RolloutPipeline, slab); O(RolloutPipeline, credits); O(RolloutPipeline, policy);
    S(PipelineSnapshot); O(PipelineSnapshot, stage_credit_headroom); O(PipelineSnapshot, credits);
    O(PipelineSnapshot, policy);
    S(RewardIndex); S(RewardRing); O(RewardRing, cons); O(RewardRing, slots);
    emit("const", "MAX_ROLLOUTS", MAX_ROLLOUTS); emit("const", "PIPELINE_RING_SIZE", PIPELINE_RING_SIZE);
    emit("const", "REWARD_RING_SIZE", REWARD_RING_SIZE); emit("enum", "ROLL_DONE", ROLL_DONE);
    emit("enum", "Q_TRAJECTORY", Q_TRAJECTORY); emit("enum", "Q_COUNT", Q_COUNT);
    emit("enum", "SCHED_FIFO", SCHED_FIFO); emit("enum", "SCHED_SHORTEST_REMAINING", SCHED_SHORTEST_REMAINING);
    emit("enum", "SCHED_PREFIX_SHARING", SCHED_PREFIX_SHARING);
    S(trace_entry_t); O(trace_entry_t, type); O(trace_entry_t, rollout_id); O(trace_entry_t, seq);
    S(TraceRing); O(TraceRing, head); emit("const", "TRACE_CAPACITY", TRACE_CAPACITY);
    emit("enum", "TRACE_COMPLETION_POLLED", TRACE_COMPLETION_POLLED); emit("enum", "TRACE_EVENT_COUNT", TRACE_EVENT_COUNT);
    printf("\n}\n");
    return 0;
}
