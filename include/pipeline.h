/*
 * pipeline.h - the host rollout pipeline: six rollout-id queues, the rollout
 * slab, per-stage credits and the scheduling policy.
 *
 * Byte-compatible with the reference (include/pipeline.h:6-117):
 *   IdRing           producer line @0 (head = next write), consumer line @64
 *                    (tail = next read), 4,096 uint32 ids @128; 16,512 B.
 *   RolloutPipeline  queues[Q_COUNT] @0, slab @99,072, credits @493,312,
 *                    policy @493,344; 493,376 B.
 *
 * Semantics (src/pipeline.c:36-269):
 *   pipeline_push/pop       single-producer single-consumer id queue; push
 *                           fails (-1) when 4,096 ids are queued, pop when
 *                           none is.
 *   pipeline_try_push       DECODE, REWARD and TRAJECTORY take one credit per
 *                           push and refuse once max credits are in use; a
 *                           max of 0 means unlimited. Other queues push plainly.
 *   pipeline_release        returns n credits of a stage, saturating at 0.
 *   pipeline_schedule       FIFO pops. Any other policy fails (-1) without
 *                           taking an id (src/pipeline.c:148-158 keeps the
 *                           older search-and-skip version disabled because it
 *                           dropped queued rollouts); pipeline_set_schedule_
 *                           policy accepts FIFO only.
 *   stage_available_credits max - used for credited stages (0 when used >=
 *                           max), UINT32_MAX for the others.
 *   stage_target_batch      min(max_batch, available credits, occupancy).
 * kv_block_limit / kv_blocks_used are carried for the caller; no function
 * here consumes them.
 *
 * Index arithmetic is modulo 2^32 and the empty test is head == tail, so a
 * queue keeps working after 2^32 operations (the reference's pop tests
 * tail >= head, which reports an empty queue once head has wrapped).
 */
#pragma once

#include <stdint.h>
#include "rl_abi.h"
#include "rollout.h"

#define PIPELINE_RING_SIZE 4096

typedef struct __attribute__((packed)) {
    volatile uint32_t head __attribute__((aligned(64)));
    uint32_t tail;
    uint8_t pad[56];
} IdRingIndex;

typedef struct {
    IdRingIndex prod __attribute__((aligned(64)));  /* prod.head: next write */
    IdRingIndex cons __attribute__((aligned(64)));  /* cons.tail: next read */
    uint32_t slots[PIPELINE_RING_SIZE] __attribute__((aligned(64)));
} IdRing;

RL_STATIC_ASSERT(RL_OFFSETOF(IdRing, cons) == 64, "IdRing.cons");
RL_STATIC_ASSERT(RL_OFFSETOF(IdRing, slots) == 128, "IdRing.slots");
RL_STATIC_ASSERT(sizeof(IdRing) == 16512, "IdRing size");

typedef enum {
    Q_FREE = 0,
    Q_PREFILL,
    Q_DECODE,
    Q_REWARD,
    Q_TRAJECTORY,
    Q_DONE,
    Q_COUNT
} pipeline_q_t;

typedef struct {
    uint32_t max_decode_credits;
    uint32_t max_reward_credits;
    uint32_t max_trajectory_credits;
    uint32_t kv_block_limit;
    uint32_t decode_used;
    uint32_t reward_used;
    uint32_t trajectory_used;
    uint32_t kv_blocks_used;
} PipelineCredits;

/* The reference's names SCHED_FIFO, SCHED_SHORTEST_REMAINING and
 * SCHED_PREFIX_SHARING are kept. <sched.h> (pulled in by <pthread.h>)
 * defines SCHED_FIFO as a macro for POSIX thread scheduling, so in a unit
 * that includes it first the enumerator SCHED_FIFO is left out and
 * PIPELINE_SCHED_FIFO, which every policy name has as a twin, is the one to
 * use. */
typedef enum {
    PIPELINE_SCHED_FIFO = 0,
    PIPELINE_SCHED_SHORTEST_REMAINING = 1,  /* rejected: see pipeline_schedule */
    PIPELINE_SCHED_PREFIX_SHARING = 2,      /* rejected: see pipeline_schedule */
#ifndef SCHED_FIFO
    SCHED_FIFO = PIPELINE_SCHED_FIFO,
#endif
    SCHED_SHORTEST_REMAINING = PIPELINE_SCHED_SHORTEST_REMAINING,
    SCHED_PREFIX_SHARING = PIPELINE_SCHED_PREFIX_SHARING,
} SchedulePolicy;

typedef struct {
    IdRing queues[Q_COUNT];
    rollout_slab_t slab;
    PipelineCredits credits;
    SchedulePolicy policy;
} RolloutPipeline;

RL_STATIC_ASSERT(RL_OFFSETOF(RolloutPipeline, slab) == 99072, "RolloutPipeline.slab");
RL_STATIC_ASSERT(RL_OFFSETOF(RolloutPipeline, credits) == 493312, "RolloutPipeline.credits");
RL_STATIC_ASSERT(RL_OFFSETOF(RolloutPipeline, policy) == 493344, "RolloutPipeline.policy");
RL_STATIC_ASSERT(sizeof(RolloutPipeline) == 493376, "RolloutPipeline size");

typedef struct {
    uint32_t queue_occupancy[Q_COUNT];
    uint32_t stage_credit_headroom[Q_COUNT];
    PipelineCredits credits;
    SchedulePolicy policy;
} PipelineSnapshot;

RL_STATIC_ASSERT(sizeof(PipelineSnapshot) == 84, "PipelineSnapshot size");

RL_EXTERN_C_BEGIN

/* src/pipeline.c:36-45: zeroed queues and credits, fresh slab, FIFO. */
int pipeline_init(RolloutPipeline *p);
/* src/pipeline.c:11-59: -1 for a queue out of range, a full push, an empty pop. */
int pipeline_push(RolloutPipeline *p, pipeline_q_t q, uint32_t rollout_id);
int pipeline_pop(RolloutPipeline *p, pipeline_q_t q, uint32_t *out_id);
/* src/pipeline.c:61-68: rollout_transition on slab record rollout_id. */
int pipeline_transition(RolloutPipeline *p, uint32_t rollout_id, rollout_state_t from, rollout_state_t to);

/* src/pipeline.c:70-79: sets the four maxima; the used counters are kept. */
void pipeline_credits_set(RolloutPipeline *p, uint32_t max_decode, uint32_t max_reward,
                          uint32_t max_trajectory, uint32_t kv_limit);
/* src/pipeline.c:81-107 */
int pipeline_try_push(RolloutPipeline *p, pipeline_q_t q, uint32_t rollout_id);
/* src/pipeline.c:109-129 */
void pipeline_release(RolloutPipeline *p, pipeline_q_t q, uint32_t n);

/* src/pipeline.c:131-138 */
int pipeline_set_schedule_policy(RolloutPipeline *p, SchedulePolicy policy);
/* src/pipeline.c:140-206 */
int pipeline_schedule(RolloutPipeline *p, pipeline_q_t q, uint32_t *out_id);

/* src/pipeline.c:208-216: queued ids; 0 for a queue out of range. */
uint32_t pipeline_occupancy(const RolloutPipeline *p, pipeline_q_t q);
/* src/pipeline.c:218-238: 0 for p == NULL. */
uint32_t pipeline_stage_available_credits(const RolloutPipeline *p, pipeline_q_t q);
/* src/pipeline.c:240-253 */
uint32_t pipeline_stage_target_batch(const RolloutPipeline *p, pipeline_q_t q, uint32_t max_batch);
/* src/pipeline.c:255-269: occupancy and headroom of every queue, credits, policy. */
void pipeline_snapshot(const RolloutPipeline *p, PipelineSnapshot *snap);

RL_EXTERN_C_END

static inline const char *
pipeline_q_name(pipeline_q_t q)
{
    static const char *const names[Q_COUNT] = {"free", "prefill", "decode", "reward", "trajectory", "done"};
    return (unsigned)q < Q_COUNT ? names[q] : "?";
}

static inline const char *
schedule_policy_name(SchedulePolicy p)
{
    static const char *const names[3] = {"FIFO", "SHORTEST_REMAINING", "PREFIX_SHARING"};
    return (unsigned)p <= PIPELINE_SCHED_PREFIX_SHARING ? names[p] : "?";
}
