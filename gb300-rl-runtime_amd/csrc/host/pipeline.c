/*
 * pipeline.c - the host rollout pipeline (reference src/pipeline.c:5-269,
 * behaviour restated in include/pipeline.h).
 *
 * Each stage queue is an IdRing driven through spsc_index.h. Credits are
 * looked up per stage as a (max, used) pair, so try_push, release and the
 * headroom queries share one path for DECODE, REWARD and TRAJECTORY; every
 * other queue is uncredited.
 */
#include <string.h>

#include "pipeline.h"
#include "spsc_index.h"

static int
q_ok(pipeline_q_t q)
{
    return (unsigned)q < (unsigned)Q_COUNT;
}

/* The credit counter of stage q and its maximum, or NULL for an uncredited
 * queue. */
static uint32_t *
stage_credit(PipelineCredits *c, pipeline_q_t q, uint32_t *max)
{
    switch (q) {
    case Q_DECODE:
        *max = c->max_decode_credits;
        return &c->decode_used;
    case Q_REWARD:
        *max = c->max_reward_credits;
        return &c->reward_used;
    case Q_TRAJECTORY:
        *max = c->max_trajectory_credits;
        return &c->trajectory_used;
    default:
        *max = 0;
        return NULL;
    }
}

int
pipeline_init(RolloutPipeline *p)
{
    if (!p)
        return -1;
    memset(p, 0, sizeof(*p));
    rollout_slab_init(&p->slab);
    p->policy = PIPELINE_SCHED_FIFO;
    return 0;
}

int
pipeline_push(RolloutPipeline *p, pipeline_q_t q, uint32_t rollout_id)
{
    uint32_t slot;
    if (!p || !q_ok(q))
        return -1;
    IdRing *r = &p->queues[q];
    if (spsc_reserve(&r->prod.head, &r->cons.tail, PIPELINE_RING_SIZE, &slot) != 0)
        return -1;
    r->slots[slot] = rollout_id;
    spsc_publish(&r->prod.head);
    return 0;
}

int
pipeline_pop(RolloutPipeline *p, pipeline_q_t q, uint32_t *out_id)
{
    uint32_t slot;
    if (!p || !out_id || !q_ok(q))
        return -1;
    IdRing *r = &p->queues[q];
    if (spsc_peek(&r->prod.head, &r->cons.tail, PIPELINE_RING_SIZE, &slot) != 0)
        return -1;
    *out_id = r->slots[slot];
    spsc_retire(&r->cons.tail);
    return 0;
}

int
pipeline_transition(RolloutPipeline *p, uint32_t rollout_id, rollout_state_t from, rollout_state_t to)
{
    rollout_t *r = p ? rollout_get(&p->slab, rollout_id) : NULL;
    return r ? rollout_transition(r, from, to) : -1;
}

void
pipeline_credits_set(RolloutPipeline *p, uint32_t max_decode, uint32_t max_reward, uint32_t max_trajectory,
                     uint32_t kv_limit)
{
    if (!p)
        return;
    p->credits.max_decode_credits = max_decode;
    p->credits.max_reward_credits = max_reward;
    p->credits.max_trajectory_credits = max_trajectory;
    p->credits.kv_block_limit = kv_limit;
}

int
pipeline_try_push(RolloutPipeline *p, pipeline_q_t q, uint32_t rollout_id)
{
    uint32_t max;
    if (!p)
        return -1;
    uint32_t *used = stage_credit(&p->credits, q, &max);
    if (used && max != 0 && *used >= max)
        return -1;                       /* no credit left; max 0 = unlimited */
    if (pipeline_push(p, q, rollout_id) != 0)
        return -1;
    if (used)
        (*used)++;
    return 0;
}

void
pipeline_release(RolloutPipeline *p, pipeline_q_t q, uint32_t n)
{
    uint32_t max;
    if (!p)
        return;
    uint32_t *used = stage_credit(&p->credits, q, &max);
    if (used)
        *used = n > *used ? 0u : *used - n;
}

int
pipeline_set_schedule_policy(RolloutPipeline *p, SchedulePolicy policy)
{
    /* Only FIFO can hand out queued ids without skipping any; the other two
     * need removal from the middle of a queue, which an IdRing cannot do. */
    if (!p || policy != PIPELINE_SCHED_FIFO)
        return -1;
    p->policy = policy;
    return 0;
}

int
pipeline_schedule(RolloutPipeline *p, pipeline_q_t q, uint32_t *out_id)
{
    if (!p || !q_ok(q) || p->policy != PIPELINE_SCHED_FIFO)
        return -1;                       /* non-FIFO: refuse, queue untouched */
    return pipeline_pop(p, q, out_id);
}

uint32_t
pipeline_occupancy(const RolloutPipeline *p, pipeline_q_t q)
{
    if (!p || !q_ok(q))
        return 0;
    const IdRing *r = &p->queues[q];
    return spsc_count(&r->prod.head, &r->cons.tail);
}

uint32_t
pipeline_stage_available_credits(const RolloutPipeline *p, pipeline_q_t q)
{
    uint32_t max;
    if (!p)
        return 0;
    const uint32_t *used = stage_credit((PipelineCredits *)&p->credits, q, &max);
    if (!used)
        return UINT32_MAX;
    return max > *used ? max - *used : 0u;
}

uint32_t
pipeline_stage_target_batch(const RolloutPipeline *p, pipeline_q_t q, uint32_t max_batch)
{
    if (!p)
        return 0;
    uint32_t n = max_batch;
    const uint32_t credit = pipeline_stage_available_credits(p, q);   /* UINT32_MAX: uncredited */
    const uint32_t occ = pipeline_occupancy(p, q);
    if (credit < n)
        n = credit;
    if (occ < n)
        n = occ;
    return n;
}

void
pipeline_snapshot(const RolloutPipeline *p, PipelineSnapshot *snap)
{
    if (!p || !snap)
        return;
    memset(snap, 0, sizeof(*snap));
    for (int q = 0; q < Q_COUNT; q++) {
        snap->queue_occupancy[q] = pipeline_occupancy(p, (pipeline_q_t)q);
        snap->stage_credit_headroom[q] = pipeline_stage_available_credits(p, (pipeline_q_t)q);
    }
    snap->credits = p->credits;
    snap->policy = p->policy;
}
