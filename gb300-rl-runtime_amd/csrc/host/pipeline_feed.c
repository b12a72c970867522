/*
 * pipeline_feed.c - the rollout pipeline feeding the device scheduler's
 * RequestRing and retiring its DoneRing (contract in pipeline_feed.h; the
 * reference's only driver of the pipeline is bench/bench_pipeline.cu:242-383).
 */
#include <string.h>

#include "pipeline_feed.h"

#define NO_ROLLOUT UINT32_MAX

int
rl_feed_init(rl_pipeline_feeder_t *f, RolloutPipeline *p, RequestRing *requests, DoneRing *dones,
             RewardRing *rewards, uint32_t *rid_of_request, uint32_t n_requests, const rl_feed_params_t *params)
{
    if (!f || !p || !requests || !dones || !rid_of_request || !params || n_requests == 0 ||
        params->block_tokens == 0 || params->top_k > 0xFFFFu)
        return -1;
    memset(f, 0, sizeof(*f));
    f->pipeline = p;
    f->requests = requests;
    f->dones = dones;
    f->rewards = rewards;
    f->rid_of_request = rid_of_request;
    f->n_requests = n_requests;
    f->params = *params;
    for (uint32_t i = 0; i < n_requests; i++)
        rid_of_request[i] = NO_ROLLOUT;
    return 0;
}

int64_t
rl_feed_register(rl_pipeline_feeder_t *f, uint32_t request_id, uint32_t seq_len, uint32_t max_tokens,
                 uint64_t rng_seed)
{
    uint32_t rid;
    if (!f || request_id >= f->n_requests || f->rid_of_request[request_id] != NO_ROLLOUT)
        return -1;
    RolloutPipeline *p = f->pipeline;
    if (rollout_alloc(&p->slab, &rid) != 0)
        return -1;
    rollout_t *ro = rollout_get(&p->slab, rid);
    ro->seq_len = seq_len;
    ro->max_tokens = max_tokens;
    ro->rng_seed = rng_seed;
    ro->reward_id = request_id;
    if (rollout_transition(ro, ROLL_FREE, ROLL_PREFILL_READY) != 0 || pipeline_push(p, Q_PREFILL, rid) != 0) {
        rollout_free(&p->slab, rid);
        return -1;
    }
    f->rid_of_request[request_id] = rid;
    f->stats.registered++;
    return rid;
}

uint32_t
rl_feed_admit(rl_pipeline_feeder_t *f, uint32_t max_n)
{
    uint32_t n = 0, rid;
    if (!f)
        return 0;
    RolloutPipeline *p = f->pipeline;
    const PipelineCredits *c = &p->credits;
    /* Pop only when pipeline_try_push will find a decode credit (max 0 =
     * unlimited), so a popped rollout always lands on Q_DECODE; the caller
     * is the single owner of both queues. */
    while (n < max_n && (c->max_decode_credits == 0 || c->decode_used < c->max_decode_credits) &&
           pipeline_pop(p, Q_PREFILL, &rid) == 0) {
        if (pipeline_transition(p, rid, ROLL_PREFILL_READY, ROLL_DECODING) != 0 ||
            pipeline_try_push(p, Q_DECODE, rid) != 0) {
            /* unreachable with a consistent pipeline; the rollout is dropped
             * rather than left half-staged */
            rollout_free(&p->slab, rid);
            continue;
        }
        n++;
    }
    f->stats.admitted += n;
    return n;
}

uint32_t
rl_feed_send(rl_pipeline_feeder_t *f, uint32_t max_n)
{
    uint32_t n = 0, rid;
    if (!f || f->end_sent)
        return 0;
    RolloutPipeline *p = f->pipeline;
    const rl_feed_params_t *fp = &f->params;
    while (n < max_n && pipeline_occupancy(p, Q_DECODE) > 0) {
        const uint32_t slot = req_ring_acquire(f->requests);
        if (slot == UINT32_MAX) {
            f->stats.req_ring_full++;
            break;
        }
        if (pipeline_schedule(p, Q_DECODE, &rid) != 0)
            break;
        const rollout_t *ro = rollout_get(&p->slab, rid);
        RolloutRequest rq;
        rq.request_id = ro->reward_id;
        rq.max_tokens = ro->max_tokens;
        rq.kv_blocks = (uint32_t)(((uint64_t)ro->seq_len + ro->max_tokens + fp->block_tokens - 1u) /
                                  fp->block_tokens);
        rq.temperature = fp->temperature;
        rq.top_k = (uint16_t)fp->top_k;
        rq.top_p = fp->top_p;
        rq.rng_seed = ro->rng_seed;
        f->requests->slots[slot] = rq;
        req_ring_commit(f->requests);
        n++;
    }
    f->stats.sent += n;
    return n;
}

int
rl_feed_end(rl_pipeline_feeder_t *f)
{
    if (!f)
        return -1;
    if (f->end_sent)
        return 0;
    const uint32_t slot = req_ring_acquire(f->requests);
    if (slot == UINT32_MAX)
        return -1;
    RolloutRequest end;
    memset(&end, 0, sizeof(end));
    end.request_id = UINT64_MAX;
    f->requests->slots[slot] = end;
    req_ring_commit(f->requests);
    f->end_sent = 1;
    return 0;
}

/* Pushes rid through one later stage: onto queue q (with its credit), off
 * it again, credit returned. */
static void
pass_stage(RolloutPipeline *p, pipeline_q_t q, uint32_t rid)
{
    uint32_t out;
    if (pipeline_try_push(p, q, rid) == 0) {
        pipeline_pop(p, q, &out);
        pipeline_release(p, q, 1);
    }
}

uint32_t
rl_feed_retire(rl_pipeline_feeder_t *f)
{
    uint32_t n = 0;
    RolloutDone d;
    if (!f)
        return 0;
    RolloutPipeline *p = f->pipeline;
    while (done_ring_pop(f->dones, &d)) {
        const uint32_t rid = d.request_id < f->n_requests ? f->rid_of_request[d.request_id] : NO_ROLLOUT;
        rollout_t *ro = rid != NO_ROLLOUT ? rollout_get(&p->slab, rid) : NULL;
        if (!ro || rollout_transition(ro, ROLL_DECODING, ROLL_REWARD_PENDING) != 0) {
            f->stats.bad_dones++;
            continue;
        }
        pass_stage(p, Q_REWARD, rid);
        if (f->rewards) {
            RewardDesc rd;
            rd.rollout_id = rid;
            rd.token_start = ro->seq_len;
            rd.token_count = d.tokens_generated;
            rd.reward_model_id = 0;
            rd.reward = d.reward;
            rd.flags = d.status;
            if (reward_push(f->rewards, &rd) == 0)
                f->stats.reward_handoffs++;
            else
                f->stats.reward_ring_full++;
        }
        rollout_transition(ro, ROLL_REWARD_PENDING, ROLL_TRAJECTORY_READY);
        pass_stage(p, Q_TRAJECTORY, rid);
        rollout_transition(ro, ROLL_TRAJECTORY_READY, ROLL_DONE);
        pass_stage(p, Q_DONE, rid);
        ro->seq_len += d.tokens_generated;
        rollout_transition(ro, ROLL_DONE, ROLL_FREE);
        rollout_free(&p->slab, rid);
        pipeline_release(p, Q_DECODE, 1);
        f->rid_of_request[d.request_id] = NO_ROLLOUT;
        n++;
    }
    f->stats.retired += n;
    return n;
}

uint32_t
rl_feed_pump(rl_pipeline_feeder_t *f)
{
    if (!f)
        return 0;
    uint32_t n = rl_feed_retire(f);
    n += rl_feed_admit(f, UINT32_MAX);
    n += rl_feed_send(f, UINT32_MAX);
    return n;
}
