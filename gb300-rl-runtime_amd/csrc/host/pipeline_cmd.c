/*
 * pipeline_cmd.c - the rollout pipeline driving the command-ring worker
 * (contract in pipeline_feed.h; the reference's loop is
 * bench/bench_pipeline.cu:170-383).
 */
#define _POSIX_C_SOURCE 199309L
#include <string.h>
#include <time.h>

#include "decode_batch.h"
#include "pipeline_feed.h"

typedef struct {
    RolloutPipeline *p;
    CommandRing *cmd;
    CompletionRing *comp;
    RewardRing *rewards;
    const rl_cmd_pipeline_cfg_t *cfg;
    rl_cmd_pipeline_stats_t *st;
    Completion *log;
    uint64_t log_cap;
    TraceRing *trace;
} Run;

static uint64_t
now_ns(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

static uint64_t
drain(Run *r)
{
    Completion c;
    uint64_t n = 0;
    while (comp_ring_poll(r->comp, &c)) {
        if (r->trace)
            trace_push(r->trace, TRACE_COMPLETION_POLLED, (uint32_t)c.seq_id, (uint32_t)c.reward_cookie);
        if (r->log && r->st->descriptors_consumed < r->log_cap)
            r->log[r->st->descriptors_consumed] = c;
        r->st->descriptors_consumed++;
        n++;
    }
    return n;
}

/* Descriptors t0 .. t0 + n - 1 of rollout rid as one decode_batch window. */
static int
dispatch_window(Run *r, uint32_t rid, uint32_t t0, uint32_t n)
{
    DecodeDispatchBatch batch;
    decode_batch_reset(&batch);
    for (uint32_t i = 0; i < n; i++) {
        Descriptor d;
        memset(&d, 0, sizeof(d));
        const uint32_t t = t0 + i;
        d.seq_id = rid;
        d.kv_block_offset = (uint32_t)(((uint64_t)rid + t) % r->cfg->kv_blocks);
        d.num_kv_blocks = 1;
        d.output_token_offset = t;
        d.reward_cookie = (uint64_t)rid << 32 | t;
        if (decode_batch_push(&batch, &d) != 0)
            return -1;
        if (r->trace)
            trace_push(r->trace, TRACE_DESC_POSTED, rid, t);
    }
    if (decode_batch_submit(r->cmd, &batch) == 0)
        goto posted;
    r->st->ring_full_spins++;
    drain(r);
    if (decode_batch_submit(r->cmd, &batch) == 0)
        goto posted;
    if (r->cfg->full_wait_ns) {
        const uint64_t until = now_ns() + r->cfg->full_wait_ns;
        do {
            drain(r);
            if (decode_batch_submit(r->cmd, &batch) == 0)
                goto posted;
        } while (now_ns() < until);
    }
    return -1;
posted:
    if (r->trace)
        for (uint32_t i = 0; i < n; i++)
            trace_push(r->trace, TRACE_DESC_COMMITTED, rid, t0 + i);
    r->st->descriptors_posted += n;
    drain(r);
    return 0;
}

static void
pass_stage(RolloutPipeline *p, pipeline_q_t q, uint32_t rid)
{
    uint32_t out;
    if (pipeline_try_push(p, q, rid) == 0) {
        pipeline_pop(p, q, &out);
        pipeline_release(p, q, 1);
    }
}

static void
finish(Run *r, uint32_t rid)
{
    RolloutPipeline *p = r->p;
    rollout_t *ro = rollout_get(&p->slab, rid);
    const uint32_t tokens = r->cfg->tokens_per_rollout;
    rollout_transition(ro, ROLL_DECODING, ROLL_REWARD_PENDING);
    pass_stage(p, Q_REWARD, rid);
    if (r->trace)
        trace_push(r->trace, TRACE_REWARD_POSTED, rid, 0);
    if (r->rewards) {
        RewardDesc rd = {rid, 0, tokens, 0, reward_score_mock(NULL, tokens), 0};
        if (reward_push(r->rewards, &rd) == 0)
            r->st->reward_handoffs++;
        else
            r->st->reward_ring_full++;
    }
    if (r->trace)
        trace_push(r->trace, TRACE_REWARD_SCORED, rid, 0);
    rollout_transition(ro, ROLL_REWARD_PENDING, ROLL_TRAJECTORY_READY);
    pass_stage(p, Q_TRAJECTORY, rid);
    rollout_transition(ro, ROLL_TRAJECTORY_READY, ROLL_DONE);
    pass_stage(p, Q_DONE, rid);
    if (r->trace)
        trace_push(r->trace, TRACE_TRAJECTORY_DONE, rid, 0);
    r->st->rollouts_completed++;
    rollout_free(&p->slab, rid);
    if (r->trace)
        trace_push(r->trace, TRACE_ROLLOUT_FREE, rid, 0);
}

/* One decode batch of pipeline_stage_target_batch rollouts, or with
 * `drain` of min(batch_max, occupancy) when that is 0; returns the rollouts
 * it took off Q_DECODE. */
static uint32_t
decode_batch_run(Run *r, int drain)
{
    RolloutPipeline *p = r->p;
    uint32_t ids[DECODE_DESCRIPTOR_BATCH_LIMIT];
    uint32_t want = pipeline_stage_target_batch(p, Q_DECODE, r->cfg->batch_max), got = 0;
    if (want == 0 && drain) {
        /* every decode credit is held by a queued rollout, so target_batch
         * (capped by the free credits) is 0: the queued rollouts already own
         * their credits and run anyway */
        const uint32_t occ = pipeline_occupancy(p, Q_DECODE);
        want = occ < r->cfg->batch_max ? occ : r->cfg->batch_max;
    }
    while (got < want && pipeline_schedule(p, Q_DECODE, &ids[got]) == 0)
        got++;
    if (got == 0)
        return 0;
    r->st->decode_batches++;
    r->st->decode_rollouts_scheduled += got;
    if (r->trace)
        trace_push(r->trace, TRACE_DECODE_BATCH, got, r->cfg->tokens_per_rollout);
    if (got > r->st->decode_batch_peak)
        r->st->decode_batch_peak = got;
    const uint32_t tokens = r->cfg->tokens_per_rollout;
    for (uint32_t i = 0; i < got; i++) {
        int posted = 1;
        for (uint32_t t = 0; t < tokens; t += DECODE_DESCRIPTOR_BATCH_LIMIT) {
            const uint32_t n = tokens - t < DECODE_DESCRIPTOR_BATCH_LIMIT ? tokens - t : DECODE_DESCRIPTOR_BATCH_LIMIT;
            if (dispatch_window(r, ids[i], t, n) != 0) {
                r->st->pipeline_overflow++;
                posted = 0;
                break;
            }
        }
        if (posted) {
            finish(r, ids[i]);
        } else {
            /* part of its decode never reached the ring: no reward, no
             * trajectory; the slot is freed and the rollout counted failed */
            rollout_transition(rollout_get(&r->p->slab, ids[i]), ROLL_DECODING, ROLL_DONE);
            rollout_free(&r->p->slab, ids[i]);
            if (r->trace)
                trace_push(r->trace, TRACE_ROLLOUT_FREE, ids[i], 0);
            r->st->rollouts_failed++;
        }
    }
    pipeline_release(p, Q_DECODE, got);
    return got;
}

int
rl_pipeline_cmd_run(RolloutPipeline *p, CommandRing *cmd, CompletionRing *comp, RewardRing *rewards,
                    const rl_cmd_pipeline_cfg_t *cfg, rl_cmd_pipeline_stats_t *stats, Completion *log,
                    uint64_t log_cap, TraceRing *trace)
{
    if (!p || !cmd || !comp || !cfg || !stats || cfg->batch_max == 0 ||
        cfg->batch_max > DECODE_DESCRIPTOR_BATCH_LIMIT || cfg->kv_blocks == 0)
        return -1;
    memset(stats, 0, sizeof(*stats));
    Run r = {p, cmd, comp, rewards, cfg, stats, log, log_cap, trace};
    const uint64_t t0 = now_ns();
    pipeline_credits_set(p, cfg->max_decode_credits, cfg->max_reward_credits, cfg->max_trajectory_credits,
                         cfg->kv_block_limit);
    for (uint32_t i = 0; i < cfg->n_rollouts; i++) {
        uint32_t rid, out;
        if (rollout_alloc(&p->slab, &rid) != 0) {
            stats->rollouts_dropped += cfg->n_rollouts - i;
            break;
        }
        stats->rollouts_started++;
        if (trace)
            trace_push(trace, TRACE_ROLLOUT_ALLOC, rid, 0);
        rollout_t *ro = rollout_get(&p->slab, rid);
        ro->max_tokens = cfg->tokens_per_rollout;
        ro->rng_seed = cfg->seed_base + i;
        rollout_transition(ro, ROLL_FREE, ROLL_PREFILL_READY);
        if (pipeline_push(p, Q_PREFILL, rid) == 0)
            pipeline_pop(p, Q_PREFILL, &out);     /* the prompt KV is already resident */
        rollout_transition(ro, ROLL_PREFILL_READY, ROLL_DECODING);
        int admitted = 0;
        for (;;) {
            if (pipeline_try_push(p, Q_DECODE, rid) == 0) {
                admitted = 1;
                break;
            }
            if (decode_batch_run(&r, 0) == 0) {
                stats->pipeline_overflow++;
                break;
            }
        }
        if (!admitted) {
            rollout_transition(ro, ROLL_DECODING, ROLL_DONE);
            rollout_free(&p->slab, rid);
            if (trace)
                trace_push(trace, TRACE_ROLLOUT_FREE, rid, 0);
            stats->rollouts_dropped++;
            continue;
        }
        if ((i + 1) % cfg->batch_max == 0)
            decode_batch_run(&r, 0);
    }
    while (pipeline_occupancy(p, Q_DECODE) > 0)
        if (decode_batch_run(&r, 1) == 0)
            break;
    uint64_t last = now_ns();
    while (stats->descriptors_consumed < stats->descriptors_posted) {
        if (drain(&r))
            last = now_ns();
        else if (now_ns() - last > cfg->drain_wait_ns)
            break;
    }
    stats->wall_ns = now_ns() - t0;
    return stats->descriptors_consumed == stats->descriptors_posted ? 0 : -1;
}
