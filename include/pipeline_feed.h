/*
 * pipeline_feed.h - the host rollout pipeline (pipeline.h) as the producer
 * of the device rollout scheduler's RequestRing and the consumer of its
 * DoneRing (request.h).
 *
 * The reference drives its pipeline only from bench/bench_pipeline.cu:
 * alloc -> FREE->PREFILL_READY -> Q_PREFILL -> PREFILL_READY->DECODING ->
 * try_push(Q_DECODE) -> FIFO schedule in windows of target_batch ->
 * dispatch -> DECODING->REWARD_PENDING -> Q_REWARD -> RewardRing ->
 * TRAJECTORY_READY -> Q_TRAJECTORY -> DONE -> Q_DONE -> free
 * (bench/bench_pipeline.cu:242-311, :348-383). Here the dispatch is a
 * RolloutRequest to the device scheduler, and a rollout leaves DECODING only
 * when its RolloutDone comes back:
 *
 *   rl_feed_admit    Q_PREFILL -> Q_DECODE while decode credits last
 *                    (PREFILL_READY -> DECODING, pipeline_try_push). A
 *                    decode credit is held from here until the rollout's done
 *                    is retired, so max_decode_credits bounds the rollouts
 *                    queued on or running in the device.
 *   rl_feed_send     FIFO pops from Q_DECODE (pipeline_schedule), one
 *                    RolloutRequest each, while the RequestRing has room:
 *                    {request_id = rollout_t.reward_id, max_tokens,
 *                     kv_blocks = ceil((seq_len + max_tokens) / block_tokens)
 *                     (the blocks of the prompt and every generated token),
 *                     temperature, top_k, top_p, rng_seed}.
 *   rl_feed_end      the end marker (request_id UINT64_MAX), once.
 *   rl_feed_retire   every RolloutDone: the rollout registered under its
 *                    request_id goes DECODING -> REWARD_PENDING (Q_REWARD,
 *                    one reward credit) -> a RewardDesc {rollout id,
 *                    token_start = seq_len, token_count = tokens_generated,
 *                    reward_model_id 0, reward, flags = status} on the
 *                    RewardRing -> TRAJECTORY_READY (Q_TRAJECTORY, one
 *                    trajectory credit) -> DONE (Q_DONE) -> freed; every
 *                    credit it held is released. The reward comes with the
 *                    done and the trajectory is the token row the device
 *                    already wrote, so each later stage completes at once.
 *
 * request_id is the caller's request index (the device scheduler indexes its
 * per-request tables by it); the feeder maps it back to the slab id through
 * rid_of_request[n_requests], which rl_feed_register fills and retirement
 * clears. Single-threaded: one host thread owns the pipeline, the producer
 * side of the RequestRing and the consumer side of the DoneRing.
 */
#pragma once

#include <stdint.h>
#include "pipeline.h"
#include "request.h"
#include "reward.h"
#include "rl_abi.h"

typedef struct {
    float temperature;
    uint32_t top_k;          /* <= 65535 (RolloutRequest.top_k is 16-bit) */
    float top_p;
    uint32_t block_tokens;   /* KV tokens per block, > 0 */
} rl_feed_params_t;

typedef struct {
    uint64_t registered;     /* rollouts allocated and queued on Q_PREFILL */
    uint64_t admitted;       /* moved to Q_DECODE with a decode credit */
    uint64_t sent;           /* RolloutRequests pushed */
    uint64_t retired;        /* dones retired to a freed slab slot */
    uint64_t reward_handoffs;
    uint64_t reward_ring_full;  /* RewardDescs the full RewardRing refused */
    uint64_t bad_dones;      /* dones naming no registered DECODING rollout */
    uint64_t req_ring_full;  /* sends stopped by a full RequestRing */
} rl_feed_stats_t;

typedef struct {
    RolloutPipeline *pipeline;
    RequestRing *requests;
    DoneRing *dones;
    RewardRing *rewards;         /* may be NULL: no reward handoff */
    uint32_t *rid_of_request;    /* [n_requests], caller-owned */
    uint32_t n_requests;
    uint32_t end_sent;
    rl_feed_params_t params;
    rl_feed_stats_t stats;
} rl_pipeline_feeder_t;

RL_EXTERN_C_BEGIN

/* Binds the rings and the map (filled with UINT32_MAX) and checks params;
 * -1 on NULL pointers, n_requests == 0, block_tokens == 0 or top_k > 65535. */
int rl_feed_init(rl_pipeline_feeder_t *f, RolloutPipeline *p, RequestRing *requests, DoneRing *dones,
                 RewardRing *rewards, uint32_t *rid_of_request, uint32_t n_requests,
                 const rl_feed_params_t *params);
/* Allocates a rollout for request_id {seq_len = prompt tokens, max_tokens,
 * rng_seed, reward_id = request_id}, FREE -> PREFILL_READY, pushes
 * Q_PREFILL. Returns the slab id, or -1 (request_id out of range or already
 * registered, slab full, Q_PREFILL full). */
int64_t rl_feed_register(rl_pipeline_feeder_t *f, uint32_t request_id, uint32_t seq_len, uint32_t max_tokens,
                         uint64_t rng_seed);
/* Stages as described above; each returns how many rollouts it moved. */
uint32_t rl_feed_admit(rl_pipeline_feeder_t *f, uint32_t max_n);
uint32_t rl_feed_send(rl_pipeline_feeder_t *f, uint32_t max_n);
uint32_t rl_feed_retire(rl_pipeline_feeder_t *f);
/* 0 once the end marker is on the ring (also when already sent), -1 when the
 * ring is full. */
int rl_feed_end(rl_pipeline_feeder_t *f);
/* One pass of retire, admit (up to the decode credits) and send. */
uint32_t rl_feed_pump(rl_pipeline_feeder_t *f);

RL_EXTERN_C_END

/* ---- the command-ring driver ----------------------------------------------
 * bench/bench_pipeline.cu's loop (:348-383, with schedule_decode_batches
 * :271-311, dispatch_decode_window :170-217 and finish_rollout :242-269) as
 * a library call over the v0.2 CommandRing / CompletionRing and the
 * persistent command-ring worker:
 *   credits (decode, reward, trajectory, kv) are set; rollout r is allocated
 *   {max_tokens = tokens_per_rollout, rng_seed = seed_base + r}, goes
 *   FREE -> PREFILL_READY (Q_PREFILL) -> DECODING and is offered to Q_DECODE;
 *   while no credit is free a decode batch is scheduled (no progress: the
 *   rollout is dropped, pipeline_overflow + 1). After every batch_max
 *   rollouts, and until Q_DECODE is empty, a batch runs: target_batch
 *   (<= batch_max <= 32) FIFO pops; per rollout, windows of up to 32
 *   descriptors {seq_id = rid, kv_block_offset = (rid + t) % kv_blocks,
 *   num_kv_blocks 1, output_token_offset = t, reward_cookie = rid << 32 | t}
 *   through decode_batch_submit, then the rollout is finished on the host
 *   (REWARD_PENDING, a RewardDesc {rid, 0, tokens, 0,
 *   reward_score_mock(tokens), 0}, TRAJECTORY_READY, DONE, freed); the batch
 *   returns its decode credits.
 * pipeline_stage_target_batch is capped by the free decode credits while
 * try_push takes a credit per queued rollout, so once every credit is held
 * no batch can run: later rollouts are dropped (as in the reference) and the
 * final "until Q_DECODE is empty" loop, which spins forever in the
 * reference, runs the queued rollouts in batches of min(batch_max,
 * occupancy) instead.
 * Other differences, all in how the host waits: completions are drained after
 * every window (the reference drains only when a submit fails, so its
 * completion ring can fill and stall the worker); a full command ring is
 * waited on for up to full_wait_ns before the window counts as an overflow
 * (0 = drain once and retry once, as the reference); and the reward, the
 * trajectory and the done queue are passed through (pushed and popped) so
 * they never fill. At the end every posted descriptor's completion is
 * awaited, giving up after drain_wait_ns without progress.
 */
#include "completion.h"
#include "ring.h"
#include "trace.h"

typedef struct {
    uint32_t n_rollouts;          /* rollouts to run (1000) */
    uint32_t tokens_per_rollout;  /* decode descriptors per rollout (128) */
    uint32_t batch_max;           /* rollouts per decode batch, 1..32 (32) */
    uint32_t kv_blocks;           /* arena blocks the descriptors walk, > 0 (128) */
    uint32_t max_decode_credits;  /* 256 */
    uint32_t max_reward_credits;  /* 128 */
    uint32_t max_trajectory_credits; /* 128 */
    uint32_t kv_block_limit;      /* 1024 */
    uint64_t seed_base;           /* 42 */
    uint64_t full_wait_ns;
    uint64_t drain_wait_ns;
} rl_cmd_pipeline_cfg_t;

typedef struct {
    uint64_t rollouts_started;
    uint64_t rollouts_completed;
    uint64_t rollouts_dropped;
    uint64_t descriptors_posted;
    uint64_t descriptors_consumed;   /* completions drained */
    uint64_t decode_batches;
    uint64_t decode_rollouts_scheduled;
    uint64_t decode_batch_peak;
    uint64_t ring_full_spins;        /* submits refused by a full command ring */
    uint64_t pipeline_overflow;
    uint64_t reward_handoffs;
    uint64_t reward_ring_full;
    uint64_t wall_ns;                /* first allocation to the last completion */
    uint64_t rollouts_failed;        /* a window of theirs was never posted (ring full
                                        past full_wait_ns): freed, no reward handoff */
} rl_cmd_pipeline_stats_t;

RL_EXTERN_C_BEGIN

/* Runs the loop above on an initialised pipeline. Completions are copied
 * to log[0 .. log_cap) in arrival order when log is not NULL. With trace set
 * the host side pushes (trace.h keys): ROLLOUT_ALLOC, DESC_POSTED when a
 * window is formed, DESC_COMMITTED when its submit succeeds,
 * COMPLETION_POLLED per completion drained (seq = low 32 bits of its
 * reward_cookie, the step), DECODE_BATCH {rollouts, tokens}, REWARD_POSTED,
 * REWARD_SCORED, TRAJECTORY_DONE and ROLLOUT_FREE. 0 when every posted
 * descriptor was completed, -1 on bad arguments or when the final drain gave
 * up (stats are filled either way). */
int rl_pipeline_cmd_run(RolloutPipeline *p, CommandRing *cmd, CompletionRing *comp, RewardRing *rewards,
                        const rl_cmd_pipeline_cfg_t *cfg, rl_cmd_pipeline_stats_t *stats, Completion *log,
                        uint64_t log_cap, TraceRing *trace);

RL_EXTERN_C_END
