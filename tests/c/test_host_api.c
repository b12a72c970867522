/*
 * test_host_api.c - the reference's CPU test scenarios, run against this
 * runtime's headers and librlrt_amd.so:
 *   test/test_hw_ring.c:12-217   (hw_desc ring, submit, doneq overflow, worker sim)
 *   test/test_smoke.c:10-199,286-322 (command/completion/done rings, windows)
 *   test/test_bench.cu:160-243, 244-308, 738-797 (ring basics, arena,
 *     completion ring, kv_prefix: the first six asserts; its final
 *     off == 0x1000 contradicts src/kv_prefix.c:83-87 and is replaced by the
 *     code's answer, -1)
 *   test/test_smoke.c:200-284, test/test_bench.cu:512-581, 739-762 (rollout
 *     slab, transitions, pipeline queues, credits and snapshot, FIFO without
 *     work loss, reward ring)
 * Exits non-zero with a message on the first failed check.
 */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "arena.h"
#include "attention_decode.h"
#include "completion.h"
#include "decode_batch.h"
#include "hw_desc.h"
#include "hw_ring.h"
#include "hw_worker_sim.h"
#include "infer_submit.h"
#include "kv_prefix.h"
#include "pipeline.h"
#include "pipeline_feed.h"
#include "request.h"
#include "reward.h"
#include "ring.h"
#include "rollout.h"

#define CHECK(c)                                                                 \
    do {                                                                         \
        if (!(c)) {                                                              \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);         \
            exit(1);                                                             \
        }                                                                        \
    } while (0)

static void
hw_ring_wraparound(void)
{
    hw_ring_t *ring = hw_ring_create();
    CHECK(ring && hw_ring_empty(ring));
    for (uint32_t i = 0; i < HW_RING_SIZE; i++) {
        hw_desc_t d;
        memset(&d, 0, sizeof d);
        d.rollout_id = i;
        CHECK(hw_ring_push(ring, &d) == 0);
    }
    CHECK(hw_ring_full(ring));
    hw_desc_t out;
    for (uint32_t i = 0; i < HW_RING_SIZE / 2u; i++) {
        CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == i);
    }
    for (uint32_t i = 0; i < HW_RING_SIZE / 2u; i++) {
        hw_desc_t d;
        memset(&d, 0, sizeof d);
        d.rollout_id = 100000u + i;
        CHECK(hw_ring_push(ring, &d) == 0);
    }
    for (uint32_t i = HW_RING_SIZE / 2u; i < HW_RING_SIZE; i++)
        CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == i);
    for (uint32_t i = 0; i < HW_RING_SIZE / 2u; i++)
        CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == 100000u + i);
    CHECK(hw_ring_empty(ring));
    hw_ring_destroy(ring);
    printf("hw_ring_wraparound OK\n");
}

static void
hw_ring_producer_observes_consumer(void)
{
    hw_ring_t *ring = hw_ring_create();
    hw_desc_t d, out;
    for (uint32_t i = 0; i < HW_RING_SIZE; i++) {
        memset(&d, 0, sizeof d);
        d.rollout_id = i;
        CHECK(hw_ring_push(ring, &d) == 0);
    }
    CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == 0u);
    memset(&out, 0, sizeof out);
    out.rollout_id = 999999u;
    CHECK(hw_ring_push(ring, &out) == 0);
    for (uint32_t i = 1; i < HW_RING_SIZE; i++)
        CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == i);
    CHECK(hw_ring_pop(ring, &out) == 0 && out.rollout_id == 999999u);
    hw_ring_destroy(ring);
    printf("hw_ring_producer_observes_consumer OK\n");
}

static void
submit_doorbell(void)
{
    hw_ring_t *cmdq = hw_ring_create(), *doneq = hw_ring_create();
    volatile uint32_t doorbell = 0;
    infer_hw_ctx_t ctx = {cmdq, doneq, &doorbell, 7u, 42u};
    hw_desc_t out;
    CHECK(infer_submit_decode(&ctx, 99u, 0x1000u, 0x2000u, 5u, 17u, 64u) == 0);
    CHECK(doorbell == 1u);
    CHECK(hw_ring_pop(cmdq, &out) == 0);
    CHECK(out.opcode == DESC_OP_DECODE && out.rollout_id == 99u && out.kv_arena_id == 42u);
    CHECK(out.prefix_id == 5u && (out.flags & DESC_FLAG_COW_PREFIX) != 0u);
    CHECK(out.seq_len == 17u && out.max_tokens == 64u);
    /* closed form of src/infer_submit.c:26-30 */
    CHECK(out.reserved0 == 7u && out.reward_model_id == 0u && out.user_data == 99u);
    CHECK(out.checksum_or_cookie == 0x6300003000ull);
    /* NULL checks and no-COW for prefix 0 */
    CHECK(infer_submit_decode(NULL, 1, 0, 0, 0, 0, 1) == -1);
    infer_hw_ctx_t bad = ctx;
    bad.doorbell = NULL;
    CHECK(infer_submit_decode(&bad, 1, 0, 0, 0, 0, 1) == -1);
    CHECK(infer_submit_decode(&ctx, 1u, 0, 0, 0u, 0u, 1u) == 0 && doorbell == 2u);
    CHECK(hw_ring_pop(cmdq, &out) == 0 && out.flags == 0u);
    hw_ring_destroy(cmdq);
    hw_ring_destroy(doneq);
    printf("submit_doorbell OK\n");
}

static void
doneq_overflow(void)
{
    hw_ring_t *q = hw_ring_create();
    hw_desc_t d;
    memset(&d, 0, sizeof d);
    for (uint32_t i = 0; i < HW_RING_SIZE; i++)
        CHECK(hw_ring_push(q, &d) == 0);
    CHECK(hw_ring_push(q, &d) == -1);
    hw_ring_destroy(q);
    printf("doneq_overflow OK\n");
}

static void *
worker_main(void *arg)
{
    hw_worker_sim_run((hw_worker_sim_t *)arg);
    return NULL;
}

static void
worker_sim_completion(void)
{
    hw_ring_t *cmdq = hw_ring_create(), *doneq = hw_ring_create();
    volatile uint32_t stop = 0;
    hw_worker_sim_t w = {cmdq, doneq, &stop, 0, 0};
    pthread_t th;
    CHECK(pthread_create(&th, NULL, worker_main, &w) == 0);
    hw_desc_t d, out;
    memset(&d, 0, sizeof d);
    d.opcode = DESC_OP_DECODE;
    d.rollout_id = 77u;
    d.seq_len = 31u;
    d.max_tokens = 96u;
    CHECK(hw_ring_push(cmdq, &d) == 0);
    while (hw_ring_pop(doneq, &out) != 0)
        ;
    CHECK(out.rollout_id == 77u);
    CHECK((out.flags & (DESC_FLAG_NEEDS_REWARD | DESC_FLAG_DONE)) != 0u);
    /* closed form: 31 -> 32 hits the 32-token reward boundary after one token */
    CHECK(out.flags == DESC_FLAG_NEEDS_REWARD && out.seq_len == 32u);
    CHECK(w.decoded_tokens == 1u && w.completions == 1u);
    memset(&d, 0, sizeof d);
    d.opcode = DESC_OP_STOP;
    CHECK(hw_ring_push(cmdq, &d) == 0);
    pthread_join(th, NULL);
    CHECK(w.completions == 1u); /* STOP produces no completion */
    hw_ring_destroy(cmdq);
    hw_ring_destroy(doneq);
    printf("worker_sim_completion OK\n");
}

static void
command_ring(void)
{
    CommandRing *ring = ring_create();
    Descriptor d;
    CHECK(ring && ring_consume(ring, &d) == 0);
    for (uint32_t i = 0; i < RING_SIZE; i++) {
        uint32_t pos = ring_acquire(ring, 1);
        CHECK(pos != UINT32_MAX);
        ring->slots[pos].seq_id = i;
        ring_commit(ring, 1);
    }
    CHECK(ring_acquire(ring, 1) == UINT32_MAX);
    for (uint32_t i = 0; i < RING_SIZE; i++)
        CHECK(ring_consume(ring, &d) == 1 && d.seq_id == i);
    CHECK(ring_acquire(ring, 1) != UINT32_MAX);
    /* wraparound (test_smoke.c:48-82) */
    for (uint32_t i = 0; i < RING_SIZE; i++) {
        uint32_t pos = ring_acquire(ring, 1);
        CHECK(pos != UINT32_MAX);
        ring->slots[pos].seq_id = 10000 + i;
        ring_commit(ring, 1);
    }
    for (uint32_t i = 0; i < RING_SIZE; i++)
        CHECK(ring_consume(ring, &d) == 1 && d.seq_id == 10000 + i);
    /* no permanent full (test_smoke.c:117-140) */
    for (uint32_t round = 0; round < 3; round++) {
        for (uint32_t i = 0; i < RING_SIZE; i++) {
            uint32_t pos = ring_acquire(ring, 1);
            CHECK(pos != UINT32_MAX);
            ring->slots[pos].seq_id = round * RING_SIZE + i;
            ring_commit(ring, 1);
        }
        CHECK(ring_acquire(ring, 1) == UINT32_MAX);
        for (uint32_t i = 0; i < RING_SIZE; i++)
            CHECK(ring_consume(ring, &d) == 1);
        CHECK(ring_consume(ring, &d) == 0);
    }
    ring_destroy(ring);
    /* producer observes consumer (test_smoke.c:84-115) */
    ring = ring_create();
    for (uint32_t i = 0; i < RING_SIZE; i++) {
        uint32_t pos = ring_acquire(ring, 1);
        ring->slots[pos].seq_id = i;
        ring_commit(ring, 1);
    }
    CHECK(ring_consume(ring, &d) == 1 && d.seq_id == 0);
    uint32_t pos = ring_acquire(ring, 1);
    CHECK(pos == 0);
    ring->slots[pos].seq_id = 99999;
    ring_commit(ring, 1);
    for (uint32_t i = 1; i < RING_SIZE; i++)
        CHECK(ring_consume(ring, &d) == 1 && d.seq_id == i);
    CHECK(ring_consume(ring, &d) == 1 && d.seq_id == 99999);
    ring_destroy(ring);
    printf("command_ring OK\n");
}

static void
completion_and_done_rings(void)
{
    CompletionRing *cr = (CompletionRing *)calloc(1, sizeof(CompletionRing));
    Completion c = {1, 7, 0, 9, 11};
    for (uint32_t i = 0; i < COMP_RING_SIZE; i++)
        CHECK(comp_ring_push(cr, &c) == 0);
    CHECK(comp_ring_push(cr, &c) == -1 && cr->overflow.value == 1);
    CHECK(comp_ring_poll(cr, &c) == 1 && comp_ring_push(cr, &c) == 0);
    free(cr);

    cr = comp_ring_create();
    Completion in = {42, 7, 3, 0xDEAD, 99}, out;
    CHECK(comp_ring_push(cr, &in) == 0 && comp_ring_poll(cr, &out) == 1);
    CHECK(out.seq_id == 42 && out.token_id == 7 && out.kv_block_offset == 3);
    CHECK(out.reward_cookie == 0xDEAD && out.cycles_taken == 99 && cr->overflow.value == 0);
    comp_ring_destroy(cr);

    DoneRing *dr = (DoneRing *)calloc(1, sizeof(DoneRing));
    RolloutDone done = {1, 2, 3, 0.5f, 0};
    for (uint32_t i = 0; i < REQUEST_RING_SIZE; i++)
        CHECK(done_ring_push(dr, &done) == 0);
    CHECK(done_ring_push(dr, &done) == -1 && dr->overflow.value == 1);
    CHECK(done_ring_pop(dr, &done) == 1 && done_ring_push(dr, &done) == 0);
    free(dr);

    RequestRing *rq = req_ring_create();
    RolloutRequest r = {5, 256, 4, 0.8f, 50, 0.9f, 42}, ro;
    uint32_t p = req_ring_acquire(rq);
    CHECK(p == 0);
    rq->slots[p] = r;
    req_ring_commit(rq);
    CHECK(req_ring_consume(rq, &ro) == 1 && ro.request_id == 5 && ro.top_k == 50 && ro.rng_seed == 42);
    CHECK(req_ring_consume(rq, &ro) == 0);
    req_ring_destroy(rq);
    printf("completion_and_done_rings OK\n");
}

static void
descriptor_windows(void)
{
    CommandRing *ring = ring_create();
    DecodeDispatchBatch batch;
    Descriptor d;
    decode_batch_reset(&batch);
    memset(&d, 0, sizeof d);
    d.seq_id = 11;
    d.output_token_offset = 3;
    CHECK(decode_batch_push(&batch, &d) == 0);
    d.seq_id = 12;
    d.output_token_offset = 4;
    CHECK(decode_batch_push(&batch, &d) == 0);
    d.seq_id = 13;
    d.output_token_offset = 5;
    CHECK(decode_batch_push(&batch, &d) == 0);
    CHECK(decode_batch_submit(ring, &batch) == 0 && ring->prod.tail == 3);
    for (uint16_t i = 0; i < 3; i++) {
        CHECK(ring_consume(ring, &d) == 1);
        CHECK(d.seq_id == 11u + i && d.output_token_offset == 3u + i);
        CHECK(d.batch_size == 3 && d.batch_index == i);
        DecodeBatchContract c = decode_batch_contract(&d);
        CHECK(c.batch_size == 3 && c.batch_index == i);
    }
    /* limits */
    decode_batch_reset(&batch);
    CHECK(decode_batch_submit(ring, &batch) == -1);
    for (int i = 0; i < 32; i++)
        CHECK(decode_batch_push(&batch, &d) == 0);
    CHECK(decode_batch_push(&batch, &d) == -1);
    DecodeBatchContract z = decode_batch_contract(NULL);
    CHECK(z.batch_size == 0 && z.batch_index == 0);
    ring_destroy(ring);
    printf("descriptor_windows OK\n");
}

static void
arena_basic(void)
{
    KVArena *a = (KVArena *)malloc(sizeof(KVArena));
    arena_init(a, 64UL << 20, 16384);
    CHECK(a->base);
    int64_t ids[100];
    for (int i = 0; i < 100; i++) {
        ids[i] = arena_acquire(a);
        CHECK(ids[i] == i); /* lowest-free-first closed form */
        memset(arena_block_ptr(a, ids[i]), 0xAB, 128);
    }
    for (int i = 0; i < 100; i++)
        arena_release(a, ids[i]);
    for (int i = 0; i < 100; i++)
        CHECK(arena_acquire(a) == i);
    arena_release(a, 37);
    CHECK(arena_acquire(a) == 37);
    arena_release(a, -1); /* ignored */
    arena_destroy(a);
    CHECK(a->base == NULL);
    free(a);
    printf("arena_basic OK\n");
}

static void
kv_prefix_basic(void)
{
    KVPrefixTable *t = (KVPrefixTable *)malloc(sizeof(KVPrefixTable));
    kv_prefix_table_init(t);
    uint32_t pid;
    CHECK(kv_prefix_register(t, 0x1000, 64, 4, &pid) == 0 && pid < MAX_PREFIXES);
    KVPrefix *p = kv_prefix_get(t, pid);
    CHECK(p && p->refcnt == 1 && p->token_len == 64);
    CHECK(kv_prefix_acquire(t, pid) == 0 && p->refcnt == 2);
    CHECK(kv_prefix_release(t, pid) == 0 && p->refcnt == 1);
    CHECK(kv_prefix_release(t, pid) == 0 && p->refcnt == 0);
    CHECK(p->kv_block_offset == -1 && p->token_len == 0 && p->kv_block_count == 4);
    uint32_t bid;
    CHECK(kv_branch_alloc(t, 0, pid, 0x2000, 16, 1, &bid) == 0 && bid < MAX_BRANCHES);
    /* reference test asserts 0x1000 here; the code answers -1 (refcount hit 0) */
    CHECK(kv_branch_total_offset(t, bid) == -1);
    CHECK(kv_branch_free(t, bid) == 0);
    CHECK(kv_prefix_acquire(t, MAX_PREFIXES) == -1 && kv_prefix_release(t, pid) == -1);
    CHECK(kv_branch_free(t, MAX_BRANCHES) == -1 && kv_branch_total_offset(t, MAX_BRANCHES) == -1);
    /* bench/bench_cow_prefix.cu: refcount after N branches is N + 1 */
    CHECK(kv_prefix_register(t, 0x4000, 512, 32, &pid) == 0 && pid == 0);
    for (uint32_t i = 0; i < 8; i++)
        CHECK(kv_branch_alloc(t, i, pid, 0x8000 + i, 0, 0, &bid) == 0);
    CHECK(kv_prefix_get(t, pid)->refcnt == 9);
    free(t);
    printf("kv_prefix_basic OK\n");
}

static void
reward_and_decode_bookkeeping(void)
{
    CHECK(reward_score_mock(NULL, 0) == 0.0f && reward_score_mock(NULL, 255) == 1.0f);
    CHECK(reward_score_mock(NULL, 256) == 0.0f && reward_score_mock(NULL, 128) == 128.0f / 255.0f);
    DecodeMicrokernelConfig c = attention_decode_config_fixed128();
    CHECK(c.head_dim == 128 && c.tokens_per_block == 32 && c.tile_tokens == 16);
    CHECK(c.prefetch_stages == 3 && c.shared_bytes == 49152);
    DecodeStepResult r = attention_decode_result_fixed128(17);
    CHECK(r.bytes_touched == 17u * 128u * 2u * 2u && r.tile_count == 2u);
    CHECK(r.cycle_estimate == 2ull * 128ull * 24ull);
    printf("reward_and_decode_bookkeeping OK\n");
}

/* test/test_bench.cu:512-534, plus the lowest-free-id order and the wipe. */
static void
rollout_slab_basic(void)
{
    static rollout_slab_t slab;
    uint32_t ids[10], id2;
    rollout_slab_init(&slab);
    for (uint32_t i = 0; i < 10; i++) {
        CHECK(rollout_alloc(&slab, &ids[i]) == 0);
        CHECK(ids[i] == i);
        rollout_get(&slab, ids[i])->seq_len = 77;
    }
    rollout_free(&slab, ids[3]);
    rollout_free(&slab, ids[7]);
    CHECK(rollout_alloc(&slab, &id2) == 0 && id2 == 3);
    CHECK(rollout_get(&slab, 3)->seq_len == 0 && rollout_get(&slab, 3)->rollout_id == 3);
    CHECK(rollout_alloc(&slab, &id2) == 0 && id2 == 7);
    CHECK(rollout_alloc(&slab, &id2) == 0 && id2 == 10);
    rollout_free(&slab, MAX_ROLLOUTS);          /* out of range: ignored */
    CHECK(rollout_get(&slab, MAX_ROLLOUTS) == NULL);
    rollout_slab_init(&slab);
    for (uint32_t i = 0; i < MAX_ROLLOUTS; i++)
        CHECK(rollout_alloc(&slab, &id2) == 0 && id2 == i);
    CHECK(rollout_alloc(&slab, &id2) == -1);
    rollout_free(&slab, 4097);
    CHECK(rollout_alloc(&slab, &id2) == 0 && id2 == 4097);
    printf("rollout_slab_basic OK\n");
}

/* test/test_bench.cu:536-557, plus the whole 6 x 6 table. */
static void
rollout_transitions(void)
{
    rollout_t r;
    memset(&r, 0, sizeof(r));
    CHECK(rollout_transition(&r, ROLL_FREE, ROLL_DECODING) != 0 && r.state == ROLL_FREE);
    CHECK(rollout_transition(&r, ROLL_FREE, ROLL_PREFILL_READY) == 0);
    CHECK(rollout_transition(&r, ROLL_PREFILL_READY, ROLL_DECODING) == 0);
    CHECK(rollout_transition(&r, ROLL_DECODING, ROLL_REWARD_PENDING) == 0);
    CHECK(rollout_transition(&r, ROLL_REWARD_PENDING, ROLL_TRAJECTORY_READY) == 0);
    CHECK(rollout_transition(&r, ROLL_TRAJECTORY_READY, ROLL_DONE) == 0);
    CHECK(rollout_transition(&r, ROLL_DONE, ROLL_FREE) == 0);
    CHECK(r.state == ROLL_FREE);
    /* a valid pair from the wrong current state fails and changes nothing */
    CHECK(rollout_transition(&r, ROLL_DECODING, ROLL_DONE) != 0 && r.state == ROLL_FREE);
    static const int allowed[6][6] = {
        {0, 1, 0, 0, 0, 0}, {0, 0, 1, 0, 0, 0}, {0, 0, 0, 1, 0, 1},
        {0, 0, 1, 0, 1, 0}, {0, 0, 0, 0, 0, 1}, {1, 0, 0, 0, 0, 0},
    };
    for (int f = 0; f < 6; f++)
        for (int t = 0; t < 6; t++) {
            CHECK(rollout_is_valid_transition((rollout_state_t)f, (rollout_state_t)t) == allowed[f][t]);
            r.state = (uint32_t)f;
            CHECK((rollout_transition(&r, (rollout_state_t)f, (rollout_state_t)t) == 0) == allowed[f][t]);
            CHECK(r.state == (uint32_t)(allowed[f][t] ? t : f));
        }
    printf("rollout_transitions OK\n");
}

/* test/test_bench.cu:559-581 and test/test_smoke.c:200-284. */
static void
pipeline_queues_credits_fifo(void)
{
    static RolloutPipeline p;
    PipelineSnapshot snap;
    uint32_t rid, rid0, rid1, rid2, out;

    CHECK(pipeline_init(&p) == 0);
    CHECK(rollout_alloc(&p.slab, &rid) == 0);
    for (int q = Q_FREE; q <= Q_DONE; q++) {
        CHECK(pipeline_push(&p, (pipeline_q_t)q, rid) == 0);
        CHECK(pipeline_pop(&p, (pipeline_q_t)q, &out) == 0 && out == rid);
    }
    CHECK(pipeline_pop(&p, Q_FREE, &out) != 0);
    CHECK(pipeline_push(&p, Q_COUNT, rid) != 0 && pipeline_occupancy(&p, Q_COUNT) == 0);
    rollout_free(&p.slab, rid);

    /* credits and snapshot (test_smoke.c:200-227) */
    CHECK(pipeline_init(&p) == 0);
    CHECK(rollout_alloc(&p.slab, &rid0) == 0 && rollout_alloc(&p.slab, &rid1) == 0);
    CHECK(rollout_alloc(&p.slab, &rid2) == 0);
    pipeline_credits_set(&p, 2, 4, 4, 32);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid0) == 0);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid1) == 0);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid2) == -1);
    pipeline_snapshot(&p, &snap);
    CHECK(snap.queue_occupancy[Q_DECODE] == 2 && snap.stage_credit_headroom[Q_DECODE] == 0);
    CHECK(snap.stage_credit_headroom[Q_REWARD] == 4 && snap.stage_credit_headroom[Q_PREFILL] == UINT32_MAX);
    CHECK(snap.credits.kv_block_limit == 32 && snap.policy == PIPELINE_SCHED_FIFO);
    CHECK(pipeline_stage_target_batch(&p, Q_DECODE, 8) == 0);
    pipeline_release(&p, Q_DECODE, 1);
    pipeline_snapshot(&p, &snap);
    CHECK(snap.stage_credit_headroom[Q_DECODE] == 1);
    CHECK(pipeline_stage_target_batch(&p, Q_DECODE, 8) == 1);
    pipeline_release(&p, Q_DECODE, 9);      /* saturates at 0 used */
    CHECK(pipeline_stage_available_credits(&p, Q_DECODE) == 2);
    CHECK(pipeline_stage_target_batch(&p, Q_DECODE, 8) == 2);
    CHECK(pipeline_stage_target_batch(&p, Q_DECODE, 1) == 1);

    /* FIFO without work loss (test_smoke.c:231-284) */
    CHECK(pipeline_init(&p) == 0);
    CHECK(rollout_alloc(&p.slab, &rid0) == 0 && rollout_alloc(&p.slab, &rid1) == 0);
    CHECK(rollout_alloc(&p.slab, &rid2) == 0);
    pipeline_credits_set(&p, 3, 4, 4, 32);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid0) == 0 && pipeline_try_push(&p, Q_DECODE, rid1) == 0);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid2) == 0 && pipeline_occupancy(&p, Q_DECODE) == 3);
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) == 0 && out == rid0 && pipeline_occupancy(&p, Q_DECODE) == 2);
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) == 0 && out == rid1);
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) == 0 && out == rid2 && pipeline_occupancy(&p, Q_DECODE) == 0);
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) != 0);
    pipeline_release(&p, Q_DECODE, 3);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid0) == 0 && pipeline_try_push(&p, Q_DECODE, rid1) == 0);
    CHECK(pipeline_try_push(&p, Q_DECODE, rid2) == 0 && pipeline_occupancy(&p, Q_DECODE) == 3);
    p.policy = PIPELINE_SCHED_SHORTEST_REMAINING;
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) != 0 && pipeline_occupancy(&p, Q_DECODE) == 3);
    CHECK(pipeline_set_schedule_policy(&p, PIPELINE_SCHED_SHORTEST_REMAINING) != 0);
    p.policy = PIPELINE_SCHED_PREFIX_SHARING;
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) != 0 && pipeline_occupancy(&p, Q_DECODE) == 3);
    CHECK(pipeline_set_schedule_policy(&p, PIPELINE_SCHED_PREFIX_SHARING) != 0);
    CHECK(pipeline_set_schedule_policy(&p, PIPELINE_SCHED_FIFO) == 0 && p.policy == PIPELINE_SCHED_FIFO);
    CHECK(pipeline_schedule(&p, Q_DECODE, &out) == 0 && out == rid0 && pipeline_occupancy(&p, Q_DECODE) == 2);

    /* a queue holds 4,096 ids */
    CHECK(pipeline_init(&p) == 0);
    for (uint32_t i = 0; i < PIPELINE_RING_SIZE; i++)
        CHECK(pipeline_push(&p, Q_REWARD, i) == 0);
    CHECK(pipeline_push(&p, Q_REWARD, 0) == -1 && pipeline_occupancy(&p, Q_REWARD) == PIPELINE_RING_SIZE);
    CHECK(pipeline_pop(&p, Q_REWARD, &out) == 0 && out == 0 && pipeline_push(&p, Q_REWARD, 9) == 0);
    printf("pipeline_queues_credits_fifo OK\n");
}

/* test/test_bench.cu:739-762, plus full and wrap. */
static void
reward_ring_basic(void)
{
    static RewardRing rr;
    RewardDesc d = {1, 0, 128, 0, 0.0f, 0}, got;
    reward_ring_init(&rr);
    CHECK(reward_push(&rr, &d) == 0);
    CHECK(reward_pop(&rr, &got) == 0 && got.rollout_id == 1 && got.token_count == 128);
    CHECK(reward_pop(&rr, &got) != 0);
    for (uint32_t i = 0; i < REWARD_RING_SIZE; i++) {
        d.rollout_id = i;
        CHECK(reward_push(&rr, &d) == 0);
    }
    CHECK(reward_push(&rr, &d) == -1);
    for (uint32_t i = 0; i < REWARD_RING_SIZE; i++)
        CHECK(reward_pop(&rr, &got) == 0 && got.rollout_id == i);
    CHECK(reward_pop(&rr, &got) == -1);
    printf("reward_ring_basic OK\n");
}

int
main(void)
{
    CHECK(sizeof(hw_desc_t) == 64u);
    hw_ring_wraparound();
    hw_ring_producer_observes_consumer();
    submit_doorbell();
    doneq_overflow();
    worker_sim_completion();
    command_ring();
    completion_and_done_rings();
    descriptor_windows();
    arena_basic();
    kv_prefix_basic();
    reward_and_decode_bookkeeping();
    rollout_slab_basic();
    rollout_transitions();
    pipeline_queues_credits_fifo();
    reward_ring_basic();
    printf("ALL OK\n");
    return 0;
}
