/*
 * orc_plumbing.c - oracle: the CPU path of the plumbing decode, timed as the
 * CPU baseline of the ring workers (test infrastructure only).
 *
 * The reference's CPU worker is hw_worker_sim_run on its own thread
 * (src/hw_worker_sim.c:23-59), fed by infer_submit_decode and polled back by
 * the submitting thread (test/test_hw_ring.c:160-217). Its decode is a
 * counter increment; here every token runs the decode math of one rollout
 * instead: fp32 online-softmax attention over the rollout's seq_len cached
 * tokens (orc_attn_decode_f32, OpenMP over heads), the greedy token of the
 * step's logits (orc_sample_row) and the append of the step's K/V token
 * (orc_kv_append). The rings are raw hw_ring_t images whose head and tail the
 * two threads exchange with acquire / release atomics.
 */
#define _GNU_SOURCE
#include <omp.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "oracle.h"

static uint32_t ld_acq(const uint8_t *p) { return __atomic_load_n((const uint32_t *)p, __ATOMIC_ACQUIRE); }
static void st_rel(uint8_t *p, uint32_t v) { __atomic_store_n((uint32_t *)p, v, __ATOMIC_RELEASE); }

static int push(uint8_t *ring, const uint8_t d[64])
{
    const uint32_t t = ld_acq(ring + 64), h = ld_acq(ring);
    if (t - h >= ORC_HW_RING_SLOTS)
        return -1;
    memcpy(ring + 128 + (size_t)(t % ORC_HW_RING_SLOTS) * 64, d, 64);
    st_rel(ring + 64, t + 1);
    return 0;
}

static int pop(uint8_t *ring, uint8_t out[64])
{
    const uint32_t h = ld_acq(ring), t = ld_acq(ring + 64);
    if (h == t)
        return -1;
    memcpy(out, ring + 128 + (size_t)(h % ORC_HW_RING_SLOTS) * 64, 64);
    st_rel(ring, h + 1);
    return 0;
}

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

typedef struct {
    const orc_plumbing_t *p;
    uint8_t *cmdq, *doneq;
    volatile int stop;
    uint32_t steps_done;
    int threads;
} worker_t;

/* src/hw_worker_sim.c:23-59 with one real decode step per token */
static void *worker(void *arg)
{
    worker_t *w = (worker_t *)arg;
    const orc_plumbing_t *p = w->p;
    const uint32_t qd = p->q_heads * p->head_dim, kvd = p->kv_heads * p->head_dim;
    float *out = malloc(sizeof(float) * qd);
    uint8_t d[64];
    /* the submitting thread keeps one core: the decode math gets the others */
    omp_set_num_threads(w->threads);
    while (!__atomic_load_n(&w->stop, __ATOMIC_ACQUIRE)) {
        if (pop(w->cmdq, d) != 0)
            continue;
        uint16_t op, flags;
        uint32_t seq, max_tokens;
        memcpy(&op, d, 2);
        if (op == 255)
            break;
        if (op != 1)
            continue;
        memcpy(&flags, d + 2, 2);
        memcpy(&seq, d + 32, 4);
        memcpy(&max_tokens, d + 36, 4);
        while (seq < max_tokens && w->steps_done < p->steps) {
            const uint32_t k = w->steps_done++;
            orc_attn_t a = {p->arena, p->block_bytes, p->token_count, p->head_dim, p->dtype, p->table,
                            p->table_stride, 1, p->q_heads, p->kv_heads, &seq, p->q + (size_t)k * qd, p->scale};
            orc_attn_decode_f32(&a, out);
            memcpy(p->attn_out + (size_t)k * qd, out, sizeof(float) * qd);
            double lp;
            p->tokens[k] = orc_sample_row(p->logits + (size_t)k * p->vocab, p->vocab, 1, 1.0f, 0, 1.0f, 0, 0, 0, &lp);
            orc_kv_append((uint8_t *)p->arena, p->block_bytes, p->token_count, p->head_dim * 2, p->table,
                          p->table_stride, 1, p->kv_heads, &seq, NULL, (const uint8_t *)(p->k_new + (size_t)k * kvd),
                          (const uint8_t *)(p->v_new + (size_t)k * kvd));
            seq++;
            if (seq >= max_tokens) {
                flags |= 2; /* DONE */
                break;
            }
            if (seq % 32u == 0) {
                flags |= 1; /* NEEDS_REWARD */
                break;
            }
        }
        memcpy(d + 32, &seq, 4);
        memcpy(d + 2, &flags, 2);
        while (push(w->doneq, d) != 0)
            ;
    }
    free(out);
    return NULL;
}

/* infer_submit_decode of step i of the rollout: (group 7, arena 42, rollout
 * 0, kv offset 0x1000 i, delta 0x40 i, no prefix, seq ctx0 + i, max ctx0 + i + 1) */
static int submit(uint8_t *cmdq, uint32_t i, uint32_t ctx0)
{
    uint8_t d[64];
    orc_decode_desc(d, 7, 42, 0, 0x1000ull * i, 0x40ull * i, 0, ctx0 + i, ctx0 + i + 1);
    return push(cmdq, d);
}

int
orc_plumbing_run(const orc_plumbing_t *p, uint32_t ctx0, uint32_t n, double *pipelined_s, double *lat_s)
{
    if (2u * n > p->steps)
        return -1;
    uint8_t *cmdq = aligned_alloc(64, ORC_HW_RING_BYTES), *doneq = aligned_alloc(64, ORC_HW_RING_BYTES);
    if (!cmdq || !doneq)
        return -1;
    memset(cmdq, 0, ORC_HW_RING_BYTES);
    memset(doneq, 0, ORC_HW_RING_BYTES);
    const int nt = omp_get_max_threads();
    worker_t w = {p, cmdq, doneq, 0, 0, nt > 1 ? nt - 1 : 1};
    pthread_t th;
    if (pthread_create(&th, NULL, worker, &w) != 0)
        return -1;
    uint8_t d[64];
    int rc = 0;
    /* pipelined: n submissions back to back, then every completion */
    double t0 = now_s();
    for (uint32_t i = 0; i < n && rc == 0; i++)
        rc = submit(cmdq, i, ctx0);
    for (uint32_t got = 0; got < n && rc == 0;) {
        if (pop(doneq, d) == 0)
            got++;
        else
            sched_yield();
    }
    *pipelined_s = now_s() - t0;
    /* lock-step: submit one, wait for its completion */
    for (uint32_t i = n; i < 2 * n && rc == 0; i++) {
        const double t1 = now_s();
        if ((rc = submit(cmdq, i, ctx0)) != 0)
            break;
        while (pop(doneq, d) != 0)
            sched_yield();
        lat_s[i - n] = now_s() - t1;
    }
    uint8_t stop[64] = {0};
    stop[0] = 255;
    while (push(cmdq, stop) != 0)
        ;
    __atomic_store_n(&w.stop, 1, __ATOMIC_RELEASE);
    pthread_join(th, NULL);
    free(cmdq);
    free(doneq);
    return rc;
}
