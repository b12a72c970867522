/*
 * oracle.h - CPU restatement of the reference rollout hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only to check results (or as the timed CPU
 * baseline), never as a fallback.
 *
 * Every function cites the reference file:line it restates. Integer parts
 * (rings, submit, worker rule, windows, arena, prefix refcounts, reward) are
 * written against raw byte images at the reference structs' byte offsets, independently
 * of the product headers. Floating-point parts: paged GQA decode attention in
 * fp64 (truth) and fp32 online softmax (CPU baseline), sampling by sorting,
 * KV append with copy-on-write, group advantage.
 *
 * Pinning (see tests/): reference test vectors (test/test_hw_ring.c,
 * test/test_smoke.c, test/test_bench.cu), traces replayed against the
 * reference C sources compiled into oracle/_ref, Philox4x32-10 known-answer
 * vectors, libm exp, brute force on tiny inputs, closed forms.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

/* ---- hw_desc ring (include/hw_ring.h:7-69) on a raw 4,194,432-byte image ---- */
#define ORC_HW_RING_BYTES 4194432u
#define ORC_HW_RING_SLOTS 65536u
int orc_hw_ring_push(uint8_t *ring, const uint8_t desc[64]);
int orc_hw_ring_pop(uint8_t *ring, uint8_t out[64]);

/* The 64-byte descriptor infer_submit_decode builds (src/infer_submit.c:12-32). */
void orc_decode_desc(uint8_t d[64], uint32_t gpu_group_id, uint32_t kv_arena_id, uint32_t rollout_id,
                     uint64_t kv_offset, uint64_t delta_offset, uint32_t prefix_id, uint32_t seq_len,
                     uint32_t max_tokens);
/* infer_submit_decode (src/infer_submit.c:3-37): builds the 64-byte
 * descriptor, pushes it, returns the doorbell value (tail) or -1. */
int64_t orc_submit_decode(uint8_t *cmdq, uint32_t gpu_group_id, uint32_t kv_arena_id,
                          uint32_t rollout_id, uint64_t kv_offset, uint64_t delta_offset,
                          uint32_t prefix_id, uint32_t seq_len, uint32_t max_tokens);

/* hw_worker_sim rule (src/hw_worker_sim.c:23-59): drains cmdq into doneq until
 * empty or STOP; returns completions, adds decoded tokens to *decoded. */
uint64_t orc_worker_sim_drain(uint8_t *cmdq, uint8_t *doneq, uint64_t *decoded, int *stopped);

/* ---- v0.2 CommandRing (include/ring.h:27-69) / CompletionRing
 * (include/completion.h:46-87) / v0.3 RequestRing, DoneRing
 * (include/request.h:54-150) on raw images. slot_size / n_slots / slot_off /
 * overflow_off (or -1) describe the ring. ---- */
typedef struct {
    uint32_t slot_size, n_slots, slot_off;
    int32_t overflow_off;
} orc_ring_shape_t;
uint32_t orc_ring_acquire(uint8_t *ring, const orc_ring_shape_t *s, uint32_t n);
void orc_ring_commit(uint8_t *ring, uint32_t n);
int orc_ring_consume(uint8_t *ring, const orc_ring_shape_t *s, uint8_t *out);
int orc_ring_push_or_overflow(uint8_t *ring, const orc_ring_shape_t *s, const uint8_t *item);
/* decode_batch_submit (src/decode_batch.c:20-42) */
int orc_decode_batch_submit(uint8_t *ring, const uint8_t *descs, uint32_t count);

/* ---- arena bitmap (src/arena.c:31-51): 16,384 words, 1 = used ---- */
int64_t orc_arena_acquire(uint64_t *bitmap);
void orc_arena_release(uint64_t *bitmap, int64_t idx);

/* ---- kv_prefix table (src/kv_prefix.c:5-149) on a raw 606,280-byte image ---- */
#define ORC_PREFIX_TABLE_BYTES 606280u
void orc_kvp_init(uint8_t *t);
int orc_kvp_register(uint8_t *t, int64_t off, uint32_t len, uint32_t nblocks, uint32_t *out_id);
int orc_kvp_acquire(uint8_t *t, uint32_t id);
int orc_kvp_release(uint8_t *t, uint32_t id);
int orc_kvb_alloc(uint8_t *t, uint32_t rollout, uint32_t prefix, int64_t delta, uint32_t dlen,
                  uint32_t dblocks, uint32_t *out_id);
int orc_kvb_free(uint8_t *t, uint32_t id);
int64_t orc_kvb_total_offset(const uint8_t *t, uint32_t id);
/* cu/kv_prefix.cu:4-23 (device kv_branch_resolve): like total_offset, but a
 * prefix whose refcnt is 0 also yields the branch's delta offset. */
int64_t orc_kvb_resolve(const uint8_t *t, uint32_t id);
/* The copy-on-write source of one (row, kv head): the prefix block whose
 * filled slots [0, token_len % tpb) the row's first own token (position ==
 * token_len) must find in its private block, or -1. Prefix blocks are
 * head-major from kv_block_offset, kv_block_count / kv_heads per head. */
int64_t orc_kvb_cow_source(const uint8_t *t, uint32_t branch, uint32_t position, uint32_t tpb,
                           uint32_t kv_heads, uint32_t head);

/* ---- reward (src/reward.c:36-41, cu/reward.cu:11) and group advantage ---- */
float orc_reward_score(uint32_t count);
uint32_t orc_match_count(const uint32_t *tokens, const uint32_t *target, uint32_t n);
void orc_group_advantage(const float *r, uint32_t n_groups, uint32_t group, float *adv);

/* ---- Philox4x32-10 (Salmon et al., SC'11), written independently of the
 * product's rl_sample_math.h ---- */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* ---- paged GQA decode attention (cu/attention_decode.cu:60-204 generalised):
 * arena of 2-byte scalars (dtype 0 bf16, 1 fp16), blocks of token_count
 * tokens of one KV head (K plane then V plane), block_table
 * [batch][kv_heads][stride]. out[batch][q_heads][head_dim]. ---- */
typedef struct {
    const uint8_t *arena;
    uint64_t block_bytes;
    uint32_t token_count, head_dim, dtype;
    const uint32_t *table;
    uint32_t table_stride, batch, q_heads, kv_heads;
    const uint32_t *ctx;
    const uint16_t *q;
    double scale;
} orc_attn_t;
void orc_attn_decode_f64(const orc_attn_t *a, double *out);
/* fp32 online softmax over 16-token tiles, OpenMP over (rollout, kv head):
 * the CPU baseline of the decode step. */
void orc_attn_decode_f32(const orc_attn_t *a, float *out);
/* decode_synth_query_component (cu/attention_decode.cu:16-28); rng_state may be NULL */
float orc_synth_query(uint64_t seq_id, uint64_t reward_cookie, const uint64_t *rng_state, uint32_t idx);

/* ---- the plumbing decode on the CPU (orc_plumbing.c): the hw_worker_sim
 * loop (src/hw_worker_sim.c:23-59) on a pthread with a real decode step per
 * token of one rollout (fp32 attention, greedy, KV append), fed through
 * hw_ring images by the calling thread. Step k uses row k of q / k_new /
 * v_new / logits and writes attn_out[k], tokens[k]. n descriptors (seq ctx0
 * + i, max ctx0 + i + 1) go in back to back (*pipelined_s = until the last
 * completion), then n more one at a time (lat_s[i] = submit to completion).
 * Needs steps >= 2n. ---- */
typedef struct {
    const uint8_t *arena;          /* written by the appends */
    uint64_t block_bytes;
    uint32_t token_count, head_dim, dtype;
    const uint32_t *table;         /* [kv_heads][table_stride] of the one rollout */
    uint32_t table_stride, q_heads, kv_heads;
    double scale;
    const uint16_t *q;             /* [steps][q_heads][head_dim] */
    const uint16_t *k_new, *v_new; /* [steps][kv_heads][head_dim] */
    const float *logits;           /* [steps][vocab] */
    uint32_t vocab, steps;
    float *attn_out;               /* [steps][q_heads][head_dim] */
    uint32_t *tokens;              /* [steps] */
} orc_plumbing_t;
int orc_plumbing_run(const orc_plumbing_t *p, uint32_t ctx0, uint32_t n, double *pipelined_s, double *lat_s);
/* OpenMP threads of the baseline kernels (omp_set_num_threads). */
void orc_set_num_threads(int n);

/* ---- sampling (specification in include/sample.h) ----
 * greedy != 0 or temperature <= 0: argmax, lowest index.
 * Returns the token; *logprob (fp64 log-sum-exp). */
uint32_t orc_sample_row(const float *logits, uint32_t vocab, int greedy, float temperature,
                        uint32_t top_k, float top_p, uint64_t seed, uint64_t step, uint32_t row,
                        double *logprob);
void orc_sample_rows(const float *logits, uint32_t rows, uint32_t vocab, uint32_t stride, int greedy,
                     float temperature, uint32_t top_k, float top_p, const uint64_t *seeds, uint64_t step,
                     uint32_t *tokens, double *logprobs);
void orc_sample_rows_v(const float *logits, uint32_t rows, uint32_t vocab, uint32_t stride, const float *temperature,
                       const uint32_t *top_k, const float *top_p, const uint64_t *seeds, const uint64_t *steps,
                       const uint32_t *draw_ids, float temperature_all, uint32_t top_k_all, float top_p_all,
                       uint64_t step_all, uint32_t *tokens, double *logprobs);

/* ---- KV append with copy-on-write (see rl_hip_kv_append) ---- */
void orc_kv_append(uint8_t *arena, uint64_t block_bytes, uint32_t token_count, uint32_t row_bytes,
                   const uint32_t *table, uint32_t stride, uint32_t batch, uint32_t kv_heads,
                   const uint32_t *positions, const int32_t *cow_src, const uint8_t *k_new,
                   const uint8_t *v_new);

/* ---- helpers ---- */
double orc_bf16_to_f64(uint16_t v);
double orc_f16_to_f64(uint16_t v);
int orc_num_threads(void);
