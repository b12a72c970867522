/*
 * rl_hip.h - thin C ABI between the host C runtime and the gfx950 kernels.
 *
 * The reference launches its kernels from CUDA translation units that
 * declare __global__ prototypes (src/main.c:39-41, test/test_bench.cu:35-37,
 * bench/bench_gpu_scheduler.cu:9-10) and allocates with cudaMalloc /
 * cudaHostAlloc inline. Here every device interaction of the C host code goes
 * through these extern "C" entry points instead: plain pointers and sizes,
 * no C++ or framework types. Conventions follow the reference: 0 on success,
 * -1 on failure (rl_hip_last_error() then holds a message); pointers to
 * device memory are marked "device".
 *
 * Threading: one host thread drives the library at a time. All work is
 * queued on one non-blocking HIP stream owned by the library (never the
 * legacy default stream, so a running persistent worker cannot deadlock a
 * synchronisation behind it).
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "hw_ring.h"
#include "kv_layout.h"
#include "kv_prefix.h"
#include "request.h"
#include "reward.h"
#include "ring.h"
#include "sample.h"
#include "trace.h"

RL_EXTERN_C_BEGIN

/* ---- session -------------------------------------------------------------
 * Replaces the reference's inline cudaSetDevice / cudaGetDeviceProperties
 * (test/test_bench.cu:333-337, src/main.c:56-60). */
typedef struct {
    int32_t device;
    uint32_t cu_count;            /* hipDeviceAttributeMultiprocessorCount */
    uint32_t wave_size;
    uint32_t lds_bytes_per_block; /* max dynamic+static LDS per workgroup */
    uint32_t clock_khz;
    uint32_t mem_clock_khz;
    uint32_t mem_bus_width_bits;
    uint32_t l2_bytes;
    uint64_t hbm_bytes;
    char arch[64];                /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} rl_hip_device_info_t;

int rl_hip_open(int device);
int rl_hip_close(void);
int rl_hip_is_open(void);
int rl_hip_device_info(rl_hip_device_info_t *out);
const char *rl_hip_last_error(void);

/* ---- memory --------------------------------------------------------------
 * Coherent host memory replaces cudaHostAlloc(Mapped)
 * (bench/bench_gpu_scheduler.cu:43-44) and the mmap'd rings of
 * src/ring.c:10-27; device memory replaces cudaMalloc (src/main.c:84-93). */
void *rl_hip_host_alloc_coherent(size_t bytes);  /* zero-filled, 4 KiB aligned */
int rl_hip_host_free(void *p);                   /* -1 if p is not such memory */
int rl_hip_is_coherent_host(const void *p);      /* 1 if p lies in such memory */
void *rl_hip_dev_alloc(size_t bytes);
int rl_hip_is_device_ptr(const void *p);         /* 1 if p is device memory */
int rl_hip_dev_free(void *p);
int rl_hip_memcpy_h2d(void *dst_device, const void *src, size_t bytes);
int rl_hip_memcpy_d2h(void *dst, const void *src_device, size_t bytes);
int rl_hip_memcpy_d2d(void *dst_device, const void *src_device, size_t bytes);
int rl_hip_memset_d(void *dst_device, int value, size_t bytes);
int rl_hip_sync(void);  /* waits for the library stream and both lanes */

/* ---- timing on the library stream (HIP events) --------------------------- */
int rl_hip_timer_begin(void);
int rl_hip_timer_end(float *elapsed_ms);

/* ---- HIP graphs of the library stream ---------------------------------------
 * No counterpart in the reference (its decode path launches one kernel per
 * descriptor). rl_hip_capture_begin records, instead of running, what this
 * thread launches on the library stream until rl_hip_capture_end, which
 * instantiates the recording into *graph; rl_hip_graph_launch replays it on
 * the library stream (same device pointers, same arguments) and
 * rl_hip_graph_destroy frees it. Only kernel entry points may be called while
 * capturing: no rl_hip_sync, timers, copies or rl_hip_memset_d. */
int rl_hip_capture_begin(void);
int rl_hip_capture_end(void **graph);
int rl_hip_graph_launch(void *graph);
int rl_hip_graph_destroy(void *graph);

#define RL_DTYPE_BF16 0u
#define RL_DTYPE_FP16 1u

/* ---- paged GQA decode attention -------------------------------------------
 * Replaces attention_decode_step_fixed128 (cu/attention_decode.cu:60-204)
 * and its per-descriptor driver process_descriptor (cu/worker.cu:26-64).
 * One query token per (rollout, q head); q head h reads KV head
 * h / (q_heads / kv_heads). Rollout b's logical block j of KV head g is
 * physical block block_table[(b * kv_heads + g) * table_stride + j] of the
 * arena; tokens [0, ctx_lens[b]) are attended. out = softmax(scale q K^T) V
 * with fp32 accumulation, stored in the input dtype (and optionally fp32).
 * ctx_lens[b] == 0 yields zeros. A rollout whose ctx_lens exceeds max_ctx or
 * whose block table names a block past arena_bytes gets NaN outputs (the
 * offending block is not read). The KV of all rows is split evenly over
 * `grid_waves` persistent waves (0: every wave the device holds at once);
 * rows shared by several waves are combined with an fp32 log-sum-exp merge
 * (a second, small kernel on the same stream). */
typedef struct {
    const void *arena_base;      /* device: KVArena.base */
    uint64_t arena_bytes;        /* KVArena.capacity: blocks past it are never read */
    KvLayoutDesc layout;         /* must pass kv_layout_check_paged */
    const uint32_t *block_table; /* device */
    uint32_t table_stride;       /* entries per (rollout, kv head) row */
    uint32_t batch;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t dtype;              /* RL_DTYPE_* of q, K, V and out */
    const uint32_t *ctx_lens;    /* device [batch] */
    uint32_t max_ctx;            /* upper bound of ctx_lens; sizes the grid */
    uint32_t grid_waves;         /* waves sharing the KV stream, <= 2^20; 0 selects a full device */
    float scale;                 /* 0 selects 1/sqrt(head_dim) */
    const void *q;               /* device [batch][q_heads][head_dim] */
    void *out;                   /* device [batch][q_heads][head_dim] */
    float *out_f32;              /* device, optional */
    void *workspace;             /* device, >= rl_hip_attn_decode_workspace() */
    size_t workspace_bytes;
} rl_attn_decode_args_t;

size_t rl_hip_attn_decode_workspace(const rl_attn_decode_args_t *args);
int rl_hip_attn_decode(const rl_attn_decode_args_t *args);

/* ---- logits projection ------------------------------------------------------
 * No reference function (the nearest analog is the fp16 GEMV
 * query_prepare_kernel, cu/query_producer.cu:5-26). logits[r][v] =
 * sum_k x[r][k] * w[v][k]: bf16 operands (w stored like an lm_head weight,
 * one row of `hidden` per vocabulary entry), fp32 accumulate and output, on
 * MFMA. `hidden` must be a multiple of 64; x and w strides multiples of 8. */
typedef struct {
    const void *x;               /* device [rows][x_stride] bf16 */
    const void *w;               /* device [vocab][w_stride] bf16 */
    float *logits;               /* device [rows][logits_stride] fp32 */
    uint32_t rows;
    uint32_t vocab;
    uint32_t hidden;
    uint32_t x_stride;           /* elements */
    uint32_t w_stride;
    uint32_t logits_stride;
} rl_logits_proj_args_t;

int rl_hip_logits_proj(const rl_logits_proj_args_t *args);

/* ---- reward and group advantage ---------------------------------------------
 * Replaces reward_score_kernel (cu/reward.cu:4-15) and adds the GRPO group
 * advantage (no reference function). Rollout r belongs to group
 * r / group_size; count_r = #{i < min(n_tokens[r], target_len, token_stride) :
 * tokens[r][i] == targets[group][i]}; reward_r = (count_r & 0xFF) / 255.0f;
 * advantage_r = (reward_r - mean) / std over the group, population std, 0 when
 * std is 0 - bit-identical to reward_match_count / reward_group_advantage in
 * reward.h. descs, when given, receives one RewardDesc per rollout.
 * target_len <= target_stride (a target row holds target_len tokens). */
typedef struct {
    const uint32_t *tokens;      /* device [rollouts][token_stride] */
    const uint32_t *n_tokens;    /* device [rollouts] */
    const uint32_t *targets;     /* device [rollouts / group_size][target_stride] */
    uint32_t rollouts;
    uint32_t group_size;         /* 1..64, divides rollouts */
    uint32_t token_stride;
    uint32_t target_stride;
    uint32_t target_len;
    RewardDesc *descs;           /* device [rollouts], optional */
    float *reward;               /* device [rollouts] */
    float *advantage;            /* device [rollouts] */
} rl_reward_args_t;

int rl_hip_reward_advantage(const rl_reward_args_t *args);

/* ---- rollout scheduler ----------------------------------------------------------
 * Restates rollout_worker (cu/gpu_scheduler.cu:26-83) as one kernel launched
 * between batched decode steps (GPU_MAX_ROLLOUTS = 256 slots of the
 * byte-compatible GpuRolloutState, request.h:67-82). Per launch: a slot that
 * took part in the last step stores `sampled[slot]` as its next generated
 * token (gen_tokens[request][t]) and counts it; slots with tokens_generated >=
 * max_tokens get reward (count & 0xFF) / 255 with count = generated tokens
 * equal to targets[request / group_size] at the same position, push
 * RolloutDone {request_id, slot, tokens_generated, reward, 0} to done_ring in
 * slot order and free the slot; requests are then consumed from req_ring
 * while a slot is free (lowest free slot first; never consumed without one;
 * request_id UINT64_MAX sets counters[2]); admitted slots copy their
 * request's kv_heads block-table rows into slot_table. Finally every slot
 * writes the next step's per-row arguments: slot_ctx / slot_pos = prompt_len
 * + tokens_generated (0 / UINT32_MAX when idle, and for a slot parked at
 * max_tokens that could not be retired for want of room on done_ring), and the sampler's
 * temperature (0 when idle), top_k, top_p, seed (the request's rng_seed) and
 * step (the index of the token being generated). Rings live in coherent host
 * memory (req_ring_create / done_ring_create after rl_hip_open).
 * counters: [0] dones pushed, [1] requests admitted, [2] end marker seen,
 * [3] status (0 ok, 2 request id >= requests, 3 done ring full for max_spin
 * polls; sticky). The launch fails (-1, error set) on a NULL pointer, a zero
 * requests / group_size / kv_heads / table_stride / gen_stride, or kv_heads x
 * table_stride >= 2^24 block-table entries per slot. */
typedef struct {
    RequestRing *req_ring;
    DoneRing *done_ring;
    GpuRolloutState *state;      /* device, zero-initialised before the first launch */
    uint32_t requests;           /* request ids index the side tables below */
    const uint32_t *prompt_len;  /* device [requests]: tokens already in the KV */
    const uint32_t *req_table;   /* device [requests][kv_heads][table_stride] */
    uint32_t kv_heads;
    uint32_t table_stride;
    uint32_t *gen_tokens;        /* device [requests][gen_stride] */
    uint32_t gen_stride;
    const uint32_t *targets;     /* device [requests / group_size][target_len] */
    uint32_t group_size;
    uint32_t target_len;
    float *rewards;              /* device [requests] */
    uint32_t *slot_table;        /* device [256][kv_heads][table_stride] */
    uint32_t *slot_ctx;          /* device [256] */
    uint32_t *slot_pos;          /* device [256] */
    float *slot_temp;            /* device [256] */
    uint32_t *slot_topk;         /* device [256] */
    float *slot_topp;            /* device [256] */
    uint64_t *slot_seed;         /* device [256] */
    uint64_t *slot_step;         /* device [256] */
    const uint32_t *sampled;     /* device [256] tokens of the last step, NULL before the first */
    uint32_t *counters;          /* device [4], zero-initialised */
    uint64_t max_spin;           /* 0 selects 2^22 */
    uint32_t *slot_request;      /* device [256] or NULL: the request id of each slot that decodes
                                    the next step, UINT32_MAX for the others */
} rl_rollout_sched_args_t;

int rl_hip_rollout_schedule(const rl_rollout_sched_args_t *args);

/* ---- persistent worker on the hw_desc rings ---------------------------------
 * Replaces hw_worker_sim_run (src/hw_worker_sim.c:23-59, include/
 * hw_worker_sim.h:6-14) and the device worker decode_worker
 * (cu/worker.cu:66-131). One persistent workgroup per ring pair: the single
 * consumer of cmdq[g] and producer of doneq[g] (rings from hw_ring_create()
 * with a device open, i.e. fine-grained coherent host memory; the two pointer
 * arrays themselves device-readable). Each DECODE descriptor gets the control
 * rule of hw_worker_sim (seq_len++ up to max_tokens, DONE / NEEDS_REWARD) with
 * one real decode step per token: attention of rollout `rollout_id` over its
 * seq_len cached tokens (block_table rows rollout * kv_heads + h), the greedy
 * token and logprob of the step's logits, and the append of the step's K/V
 * token at position seq_len. Group g's k-th step reads q/k_new/v_new/logits
 * row g * max_steps + k and writes attn_out / token_out / logprob_out there.
 * STOP ends the worker without a completion; other opcodes are dropped.
 * The launch returns at once; rl_hip_sync() waits until every worker exited:
 * on STOP, when *stop becomes nonzero, or after max_idle_polls consecutive
 * empty polls (a full completion ring likewise). stats[g] = {decoded tokens,
 * completions, steps, status}; status 0 stopped, 1 idle limit, 2 inputs
 * exhausted or rollout id >= rollouts, 3 completion ring full, 4 appended
 * token outside the block table or arena. With stamps set, worker g writes
 * the GPU's 100 MHz clock (s_memrealtime ticks) to stamps[g][0] when a poll
 * first sees a new descriptor and to stamps[g][1] just before it releases
 * that descriptor's completion (ring_lockstep_hw in trace.h reads them). */
typedef struct {
    hw_ring_t *const *cmdq;      /* device-readable [groups] */
    hw_ring_t *const *doneq;     /* device-readable [groups] */
    uint32_t groups;             /* <= compute units */
    const volatile uint32_t *stop; /* coherent host memory */
    uint64_t max_idle_polls;     /* 0 selects 2^22 */
    void *arena_base;            /* device: KVArena.base (appended tokens are written) */
    uint64_t arena_bytes;
    KvLayoutDesc layout;
    const uint32_t *block_table; /* device [rollouts * kv_heads][table_stride] */
    uint32_t table_stride;
    uint32_t rollouts;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t dtype;              /* RL_DTYPE_* of q, K, V */
    float scale;                 /* 0 selects 1/sqrt(head_dim) */
    uint32_t max_steps;          /* decode steps per group the inputs hold */
    const void *q;               /* device [groups][max_steps][q_heads][head_dim] */
    const void *k_new;           /* device [groups][max_steps][kv_heads][head_dim] */
    const void *v_new;
    const float *logits;         /* device [groups][max_steps][vocab] */
    uint32_t vocab;
    float *attn_out;             /* device [groups][max_steps][q_heads][head_dim] */
    uint32_t *token_out;         /* device [groups][max_steps] */
    float *logprob_out;          /* device [groups][max_steps] */
    uint64_t *stats;             /* device or coherent [groups][4] */
    void *workspace;             /* device, >= rl_hip_hw_worker_workspace() */
    size_t workspace_bytes;
    uint64_t *stamps;            /* coherent host [groups][2] or NULL: see below */
} rl_hw_worker_args_t;

size_t rl_hip_hw_worker_workspace(const rl_hw_worker_args_t *args);
int rl_hip_hw_worker_launch(const rl_hw_worker_args_t *args);

/* ---- the batched decode step driven through the hw_desc rings ---------------
 * Replaces the one-descriptor-per-SM device worker (cu/worker.cu:66-131) and
 * applies the hw_worker_sim rule (src/hw_worker_sim.c:23-59) token by token,
 * with up to `batch` DECODE descriptors sharing one decode step that spans
 * every compute unit. rl_hip_ring_step_enqueue queues `steps` steps on the
 * library stream and returns at once; each step:
 *  - takes descriptors from cmdq into free rows (lowest row first, ring
 *    order), waiting (bounded by max_idle_polls) only while no row is active:
 *    DECODE with seq_len < max_tokens decodes; DECODE with seq_len >=
 *    max_tokens passes through unchanged; STOP, the host *stop flag, an idle
 *    limit or a rollout_id >= rollouts end admission (stats status 4, 4, 1, 2)
 *    while active rows finish; other opcodes are dropped;
 *  - decodes one token for every active row: paged GQA attention of rollout
 *    rollout_id over its seq_len cached tokens (block_table rows rollout *
 *    kv_heads + h) with the K/V token appended at position seq_len, and
 *    sampling of the step's logits (greedy, or temperature / top_k / top_p
 *    with Philox key seeds[rollout] and counter (seq_len, rollout): the draw
 *    depends on the descriptor, never on the batch row it was admitted
 *    into), together as rl_hip_decode_sample_step (one launch streams the
 *    attention beside the sampling, a second merges and appends; its
 *    results on the rows of the step);
 *  - applies the rule for that token (seq_len++; DONE at max_tokens;
 *    NEEDS_REWARD at a multiple of 32; otherwise the row decodes again next
 *    step) and pushes finished descriptors to doneq in row order (bounded
 *    wait for room; status 3 if it never comes, and the finished descriptors
 *    then stay in their rows, unchanged, for a later step or call to push).
 * Step k (counting from first_step) reads input slot k % input_slots and
 * writes output slot k % output_slots; row i of a slot belongs to whatever
 * descriptor holds row i in that step, which row_rollout_out records
 * (UINT32_MAX for a row that did not decode). The workspace (from
 * rl_hip_ring_step_workspace) holds the row table and the pipeline's ring
 * indexes across calls: zero it before the first enqueue of a run. stats =
 * {tokens decoded, completions pushed, steps with work, status}. */
typedef struct {
    hw_ring_t *cmdq;             /* coherent host (hw_ring_create after rl_hip_open) */
    hw_ring_t *doneq;            /* coherent host */
    const volatile uint32_t *stop; /* coherent host */
    uint64_t max_idle_polls;     /* 0 selects 2^22 */
    uint32_t batch;              /* rows per step, 1..1024 */
    void *arena_base;            /* device: KVArena.base */
    uint64_t arena_bytes;
    KvLayoutDesc layout;
    const uint32_t *block_table; /* device [rollouts][kv_heads][table_stride] */
    uint32_t table_stride;
    uint32_t rollouts;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t dtype;              /* RL_DTYPE_* of q, K, V and attn_out */
    float scale;                 /* 0 selects 1/sqrt(head_dim) */
    uint32_t max_ctx;            /* upper bound of every seq_len */
    uint32_t input_slots;
    const void *q;               /* device [input_slots][batch][q_heads][head_dim] */
    const void *k_new;           /* device [input_slots][batch][kv_heads][head_dim] */
    const void *v_new;
    const float *logits;         /* device [input_slots][batch][vocab] */
    uint32_t vocab;              /* multiple of 4 */
    uint32_t greedy;
    float temperature;
    uint32_t top_k;
    float top_p;
    const uint64_t *seeds;       /* device [rollouts] or NULL: the rollout id is the seed */
    uint32_t output_slots;
    void *attn_out;              /* device [output_slots][batch][q_heads][head_dim] */
    float *attn_out_f32;         /* device, optional, same shape */
    uint32_t *token_out;         /* device [output_slots][batch] */
    float *logprob_out;          /* device [output_slots][batch] */
    uint32_t *row_rollout_out;   /* device [output_slots][batch] or NULL */
    uint64_t *stats;             /* device [4] */
    void *workspace;             /* device, >= rl_hip_ring_step_workspace(), zeroed before the first enqueue */
    size_t workspace_bytes;
} rl_ring_step_args_t;

size_t rl_hip_ring_step_workspace(const rl_ring_step_args_t *args);
int rl_hip_ring_step_enqueue(const rl_ring_step_args_t *args, uint32_t steps, uint64_t first_step);

/* The same pipeline as one self-scheduled launch, like the reference's
 * persistent device worker (cu/worker.cu:66-131) but with every compute unit
 * on each step: a persistent grid of one workgroup per compute unit (a
 * cooperative launch) in which one wave runs the turns beside the steps, a
 * few service waves append the K/V tokens, and the other workgroups stream
 * the fused steps back to back, a step released as soon as the previous
 * step's tokens are appended (so consecutive steps overlap) and merged by
 * the next step's sampling waves. It runs up to max_steps steps and ends
 * earlier once admission has ended and every row is free (later steps would
 * decode nothing); the last turn publishes the last step. Turns, stats, the
 * row table, completions, rows, tokens, logprobs and the arena are those of
 * rl_hip_ring_step_enqueue(args, s, first_step) for the s steps the loop
 * ran, which it writes to *steps_run (device, may be NULL) at its end; the
 * attention outputs agree to fp32 rounding (the steps' split differs). A
 * step's completions become visible once its results are written, possibly a
 * few steps later than the launched pipeline would show them; all of them
 * before the launch ends. A following enqueue or loop continues at
 * first_step + s on the same workspace. Requires output_slots >= 3 (a step's
 * split rows are merged while the next two run) and a shape that fits the
 * fused kernel (as rl_hip_decode_sample_step's fused path: batch <= 1024 and
 * the GQA group, head_dim and block size it takes); others return -1. Every
 * wait is bounded; one that runs out ends the loop with stats status 5 (the
 * run's ring state is then undefined). Queued on the library stream; returns
 * at once. */
int rl_hip_ring_loop_launch(const rl_ring_step_args_t *args, uint32_t max_steps, uint64_t first_step,
                            uint32_t *steps_run);

/* ---- persistent worker on the v0.2 command / completion rings ---------------
 * Replaces decode_worker and process_descriptor (cu/worker.cu:25-131): one
 * persistent workgroup per (CommandRing, CompletionRing) pair - the single
 * consumer and the single producer of that pair - that takes every window of
 * committed Descriptors at the head (up to 32, the decode_batch window),
 * runs the fixed128 decode step of each (attention_decode_step_fixed128,
 * cu/attention_decode.cu:60-204: one head, d128, fp16 K/V of the 16 KiB arena
 * block kv_block_offset, seq_len = num_kv_blocks clamped to [1, 32], q from
 * q_buffer slot output_token_offset & (io_slots - 1) or, with no q buffer,
 * the reference's synthesized query seeded by seq_id, reward_cookie and
 * sample_state->rng_state; fp32 output to the o buffer; token = lowest index
 * of the output's maximum; cycles = ceil(seq_len / 16) * 128 * 24) and
 * pushes the Completions {seq_id, token_id, kv_block_offset, reward_cookie,
 * cycles} in descriptor order. seq_id == UINT64_MAX is consumed and stops the
 * worker without a completion. A block past arena_bytes gives NaN outputs and
 * token 0 (it is not read). The launch returns at once; rl_hip_sync() waits
 * for every worker to exit (sentinel, *stop, max_idle_polls empty polls, or
 * a completion ring full for as long). stats per group: {descriptors run,
 * completions pushed, windows, status (0 stopped, 1 idle, 3 ring full)}.
 * With trace set, worker g appends to trace[g] (trace.h records; the worker is
 * that ring's only producer and starts at its head) a DESC_CONSUMED record per
 * descriptor when its window has been read and a COMPLETION_POSTED record per
 * completion just before the completion tail is released, {tsc = the GPU's
 * 100 MHz s_memrealtime ticks, rollout_id = low 32 bits of seq_id, seq =
 * output_token_offset}; the ring head is release-stored after each batch of
 * records. With stamps set, worker g writes the GPU's 100 MHz clock to
 * stamps[g][0] when a poll first sees a new tail and to stamps[g][1] just
 * before it releases a window's completions (ring_lockstep_cmd in trace.h
 * reads them). */
typedef struct {
    CommandRing *const *rings;          /* coherent host [groups] (ring_create after rl_hip_open) */
    CompletionRing *const *comp_rings;  /* coherent host [groups] (comp_ring_create) */
    uint32_t groups;                    /* 1 .. workers resident at once (one per compute unit) */
    const volatile uint32_t *stop;      /* coherent host: nonzero ends every worker */
    uint64_t max_idle_polls;            /* 0 selects 2^22 */
    const void *arena_base;             /* device: fixed128 blocks of 16,384 bytes */
    uint64_t arena_bytes;
    const SampleState *sample_state;    /* device, optional (synthesized queries only) */
    const void *q_buffer;               /* device fp16 [io_slots][128], or NULL */
    float *o_buffer;                    /* device fp32 [io_slots][128], or NULL */
    uint32_t io_slots;                  /* a power of two; 0 uses slot 0 */
    uint64_t *stats;                    /* device [groups][4] */
    TraceRing *trace;                   /* coherent host [groups] rings, or NULL (see below) */
    uint64_t *stamps;                   /* coherent host [groups][2] or NULL (see below) */
} rl_cmd_worker_args_t;

int rl_hip_cmd_worker_launch(const rl_cmd_worker_args_t *args);

/* ---- clock samples for device-stamped traces ---------------------------------
 * No counterpart in the reference (its tracing is host-only; docs/tracing.md
 * lists device timestamps as future work). Takes `samples` ping-pong rounds
 * between the host and a one-wave kernel on a private stream and returns the
 * round with the shortest trip: the GPU's 100 MHz s_memrealtime reading, the
 * host CLOCK_MONOTONIC ns at the middle of that trip, and the trip (the
 * sample's uncertainty is at most half of it). Two calls, before and after a
 * run, feed trace_clock_fit (trace.h). samples 1..1024. */
int rl_hip_trace_clock_sample(uint32_t samples, uint64_t *ticks, double *host_ns, uint64_t *rtt_ns);

/* ---- wave broadcast self-test ---------------------------------------------
 * The ring workers hand the values one lane reads from a ring to the whole
 * wave with a lane broadcast (rl_wave_bcast_u32 / _u64, in place of the
 * reference's warp_broadcast_u32 / _u64, include/warp_broadcast.cuh). This
 * runs it in the shape of the reference's test (test/test_bench.cu:47-59,
 * 623-656) on two 64-lane waves: in wave w, lane (w ? 37 : 0) holds seq
 * 0x123456789ABCDEF0 + w, offset 77 + w and cookie 0x0FEDCBA987654321 ^ w,
 * the other lanes zeros, and every lane writes what it receives to element
 * 64 w + lane of each device array (128 entries each). Synchronous. */
int rl_hip_wave_broadcast_selftest(uint64_t *seq_out, uint32_t *offset_out, uint64_t *cookie_out);

/* ---- sampling -------------------------------------------------------------
 * Replaces sample_token (cu/sample.cu:41-123) with the specification in
 * sample.h: greedy, or temperature / top-k (k <= 256) / top-p with a
 * Philox4x32-10 draw and an integer CDF, plus the token's logprob.
 * Per-row parameter arrays may be NULL, in which case the *_all scalar is
 * used for every row. Rows with top_k == 0 or top_k >= vocab and top_p < 1
 * (a whole-vocabulary nucleus) take an exact full-row path, as do rows whose
 * top-k candidates overflow the per-slice lists. vocab <= 64 * 8192. */
typedef struct {
    const float *logits;         /* device [rows][row_stride] fp32 */
    uint32_t rows;
    uint32_t vocab;
    uint32_t row_stride;         /* elements; multiple of 4 */
    uint32_t greedy;             /* 1: argmax path, parameters ignored */
    const float *temperature;    /* device [rows] or NULL */
    const uint32_t *top_k;       /* device [rows] or NULL */
    const float *top_p;          /* device [rows] or NULL */
    const uint64_t *seed;        /* device [rows] or NULL */
    float temperature_all;
    uint32_t top_k_all;
    float top_p_all;
    uint64_t seed_all;
    uint64_t step;               /* Philox counter of this sampling event */
    const uint64_t *steps;       /* device [rows] per-row step counters, or NULL: `step` for every row */
    uint32_t *token_out;         /* device [rows] */
    float *logprob_out;          /* device [rows] */
    void *workspace;             /* device, >= rl_hip_sample_workspace() */
    size_t workspace_bytes;
    const uint32_t *draw_ids;    /* device [rows] or NULL: row r's Philox counter is (step, draw_ids[r])
                                    instead of (step, r), so a sampling stream (a rollout) draws the
                                    same numbers whichever batch row it occupies */
} rl_sample_args_t;

size_t rl_hip_sample_workspace(const rl_sample_args_t *args);
int rl_hip_sample(const rl_sample_args_t *args);

/* ---- KV append with copy-on-write ----------------------------------------
 * Writes one new token per (rollout, kv head): K row and V row into slot
 * positions[b] % token_count of physical block
 * block_table[(b * kv_heads + g) * table_stride + positions[b] / token_count].
 * When cow_src is non-NULL and cow_src[b * kv_heads + g] >= 0, the slots
 * [0, positions[b] % token_count) of that (shared) source block are first
 * copied into the destination block: the copy-on-write of a partially
 * filled prefix block. The reference keeps the sharing state (refcounts of
 * src/kv_prefix.c:46-133, the offset rule of kv_branch_resolve,
 * cu/kv_prefix.cu:4-23) but never copies a block; the copy is this library's.
 * At the copy-on-write step the destination block holds nothing yet: an
 * attention in the same step must read the prefix through a table that still
 * maps the shared source block (the append's table maps the private
 * destination), and from the next step on the private block holds the
 * prefix slots and the new token. rl_hip_kv_cow (below) instead copies before
 * the attention, so that one table serves both. */
typedef struct {
    void *arena_base;            /* device */
    uint64_t arena_bytes;        /* blocks past it are never written */
    KvLayoutDesc layout;
    const uint32_t *block_table; /* device */
    uint32_t table_stride;
    uint32_t batch;
    uint32_t kv_heads;
    const uint32_t *positions;   /* device [batch]; >= table_stride * token_count: skipped */
    const int32_t *cow_src;      /* device [batch][kv_heads] or NULL */
    const void *k_new;           /* device [batch][kv_heads][head_dim] */
    const void *v_new;           /* device [batch][kv_heads][head_dim] */
} rl_kv_append_args_t;

int rl_hip_kv_append(const rl_kv_append_args_t *args);

/* ---- prefix table on the device ------------------------------------------
 * rl_hip_kv_branch_resolve replaces kv_branch_resolve (cu/kv_prefix.cu:4-23)
 * on a byte-compatible KVPrefixTable image in device memory (copied from the
 * host table that kv_prefix_register / kv_branch_alloc maintain):
 * out_offsets[i] = -1 when branch_ids[i] >= MAX_BRANCHES; the branch's
 * delta_kv_offset when its prefix_id >= MAX_PREFIXES or that prefix's refcnt
 * is 0; otherwise the prefix's kv_block_offset. (The host
 * kv_branch_total_offset ignores the refcount; the device rule does not.)
 *
 * rl_hip_kv_cow is the copy-on-write of a shared prefix's partially filled
 * last block, run before a step whose attention reads it (no reference
 * function: the reference keeps the refcounts, src/kv_prefix.c:46-133, and
 * copies nothing). Row b's branch is row_key[b] (or branch_of_key[row_key[b]]
 * when that side table is given; keys bounds it). When the branch resolves to
 * a live prefix of token_len P with P % token_count != 0 and positions[b] ==
 * P (the branch's first own token lands in that block), kv head g's slots
 * [0, P % token_count) of the prefix block kv_block_offset + g *
 * (kv_block_count / kv_heads) + P / token_count (prefix blocks head-major
 * from kv_block_offset, in arena block units) are copied into the row's
 * block block_table[(b * kv_heads + g) * table_stride + P / token_count].
 * Every other row is left alone, as are blocks past the arena or the table.
 * That table entry must be a private block: when it is the prefix block
 * itself, nothing is copied and the step's append would write the branch's
 * token into the block every sibling reads. With row_status set, entry
 * b * kv_heads + g reports what happened to (row b, kv head g):
 * RL_COW_NONE (nothing to copy: no live prefix, a prefix ending on a block
 * boundary, or not the branch's first own token), RL_COW_COPIED,
 * RL_COW_SHARED (the row's entry is the prefix block: not copied) or
 * RL_COW_OUT_OF_RANGE (a block past the arena, or P / token_count past the
 * table or the prefix's blocks: not copied). */
#define RL_COW_NONE 0u
#define RL_COW_COPIED 1u
#define RL_COW_SHARED 2u
#define RL_COW_OUT_OF_RANGE 3u
int rl_hip_kv_branch_resolve(const KVPrefixTable *table, const uint32_t *branch_ids, int64_t *out_offsets,
                             uint32_t n);

typedef struct {
    void *arena_base;               /* device */
    uint64_t arena_bytes;
    KvLayoutDesc layout;
    const KVPrefixTable *prefixes;  /* device image of the host table */
    const uint32_t *row_key;        /* device [batch] */
    const uint32_t *branch_of_key;  /* device [keys] branch ids, or NULL: row_key holds the branch id */
    uint32_t keys;
    const uint32_t *block_table;    /* device [batch][kv_heads][table_stride]: private blocks */
    uint32_t table_stride;
    uint32_t batch;
    uint32_t kv_heads;
    const uint32_t *positions;      /* device [batch]: the position the step appends */
    uint32_t *row_status;           /* device [batch][kv_heads] RL_COW_*, or NULL */
} rl_kv_cow_args_t;

int rl_hip_kv_cow(const rl_kv_cow_args_t *args);

/* ---- fused decode step: attention, then the KV append ---------------------
 * Replaces the per-descriptor decode of process_descriptor
 * (cu/worker.cu:25-64: attention_decode_step_fixed128 over the rollout's
 * cached tokens) followed by the append of the step's K/V token (with the
 * copy-on-write described above), batched. Results equal
 * rl_hip_attn_decode(attn) then rl_hip_kv_append(append) byte for byte: the
 * append runs inside the attention's merge kernel, after every context has
 * been read, so the step takes one launch less. append->batch and kv_heads
 * must equal attn's. The attention reads through attn->block_table and the
 * append writes through append->block_table: at a copy-on-write step the
 * first still maps the shared source block, the second the private one. */
int rl_hip_decode_step(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append);

/* ---- decode step of one micro-batch with the sampling of another ----------
 * Replaces, for a rollout loop that keeps two micro-batches in flight, the
 * per-descriptor decode (cu/worker.cu:25-64) of one micro-batch together with
 * sample_token (cu/sample.cu:41-123) of the other, whose logits the previous
 * step produced: rl_hip_decode_step(attn, append) and rl_hip_sample(samp) in
 * one persistent launch that streams both from HBM side by side, plus the
 * attention merge with the append. samp must not read what attn writes (its
 * logits are the other micro-batch's). Tokens, logprobs and the appended
 * KV equal the two calls'; the attention is the same fp32 online-softmax
 * math with the rows split at other tile positions (fixed for a given set
 * of contexts, so repeated calls give the same bits), within 1e-4 of fp64
 * like rl_hip_attn_decode. The workspace (size from
 * rl_hip_decode_sample_step_workspace) holds the step's tile prefix and
 * partials; it needs no initialisation. append may be NULL: the attention
 * and the sampling without a KV append. Shapes whose tiles do not fit the
 * fused kernel's LDS (GQA groups of 8 at head_dim 128, batches above 1,024)
 * run rl_hip_decode_step (rl_hip_attn_decode without an append) and then
 * rl_hip_sample on the same workspace, with exactly their results. */
size_t rl_hip_decode_sample_step_workspace(const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp);
int rl_hip_decode_sample_step(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                              const rl_sample_args_t *samp, void *workspace, size_t workspace_bytes);

/* ---- the same step pipelined over two micro-batches ------------------------
 * The launch of rl_hip_decode_sample_step without its second kernel: step t
 * streams attn's tiles (partials into `workspace`) and samples `samp`, and
 * its sampling waves first merge the previous step's split rows and append
 * its K/V token (prev_attn / prev_append, partials in prev_workspace, which
 * that step was given as its workspace). So the rows of attn are complete
 * only after the next step (or rl_hip_decode_pipeline_flush) has run; rows
 * that one piece covered are written at once. Tokens, logprobs and the
 * appended KV equal rl_hip_decode_sample_step's; the attention is its fp32
 * math (bit for bit when the split is the same, as at the first step: the
 * merge work of the sampling waves shifts the split otherwise), within 1e-4
 * of fp64. prev_attn NULL: nothing to merge (the first step). The two micro-batches alternate, each with its own
 * workspace of rl_hip_decode_sample_step_workspace bytes; prev_attn must
 * have attn's heads, dtype and layout, and prev_append must not write what
 * attn reads (the other micro-batch's blocks; a slot at or past a row's
 * context is never read). Shapes outside the fused kernel are refused.
 * rl_hip_decode_pipeline_flush merges and appends the last step. Replaces
 * the same reference functions as rl_hip_decode_sample_step. */
int rl_hip_decode_pipeline_step(const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp,
                                const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append,
                                void *workspace, void *prev_workspace, size_t workspace_bytes);
int rl_hip_decode_pipeline_flush(const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append,
                                 void *prev_workspace, size_t workspace_bytes);

/* ---- two lanes of pipelined steps ------------------------------------------
 * No counterpart in the reference (its worker runs one descriptor at a time).
 * The session owns RL_HIP_LANES extra streams (default priority). Work queued
 * on different lanes may run at the same time: a step's launch fills the
 * compute units that the other lane's step leaves idle while its last waves
 * drain, which one stream cannot do (each launch waits for the previous one
 * to finish). rl_hip_lanes_fork makes every lane wait for what was queued on
 * the library stream so far; rl_hip_lanes_join makes the library stream wait
 * for what was queued on the lanes so far (so rl_hip_timer_end, copies and
 * rl_hip_sync after it see the lanes' results). rl_hip_decode_lane_step and
 * rl_hip_decode_lane_flush are rl_hip_decode_pipeline_step and
 * rl_hip_decode_pipeline_flush on lane `lane` (0 or 1), with the same
 * arguments and results. Lanes are ordered only by fork and join, so each
 * lane runs its own pipeline: a micro-batch's steps, the step that merges
 * them and its flush go to one lane, and the lanes' micro-batches, workspaces,
 * logits and outputs are disjoint. Four micro-batches m = 0..3 at steps
 * t = 0, 1, 2, ...: step t runs micro-batch t % 4 on lane t % 2 and merges
 * step t - 2 (the same lane's previous step). */
#define RL_HIP_LANES 2
int rl_hip_lanes_fork(void);
int rl_hip_lanes_join(void);
int rl_hip_decode_lane_step(int lane, const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp,
                            const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append,
                            void *workspace, void *prev_workspace, size_t workspace_bytes);
int rl_hip_decode_lane_flush(int lane, const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append,
                             void *prev_workspace, size_t workspace_bytes);

/* ---- fused decode step that allocates nothing ------------------------------
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and results as rl_hip_decode_step, but
 * the workspace is a fixed device array of RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES
 * inside the library (one per device, held until the process ends; its address
 * is taken at rl_hip_open). attn->workspace and attn->workspace_bytes are
 * ignored. The call fails (-1, error set) when the step needs more workspace
 * than that (rl_hip_attn_decode_workspace tells how much): about 2 KiB per
 * (wave + rollout x kv head) at GQA group 4 and head_dim 128, so 16 MiB covers
 * every full-device grid up to ~6,000 rows. It calls no hipMalloc, hipFree or
 * other allocating routine. All calls on one device share its scratch: calls
 * that overlap on one device (other threads, other streams, graphs replayed
 * concurrently) race and corrupt each other's results; calls queued on the
 * library stream one after another do not. */
#define RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES (16u << 20)
int rl_hip_decode_step_noalloc(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append);

RL_EXTERN_C_END
