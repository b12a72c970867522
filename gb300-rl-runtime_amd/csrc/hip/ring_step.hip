// ring_step.hip - the batched decode step driven through the hw_desc rings.
//
// The reference's device worker takes one descriptor at a time on one SM
// (cu/worker.cu:66-131) and its CPU model applies the hw_worker_sim rule per
// descriptor (src/hw_worker_sim.c:23-59). Here up to `batch` DECODE
// descriptors share one decode step that spreads over every compute unit,
// in a stream-ordered pipeline the host enqueues ahead of time:
//
//  poll     one wave drains the command ring (coherent host memory, system-
//           scope loads) into free rows of a device row table, lowest row
//           first, in ring order: DECODE descriptors with seq_len <
//           max_tokens decode, those at max_tokens pass through unchanged,
//           other opcodes are dropped, STOP ends admission. It waits (bounded)
//           only while no row is active; once rows are active it takes what
//           the ring holds and goes.
//  gather   one wave per (row, kv head): the row's block-table row (by the
//           descriptor's rollout_id) into a batch-ordered table, and the
//           row's context (= seq_len), append position, Philox seed and
//           counter.
//  step     rl_hip_decode_step (paged GQA attention over all compute units,
//           the KV append in its merge kernel) and rl_hip_sample over the
//           batch rows.
//  publish  one wave applies the hw_worker_sim rule for the token just
//           decoded to every active row (seq_len++, DONE at max_tokens,
//           NEEDS_REWARD at a multiple of 32, else the row stays for the next
//           step), pushes the finished descriptors to the completion ring in
//           row order (bounded wait for room) and frees their rows.
//
// Each kernel boundary makes the previous kernel's writes visible on every
// XCD, which an in-kernel hand-off between workgroups would have to buy with
// L2 write-backs and invalidations. Waits are bounded: the poll gives up after
// max_idle_polls empty polls (status 1), the publish after as many polls of a
// full completion ring (status 3); a STOP, the host stop flag, an idle limit
// or a bad rollout id end admission while active rows finish.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hw_desc.h"
#include "hw_ring.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

enum : uint32_t { kRunning = 0, kIdle = 1, kBadInput = 2, kDoneqFull = 3, kStopped = 4 };
enum : uint32_t { kFree = 0, kDecode = 1, kPass = 2 };

struct RingCtl {
    uint32_t status;       // kRunning until admission ends (sticky)
    uint32_t head;         // the command ring's consumer index (this pipeline owns it)
    uint32_t dtail;        // the completion ring's producer index (owned too)
    uint32_t init;
    uint64_t decoded, completions, steps;
};

struct RingParams {
    hw_ring_t *cq;
    hw_ring_t *dq;
    const volatile uint32_t *stop;
    uint64_t max_idle;
    uint32_t batch;
    uint32_t rollouts;
    uint32_t kv_heads;
    uint32_t table_stride;
    const uint32_t *table;      // [rollouts][kv_heads][table_stride]
    const uint64_t *seeds;      // [rollouts] or NULL (seed = rollout id)
    RingCtl *ctl;
    hw_desc_t *rows;            // [batch]
    uint32_t *kind;             // [batch]
    uint32_t *btab;             // [batch][kv_heads][table_stride]
    uint32_t *ctx;              // [batch]
    uint32_t *pos;              // [batch]
    uint64_t *rseed;            // [batch]
    uint64_t *rstep;            // [batch]
    uint32_t *row_rollout;      // [batch] of this step's output slot, or NULL
    uint64_t *stats;            // [4]
};

__device__ __forceinline__ uint32_t sys_load(const volatile uint32_t *p)
{
    return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void sys_store_release(volatile uint32_t *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kMaxBatch = 1024;

// One wave: admission of ring descriptors into free rows.
__global__ __launch_bounds__(64) void ring_poll_kernel(RingParams p)
{
    __shared__ uint16_t s_free[kMaxBatch];  // free rows, ascending
    const uint32_t lane = threadIdx.x;
    RingCtl *c = p.ctl;
    uint32_t status = c->status, head = c->head;
    if (!c->init) {
        head = rl_wave_bcast_u32(lane == 0 ? sys_load(&p.cq->head) : 0u, 0);
        const uint32_t dt = rl_wave_bcast_u32(lane == 0 ? sys_load(&p.dq->tail) : 0u, 0);
        if (lane == 0) {
            c->dtail = dt;
            c->init = 1;
        }
    }
    // free rows in ascending order, active count
    uint32_t nfree = 0;
    for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
        const uint32_t i = i0 + lane;
        const bool f = i < p.batch && p.kind[i] == kFree;
        const uint64_t m = __ballot(f);
        if (f)
            s_free[nfree + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] =
                (uint16_t)i;
        nfree += (uint32_t)__builtin_popcountll(m);
    }
    uint32_t active = p.batch - nfree, taken = 0;
    rl_wave_lds_fence();
    uint64_t idle = 0;
    while (status == kRunning && taken < nfree) {
        const uint32_t tail = rl_wave_bcast_u32(lane == 0 ? sys_load(&p.cq->tail) : 0u, 0);
        const uint32_t avail = tail - head;
        if (avail == 0) {
            if (active > 0)
                break;  // rows to decode: go with them
            const uint32_t stop = rl_wave_bcast_u32(lane == 0 ? sys_load(p.stop) : 0u, 0);
            if (stop) {
                status = kStopped;
                break;
            }
            if (++idle > p.max_idle) {
                status = kIdle;
                break;
            }
            __builtin_amdgcn_s_sleep(8);
            continue;
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        const uint32_t take = min(min(avail, 64u), nfree - taken);
        hw_desc_t d;
        const bool in = lane < take;
        if (in) {
            const volatile rl_u32x4 *src = (const volatile rl_u32x4 *)&p.cq->desc[(head + lane) & HW_RING_MASK];
            rl_u32x4 w[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                w[j] = src[j];
            __builtin_memcpy(&d, w, sizeof(d));
        } else {
            __builtin_memset(&d, 0, sizeof(d));
        }
        const bool is_stop = in && d.opcode == DESC_OP_STOP;
        const bool is_dec = in && d.opcode == DESC_OP_DECODE;
        const bool bad = is_dec && d.rollout_id >= p.rollouts;
        const uint64_t ends = __ballot(is_stop || bad);
        const uint32_t f = ends ? (uint32_t)__builtin_ctzll(ends) : take;  // first STOP or bad id
        const uint32_t consumed = ends ? f + 1 : take;
        const bool use = is_dec && lane < f;
        const uint64_t um = __ballot(use);
        if (use) {
            const uint32_t k = __builtin_amdgcn_mbcnt_hi((uint32_t)(um >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)um, 0));
            const uint32_t row = s_free[taken + k];
            p.rows[row] = d;
            p.kind[row] = d.seq_len < d.max_tokens ? kDecode : kPass;
        }
        const uint32_t n = (uint32_t)__builtin_popcountll(um);
        taken += n;
        active += n;
        head += consumed;
        if (lane == 0)
            sys_store_release(&p.cq->head, head);
        if (ends) {
            const bool was_bad = ((__ballot(bad) >> f) & 1ull) != 0;
            status = was_bad ? kBadInput : kStopped;
        }
        idle = 0;
    }
    if (status == kRunning && taken < nfree && active == 0) {
        // nothing admitted and nothing running: the host flag still ends the run
        if (rl_wave_bcast_u32(lane == 0 ? sys_load(p.stop) : 0u, 0))
            status = kStopped;
    }
    if (lane == 0) {
        c->status = status;
        c->head = head;
    }
}

// One wave per (row, kv head): the batch-ordered step arguments.
__global__ __launch_bounds__(64) void ring_gather_kernel(RingParams p)
{
    const uint32_t g = blockIdx.x, i = blockIdx.y, lane = threadIdx.x;
    const uint32_t k = p.kind[i];
    const uint32_t r = p.rows[i].rollout_id;
    const uint32_t seq = p.rows[i].seq_len;
    if (k == kDecode) {
        const uint32_t *src = p.table + ((size_t)r * p.kv_heads + g) * p.table_stride;
        uint32_t *dst = p.btab + ((size_t)i * p.kv_heads + g) * p.table_stride;
        for (uint32_t e = lane; e < p.table_stride; e += 64)
            dst[e] = src[e];
    }
    if (g == 0 && lane == 0) {
        const bool dec = k == kDecode;
        p.ctx[i] = dec ? seq : 0u;
        p.pos[i] = dec ? seq : 0xFFFFFFFFu;
        p.rseed[i] = dec ? (p.seeds ? p.seeds[r] : (uint64_t)r) : 0ull;
        p.rstep[i] = dec ? (uint64_t)seq : 0ull;
        if (p.row_rollout)
            p.row_rollout[i] = dec ? r : 0xFFFFFFFFu;
    }
}

// One wave: the hw_worker_sim rule for the decoded token, completions in row order.
__global__ __launch_bounds__(64) void ring_publish_kernel(RingParams p)
{
    const uint32_t lane = threadIdx.x;
    RingCtl *c = p.ctl;
    uint32_t status = c->status;
    uint32_t dtail = c->dtail;
    // pass 1: how many rows finish, how many decoded
    uint32_t n_done = 0, n_dec = 0;
    for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
        const uint32_t i = i0 + lane;
        uint32_t k = i < p.batch ? p.kind[i] : kFree;
        bool fin = k == kPass;
        if (k == kDecode) {
            const uint32_t s = p.rows[i].seq_len + 1;
            fin = s >= p.rows[i].max_tokens || (s & 31u) == 0u;
        }
        n_done += (uint32_t)__builtin_popcountll(__ballot(fin));
        n_dec += (uint32_t)__builtin_popcountll(__ballot(k == kDecode));
    }
    // room on the completion ring (bounded wait)
    bool room = true;
    if (n_done) {
        uint32_t ok = 1;
        if (lane == 0) {
            uint64_t spin = 0;
            while (dtail - sys_load(&p.dq->head) > HW_RING_SIZE - n_done) {
                if (++spin > p.max_idle) {
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        room = rl_wave_bcast_u32(ok, 0) != 0;
        if (!room)
            status = kDoneqFull;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    }
    // pass 2: apply the rule, write the completions, free finished rows
    uint32_t rank0 = 0;
    for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
        const uint32_t i = i0 + lane;
        const uint32_t k = i < p.batch ? p.kind[i] : kFree;
        hw_desc_t d;
        bool fin = false;
        if (k != kFree) {
            d = p.rows[i];
            fin = k == kPass;
            if (k == kDecode) {
                d.seq_len++;
                if (d.seq_len >= d.max_tokens) {
                    d.flags |= (uint16_t)DESC_FLAG_DONE;
                    fin = true;
                } else if ((d.seq_len & 31u) == 0u) {
                    d.flags |= (uint16_t)DESC_FLAG_NEEDS_REWARD;
                    fin = true;
                }
                p.rows[i] = d;
            }
        }
        const uint64_t fm = __ballot(fin);
        if (fin) {
            const uint32_t rk = rank0 + __builtin_amdgcn_mbcnt_hi((uint32_t)(fm >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)fm, 0));
            if (room) {
                volatile rl_u32x4 *dst = (volatile rl_u32x4 *)&p.dq->desc[(dtail + rk) & HW_RING_MASK];
                rl_u32x4 w[4];
                __builtin_memcpy(w, &d, sizeof(d));
#pragma unroll
                for (int j = 0; j < 4; j++)
                    dst[j] = w[j];
            }
            p.kind[i] = kFree;  // a finished row is freed even when its completion is lost
        }
        rank0 += (uint32_t)__builtin_popcountll(fm);
    }
    if (n_done && room) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        dtail += n_done;
        if (lane == 0)
            sys_store_release(&p.dq->tail, dtail);
    }
    if (lane == 0) {
        c->status = status;
        c->dtail = dtail;
        c->decoded += n_dec;
        c->completions += room ? n_done : 0u;
        c->steps += n_dec || n_done ? 1u : 0u;
        p.stats[0] = c->decoded;
        p.stats[1] = c->completions;
        p.stats[2] = c->steps;
        p.stats[3] = status;
    }
}

// ---- host side -------------------------------------------------------------

struct RingWs {
    size_t ctl, rows, kind, btab, ctx, pos, rseed, rstep, attn, samp, total;
    size_t attn_bytes, samp_bytes;
};

size_t up256(size_t x) { return (x + 255) / 256 * 256; }

rl_attn_decode_args_t attn_of(const rl_ring_step_args_t *a, void *ws, size_t ws_bytes)
{
    rl_attn_decode_args_t t = {};
    t.arena_base = a->arena_base;
    t.arena_bytes = a->arena_bytes;
    t.layout = a->layout;
    t.block_table = (const uint32_t *)1;  // placeholders for the workspace query; set per launch
    t.table_stride = a->table_stride;
    t.batch = a->batch;
    t.q_heads = a->q_heads;
    t.kv_heads = a->kv_heads;
    t.dtype = a->dtype;
    t.ctx_lens = (const uint32_t *)1;
    t.max_ctx = a->max_ctx;
    t.grid_waves = 0;
    t.scale = a->scale;
    t.q = a->q;
    t.out = a->attn_out;
    t.out_f32 = nullptr;
    t.workspace = ws;
    t.workspace_bytes = ws_bytes;
    return t;
}

rl_sample_args_t samp_of(const rl_ring_step_args_t *a)
{
    rl_sample_args_t s = {};
    s.logits = a->logits;
    s.rows = a->batch;
    s.vocab = a->vocab;
    s.row_stride = a->vocab;
    s.greedy = a->greedy;
    s.temperature_all = a->temperature;
    s.top_k_all = a->top_k;
    s.top_p_all = a->top_p;
    s.seed = (const uint64_t *)1;
    s.steps = (const uint64_t *)1;
    s.token_out = a->token_out;
    s.logprob_out = a->logprob_out;
    return s;
}

int ring_validate(const rl_ring_step_args_t *a, const char *who)
{
    if (!a || !a->cmdq || !a->doneq || !a->stop || !a->arena_base || !a->block_table || !a->q || !a->k_new ||
        !a->v_new || !a->logits || !a->attn_out || !a->token_out || !a->logprob_out || !a->stats) {
        rl_set_error("%s: NULL argument", who);
        return -1;
    }
    if (a->batch == 0 || a->batch > (uint32_t)kMaxBatch) {
        rl_set_error("%s: batch %u not in 1..%d", who, a->batch, kMaxBatch);
        return -1;
    }
    if (a->rollouts == 0 || a->input_slots == 0 || a->output_slots == 0 || a->vocab == 0) {
        rl_set_error("%s: rollouts %u, input_slots %u, output_slots %u, vocab %u must be positive", who,
                     a->rollouts, a->input_slots, a->output_slots, a->vocab);
        return -1;
    }
    if (a->vocab % 4 != 0) {
        rl_set_error("%s: vocab %u is not a multiple of 4", who, a->vocab);
        return -1;
    }
    return 0;
}

int ring_layout(const rl_ring_step_args_t *a, RingWs &w)
{
    const size_t B = a->batch;
    w.ctl = 0;
    w.rows = 256;
    w.kind = w.rows + up256(B * sizeof(hw_desc_t));
    w.btab = w.kind + up256(B * 4);
    w.ctx = w.btab + up256(B * a->kv_heads * (size_t)a->table_stride * 4);
    w.pos = w.ctx + up256(B * 4);
    w.rseed = w.pos + up256(B * 4);
    w.rstep = w.rseed + up256(B * 8);
    w.attn = w.rstep + up256(B * 8);
    rl_attn_decode_args_t t = attn_of(a, nullptr, 0);
    w.attn_bytes = rl_hip_attn_decode_workspace(&t);
    if (w.attn_bytes == 0)
        return -1;
    w.samp = w.attn + up256(w.attn_bytes);
    rl_sample_args_t s = samp_of(a);
    w.samp_bytes = rl_hip_sample_workspace(&s);
    if (w.samp_bytes == 0)
        return -1;
    w.total = w.samp + up256(w.samp_bytes);
    return 0;
}

}  // namespace

extern "C" size_t rl_hip_ring_step_workspace(const rl_ring_step_args_t *a)
{
    if (rl_require_open("rl_hip_ring_step_workspace") || ring_validate(a, "rl_hip_ring_step_workspace"))
        return 0;
    RingWs w;
    if (ring_layout(a, w))
        return 0;
    return w.total;
}

extern "C" int rl_hip_ring_step_enqueue(const rl_ring_step_args_t *a, uint32_t steps, uint64_t first_step)
{
    if (rl_require_open("rl_hip_ring_step_enqueue") || ring_validate(a, "rl_hip_ring_step_enqueue"))
        return -1;
    RingWs w;
    if (ring_layout(a, w))
        return -1;
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_ring_step_enqueue: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    uint8_t *ws = (uint8_t *)a->workspace;
    RingParams p;
    p.cq = a->cmdq;
    p.dq = a->doneq;
    p.stop = a->stop;
    p.max_idle = a->max_idle_polls ? a->max_idle_polls : (1ull << 22);
    p.batch = a->batch;
    p.rollouts = a->rollouts;
    p.kv_heads = a->kv_heads;
    p.table_stride = a->table_stride;
    p.table = a->block_table;
    p.seeds = a->seeds;
    p.ctl = (RingCtl *)(ws + w.ctl);
    p.rows = (hw_desc_t *)(ws + w.rows);
    p.kind = (uint32_t *)(ws + w.kind);
    p.btab = (uint32_t *)(ws + w.btab);
    p.ctx = (uint32_t *)(ws + w.ctx);
    p.pos = (uint32_t *)(ws + w.pos);
    p.rseed = (uint64_t *)(ws + w.rseed);
    p.rstep = (uint64_t *)(ws + w.rstep);
    p.stats = a->stats;

    const size_t B = a->batch;
    const size_t qrow = (size_t)a->q_heads * a->layout.head_dim * 2;
    const size_t kvrow = (size_t)a->kv_heads * a->layout.head_dim * 2;
    for (uint32_t n = 0; n < steps; n++) {
        const uint64_t k = first_step + n;
        const size_t si = k % a->input_slots, so = k % a->output_slots;
        p.row_rollout = a->row_rollout_out ? a->row_rollout_out + so * B : nullptr;
        hipLaunchKernelGGL(ring_poll_kernel, dim3(1), dim3(64), 0, rl_stream(), p);
        if (rl_check_launch("ring_poll_kernel launch"))
            return -1;
        hipLaunchKernelGGL(ring_gather_kernel, dim3(a->kv_heads, a->batch), dim3(64), 0, rl_stream(), p);
        if (rl_check_launch("ring_gather_kernel launch"))
            return -1;
        rl_attn_decode_args_t t = attn_of(a, ws + w.attn, w.attn_bytes);
        t.block_table = p.btab;
        t.ctx_lens = p.ctx;
        t.q = (const uint8_t *)a->q + si * B * qrow;
        t.out = (uint8_t *)a->attn_out + so * B * qrow;
        t.out_f32 = a->attn_out_f32 ? a->attn_out_f32 + so * B * (qrow / 2) : nullptr;
        rl_kv_append_args_t ap = {};
        ap.arena_base = a->arena_base;
        ap.arena_bytes = a->arena_bytes;
        ap.layout = a->layout;
        ap.block_table = p.btab;
        ap.table_stride = a->table_stride;
        ap.batch = a->batch;
        ap.kv_heads = a->kv_heads;
        ap.positions = p.pos;
        ap.cow_src = nullptr;
        ap.k_new = (const uint8_t *)a->k_new + si * B * kvrow;
        ap.v_new = (const uint8_t *)a->v_new + si * B * kvrow;
        if (rl_hip_decode_step(&t, &ap))
            return -1;
        rl_sample_args_t s = samp_of(a);
        s.logits = a->logits + si * B * a->vocab;
        s.seed = p.rseed;
        s.steps = p.rstep;
        s.token_out = a->token_out + so * B;
        s.logprob_out = a->logprob_out + so * B;
        s.workspace = ws + w.samp;
        s.workspace_bytes = w.samp_bytes;
        if (rl_hip_sample(&s))
            return -1;
        hipLaunchKernelGGL(ring_publish_kernel, dim3(1), dim3(64), 0, rl_stream(), p);
        if (rl_check_launch("ring_publish_kernel launch"))
            return -1;
    }
    return 0;
}
