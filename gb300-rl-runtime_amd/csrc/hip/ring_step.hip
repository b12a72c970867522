// ring_step.hip - the batched decode step driven through the hw_desc rings.
//
// The reference's device worker takes one descriptor at a time on one SM
// (cu/worker.cu:66-131) and its CPU model applies the hw_worker_sim rule per
// descriptor (src/hw_worker_sim.c:23-59). Here up to `batch` DECODE
// descriptors share one decode step that spreads over every compute unit,
// in a stream-ordered pipeline the host enqueues ahead of time. Per step:
//
//  turn     one wave (ring_turn_kernel). First the publish of the step just
//           decoded: the hw_worker_sim rule for its token on every active
//           row (seq_len++, DONE at max_tokens, NEEDS_REWARD at a multiple of
//           32, else the row stays for the next step), the finished
//           descriptors pushed to the completion ring in row order (bounded
//           wait for room) and their rows freed. Then the admission: the
//           command ring (coherent host memory, system-scope loads) drained
//           into the free rows, lowest row first, in ring order: DECODE
//           descriptors with seq_len < max_tokens decode, those at
//           max_tokens pass through unchanged, other opcodes are dropped,
//           STOP ends admission. It waits (bounded) only while no row is
//           active; once rows are active it takes what the ring holds and
//           goes. Last, every row's step arguments: its rollout (the
//           block-table row the step reads), context (= seq_len), append
//           position, Philox seed and counter. The three ring indexes and
//           the stop flag it needs are read in one round trip, and both
//           ring releases share one fence.
//  step     rl_hip_decode_sample_step over the batch rows with the
//           rollout-ordered block table read through the row map: one launch
//           streams the paged GQA attention's tiles beside the sampling of
//           the step's logits (an input of the step, not the attention's
//           output), a second merges the split rows and appends the K/V
//           token. Shapes outside the fused kernel take rl_hip_decode_step
//           and rl_hip_sample.
//
// A call of `steps` steps launches steps + 1 turns: the last one only
// publishes. Each kernel boundary makes the previous kernel's writes visible
// on every XCD, which an in-kernel hand-off between workgroups would have to
// buy with L2 write-backs and invalidations. Waits are bounded: the
// admission gives up after max_idle_polls empty polls (status 1), the publish
// after as many polls of a full completion ring (status 3); a STOP, the host
// stop flag, an idle limit or a bad rollout id end admission while active
// rows finish.
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
    const uint64_t *seeds;      // [rollouts] or NULL (seed = rollout id)
    RingCtl *ctl;
    hw_desc_t *rows;            // [batch]
    uint32_t *kind;             // [batch]
    uint32_t *rmap;             // [batch] rollout of each row (the block-table row the step reads)
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

__device__ __forceinline__ void sys_store(volatile uint32_t *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kMaxBatch = 1024;

__device__ __forceinline__ uint32_t lanes_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// Step arguments of a row that decodes seq_len next (rollout r), or of a row
// that does not decode.
__device__ __forceinline__ void set_row_args(const RingParams &p, uint32_t i, bool dec, uint32_t r, uint32_t seq)
{
    p.ctx[i] = dec ? seq : 0u;
    p.pos[i] = dec ? seq : 0xFFFFFFFFu;
    p.rstep[i] = dec ? (uint64_t)seq : 0ull;
    if (p.row_rollout)
        p.row_rollout[i] = dec ? r : 0xFFFFFFFFu;
}

// One wave, between two decode steps: the publish of the step just decoded
// (the hw_worker_sim rule for its token, completions in row order, finished
// rows freed), then the admission of ring descriptors into the free rows for
// the next step. Every row's step arguments are written where the row is
// updated: continuing rows in the publish pass, new rows at admission, rows
// left free at the end. The producer's tail, the consumer's head and the
// stop flag are read together in one round trip; ring records move as
// relaxed system-scope 8-byte accesses issued back to back; the completion
// ring's tail and the command ring's head are released together behind one
// fence at the end - or the completions first, when the admission has to
// wait for the host.
__global__ __launch_bounds__(64) void ring_turn_kernel(RingParams p, uint32_t do_publish, uint32_t do_poll)
{
    __shared__ uint16_t s_free[kMaxBatch];  // free rows, ascending
    const uint32_t lane = threadIdx.x;
    RingCtl *c = p.ctl;
    uint32_t status = c->status, head = c->head, dtail = c->dtail;
    if (!c->init) {
        const volatile uint32_t *ia = lane == 0 ? &p.cq->head : &p.dq->tail;
        const uint32_t iv = lane < 2 ? sys_load(ia) : 0u;
        head = rl_wave_bcast_u32(iv, 0);
        dtail = rl_wave_bcast_u32(iv, 1);
    }
    const uint32_t head0 = head;
    // the first 64 rows, loaded before the ring indexes so that the two
    // round trips overlap
    const uint32_t k_first = lane < p.batch ? p.kind[lane] : kFree;
    const hw_desc_t d_first = p.rows[lane < p.batch ? lane : 0];
    // the command ring's tail, the completion ring's head and the stop flag
    const volatile uint32_t *ra = lane == 0 ? &p.cq->tail : lane == 1 ? &p.dq->head : p.stop;
    const uint32_t rv = lane < 3 ? sys_load(ra) : 0u;
    const uint32_t cq_tail = rl_wave_bcast_u32(rv, 0);
    const uint32_t dq_head = rl_wave_bcast_u32(rv, 1);
    const uint32_t stop0 = rl_wave_bcast_u32(rv, 2);

    // ---- room on the completion ring -----------------------------------------
    // A whole batch of completions fits (the usual case): no count needed.
    // Otherwise count the rows that finish and wait (bounded) for their room.
    bool room = true;
    if (do_publish && HW_RING_SIZE - (dtail - dq_head) < p.batch) {
        uint32_t need = 0;
        for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
            const uint32_t i = i0 + lane;
            const uint32_t k = i < p.batch ? p.kind[i] : kFree;
            const uint32_t s1 = i < p.batch ? p.rows[i].seq_len + 1 : 0u;
            const uint32_t mt = i < p.batch ? p.rows[i].max_tokens : 0u;
            const bool fin = k == kPass || (k == kDecode && (s1 >= mt || (s1 & 31u) == 0u));
            need += (uint32_t)__builtin_popcountll(__ballot(fin));
        }
        if (need) {
            uint32_t ok = 1;
            if (lane == 0) {
                uint64_t spin = 0;
                uint32_t h = dq_head;
                while (dtail - h > HW_RING_SIZE - need) {
                    if (++spin > p.max_idle) {
                        ok = 0;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                    h = sys_load(&p.dq->head);
                }
            }
            room = rl_wave_bcast_u32(ok, 0) != 0;
            if (!room)
                status = kDoneqFull;
        }
    }
    // Every access to the rings' host memory is a system-scope atomic, which
    // bypasses the caches, and each one is issued after the index it depends
    // on has returned: the completions are written after the consumer's head
    // was read, the descriptors read after the producer's tail. No cache
    // needs invalidating for that, so the acquire sides are wavefront-scope
    // fences (the order of this wave's own accesses).
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- publish: the rule, the completions, the free-row list ---------------
    uint32_t nfree = 0, n_done = 0, n_dec = 0;
    for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
        const uint32_t i = i0 + lane;
        const bool valid = i < p.batch;
        const uint32_t k = i0 == 0 ? k_first : valid ? p.kind[i] : kFree;
        hw_desc_t d = i0 == 0 ? d_first : p.rows[valid ? i : 0];
        bool fin = false;
        if (do_publish && k != kFree) {
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
            if (room) {
                uint64_t w[8];
                __builtin_memcpy(w, &d, sizeof(d));
                rl_sys_store_64B(&p.dq->desc[(dtail + n_done + lanes_below(fm)) & HW_RING_MASK], w);
                p.kind[i] = kFree;
            } else {
                // no room: the finished descriptor stays in its row as a
                // pass-through, which a later turn's publish pushes
                p.kind[i] = kPass;
                set_row_args(p, i, false, 0u, 0u);
            }
        } else if (k == kDecode) {
            set_row_args(p, i, true, d.rollout_id, d.seq_len);  // the row decodes again
        }
        n_done += (uint32_t)__builtin_popcountll(fm);
        n_dec += do_publish ? (uint32_t)__builtin_popcountll(__ballot(k == kDecode)) : 0u;
        const bool f = valid && (k == kFree || (fin && room));
        const uint64_t m = __ballot(f);
        if (f)
            s_free[nfree + lanes_below(m)] = (uint16_t)i;
        nfree += (uint32_t)__builtin_popcountll(m);
    }
    bool dq_pending = false;
    if (n_done && room) {
        dtail += n_done;
        dq_pending = true;
    }
    rl_wave_lds_fence();

    // ---- admission -----------------------------------------------------------
    uint32_t active = p.batch - nfree, taken = 0;
    if (do_poll) {
        uint64_t idle = 0;
        bool fresh = true;  // cq_tail and stop0 were read at entry
        while (status == kRunning && taken < nfree) {
            const uint32_t tail = fresh ? cq_tail : rl_wave_bcast_u32(lane == 0 ? sys_load(&p.cq->tail) : 0u, 0);
            const uint32_t avail = tail - head;
            if (avail == 0) {
                if (active > 0)
                    break;  // rows to decode: go with them
                if (dq_pending) {
                    // the host may wait for these completions before it submits more
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
                    if (lane == 0)
                        sys_store(&p.dq->tail, dtail);
                    dq_pending = false;
                }
                const uint32_t stop = fresh ? stop0 : rl_wave_bcast_u32(lane == 0 ? sys_load(p.stop) : 0u, 0);
                fresh = false;
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
            fresh = false;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const uint32_t take = min(min(avail, 64u), nfree - taken);
            hw_desc_t d;
            const bool in = lane < take;
            if (in) {
                uint64_t w[8];
                rl_sys_load_64B(&p.cq->desc[(head + lane) & HW_RING_MASK], w);
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
                const uint32_t row = s_free[taken + lanes_below(um)];
                const bool dec = d.seq_len < d.max_tokens;
                p.rows[row] = d;
                p.kind[row] = dec ? kDecode : kPass;
                p.rmap[row] = dec ? d.rollout_id : 0u;
                p.rseed[row] = dec ? (p.seeds ? p.seeds[d.rollout_id] : (uint64_t)d.rollout_id) : 0ull;
                set_row_args(p, row, dec, d.rollout_id, d.seq_len);
            }
            const uint32_t n = (uint32_t)__builtin_popcountll(um);
            taken += n;
            active += n;
            head += consumed;
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
    }

    // ---- releases: the completions, then the consumed descriptors ------------
    if (dq_pending || head != head0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        if (lane == 0) {
            if (dq_pending)
                sys_store(&p.dq->tail, dtail);
            if (head != head0)
                sys_store(&p.cq->head, head);
        }
    }

    // ---- rows left free decode nothing next step --------------------------------
    for (uint32_t j = taken + lane; j < nfree; j += 64) {
        const uint32_t i = s_free[j];
        p.rmap[i] = 0u;
        set_row_args(p, i, false, 0u, 0u);
    }
    if (lane == 0) {
        c->init = 1;
        c->status = status;
        c->head = head;
        c->dtail = dtail;
        if (do_publish) {
            c->decoded += n_dec;
            c->completions += room ? n_done : 0u;
            c->steps += n_dec || n_done ? 1u : 0u;
        }
        p.stats[0] = c->decoded;
        p.stats[1] = c->completions;
        p.stats[2] = c->steps;
        p.stats[3] = status;
    }
}

// ---- host side -------------------------------------------------------------

struct RingWs {
    size_t ctl, rows, kind, rmap, ctx, pos, rseed, rstep, step, total;
    size_t step_bytes;
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
    w.rmap = w.kind + up256(B * 4);
    w.ctx = w.rmap + up256(B * 4);
    w.pos = w.ctx + up256(B * 4);
    w.rseed = w.pos + up256(B * 4);
    w.rstep = w.rseed + up256(B * 8);
    w.step = w.rstep + up256(B * 8);
    rl_attn_decode_args_t t = attn_of(a, nullptr, 0);
    rl_sample_args_t s = samp_of(a);
    w.step_bytes = rl_hip_decode_sample_step_workspace(&t, &s);
    if (w.step_bytes == 0)
        return -1;
    w.total = w.step + up256(w.step_bytes);
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
    p.seeds = a->seeds;
    p.ctl = (RingCtl *)(ws + w.ctl);
    p.rows = (hw_desc_t *)(ws + w.rows);
    p.kind = (uint32_t *)(ws + w.kind);
    p.rmap = (uint32_t *)(ws + w.rmap);
    p.ctx = (uint32_t *)(ws + w.ctx);
    p.pos = (uint32_t *)(ws + w.pos);
    p.rseed = (uint64_t *)(ws + w.rseed);
    p.rstep = (uint64_t *)(ws + w.rstep);
    p.stats = a->stats;

    const size_t B = a->batch;
    const size_t qrow = (size_t)a->q_heads * a->layout.head_dim * 2;
    const size_t kvrow = (size_t)a->kv_heads * a->layout.head_dim * 2;
    if (steps == 0)
        return 0;
    for (uint32_t n = 0; n < steps; n++) {
        const uint64_t k = first_step + n;
        const size_t si = k % a->input_slots, so = k % a->output_slots;
        p.row_rollout = a->row_rollout_out ? a->row_rollout_out + so * B : nullptr;
        // publish the previous step of this call (if any), admit for this one
        hipLaunchKernelGGL(ring_turn_kernel, dim3(1), dim3(64), 0, rl_stream(), p, n > 0 ? 1u : 0u, 1u);
        if (rl_check_launch("ring_turn_kernel launch"))
            return -1;
        rl_attn_decode_args_t t = attn_of(a, nullptr, 0);
        t.block_table = a->block_table;
        t.ctx_lens = p.ctx;
        t.q = (const uint8_t *)a->q + si * B * qrow;
        t.out = (uint8_t *)a->attn_out + so * B * qrow;
        t.out_f32 = a->attn_out_f32 ? a->attn_out_f32 + so * B * (qrow / 2) : nullptr;
        rl_kv_append_args_t ap = {};
        ap.arena_base = a->arena_base;
        ap.arena_bytes = a->arena_bytes;
        ap.layout = a->layout;
        ap.block_table = a->block_table;
        ap.table_stride = a->table_stride;
        ap.batch = a->batch;
        ap.kv_heads = a->kv_heads;
        ap.positions = p.pos;
        ap.cow_src = nullptr;
        ap.k_new = (const uint8_t *)a->k_new + si * B * kvrow;
        ap.v_new = (const uint8_t *)a->v_new + si * B * kvrow;
        rl_sample_args_t s = samp_of(a);
        s.logits = a->logits + si * B * a->vocab;
        s.seed = p.rseed;
        s.steps = p.rstep;
        s.draw_ids = p.rmap;  // the draw follows the rollout, not the row it was admitted into
        s.token_out = a->token_out + so * B;
        s.logprob_out = a->logprob_out + so * B;
        // batch row i reads the block-table row of the rollout it holds
        if (rl_decode_sample_step_mapped(&t, &ap, &s, p.rmap, ws + w.step, w.step_bytes,
                                         "rl_hip_ring_step_enqueue"))
            return -1;
    }
    // publish the last step
    p.row_rollout = nullptr;
    hipLaunchKernelGGL(ring_turn_kernel, dim3(1), dim3(64), 0, rl_stream(), p, 1u, 0u);
    if (rl_check_launch("ring_turn_kernel launch"))
        return -1;
    return 0;
}
