// ring_core.h - the turn of the ring-driven batched step: the publish of the
// step just decoded and the admission of descriptors for the next one, run
// by one wave (ring_step.hip launches it as a kernel between steps; the
// self-scheduled loop in decode_fused.hip calls it inside its persistent
// kernel).
#pragma once

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
// that does not decode: all five written every turn, so that a turn may
// write a fresh set while the previous step still reads another.
__device__ __forceinline__ void set_row_args(const RingParams &p, uint32_t i, bool dec, uint32_t r, uint32_t seq)
{
    p.ctx[i] = dec ? seq : 0u;
    p.pos[i] = dec ? seq : 0xFFFFFFFFu;
    p.rstep[i] = dec ? (uint64_t)seq : 0ull;
    p.rmap[i] = dec ? r : 0u;
    p.rseed[i] = dec ? (p.seeds ? p.seeds[r] : (uint64_t)r) : 0ull;
    if (p.row_rollout)
        p.row_rollout[i] = dec ? r : 0xFFFFFFFFu;
}

// When the completions of a turn become visible. ReleaseNow: at the end of
// the turn (and before an admission wait for the host). A deferring caller
// (kDefer) releases them itself once the step they complete has all its
// results written; ready() waits (bounded) for that, for the one case the
// turn cannot defer: no row active and the host possibly waiting for those
// completions before it submits more.
struct ReleaseNow {
    static constexpr bool kDefer = false;
    __device__ bool ready() const { return true; }
};

struct TurnOut {
    uint32_t status;    // admission status after the turn
    uint32_t pending;   // completions written but not released (deferring callers)
    uint32_t dtail;     // the completion ring tail that releases them
    uint32_t released;  // the turn stored the completion ring tail (every completion so far is visible)
};

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
// Run by one wave (lane = threadIdx.x % 64 of that wave); s_free is LDS of
// kMaxBatch entries. Returns (in every lane) how many rows the turn leaves
// held - decoding next step, or a finished descriptor still to be pushed -
// and the admission status (and, for deferring callers, the completions left
// to release) in *out when given.
template <class Rel = ReleaseNow>
__device__ uint32_t ring_turn(const RingParams &p, uint32_t do_publish, uint32_t do_poll, uint16_t *s_free,
                              TurnOut *out = nullptr, const Rel &rel = Rel())
{
    const uint32_t lane = threadIdx.x & 63;
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
    bool released = false;
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
        } else if (k == kPass) {
            set_row_args(p, i, false, 0u, 0u);  // held for a publish (turns that do not publish)
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
                if (dq_pending && rel.ready()) {
                    // the host may wait for these completions before it submits more
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
                    if (lane == 0)
                        sys_store(&p.dq->tail, dtail);
                    dq_pending = false;
                    released = true;
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
    const bool release_dq = dq_pending && !Rel::kDefer;
    released |= release_dq;
    if (release_dq || head != head0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        if (lane == 0) {
            if (release_dq)
                sys_store(&p.dq->tail, dtail);
            if (head != head0)
                sys_store(&p.cq->head, head);
        }
    }

    // ---- rows left free decode nothing next step --------------------------------
    for (uint32_t j = taken + lane; j < nfree; j += 64)
        set_row_args(p, s_free[j], false, 0u, 0u);
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
    if (out) {
        out->status = status;
        out->pending = dq_pending && Rel::kDefer ? 1u : 0u;
        out->dtail = dtail;
        out->released = released ? 1u : 0u;
    }
    return active;
}

// ---- host side -------------------------------------------------------------

// The ring step's workspace: the control record at ctl (the self-scheduled
// loop's sync words at ctl + kLoopSyncOff), the row table and the rows' step
// arguments, the fused step's workspace at step; then two more sets of step
// arguments and step workspaces (set[i]: rmap, ctx, pos, rseed, rstep and
// step), which the self-scheduled loop rotates with the first (the launched
// pipeline uses the first only).
struct RingWs {
    size_t ctl, rows, kind, rmap, ctx, pos, rseed, rstep, step;
    struct Set {
        size_t rmap, ctx, pos, rseed, rstep, step;
    } set[2];
    size_t total;
    size_t step_bytes;
};
constexpr size_t kLoopSyncOff = 128;  // past the 40-byte RingCtl, before the rows at 256


inline size_t up256(size_t x) { return (x + 255) / 256 * 256; }

inline rl_attn_decode_args_t attn_of(const rl_ring_step_args_t *a, void *ws, size_t ws_bytes)
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

inline rl_sample_args_t samp_of(const rl_ring_step_args_t *a)
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

inline int ring_validate(const rl_ring_step_args_t *a, const char *who)
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

inline int ring_layout(const rl_ring_step_args_t *a, RingWs &w)
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
    size_t o = w.step + up256(w.step_bytes);
    for (RingWs::Set &x : w.set) {
        x.rmap = o;
        x.ctx = x.rmap + up256(B * 4);
        x.pos = x.ctx + up256(B * 4);
        x.rseed = x.pos + up256(B * 4);
        x.rstep = x.rseed + up256(B * 8);
        x.step = x.rstep + up256(B * 8);
        o = x.step + up256(w.step_bytes);
    }
    w.total = o;
    return 0;
}

// The turn's arguments over the workspace of layout w (the per-step output
// slot's row_rollout is set by the caller).
inline RingParams ring_params_of(const rl_ring_step_args_t *a, uint8_t *ws, const RingWs &w)
{
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
    p.row_rollout = nullptr;
    p.stats = a->stats;
    return p;
}

}  // namespace
