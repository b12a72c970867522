// hw_worker.hip - the persistent gfx950 worker on the hw_desc rings.
//
// Replaces the CPU worker hw_worker_sim_run (src/hw_worker_sim.c:23-59) and
// the reference's per-SM device worker (cu/worker.cu:66-131) with one
// persistent workgroup (8 wave64s) per ring pair. Each workgroup is the
// single consumer of its command ring and the single producer of its
// completion ring, both in fine-grained coherent host memory, so the SPSC
// contract of hw_ring.h holds on the device side too:
//
//  poll    thread 0 reads the producer's tail with system-scope loads
//          (s_sleep between empty polls, the host's stop flag on every 16th
//          of them), acquires, copies the 64-byte descriptor and
//          release-stores head + 1. Every load of an idle worker crosses
//          PCIe: with one worker per compute unit, reading the stop flag on
//          every poll as well loaded the link enough to slow the one busy
//          ring's round trip from 6.7 to 39 us.
//  decode  for DECODE, the control rule of hw_worker_sim - while seq_len <
//          max_tokens: one decode step, seq_len++, stop at max_tokens (DONE)
//          or at a multiple of 32 (NEEDS_REWARD) - with a real step for every
//          token: paged attention of the rollout over its seq_len tokens (the
//          batched kernel's MFMA tile stream, eight waves, split rows merged in
//          the workgroup), the greedy token and its logprob over the step's
//          logits, and the append of the step's K/V token at position seq_len.
//  publish thread 0 writes the updated descriptor into the completion ring
//          and release-stores tail + 1 at system scope.
//  stamps  optional: thread 0 writes the GPU's 100 MHz clock (s_memrealtime)
//          when a poll first sees a new descriptor and just before the
//          completion's tail is released, to stamps[g][0] and [1] in
//          coherent host memory (the release orders both before the tail),
//          for the host's unloaded-latency measurement.
//  exit    on STOP (no completion, like the simulator), when the host sets
//          *stop, or - so that no wave can spin forever - after
//          max_idle_polls consecutive empty polls or a completion ring that
//          stays full for as long; the reason is left in the stats.
// Other opcodes are dropped without a completion, as in the simulator.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_core.h"
#include "hw_desc.h"
#include "hw_ring.h"
#include "kv_layout.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr int kWorkerWavesMax = 8;  // a step's tiles are shared by up to this many waves
constexpr int kWorkerThreadsMax = kWorkerWavesMax * 64;
constexpr uint64_t kDefaultIdlePolls = 1ull << 22;

enum : uint32_t {
    kStatusStopped = 0,      // STOP descriptor or host stop flag
    kStatusIdle = 1,         // max_idle_polls empty polls in a row
    kStatusInputs = 2,       // more decode steps than the inputs hold, or a rollout id out of range
    kStatusDoneqFull = 3,    // completion ring full for max_idle_polls polls
    kStatusAppend = 4,       // an appended token's block outside the table or the arena
};

struct WorkerParams {
    hw_ring_t *const *cmdq;
    hw_ring_t *const *doneq;
    const volatile uint32_t *stop;
    uint64_t max_idle_polls;
    AttnParams attn;  // arena, table, heads, scale; per-step fields are set per descriptor
    uint32_t rollouts;
    uint32_t max_steps;
    const uint16_t *q;
    const uint16_t *k_new;
    const uint16_t *v_new;
    const float *logits;
    uint32_t vocab;
    float *attn_out;
    uint32_t *token_out;
    float *logprob_out;
    uint64_t *stats;
    float *part;  // [groups][kWorkerWavesMax + kv_heads][G * D + 2 * G]
    uint64_t *stamps;  // coherent host [groups][2] or nullptr
};

__device__ __forceinline__ uint32_t sys_load(const volatile uint32_t *p)
{
    return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void sys_store_release(volatile uint32_t *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// (value desc, index asc) argmax across the wave
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(v, off);
        const uint32_t oi = __shfl_xor(i, off);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
}

__device__ __forceinline__ float wave_sum_f(float v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
        v += __shfl_xor(v, off);
    return v;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kGreedyBatch = 8;  // 16-byte loads in flight per thread

// Folds a batch of n values (at indices idx[j], increasing) into a running
// (best, bidx, z): best the max, bidx the lowest index holding it, z the sum
// of exp(v - best). The batch max comes first, so each value costs one exp
// and no branch.
template <int N>
__device__ __forceinline__ void greedy_fold_batch(const float (&v)[N], const uint32_t (&idx)[N], float &best,
                                                  uint32_t &bidx, float &z)
{
    float bm = v[0];
    uint32_t bi = idx[0];
#pragma unroll
    for (int j = 1; j < N; j++) {
        const bool gt = v[j] > bm;  // strict: the earlier (lower) index keeps a tie
        bm = gt ? v[j] : bm;
        bi = gt ? idx[j] : bi;
    }
    const bool take = bm > best;
    const float nb = take ? bm : best;
    bidx = take ? bi : bidx;
    if (nb != -INFINITY) {
        float zz = best == -INFINITY ? 0.f : z * __builtin_amdgcn_exp2f((best - nb) * kLog2e);
#pragma unroll
        for (int j = 0; j < N; j++)
            zz += v[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((v[j] - nb) * kLog2e);
        z = zz;
    }
    best = nb;
}

// One thread's share of a greedy scan over lg[0, n): 16-byte loads of
// consecutive quads (quad q at thread q % threads) when the row is 16-byte
// aligned, kGreedyBatch of them issued before any is used (a quad past the
// end re-reads the last whole quad and is masked, so no load is
// conditional); scalar loads for the remainder or an unaligned row.
template <uint32_t T>
__device__ void greedy_scan(const float *lg, uint32_t n, uint32_t tid, float &best, uint32_t &bidx, float &z)
{
    uint32_t done = 0;
    const uint32_t quads = n / 4;
    if (((uintptr_t)lg & 15u) == 0 && quads > 0) {
        const RL_GLOBAL rl_f32x4 *l4 = (const RL_GLOBAL rl_f32x4 *)lg;
        for (uint32_t q0 = 0; q0 < quads; q0 += T * kGreedyBatch) {
            rl_f32x4 r[kGreedyBatch];
#pragma unroll
            for (int j = 0; j < kGreedyBatch; j++)
                r[j] = l4[min(q0 + j * T + tid, quads - 1)];
            float v[4 * kGreedyBatch];
            uint32_t idx[4 * kGreedyBatch];
#pragma unroll
            for (int j = 0; j < kGreedyBatch; j++) {
                const uint32_t q = q0 + j * T + tid;
                const bool in = q < quads;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[4 * j + e] = in ? r[j][e] : -INFINITY;
                    idx[4 * j + e] = q * 4 + e;
                }
            }
            greedy_fold_batch(v, idx, best, bidx, z);
        }
        done = quads * 4;
    }
    for (uint32_t i0 = done; i0 < n; i0 += T * kGreedyBatch) {
        float v[kGreedyBatch];
        uint32_t idx[kGreedyBatch];
#pragma unroll
        for (int j = 0; j < kGreedyBatch; j++) {
            const uint32_t i = i0 + j * T + tid;
            v[j] = lg[min(i, n - 1)];
            v[j] = i < n ? v[j] : -INFINITY;
            idx[j] = i;
        }
        greedy_fold_batch(v, idx, best, bidx, z);
    }
}

// LDS of the worker beside the tile stages: the merge weights and the small
// per-step buffers.
template <int G>
constexpr int worker_fixed_lds()
{
    return kMergeLds * G * 4 + 2048;
}

// Waves of the worker: a decode step's attention is latency-bound (one
// workgroup per ring pair), so its tiles are shared by eight waves when two
// tile stages per wave fit the LDS, else by four.
template <int D, int G, int DT, int TPB>
constexpr int worker_waves()
{
    using C = Cfg<D, G, DT, TPB>;
    return (C::LDS_CU - worker_fixed_lds<G>()) / (kWorkerWavesMax * (C::STAGE + C::QSLOT)) >= 2 ? kWorkerWavesMax
                                                                                                : 4;
}

// Stages of each wave's tile ring: two with eight waves; with four, up to
// four as the LDS and the vmcnt range of the copies allow. Beyond two stages
// the stream's per-stage state is indexed at run time and lives in scratch
// memory, so eight waves of two stages keep the same 16 tiles in flight
// without it.
template <int D, int G, int DT, int TPB>
constexpr int worker_stages()
{
    using C = Cfg<D, G, DT, TPB>;
    constexpr int W = worker_waves<D, G, DT, TPB>();
    constexpr int per = W * (C::STAGE + C::QSLOT);
    int ns = (C::LDS_CU - worker_fixed_lds<G>()) / per;
    const int cap = W == kWorkerWavesMax ? 2 : 4;
    ns = ns > cap ? cap : ns;
    while (ns > 2 && (ns - 1) * C::UNIT_OPS >= 64)
        ns--;
    return ns < 2 ? 2 : ns;
}

template <int D, int G, int DT, int TPB>
__global__ __launch_bounds__(kWorkerThreadsMax) void hw_worker_kernel(WorkerParams wp)
{
    using C = Cfg<D, G, DT, TPB>;
    constexpr int W = worker_waves<D, G, DT, TPB>();
    constexpr uint32_t kThreads = W * 64;
    constexpr int NS = worker_stages<D, G, DT, TPB>();
    constexpr int PART = C::PART;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_st[NS][W * C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_q[W * NS * C::QSLOT];
    __shared__ float s_f[kMergeLds * G];
    __shared__ float s_L[G];
    __shared__ uint32_t s_desc[16];
    __shared__ uint32_t s_out[16];
    __shared__ uint32_t s_ctl;
    __shared__ float s_red[W];
    __shared__ uint32_t s_redi[W];
    __shared__ float s_z[W];

    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t grp = blockIdx.x;
    hw_ring_t *cq = wp.cmdq[grp];
    hw_ring_t *dq = wp.doneq[grp];
    const uint32_t kvh = wp.attn.kv_heads;
    const uint32_t qh = wp.attn.q_heads;

    uint64_t decoded = 0, completions = 0;
    uint32_t steps = 0, status = kStatusStopped;
    // the worker owns cmdq.head and doneq.tail: start from their current values
    uint32_t head = 0, dtail = 0;
    if (tid == 0) {
        head = sys_load(&cq->head);
        dtail = sys_load(&dq->tail);
    }

    RL_LDS uint8_t *st = (RL_LDS uint8_t *)lds_st[0] + wave * C::STAGE;
    RL_LDS uint8_t *qs = (RL_LDS uint8_t *)lds_q + wave * NS * C::QSLOT;

    for (;;) {
        // ---- next descriptor (wave 0), bounded wait -------------------------
        // Lane 0 polls the producer's tail (the stop flag only while the ring
        // is empty, on every 16th empty poll); after the acquire, lanes 0-15 read the 16 dwords of the
        // descriptor in one load instruction, then lane 0 releases the slot.
        if (wave == 0) {
            uint32_t ctl = 0, got = 0;
            if (lane == 0) {
                uint64_t idle = 0;
                for (;;) {
                    if (sys_load(&cq->tail) != head) {
                        got = 1;
                        if (wp.stamps)
                            wp.stamps[(size_t)grp * 2] = __builtin_amdgcn_s_memrealtime();
                        break;
                    }
                    if ((idle & 15) == 15 && sys_load(wp.stop) != 0) {
                        ctl = 1;
                        break;
                    }
                    if (++idle > wp.max_idle_polls) {
                        ctl = 1;
                        status = kStatusIdle;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
            }
            got = rl_wave_bcast_u32(got, 0);
            if (got) {
                // the descriptor's dwords are read with system-scope
                // (volatile) loads, which bypass the caches, after the tail
                // that covers them: no cache needs invalidating
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const uint32_t h = rl_wave_bcast_u32(head, 0);
                if (lane < 16)
                    s_desc[lane] = ((const volatile uint32_t *)&cq->desc[h & HW_RING_MASK])[lane];
                rl_wave_lds_fence();
                if (lane == 0) {
                    head++;
                    sys_store_release(&cq->head, head);
                }
            }
            if (lane == 0)
                s_ctl = ctl;
        }
        __syncthreads();
        if (s_ctl)
            break;
        hw_desc_t d;
        {
            uint32_t *dw = (uint32_t *)&d;
#pragma unroll
            for (int i = 0; i < 16; i++)
                dw[i] = s_desc[i];
        }
        __syncthreads();  // s_desc is rewritten by the next poll
        if (d.opcode == DESC_OP_STOP)
            break;
        if (d.opcode != DESC_OP_DECODE)
            continue;

        // ---- the control rule, one real decode step per token ----------------
        bool fail = false;
        while (d.seq_len < d.max_tokens) {
            if (steps >= wp.max_steps || d.rollout_id >= wp.rollouts) {
                status = kStatusInputs;
                fail = true;
                break;
            }
            const uint32_t r = d.rollout_id;
            const uint32_t pos = d.seq_len;  // tokens in the cache before this step
            const size_t step_row = (size_t)grp * wp.max_steps + steps;

            // attention of rollout r over its pos tokens
            AttnParams a = wp.attn;
            a.batch = 1;
            a.max_ctx = pos;
            a.table = wp.attn.table + (size_t)r * kvh * wp.attn.table_stride;
            a.q = wp.q + step_row * qh * D;
            a.out = nullptr;
            a.out_f32 = wp.attn_out + step_row * qh * D;
            a.part = wp.part + (size_t)grp * (kWorkerWavesMax + kvh) * PART;
            const uint32_t nu = (pos + kTile - 1) / kTile;
            const uint32_t U = kvh * nu;
            if (U == 0) {
                for (uint32_t g = 0; g < kvh; g++)
                    empty_row<D, G, DT, G>(a, 0, g, 0, false, tid, kThreads);
            } else {
                const uint32_t NW = min((uint32_t)W, U);
                if ((uint32_t)wave < NW) {
                    const uint32_t sb = (uint32_t)(((uint64_t)wave * U) / NW);
                    const uint32_t se = (uint32_t)(((uint64_t)(wave + 1) * U) / NW);
                    attn_stream<D, G, DT, TPB, NS>(a, CtxFixed{pos}, wave, sb, se, 0, 0, st, W * C::STAGE, qs, lane);
                }
                __syncthreads();
                for (uint32_t g = 0; g < kvh; g++)
                    merge_row<D, G, DT, kThreads, G>(a, 0, g, 0, g * nu, nu, U, NW, false, tid, s_f, s_L);
            }

            // greedy token (lowest index among maxima) and its logprob: one
            // pass over the logits with kGreedyBatch independent loads in
            // flight per thread and an online log-sum-exp (per-thread running
            // max, sum rescaled when the max grows)
            {
                const float *lg = wp.logits + step_row * wp.vocab;
                float best = -INFINITY, z = 0.f;
                uint32_t bidx = 0xFFFFFFFFu;
                greedy_scan<kThreads>(lg, wp.vocab, tid, best, bidx, z);
                // combine (best, bidx, z) over the workgroup; z is relative to best
                float m = best;
                wave_argmax(m, bidx);
                z = wave_sum_f(best == -INFINITY ? 0.f : z * exp2f((best - m) * kLog2e));
                if (lane == 0) {
                    s_red[wave] = m;
                    s_redi[wave] = bidx;
                    s_z[wave] = z;
                }
                __syncthreads();
                float gm = s_red[0];
                uint32_t mi = s_redi[0];
#pragma unroll
                for (int w = 1; w < W; w++)
                    if (s_red[w] > gm || (s_red[w] == gm && s_redi[w] < mi)) {
                        gm = s_red[w];
                        mi = s_redi[w];
                    }
                if (tid == 0) {
                    float zs = 0.f;
#pragma unroll
                    for (int w = 0; w < W; w++)
                        zs += s_red[w] == -INFINITY ? 0.f : s_z[w] * exp2f((s_red[w] - gm) * kLog2e);
                    const uint32_t tok = mi >= wp.vocab ? 0u : mi;  // no finite maximum: token 0
                    wp.token_out[step_row] = tok;
                    wp.logprob_out[step_row] = lg[tok] - (gm + logf(zs));
                }
                __syncthreads();  // s_red is reused by the next step
            }

            // append the step's K and V token at position pos
            {
                constexpr int CH = D * 2 / 16;  // 16-byte chunks per row
                bool bad = false;
                for (uint32_t t = tid; t < kvh * CH * 2; t += kThreads) {
                    const uint32_t h = t / (CH * 2);
                    const uint32_t c = t % (CH * 2);
                    const bool isv = c >= (uint32_t)CH;
                    const uint32_t cc = isv ? c - CH : c;
                    const uint32_t lb = pos / TPB;
                    if (lb >= a.table_stride) {
                        bad = true;
                        continue;
                    }
                    const uint32_t blk = a.table[(size_t)h * a.table_stride + lb];
                    if (blk >= a.arena_blocks) {
                        bad = true;
                        continue;
                    }
                    const uint16_t *srcp = (isv ? wp.v_new : wp.k_new) + (step_row * kvh + h) * D;
                    uint8_t *dst = (uint8_t *)a.arena + (uint64_t)blk * a.block_bytes + (isv ? TPB * C::RB : 0) +
                                   (pos % TPB) * C::RB;
                    *(rl_u32x4 *)(dst + cc * 16) = *(const rl_u32x4 *)((const uint8_t *)srcp + cc * 16);
                }
                // the next step's copies, issued by the waves of this
                // workgroup, read the appended token: release before the
                // barrier, acquire after it, both at workgroup scope
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                if (__syncthreads_or(bad)) {
                    status = kStatusAppend;
                    fail = true;
                    break;
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            }

            d.seq_len++;
            decoded++;
            steps++;
            if (d.seq_len >= d.max_tokens) {
                d.flags |= (uint16_t)DESC_FLAG_DONE;
                break;
            }
            if ((d.seq_len & 31u) == 0u) {
                d.flags |= (uint16_t)DESC_FLAG_NEEDS_REWARD;
                break;
            }
        }
        if (fail)
            break;

        // ---- publish the completion (wave 0), bounded wait while full --------
        // Lanes 0-15 write the descriptor's 16 dwords with one store
        // instruction; lane 0 then release-stores the new tail.
        if (wave == 0) {
            uint32_t ctl = 1, room = 0;
            if (lane == 0) {
                uint64_t idle = 0;
                for (;;) {
                    if (dtail - sys_load(&dq->head) < HW_RING_SIZE) {
                        room = 1;
                        break;
                    }
                    if (sys_load(wp.stop) != 0)
                        break;
                    if (++idle > wp.max_idle_polls) {
                        status = kStatusDoneqFull;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
            }
            if (rl_wave_bcast_u32(room, 0)) {
                const uint32_t t = rl_wave_bcast_u32(dtail, 0);
                if (lane == 0) {
                    const uint32_t *dw = (const uint32_t *)&d;
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        s_out[i] = dw[i];
                }
                rl_wave_lds_fence();
                if (lane < 16)
                    ((volatile uint32_t *)&dq->desc[t & HW_RING_MASK])[lane] = s_out[lane];
                if (lane == 0) {
                    dtail++;
                    if (wp.stamps)
                        wp.stamps[(size_t)grp * 2 + 1] = __builtin_amdgcn_s_memrealtime();
                    sys_store_release(&dq->tail, dtail);
                }
                ctl = 0;
            }
            if (lane == 0)
                s_ctl = ctl;
        }
        __syncthreads();
        if (s_ctl)
            break;
        completions++;
    }
    if (tid == 0) {
        uint64_t *st = wp.stats + (size_t)grp * 4;
        st[0] = decoded;
        st[1] = completions;
        st[2] = steps;
        st[3] = status;
    }
}

// ---- launcher ------------------------------------------------------------------

size_t part_bytes(const rl_hw_worker_args_t *a)
{
    const uint32_t G = a->q_heads / a->kv_heads;
    return (size_t)a->groups * (kWorkerWavesMax + a->kv_heads) * (G * a->layout.head_dim + 2 * G) * 4;
}

template <int D, int G, int DT, int TPB>
int launch(const WorkerParams &wp, uint32_t groups)
{
    hipLaunchKernelGGL((hw_worker_kernel<D, G, DT, TPB>), dim3(groups), dim3(worker_waves<D, G, DT, TPB>() * 64), 0,
                       rl_stream(), wp);
    return rl_check_launch("hw_worker_kernel launch");
}

template <int D, int G, int DT>
int dispatch_tpb(const WorkerParams &wp, uint32_t groups, uint32_t tpb)
{
    return tpb == 16 ? launch<D, G, DT, 16>(wp, groups) : launch<D, G, DT, 32>(wp, groups);
}

template <int D, int G>
int dispatch_dt(const WorkerParams &wp, uint32_t groups, uint32_t dt, uint32_t tpb)
{
    return dt == RL_DTYPE_BF16 ? dispatch_tpb<D, G, 0>(wp, groups, tpb) : dispatch_tpb<D, G, 1>(wp, groups, tpb);
}

template <int D>
int dispatch_g(const WorkerParams &wp, uint32_t groups, uint32_t G, uint32_t dt, uint32_t tpb)
{
    switch (G) {
    case 1: return dispatch_dt<D, 1>(wp, groups, dt, tpb);
    case 2: return dispatch_dt<D, 2>(wp, groups, dt, tpb);
    case 4: return dispatch_dt<D, 4>(wp, groups, dt, tpb);
    default: return dispatch_dt<D, 8>(wp, groups, dt, tpb);
    }
}

int validate(const rl_hw_worker_args_t *a)
{
    if (!a) {
        rl_set_error("rl_hip_hw_worker: NULL args");
        return -1;
    }
    if (!a->cmdq || !a->doneq || !a->stop || !a->stats) {
        rl_set_error("rl_hip_hw_worker: NULL ring array, stop flag or stats");
        return -1;
    }
    if (a->groups == 0 || a->groups > 65535) {
        rl_set_error("rl_hip_hw_worker: groups %u out of range", a->groups);
        return -1;
    }
    if (kv_layout_check_paged(&a->layout) != 0) {
        rl_set_error("rl_hip_hw_worker: unsupported KV layout (token_count %u, head_dim %u, scalar %u)",
                     a->layout.token_count, a->layout.head_dim, a->layout.scalar_bytes);
        return -1;
    }
    if (a->kv_heads == 0 || a->q_heads % a->kv_heads != 0) {
        rl_set_error("rl_hip_hw_worker: q_heads %u not a multiple of kv_heads %u", a->q_heads, a->kv_heads);
        return -1;
    }
    const uint32_t G = a->q_heads / a->kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) {
        rl_set_error("rl_hip_hw_worker: GQA group %u not in {1,2,4,8}", G);
        return -1;
    }
    if (a->dtype != RL_DTYPE_BF16 && a->dtype != RL_DTYPE_FP16) {
        rl_set_error("rl_hip_hw_worker: dtype %u", a->dtype);
        return -1;
    }
    if (!a->arena_base || a->arena_bytes < a->layout.block_bytes || !a->block_table || a->table_stride == 0) {
        rl_set_error("rl_hip_hw_worker: arena or block table missing");
        return -1;
    }
    if (a->max_steps == 0 || !a->q || !a->k_new || !a->v_new || !a->logits || a->vocab == 0 || !a->attn_out ||
        !a->token_out || !a->logprob_out || a->rollouts == 0) {
        rl_set_error("rl_hip_hw_worker: step inputs or outputs missing");
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" size_t rl_hip_hw_worker_workspace(const rl_hw_worker_args_t *a)
{
    if (validate(a))
        return 0;
    return part_bytes(a);
}

extern "C" int rl_hip_hw_worker_launch(const rl_hw_worker_args_t *a)
{
    if (rl_require_open("rl_hip_hw_worker_launch") || validate(a))
        return -1;
    if (!a->workspace || a->workspace_bytes < part_bytes(a)) {
        rl_set_error("rl_hip_hw_worker_launch: workspace %zu bytes < %zu required", a->workspace_bytes,
                     part_bytes(a));
        return -1;
    }
    if (a->groups > rl_cu_count()) {
        // every worker must be resident at once: each may wait on its rings
        rl_set_error("rl_hip_hw_worker_launch: %u groups exceed the %u compute units", a->groups, rl_cu_count());
        return -1;
    }
    WorkerParams wp;
    wp.cmdq = a->cmdq;
    wp.doneq = a->doneq;
    wp.stop = a->stop;
    wp.max_idle_polls = a->max_idle_polls ? a->max_idle_polls : kDefaultIdlePolls;
    AttnParams &p = wp.attn;
    p.arena = (const uint8_t *)a->arena_base;
    p.block_bytes = a->layout.block_bytes;
    p.arena_blocks = a->arena_bytes / a->layout.block_bytes;
    p.table = a->block_table;
    p.table_stride = a->table_stride;
    p.row_map = nullptr;
    p.ctx = nullptr;
    p.max_ctx = 0;
    p.batch = 1;
    p.q_heads = a->q_heads;
    p.kv_heads = a->kv_heads;
    p.q = nullptr;
    p.out = nullptr;
    p.out_f32 = nullptr;
    const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)a->layout.head_dim);
    p.scale_log2 = scale * 1.4426950408889634f;
    p.nwaves = 4;
    p.part = nullptr;
    p.cum = nullptr;
    wp.rollouts = a->rollouts;
    wp.max_steps = a->max_steps;
    wp.q = (const uint16_t *)a->q;
    wp.k_new = (const uint16_t *)a->k_new;
    wp.v_new = (const uint16_t *)a->v_new;
    wp.logits = a->logits;
    wp.vocab = a->vocab;
    wp.attn_out = a->attn_out;
    wp.token_out = a->token_out;
    wp.logprob_out = a->logprob_out;
    wp.stats = a->stats;
    wp.stamps = a->stamps;
    wp.part = (float *)a->workspace;

    const uint32_t G = a->q_heads / a->kv_heads;
    if (a->layout.head_dim == 128)
        return dispatch_g<128>(wp, a->groups, G, a->dtype, a->layout.token_count);
    return dispatch_g<64>(wp, a->groups, G, a->dtype, a->layout.token_count);
}
