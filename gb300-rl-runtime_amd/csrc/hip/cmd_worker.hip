// cmd_worker.hip - the persistent gfx950 worker on the v0.2 rings: 32-byte
// Descriptors in from a CommandRing, 32-byte Completions out to a
// CompletionRing, both in fine-grained coherent host memory.
//
// Replaces decode_worker / process_descriptor (cu/worker.cu:25-131: one warp
// per SM, lane 0 consumes one descriptor at a time, runs
// attention_decode_step_fixed128 and pushes the completion) with one
// persistent workgroup (16 wave64s) per ring pair - the single consumer of its
// command ring and the single producer of its completion ring, so the SPSC
// contract of ring.h / completion.h holds on the device side:
//
//  poll    lane 0 of wave 0 reads the producer's tail with system-scope loads
//          (the stop flag only while the ring is empty, on every 16th empty
//          poll: each idle worker's loads cross PCIe, and with one worker per
//          compute unit a stop read on every poll slowed the busy ring's
//          round trip from 8.4 to 44 us); after the acquire the
//          whole window of descriptors already committed - up to 32, the
//          decode_batch window (src/decode_batch.c:3-51) - is read with one
//          16-byte load per lane, and the head is released once. The tail
//          and the completion ring's head are read again while each window
//          decodes, so the next poll and the room check rarely wait.
//  decode  wave w takes descriptors w, w + 16, ... of the window: the fixed128
//          step of the reference (cu/attention_decode.cu:60-204) - one head,
//          d128, fp16 K/V of arena block kv_block_offset (K plane, V plane at
//          +8 KiB, 32 tokens), seq_len = num_kv_blocks clamped to [1, 32]
//          ("seq_len" is what the reference passes there), q from slot
//          output_token_offset & (io_slots - 1) of the q buffer or the
//          reference's synthesized query, fp32 softmax(q K^T / sqrt(128)) V to
//          the o buffer, token = the lowest index of the output's maximum,
//          cycles = tiles * 128 * 24. Scores: lane l takes token l % 32 and
//          half l / 32 of its K row (one 128-byte line, 16-byte loads), the
//          halves add across the wave, one max and one sum for the softmax;
//          the output: lane l owns dims 2l and 2l + 1, the weights broadcast
//          from the token lanes.
//  publish wave 0 writes the window's completions {seq_id, token_id,
//          kv_block_offset, reward_cookie, cycles} in descriptor order with
//          one 16-byte store per lane and release-stores tail + n at system
//          scope. A descriptor with seq_id == UINT64_MAX is consumed and ends
//          the worker without a completion, as in the reference; the ones
//          before it in its window are completed first.
//  exit    also on the host's stop flag, after max_idle_polls empty polls, or
//          when the completion ring stays full for as long (stats status).
//  trace   optional: wave 0 appends 20-byte trace records (trace.h) to the
//          worker's own TraceRing in coherent host memory - DESC_CONSUMED per
//          descriptor once its window is read, COMPLETION_POSTED per
//          completion before the tail release - stamped with s_memrealtime
//          (100 MHz) and keyed {low 32 bits of seq_id, output_token_offset};
//          one 32-bit word per lane, then a release store of the ring head.
//  stamps  optional: lane 0 of wave 0 writes s_memrealtime when a poll finds
//          a new tail and just before a window's completions are released,
//          to stamps[g][0] and [1] in coherent host memory, for the host's
//          unloaded-latency measurement.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "completion.h"
#include "descriptor.h"
#include "ring.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"
#include "sample.h"
#include "trace.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kWindow = 32;          // descriptors per poll at most (the decode_batch window)
constexpr uint32_t kD = 128;              // fixed128 head dim
constexpr uint32_t kTokens = 32;          // tokens per fixed128 block
constexpr uint32_t kRowBytes = kD * 2;    // fp16
constexpr uint32_t kBlockBytes = 2 * kTokens * kRowBytes;  // 16 KiB: K plane, V plane
constexpr uint64_t kDefaultIdlePolls = 1ull << 22;

enum : uint32_t { kStatusStopped = 0, kStatusIdle = 1, kStatusCompFull = 3 };

struct CmdParams {
    CommandRing *const *rings;
    CompletionRing *const *comp_rings;
    const volatile uint32_t *stop;
    uint64_t max_idle_polls;
    const uint8_t *arena;
    uint64_t arena_blocks;
    const SampleState *sample_state;
    const uint16_t *q;
    float *o;
    uint32_t io_mask;
    uint64_t *stats;
    TraceRing *trace;
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

// Appends the records {tsc, type, low 32 bits of seq_id, output_token_offset}
// of descriptors d[0..n) at the ring's head (wave 0; the worker is the ring's
// only producer), one 32-bit word per lane, and release-stores the new head.
__device__ void trace_append(TraceRing *tr, uint64_t &thead, const Descriptor *d, uint32_t n, uint32_t type,
                             int lane)
{
    const uint64_t tsc = __builtin_amdgcn_s_memrealtime();
    volatile uint32_t *words = (volatile uint32_t *)tr->entries;
    for (uint32_t w = (uint32_t)lane; w < 5u * n; w += 64u) {
        const uint32_t i = w / 5u, f = w - 5u * i;
        const uint32_t v = f == 0 ? (uint32_t)tsc
                         : f == 1 ? (uint32_t)(tsc >> 32)
                         : f == 2 ? type
                         : f == 3 ? (uint32_t)d[i].seq_id
                                  : d[i].output_token_offset;
        words[((thead + i) & (TRACE_CAPACITY - 1)) * 5u + f] = v;
    }
    thead += n;
    if (lane == 0)
        __hip_atomic_store((uint64_t *)&tr->head, thead, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ float wave_sum(float v)
{
    v = rl_row_sum(v);
    return (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))) +
           (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48)));
}

// The reference's query when no q buffer is given
// (decode_synth_query_component, cu/attention_decode.cu:16-28).
__device__ __forceinline__ float synth_query(const Descriptor &d, const SampleState *st, uint32_t idx)
{
    uint64_t seed = d.seq_id ^ d.reward_cookie ^ ((uint64_t)(idx + 1u) * 0x9e3779b97f4a7c15ull);
    if (st)
        seed ^= st->rng_state[idx & 3u];
    const uint32_t bits = (uint32_t)(seed ^ (seed >> 32));
    const int centered = (int)(bits & 0xFFu) - 127;
    return (float)centered / 127.0f;
}

__device__ __forceinline__ float wave_max(float v)
{
    v = rl_row_max(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}

// One fixed128 decode step by one wave (qs: this wave's 128-float LDS slot,
// vs: its 8 KiB slot for the V plane). Returns the completion record's token
// and cycle fields.
__device__ void fixed128_step(const CmdParams &p, const Descriptor &d, RL_LDS float *qs, RL_LDS uint8_t *vs, int lane,
                              uint32_t &token, uint64_t &cycles)
{
    const uint32_t seq = d.num_kv_blocks == 0 ? 1u : (d.num_kv_blocks > kTokens ? kTokens : d.num_kv_blocks);
    const uint32_t slot = d.output_token_offset & p.io_mask;
    const bool bad = d.kv_block_offset >= p.arena_blocks;
    const uint8_t *blk = p.arena + (uint64_t)(bad ? 0u : d.kv_block_offset) * kBlockBytes;
    const uint32_t t = (uint32_t)lane & (kTokens - 1);   // this lane's token
    const uint32_t h = (uint32_t)lane / kTokens;         // and half of its K row

    // every load issued before the first use: the V plane straight to LDS
    // (eight 1 KiB copies), then the lane's K half row (8 x 16 B)
    const uint8_t *vp = blk + kTokens * kRowBytes;
#pragma unroll
    for (int i = 0; i < 8; i++)
        rl_g2lds_16_off(vp, (uint32_t)(i * 1024 + lane * 16), vs + i * 1024);
    rl_u32x4 kq[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        kq[i] = *(const RL_GLOBAL rl_u32x4 *)(blk + t * kRowBytes + h * (kRowBytes / 2) + i * 16);
    float q0, q1;
    if (p.q) {
        const uint32_t qw = *(const RL_GLOBAL uint32_t *)(p.q + (size_t)slot * kD + 2u * lane);
        rl_unpack2<1>(qw, q0, q1);
    } else {
        q0 = synth_query(d, p.sample_state, 2u * lane);
        q1 = synth_query(d, p.sample_state, 2u * lane + 1u);
    }
    qs[2 * lane] = q0;
    qs[2 * lane + 1] = q1;
    rl_wave_lds_fence();

    // q . k_t over this half, then the other half's partial
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const rl_f32x4 qa = *(RL_LDS const rl_f32x4 *)(qs + h * 64 + 8 * i);
        const rl_f32x4 qb = *(RL_LDS const rl_f32x4 *)(qs + h * 64 + 8 * i + 4);
        float k0, k1, k2, k3, k4, k5, k6, k7;
        rl_unpack2<1>(kq[i].x, k0, k1);
        rl_unpack2<1>(kq[i].y, k2, k3);
        rl_unpack2<1>(kq[i].z, k4, k5);
        rl_unpack2<1>(kq[i].w, k6, k7);
        dot = fmaf(qa.x, k0, dot);
        dot = fmaf(qa.y, k1, dot);
        dot = fmaf(qa.z, k2, dot);
        dot = fmaf(qa.w, k3, dot);
        dot = fmaf(qb.x, k4, dot);
        dot = fmaf(qb.y, k5, dot);
        dot = fmaf(qb.z, k6, dot);
        dot = fmaf(qb.w, k7, dot);
        // two query reads in flight at a time: hoisting all sixteen costs
        // 64 VGPRs, which the 16-wave workgroup does not have
        __builtin_amdgcn_sched_barrier(0);
    }
    dot += __shfl_xor(dot, 32);
    const float scale = 0.08838834764831845f;  // 1 / sqrt(128)
    const float sc = t < seq ? dot * scale : -INFINITY;
    const float m = wave_max(sc);
    const float e = (h == 0 && t < seq) ? __expf(sc - m) : 0.f;
    const float l = wave_sum(e);
    rl_wait_vmcnt<0>();  // the V copies have landed (issued first, they retire first)
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (uint32_t tt = 0; tt < kTokens; tt++) {
        const float et = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), (int)tt));
        float v0, v1;
        rl_unpack2<1>(*(RL_LDS const uint32_t *)(vs + tt * kRowBytes + lane * 4u), v0, v1);
        o0 = fmaf(et, v0, o0);
        o1 = fmaf(et, v1, o1);
    }
    o0 /= l;
    o1 /= l;
    if (bad) {
        o0 = __builtin_nanf("");
        o1 = o0;
    }
    if (p.o) {
        float *orow = p.o + (size_t)slot * kD;
        orow[2u * lane] = o0;
        orow[2u * lane + 1u] = o1;
    }
    // lowest index of the maximum (the pair's first element wins a tie)
    float best = o1 > o0 ? o1 : o0;
    uint32_t bidx = o1 > o0 ? 2u * lane + 1u : 2u * lane;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float ob = __shfl_xor(best, off);
        const uint32_t oi = __shfl_xor(bidx, off);
        if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bidx = oi;
        }
    }
    token = bad ? 0u : bidx;
    cycles = (uint64_t)((seq + 15u) / 16u) * kD * 24u;
}

__global__ __launch_bounds__(kThreads) void cmd_worker_kernel(CmdParams p)
{
    __shared__ __attribute__((aligned(16))) Descriptor s_desc[kWindow];
    __shared__ __attribute__((aligned(16))) Completion s_comp[kWindow];
    __shared__ __attribute__((aligned(16))) float s_q[kWaves][kD];  // each wave's query
    __shared__ __attribute__((aligned(1024))) uint8_t s_v[kWaves][kTokens * kRowBytes];  // each wave's V plane
    __shared__ uint32_t s_ctl[2];  // descriptors to run, exit flag

    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    CommandRing *ring = p.rings[blockIdx.x];
    CompletionRing *cr = p.comp_rings[blockIdx.x];

    uint64_t descs = 0, completions = 0, windows = 0;
    uint32_t status = kStatusStopped;
    uint32_t head = 0, ctail = 0;  // lane 0 of wave 0: this worker owns cons.head and the completion tail
    // lane 0 of wave 0: the producer's tail and the host's completion head as
    // last read; both are read again while the window decodes, so the next
    // poll and the room check usually find their answer already there (an
    // older value only means fewer descriptors or less room, then re-read)
    uint32_t tail_seen = 0, chead_seen = 0;
    if (tid == 0) {
        head = sys_load(&ring->cons.head);
        ctail = sys_load(&cr->prod.tail);
        tail_seen = head;
        chead_seen = sys_load(&cr->cons.head);
    }
    TraceRing *tr = p.trace ? p.trace + blockIdx.x : nullptr;
    uint64_t thead = 0;            // wave 0, uniform: the trace ring's head
    if (tr && wave == 0)
        thead = __hip_atomic_load((uint64_t *)&tr->head, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);

    for (;;) {
        // ---- the committed window at the head (wave 0) ------------------------
        if (wave == 0) {
            uint32_t avail = 0, ctl = 0;
            if (lane == 0) {
                uint64_t idle = 0;
                avail = tail_seen - head;
                for (; avail == 0;) {
                    avail = sys_load(&ring->prod.tail) - head;
                    if (avail != 0)
                        break;
                    if ((idle & 15) == 15 && sys_load(p.stop) != 0) {
                        ctl = 1;
                        break;
                    }
                    if (++idle > p.max_idle_polls) {
                        ctl = 1;
                        status = kStatusIdle;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
                if (avail != 0 && p.stamps)
                    p.stamps[(size_t)blockIdx.x * 2] = __builtin_amdgcn_s_memrealtime();
            }
            avail = rl_wave_bcast_u32(avail, 0);
            ctl = rl_wave_bcast_u32(ctl, 0);
            uint32_t n = 0;
            if (!ctl) {
                // The slots are read with system-scope (volatile) loads, which
                // bypass the caches, after the tail that covers them has
                // returned: no cache needs invalidating, so the acquire is a
                // wavefront-scope fence.
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const uint32_t h = rl_wave_bcast_u32(head, 0);
                // the window ends where the ring wraps or after kWindow descriptors
                n = min(min(avail, kWindow), RING_SIZE - (h & (RING_SIZE - 1)));
                if ((uint32_t)lane < 2 * n) {
                    const volatile rl_u32x4 *src = (const volatile rl_u32x4 *)&ring->slots[h & (RING_SIZE - 1)];
                    ((rl_u32x4 *)s_desc)[lane] = src[lane];
                }
                rl_wave_lds_fence();
                // a shutdown sentinel ends the window (it is consumed, not run)
                uint32_t run = n;
                for (uint32_t i = 0; i < n; i++)
                    if (s_desc[i].seq_id == ~0ull) {
                        run = i;
                        ctl = 1;
                        n = i + 1;
                        break;
                    }
                if (lane == 0) {
                    head += n;
                    sys_store_release(&ring->cons.head, head);
                }
                n = run;
                if (tr && n)
                    trace_append(tr, thead, s_desc, n, TRACE_DESC_CONSUMED, lane);
            }
            if (lane == 0) {
                s_ctl[0] = n;
                s_ctl[1] = ctl;
            }
        }
        __syncthreads();
        const uint32_t n = s_ctl[0];
        const uint32_t stop_now = s_ctl[1];

        if (tid == 0 && n && !stop_now) {
            tail_seen = sys_load(&ring->prod.tail);
            chead_seen = sys_load(&cr->cons.head);
        }

        // ---- decode: one descriptor per wave at a time ---------------------------
        for (uint32_t i = wave; i < n; i += kWaves) {
            const Descriptor d = s_desc[i];
            uint32_t token;
            uint64_t cycles;
            fixed128_step(p, d, (RL_LDS float *)s_q[wave], (RL_LDS uint8_t *)s_v[wave], lane, token, cycles);
            if (lane == 0) {
                Completion c;
                c.seq_id = d.seq_id;
                c.token_id = token;
                c.kv_block_offset = d.kv_block_offset;
                c.reward_cookie = d.reward_cookie;
                c.cycles_taken = cycles;
                s_comp[i] = c;
            }
        }
        __syncthreads();

        // ---- publish the window's completions (wave 0), bounded wait while full --
        uint32_t fail = 0;
        if (wave == 0 && n) {
            uint32_t room = 0;
            if (lane == 0) {
                uint64_t idle = 0;
                for (;;) {
                    if (ctail - chead_seen <= (uint32_t)COMP_RING_SIZE - n) {
                        room = 1;
                        break;
                    }
                    chead_seen = sys_load(&cr->cons.head);
                    if (ctail - chead_seen <= (uint32_t)COMP_RING_SIZE - n) {
                        room = 1;
                        break;
                    }
                    if (sys_load(p.stop) != 0)
                        break;
                    if (++idle > p.max_idle_polls) {
                        status = kStatusCompFull;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
            }
            if (rl_wave_bcast_u32(room, 0)) {
                if (tr)
                    trace_append(tr, thead, s_desc, n, TRACE_COMPLETION_POSTED, lane);
                const uint32_t t = rl_wave_bcast_u32(ctail, 0);
                // two lanes per record; records may wrap around the ring
                if ((uint32_t)lane < 2 * n) {
                    const uint32_t rec = (uint32_t)lane / 2;
                    volatile rl_u32x4 *dst = (volatile rl_u32x4 *)&cr->slots[(t + rec) & (COMP_RING_SIZE - 1)];
                    dst[lane & 1] = ((const rl_u32x4 *)s_comp)[lane];
                }
                if (lane == 0) {
                    ctail += n;
                    if (p.stamps)
                        p.stamps[(size_t)blockIdx.x * 2 + 1] = __builtin_amdgcn_s_memrealtime();
                    sys_store_release(&cr->prod.tail, ctail);
                }
            } else {
                fail = 1;
            }
            if (lane == 0)
                s_ctl[1] = fail;
        }
        if (n) {
            __syncthreads();
            fail = s_ctl[1];
        }
        descs += n;
        if (!fail && n) {
            completions += n;
            windows++;
        }
        if (stop_now || fail)
            break;
        __syncthreads();  // s_desc / s_ctl are rewritten by the next poll
    }
    if (tid == 0) {
        uint64_t *st = p.stats + (size_t)blockIdx.x * 4;
        st[0] = descs;
        st[1] = completions;
        st[2] = windows;
        st[3] = status;
    }
}

}  // namespace

extern "C" int rl_hip_cmd_worker_launch(const rl_cmd_worker_args_t *a)
{
    if (rl_require_open("rl_hip_cmd_worker_launch"))
        return -1;
    if (!a || !a->rings || !a->comp_rings || !a->stop || !a->stats || !a->arena_base) {
        rl_set_error("rl_hip_cmd_worker_launch: NULL argument");
        return -1;
    }
    if (a->groups == 0) {
        rl_set_error("rl_hip_cmd_worker_launch: groups 0");
        return -1;
    }
    // Every worker must be resident at once: a worker that waits for a free
    // compute unit leaves its ring pair unserved until another worker exits.
    int per_cu = 0;
    if (rl_check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, cmd_worker_kernel, kThreads, 0),
                     "hipOccupancyMaxActiveBlocksPerMultiprocessor(cmd_worker_kernel)"))
        return -1;
    const uint64_t resident = (uint64_t)(per_cu > 0 ? per_cu : 0) * rl_cu_count();
    if (a->groups > resident) {
        rl_set_error("rl_hip_cmd_worker_launch: %u groups exceed the %llu workers the device holds at once "
                     "(%d per compute unit x %u compute units)",
                     a->groups, (unsigned long long)resident, per_cu, rl_cu_count());
        return -1;
    }
    if (a->io_slots & (a->io_slots - 1)) {
        rl_set_error("rl_hip_cmd_worker_launch: io_slots %u is not a power of two", a->io_slots);
        return -1;
    }
    if (a->arena_bytes < kBlockBytes) {
        rl_set_error("rl_hip_cmd_worker_launch: arena of %llu bytes holds no 16 KiB block",
                     (unsigned long long)a->arena_bytes);
        return -1;
    }
    CmdParams p;
    p.rings = a->rings;
    p.comp_rings = a->comp_rings;
    p.stop = a->stop;
    p.max_idle_polls = a->max_idle_polls ? a->max_idle_polls : kDefaultIdlePolls;
    p.arena = (const uint8_t *)a->arena_base;
    p.arena_blocks = a->arena_bytes / kBlockBytes;
    p.sample_state = a->sample_state;
    p.q = (const uint16_t *)a->q_buffer;
    p.o = a->o_buffer;
    p.io_mask = a->io_slots ? a->io_slots - 1 : 0;
    p.stats = a->stats;
    p.trace = a->trace;
    p.stamps = a->stamps;
    hipLaunchKernelGGL(cmd_worker_kernel, dim3(a->groups), dim3(kThreads), 0, rl_stream(), p);
    return rl_check_launch("cmd_worker_kernel launch");
}
