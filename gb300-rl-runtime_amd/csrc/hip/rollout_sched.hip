// rollout_sched.hip - the device rollout scheduler between two decode steps.
//
// Restates rollout_worker (cu/gpu_scheduler.cu:26-83: one thread consumes at
// most one request per iteration, sweeps 256 slots, emits a done and frees
// the slot when tokens_generated >= max_tokens) as one step-synchronous
// kernel of 256 threads, thread s owning slot s of the byte-compatible
// GpuRolloutState. Each launch, between two batched decode steps:
//  commit  a slot that took part in the last step (append position set)
//          records the token sampled for it and counts it;
//  retire  slots with tokens_generated >= max_tokens get their reward - the
//          reference rule (count & 0xFF) / 255 applied to the number of
//          generated tokens equal to the group's target at the same position,
//          counted by whole waves four slots at a time - and write their
//          RolloutDone records in parallel, slot s at done-ring position tail
//          + (retiring slots below s), so the ring holds them in slot order;
//          after a barrier thread 0 publishes the new tail (coherent host
//          memory) and the slots are freed;
//  admit   the free slots (after retirement) are ranked in slot order;
//          threads read up to that many requests from the ring in parallel,
//          the first end marker (request_id UINT64_MAX) or bad id stops the
//          admission (a ballot finds it), thread 0 publishes the new head, and
//          the i-th request goes to the i-th free slot - the lowest free slot
//          first, as in the reference, whose seeding of the slot fields is
//          kept. Unlike the reference, a request is never consumed without a
//          free slot, so none is dropped;
//  prepare every slot writes the next step's arguments: attention context and
//          append position (prompt tokens + generated tokens; none for a slot
//          parked at max_tokens because the done ring had no room), sampler
//          temperature / top-k / top-p / seed / step (temperature 0 for an
//          idle slot: the cheap greedy path), and the admitted slots' rows of
//          the block table are copied from their requests' rows.
// Latency is the whole cost of this kernel, so every device input is loaded
// up front in one batch, the four host-ring indexes a launch needs are read
// together while the rewards are counted, host records are read and written
// with relaxed system-scope accesses that stay in flight together (one fence
// orders them), and work lists are compact: a launch that retires and admits
// nothing touches no host memory and loops over nothing.
// Waits on the done ring are bounded by max_spin polls (status 3).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "request.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr int kSlots = GPU_MAX_ROLLOUTS;
static_assert(kSlots == 256, "one thread per slot");

enum : uint32_t { kOk = 0, kBadRequest = 2, kDoneFull = 3 };

__device__ __forceinline__ uint32_t sys_load(const volatile uint32_t *p)
{
    return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ uint16_t sys_load16(const volatile uint16_t *p)
{
    return __hip_atomic_load((uint16_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void sys_store(volatile uint32_t *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A packed 34-byte request (2-byte aligned in the ring) read as 17 halves.
// Relaxed system-scope loads are all in flight together; volatile loads would
// each wait for the one before, one PCIe round trip apiece.
__device__ RolloutRequest read_request(const RolloutRequest *src)
{
    union {
        RolloutRequest r;
        uint16_t h[17];
    } u;
    const volatile uint16_t *s = (const volatile uint16_t *)src;
#pragma unroll
    for (int i = 0; i < 17; i++)
        u.h[i] = sys_load16(s + i);
    return u.r;
}

constexpr int kWaves = kSlots / 64;
constexpr int kRewardSlots = 4;   // retiring slots a wave counts per round
constexpr int kCopyDepth = 32;    // block-table entries per thread and round

__global__ __launch_bounds__(kSlots) void rollout_schedule_kernel(rl_rollout_sched_args_t p)
{
    __shared__ uint32_t s_w[kWaves];
    __shared__ uint32_t s_stop[kWaves];
    __shared__ uint32_t s_ctl[4];
    __shared__ uint32_t s_rslot[kSlots];     // retiring slots in slot order
    __shared__ uint32_t s_rreq[kSlots];      // ... their request ids
    __shared__ uint32_t s_rlen[kSlots];      // ... the number of generated tokens the reward compares
    __shared__ float s_reward[kSlots];       // ... their rewards
    __shared__ uint32_t s_aslot[kSlots];     // admitted slots in admission order
    __shared__ uint32_t s_arid[kSlots];      // request ids read this launch, in ring order
    __shared__ RolloutRequest s_req[kSlots]; // requests read from the ring this launch, in ring order
    const uint32_t s = threadIdx.x;
    const int lane = s & 63, wave = s >> 6;
    GpuRolloutSlot *slot = &p.state->slots[s];
    const uint32_t row_entries = p.kv_heads * p.table_stride;
    DoneRing *dr = p.done_ring;
    RequestRing *rr = p.req_ring;

    // ---- every device-side input of the launch, loaded together -------------
    const uint32_t cnt_done = p.counters[0], cnt_adm = p.counters[1];
    const uint32_t ended = p.counters[2], status0 = p.counters[3];
    const uint64_t bits = p.state->bitmap[wave];
    const uint32_t active = slot->active;
    const uint32_t req0 = slot->request_id;
    uint32_t t = slot->tokens_generated;
    const uint32_t max_tok = slot->max_tokens;
    const uint64_t seed0 = slot->rng_state[0];
    const float temp0 = slot->temperature;
    const uint32_t topk0 = slot->top_k;
    const float topp0 = slot->top_p;
    const uint32_t pos = p.slot_pos[s];
    const uint32_t tok = p.sampled ? p.sampled[s] : 0u;
    const uint32_t plen0 = p.prompt_len[min(req0, p.requests - 1)];

    // ---- commit the last step's token ------------------------------------
    if (p.sampled && active && pos != 0xFFFFFFFFu) {
        if (req0 < p.requests && t < p.gen_stride)
            p.gen_tokens[(size_t)req0 * p.gen_stride + t] = tok;
        t += 1;
        slot->tokens_generated = t;
    }

    // ---- rank the retiring slots and the slots free after retirement -----------
    // (one scan: retiring count in the low half, free count in the high half)
    const bool retire = status0 == kOk && active && t >= max_tok;
    const bool maybe_free = status0 == kOk && ended == 0 && (((bits >> lane) & 1ull) == 0 || retire);
    const uint32_t v = (retire ? 1u : 0u) | (maybe_free ? 0x10000u : 0u);
    const uint32_t incl = rl_wave_incl_scan_u32(v);
    if (lane == 63)
        s_w[wave] = incl;
    __syncthreads();
    uint32_t ex = incl - v, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        ex += w < wave ? s_w[w] : 0u;
        tot += s_w[w];
    }
    const uint32_t rank = ex & 0xFFFFu, frank = ex >> 16;
    const uint32_t n_ret = tot & 0xFFFFu, n_free = tot >> 16;
    if (retire) {
        s_rslot[rank] = s;
        s_rreq[rank] = req0;
        s_rlen[rank] = req0 < p.requests ? min(min(t, p.gen_stride), p.target_len) : 0u;
    }
    // the host-ring indexes this launch needs, in flight while the rewards are counted
    uint32_t dtail = 0, dhead = 0, rhead = 0, rtail = 0;
    if (s == 0) {
        if (n_ret) {
            dtail = sys_load(&dr->prod.tail);
            dhead = sys_load(&dr->cons.head);
        }
        if (n_free) {
            rhead = sys_load(&rr->cons.head);
            rtail = sys_load(&rr->prod.tail);
        }
    }
    __syncthreads();

    // ---- rewards: (count & 0xFF) / 255 over the generated tokens equal to the
    // group's target; wave w counts retiring slots 4w .. 4w + 3, 4w + 16 .., 256
    // tokens of four slots per round with all their loads in flight ------------
    for (uint32_t j0 = (uint32_t)wave * kRewardSlots; j0 < n_ret; j0 += kWaves * kRewardSlots) {
        const uint32_t *ga[kRewardSlots], *ta[kRewardSlots];
        uint32_t n[kRewardSlots], cnt[kRewardSlots], nmax = 0;
#pragma unroll
        for (int g = 0; g < kRewardSlots; g++) {
            const uint32_t j = j0 + g;
            n[g] = j < n_ret ? s_rlen[j] : 0u;
            const uint32_t rq = j < n_ret ? s_rreq[j] : 0u;
            // a slot with nothing to compare reads element 0 of gen_tokens, masked out
            ga[g] = n[g] ? p.gen_tokens + (size_t)rq * p.gen_stride : p.gen_tokens;
            ta[g] = n[g] ? p.targets + (size_t)(rq / p.group_size) * p.target_len : p.gen_tokens;
            cnt[g] = 0;
            nmax = max(nmax, n[g]);
        }
        for (uint32_t c0 = 0; c0 < nmax; c0 += 256) {
            uint32_t a[kRewardSlots][4], b[kRewardSlots][4];
#pragma unroll
            for (int g = 0; g < kRewardSlots; g++)
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t i = c0 + (uint32_t)u * 64 + (uint32_t)lane;
                    const uint32_t k = i < n[g] ? i : 0u;
                    a[g][u] = ga[g][k];
                    b[g][u] = ta[g][k];
                }
#pragma unroll
            for (int g = 0; g < kRewardSlots; g++)
#pragma unroll
                for (int u = 0; u < 4; u++)
                    cnt[g] += (c0 + (uint32_t)u * 64 + (uint32_t)lane < n[g] && a[g][u] == b[g][u]) ? 1u : 0u;
        }
#pragma unroll
        for (int g = 0; g < kRewardSlots; g++) {
            const uint32_t c = rl_wave_sum_u32(cnt[g]);
            if (lane == 0 && j0 + g < n_ret)
                s_reward[j0 + g] = (float)(c & 0xFFu) / 255.0f;
        }
    }

    // ---- room on the done ring (bounded wait), requests available ------------
    if (s == 0) {
        uint32_t st = status0;
        if (n_ret) {
            uint64_t spin = 0;
            while (dtail - dhead > (uint32_t)REQUEST_RING_SIZE - n_ret) {
                if (++spin > p.max_spin) {
                    st = kDoneFull;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
                dhead = sys_load(&dr->cons.head);
            }
        }
        uint32_t n_try = 0;
        if (n_free && st == kOk) {
            n_try = min(n_free, rtail - rhead);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        }
        s_ctl[0] = dtail;
        s_ctl[1] = st;
        s_ctl[2] = rhead;
        s_ctl[3] = n_try;
    }
    __syncthreads();
    const uint32_t st = s_ctl[1], n_try = s_ctl[3];

    // ---- retire: RolloutDone records in slot order; read the requests ----------
    const bool pushed = retire && st == kOk;
    if (pushed) {
        const uint32_t req = req0;
        const float reward = s_reward[rank];
        volatile uint32_t *dst = (volatile uint32_t *)&dr->slots[(s_ctl[0] + rank) & (REQUEST_RING_SIZE - 1)];
        sys_store(dst + 0, req);  // request_id (the slot keeps its low 32 bits, as in the reference)
        sys_store(dst + 1, 0);
        sys_store(dst + 2, s);    // rollout_id = slot
        sys_store(dst + 3, t);
        sys_store(dst + 4, __float_as_uint(reward));
        sys_store(dst + 5, 0);    // status
        // this wave's records are complete before the barrier, ahead of the tail
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        if (req < p.requests)
            p.rewards[req] = reward;
        slot->active = 0;
    }
    // requests in ring order; the first end marker or bad id stops the admission
    bool stop = false, bad = false;
    if (s < n_try) {
        const RolloutRequest q = read_request(&rr->slots[(s_ctl[2] + s) & (REQUEST_RING_SIZE - 1)]);
        s_req[s] = q;
        s_arid[s] = (uint32_t)(q.request_id & 0xFFFFFFFFu);
        stop = q.request_id == ~0ull || (uint32_t)(q.request_id & 0xFFFFFFFFu) >= p.requests;
        bad = stop && q.request_id != ~0ull;
    }
    const uint64_t sb = __ballot(stop), bb = __ballot(bad);
    if (lane == 0) {
        const uint32_t f = (uint32_t)__builtin_ctzll(sb | (1ull << 63));
        s_stop[wave] = sb ? (((uint32_t)wave * 64 + f) << 1) | (uint32_t)((bb >> f) & 1ull) : 0xFFFFFFFFu;
    }
    __syncthreads();

    // ---- publish, admit: the i-th request into the i-th free slot ---------------
    uint32_t key = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < kWaves; w++)
        key = min(key, s_stop[w]);
    const uint32_t n_adm = key == 0xFFFFFFFFu ? n_try : key >> 1;
    const uint32_t used = key == 0xFFFFFFFFu ? n_try : (key >> 1) + 1;
    if (s == 0) {
        const bool publish = st == kOk && n_ret;
        if (publish || used) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
            if (publish)
                sys_store(&dr->prod.tail, s_ctl[0] + n_ret);
            if (used)
                sys_store(&rr->cons.head, s_ctl[2] + used);
        }
        if (publish)
            p.counters[0] = cnt_done + n_ret;
        p.counters[1] = cnt_adm + n_adm;
        if (key != 0xFFFFFFFFu && !(key & 1u))
            p.counters[2] = 1;
        p.counters[3] = key != 0xFFFFFFFFu && (key & 1u) ? (uint32_t)kBadRequest : st;
    }
    const bool admit = maybe_free && frank < n_adm;
    uint32_t rid = req0, tg = t, maxt = max_tok;
    float temp = temp0, topp = topp0;
    uint32_t topk = topk0;
    uint64_t seed = seed0;
    if (admit) {
        const RolloutRequest &q = s_req[frank];
        rid = (uint32_t)(q.request_id & 0xFFFFFFFFu);
        tg = 0;
        maxt = q.max_tokens;
        temp = q.temperature;
        topk = q.top_k;
        topp = q.top_p;
        seed = q.rng_seed;
        slot->active = 1;
        slot->request_id = rid;
        slot->tokens_generated = 0;
        slot->max_tokens = q.max_tokens;
        slot->kv_blocks = q.kv_blocks;
        slot->rng_state[0] = q.rng_seed;
        slot->rng_state[1] = q.rng_seed ^ 0x9e3779b97f4a7c15ull;
        slot->rng_state[2] = (q.rng_seed << 17) ^ 0x3c6ef372fe94f82aull;
        slot->rng_state[3] = ~q.rng_seed;
        slot->temperature = q.temperature;
        slot->top_k = q.top_k;
        slot->top_p = q.top_p;
        s_aslot[frank] = s;
    }
    const uint64_t freed = __ballot(pushed), taken = __ballot(admit);
    if (lane == 0 && (freed | taken))
        p.state->bitmap[wave] = (bits & ~freed) | taken;

    // ---- block-table rows of the slots admitted now ---------------------------
    if (n_adm) {
        __syncthreads();
        const uint32_t total = n_adm * row_entries;  // < 2^32: row_entries < 2^24
        // entry e belongs to admitted row e / row_entries < 256: the float
        // quotient is within 1e-4 of it, and one step either way corrects it
        const float inv_row = 1.0f / (float)row_entries;
        auto row_of = [&](uint32_t e) {
            uint32_t i = (uint32_t)((float)e * inv_row);
            i -= i * row_entries > e ? 1u : 0u;
            i += (i + 1) * row_entries <= e ? 1u : 0u;
            return i;
        };
        for (uint32_t e0 = s; e0 < total; e0 += kSlots * kCopyDepth) {
            uint32_t val[kCopyDepth], row[kCopyDepth];
#pragma unroll
            for (int u = 0; u < kCopyDepth; u++) {
                const uint32_t e = min(e0 + (uint32_t)u * kSlots, total - 1);
                row[u] = row_of(e);
                val[u] = p.req_table[(size_t)s_arid[row[u]] * row_entries + (e - row[u] * row_entries)];
            }
#pragma unroll
            for (int u = 0; u < kCopyDepth; u++) {
                const uint32_t e = e0 + (uint32_t)u * kSlots;
                if (e < total)
                    p.slot_table[(size_t)s_aslot[row[u]] * row_entries + (e - row[u] * row_entries)] = val[u];
            }
        }
    }

    // ---- the next step's arguments ------------------------------------------------
    // A slot decodes the next step while it holds fewer than max_tokens tokens.
    // One that reached max_tokens and could not be retired (no room on the done
    // ring) stays active but parked: no context, no append position, so it
    // neither grows nor writes past its blocks.
    const bool decodes = (admit || (active && !pushed)) && tg < maxt;
    if (p.slot_request)
        p.slot_request[s] = decodes ? rid : 0xFFFFFFFFu;
    if (decodes) {
        const uint32_t ctx = (admit ? p.prompt_len[rid] : plen0) + tg;
        p.slot_ctx[s] = ctx;
        p.slot_pos[s] = ctx;
        p.slot_temp[s] = temp;
        p.slot_topk[s] = topk;
        p.slot_topp[s] = topp;
        p.slot_seed[s] = seed;
        p.slot_step[s] = tg;
    } else {
        p.slot_ctx[s] = 0;
        p.slot_pos[s] = 0xFFFFFFFFu;
        p.slot_temp[s] = 0.f;
        p.slot_topk[s] = 0;
        p.slot_topp[s] = 1.f;
        p.slot_seed[s] = 0;
        p.slot_step[s] = 0;
    }
}

}  // namespace

extern "C" int rl_hip_rollout_schedule(const rl_rollout_sched_args_t *a)
{
    if (rl_require_open("rl_hip_rollout_schedule"))
        return -1;
    if (!a || !a->req_ring || !a->done_ring || !a->state || !a->prompt_len || !a->req_table || !a->gen_tokens ||
        !a->targets || !a->rewards || !a->slot_table || !a->slot_ctx || !a->slot_pos || !a->slot_temp ||
        !a->slot_topk || !a->slot_topp || !a->slot_seed || !a->slot_step || !a->counters) {
        rl_set_error("rl_hip_rollout_schedule: NULL argument");
        return -1;
    }
    if ((uint64_t)a->kv_heads * a->table_stride >= (1ull << 24)) {
        rl_set_error("rl_hip_rollout_schedule: kv_heads %u x table_stride %u block-table entries per slot "
                     "(at most 2^24 - 1)", a->kv_heads, a->table_stride);
        return -1;
    }
    if (a->requests == 0 || a->group_size == 0 || a->kv_heads == 0 || a->table_stride == 0 || a->gen_stride == 0) {
        rl_set_error("rl_hip_rollout_schedule: requests %u, group_size %u, kv_heads %u, table_stride %u, "
                     "gen_stride %u must be positive",
                     a->requests, a->group_size, a->kv_heads, a->table_stride, a->gen_stride);
        return -1;
    }
    rl_rollout_sched_args_t p = *a;
    if (p.max_spin == 0)
        p.max_spin = 1ull << 22;
    hipLaunchKernelGGL(rollout_schedule_kernel, dim3(1), dim3(kSlots), 0, rl_stream(), p);
    return rl_check_launch("rollout_schedule_kernel launch");
}
