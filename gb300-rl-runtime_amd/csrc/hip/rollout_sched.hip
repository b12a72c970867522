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
//          generated tokens equal to the group's target at the same position
//          - and write their RolloutDone records in parallel, slot s at
//          done-ring position tail + (retiring slots below s), so the ring
//          holds them in slot order; after a barrier thread 0 publishes the
//          new tail with one system-scope release (coherent host memory) and
//          the slots are freed;
//  admit   the free slots (after retirement) are ranked in slot order;
//          threads read up to that many requests from the ring in parallel,
//          thread 0 stops at the end marker (request_id UINT64_MAX) or a bad
//          id and publishes the new head, and the i-th request goes to the
//          i-th free slot - the lowest free slot first, as in the reference,
//          whose seeding of the slot fields is kept. Unlike the reference, a
//          request is never consumed without a free slot, so none is dropped;
//  prepare every slot writes the next step's arguments: attention context and
//          append position (prompt tokens + generated tokens), sampler
//          temperature / top-k / top-p / seed / step (temperature 0 for an
//          idle slot: the cheap greedy path), and an admitted slot copies its
//          request's block-table rows.
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

__device__ __forceinline__ void sys_store_release(volatile uint32_t *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A packed 34-byte request (2-byte aligned in the ring) read as 17 halves.
__device__ RolloutRequest read_request(const RolloutRequest *src)
{
    union {
        RolloutRequest r;
        uint16_t h[17];
    } u;
    const volatile uint16_t *s = (const volatile uint16_t *)src;
#pragma unroll
    for (int i = 0; i < 17; i++)
        u.h[i] = s[i];
    return u.r;
}

// Exclusive prefix of v over the workgroup in thread order; total in `total`.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t &total, uint32_t *s_w)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t incl = rl_wave_incl_scan_u32(v);
    if (lane == 63)
        s_w[wave] = incl;
    __syncthreads();
    uint32_t base = 0, t = 0;
#pragma unroll
    for (int w = 0; w < kSlots / 64; w++) {
        base += w < wave ? s_w[w] : 0u;
        t += s_w[w];
    }
    __syncthreads();
    total = t;
    return base + incl - v;
}

__global__ __launch_bounds__(kSlots) void rollout_schedule_kernel(rl_rollout_sched_args_t p)
{
    __shared__ uint32_t s_w[kSlots / 64];
    __shared__ uint32_t s_ctl[4];
    __shared__ uint32_t s_admit[kSlots];           // request index admitted into the slot this launch, or ~0
    __shared__ RolloutRequest s_req[kSlots];       // requests read from the ring this launch, in ring order
    const uint32_t s = threadIdx.x;
    const int lane = s & 63, wave = s >> 6;
    GpuRolloutSlot *slot = &p.state->slots[s];
    const uint32_t row_entries = p.kv_heads * p.table_stride;
    const uint32_t status0 = p.counters[3];

    // ---- commit the last step's token ------------------------------------
    uint32_t active = slot->active;
    if (p.sampled && active && p.slot_pos[s] != 0xFFFFFFFFu) {
        const uint32_t req = slot->request_id;
        const uint32_t t = slot->tokens_generated;
        if (req < p.requests && t < p.gen_stride)
            p.gen_tokens[(size_t)req * p.gen_stride + t] = p.sampled[s];
        slot->tokens_generated = t + 1;
    }

    // ---- retire: reward, then the dones in slot order -------------------------
    const bool retire = status0 == kOk && active && slot->tokens_generated >= slot->max_tokens;
    float reward = 0.f;
    if (retire) {
        const uint32_t req = slot->request_id;
        uint32_t count = 0;
        if (req < p.requests) {
            const uint32_t *tok = p.gen_tokens + (size_t)req * p.gen_stride;
            const uint32_t *tgt = p.targets + (size_t)(req / p.group_size) * p.target_len;
            const uint32_t n = min(min(slot->tokens_generated, p.gen_stride), p.target_len);
            for (uint32_t i = 0; i < n; i++)
                count += tok[i] == tgt[i] ? 1u : 0u;
        }
        reward = (float)(count & 0xFFu) / 255.0f;
    }
    uint32_t n_ret;
    const uint32_t rank = block_excl_scan(retire ? 1u : 0u, n_ret, s_w);
    DoneRing *dr = p.done_ring;
    if (s == 0) {
        uint32_t status = status0;
        const uint32_t dtail = n_ret ? sys_load(&dr->prod.tail) : 0u;
        uint64_t spin = 0;
        while (n_ret && status == kOk && dtail - sys_load(&dr->cons.head) > (uint32_t)REQUEST_RING_SIZE - n_ret) {
            if (++spin > p.max_spin)
                status = kDoneFull;
            else
                __builtin_amdgcn_s_sleep(8);
        }
        s_ctl[0] = dtail;
        s_ctl[1] = status;
    }
    __syncthreads();
    const uint32_t dtail = s_ctl[0];
    const bool pushed = retire && s_ctl[1] == kOk;
    if (pushed) {
        volatile uint32_t *dst = (volatile uint32_t *)&dr->slots[(dtail + rank) & (REQUEST_RING_SIZE - 1)];
        const uint32_t req = slot->request_id;
        dst[0] = req;  // request_id (the slot keeps its low 32 bits, as in the reference)
        dst[1] = 0;
        dst[2] = s;    // rollout_id = slot
        dst[3] = slot->tokens_generated;
        dst[4] = __float_as_uint(reward);
        dst[5] = 0;    // status
        if (req < p.requests)
            p.rewards[req] = reward;
        slot->active = 0;
    }
    const uint64_t freed = __ballot(pushed);  // wave w owns bitmap word w
    if (lane == 0 && freed)
        p.state->bitmap[wave] &= ~freed;
    __syncthreads();  // every record is written before the tail moves
    if (s == 0 && s_ctl[1] == kOk && n_ret) {
        sys_store_release(&dr->prod.tail, dtail + n_ret);
        p.counters[0] += n_ret;
    }

    // ---- admit: requests in ring order into the free slots in slot order ------
    const bool is_free = s_ctl[1] == kOk && p.counters[2] == 0 &&
                         ((p.state->bitmap[wave] >> lane) & 1ull) == 0;
    uint32_t n_free;
    const uint32_t frank = block_excl_scan(is_free ? 1u : 0u, n_free, s_w);
    RequestRing *rr = p.req_ring;
    if (s == 0) {
        uint32_t head = 0, n_try = 0;
        if (n_free) {
            head = sys_load(&rr->cons.head);
            n_try = min(n_free, sys_load(&rr->prod.tail) - head);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        }
        s_ctl[2] = head;
        s_ctl[3] = n_try;
    }
    __syncthreads();
    const uint32_t head = s_ctl[2], n_try = s_ctl[3];
    if (s < n_try)
        s_req[s] = read_request(&rr->slots[(head + s) & (REQUEST_RING_SIZE - 1)]);
    __syncthreads();
    if (s == 0) {
        uint32_t status = s_ctl[1], n_adm = 0, used = 0;
        for (; used < n_try; used++) {
            const RolloutRequest &q = s_req[used];
            if (q.request_id == ~0ull) {
                p.counters[2] = 1;
                used++;
                break;
            }
            if ((uint32_t)(q.request_id & 0xFFFFFFFFu) >= p.requests) {
                status = kBadRequest;
                used++;
                break;
            }
            n_adm++;
        }
        if (used)
            sys_store_release(&rr->cons.head, head + used);
        p.counters[1] += n_adm;
        p.counters[3] = status;
        s_ctl[3] = n_adm;
    }
    __syncthreads();
    const uint32_t n_adm = s_ctl[3];
    const bool admit = is_free && frank < n_adm;
    s_admit[s] = 0xFFFFFFFFu;
    if (admit) {
        const RolloutRequest &q = s_req[frank];
        const uint32_t rid = (uint32_t)(q.request_id & 0xFFFFFFFFu);
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
        s_admit[s] = rid;
    }
    const uint64_t taken = __ballot(admit);
    if (lane == 0 && taken)
        p.state->bitmap[wave] |= taken;
    __syncthreads();

    // ---- block-table rows of the slots admitted now ---------------------------
    for (uint32_t i = 0; i < (uint32_t)kSlots; i++) {
        const uint32_t rid = s_admit[i];
        if (rid == 0xFFFFFFFFu)
            continue;
        const uint32_t *src = p.req_table + (size_t)rid * row_entries;
        uint32_t *dst = p.slot_table + (size_t)i * row_entries;
        for (uint32_t e = s; e < row_entries; e += kSlots)
            dst[e] = src[e];
    }

    // ---- the next step's arguments ------------------------------------------------
    active = slot->active;
    if (active) {
        const uint32_t rid = slot->request_id;
        const uint32_t ctx = p.prompt_len[rid] + slot->tokens_generated;
        p.slot_ctx[s] = ctx;
        p.slot_pos[s] = ctx;
        p.slot_temp[s] = slot->temperature;
        p.slot_topk[s] = slot->top_k;
        p.slot_topp[s] = slot->top_p;
        p.slot_seed[s] = slot->rng_state[0];
        p.slot_step[s] = slot->tokens_generated;
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
