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
//          - and thread 0 pushes their RolloutDone records in slot order to
//          the done ring (coherent host memory, system-scope release), then
//          frees the slots;
//  admit   thread 0 consumes requests while a slot is free, each into the
//          lowest free slot (slot fields seeded as in the reference). Unlike
//          the reference, a request is never consumed without a free slot,
//          so none is dropped. request_id UINT64_MAX marks the end;
//  prepare every slot writes the next step's arguments: attention context and
//          append position (prompt tokens + generated tokens), sampler
//          temperature / top-k / top-p / seed / step (temperature 0 for an
//          idle slot: the cheap greedy path), and an admitted slot copies its
//          request's block-table rows.
// Waits on the done ring are bounded by max_spin polls (status 3).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "request.h"
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

__global__ __launch_bounds__(kSlots) void rollout_schedule_kernel(rl_rollout_sched_args_t p)
{
    __shared__ uint32_t s_retire[kSlots];
    __shared__ float s_reward[kSlots];
    __shared__ uint32_t s_admit[kSlots];  // request index admitted into the slot this launch, or ~0
    const uint32_t s = threadIdx.x;
    GpuRolloutSlot *slot = &p.state->slots[s];
    const uint32_t row_entries = p.kv_heads * p.table_stride;

    // ---- commit the last step's token ------------------------------------
    uint32_t active = slot->active;
    if (p.sampled && active && p.slot_pos[s] != 0xFFFFFFFFu) {
        const uint32_t req = slot->request_id;
        const uint32_t t = slot->tokens_generated;
        if (req < p.requests && t < p.gen_stride)
            p.gen_tokens[(size_t)req * p.gen_stride + t] = p.sampled[s];
        slot->tokens_generated = t + 1;
    }

    // ---- retire ----------------------------------------------------------------
    bool retire = false;
    if (active && slot->tokens_generated >= slot->max_tokens) {
        retire = true;
        const uint32_t req = slot->request_id;
        uint32_t count = 0;
        if (req < p.requests) {
            const uint32_t *tok = p.gen_tokens + (size_t)req * p.gen_stride;
            const uint32_t *tgt = p.targets + (size_t)(req / p.group_size) * p.target_len;
            const uint32_t n = min(min(slot->tokens_generated, p.gen_stride), p.target_len);
            for (uint32_t i = 0; i < n; i++)
                count += tok[i] == tgt[i] ? 1u : 0u;
        }
        s_reward[s] = (float)(count & 0xFFu) / 255.0f;
    }
    s_retire[s] = retire ? 1u : 0u;
    s_admit[s] = 0xFFFFFFFFu;
    __syncthreads();

    if (s == 0) {
        uint32_t status = p.counters[3];
        // dones, in slot order
        DoneRing *dr = p.done_ring;
        uint32_t dtail = sys_load(&dr->prod.tail);
        for (uint32_t i = 0; i < (uint32_t)kSlots && status == kOk; i++) {
            if (!s_retire[i])
                continue;
            GpuRolloutSlot *rs = &p.state->slots[i];
            uint64_t spin = 0;
            while (dtail - sys_load(&dr->cons.head) >= (uint32_t)REQUEST_RING_SIZE) {
                if (++spin > p.max_spin) {
                    status = kDoneFull;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
            if (status != kOk)
                break;
            volatile uint32_t *dst = (volatile uint32_t *)&dr->slots[dtail & (REQUEST_RING_SIZE - 1)];
            const uint32_t req = rs->request_id;
            dst[0] = req;  // request_id (low 32 bits kept by the slot, as in the reference)
            dst[1] = 0;
            dst[2] = i;    // rollout_id = slot
            dst[3] = rs->tokens_generated;
            dst[4] = __float_as_uint(s_reward[i]);
            dst[5] = 0;    // status
            dtail++;
            sys_store_release(&dr->prod.tail, dtail);
            if (req < p.requests)
                p.rewards[req] = s_reward[i];
            rs->active = 0;
            p.state->bitmap[i / 64] &= ~(1ull << (i % 64));
            p.counters[0]++;
        }
        // admissions
        RequestRing *rr = p.req_ring;
        uint32_t head = sys_load(&rr->cons.head);
        while (status == kOk && p.counters[2] == 0) {
            int free_slot = -1;
            for (int w = 0; w < kSlots / 64 && free_slot < 0; w++) {
                const uint64_t bits = ~p.state->bitmap[w];
                if (bits)
                    free_slot = w * 64 + __ffsll((long long)bits) - 1;
            }
            if (free_slot < 0)
                break;
            if (sys_load(&rr->prod.tail) == head)
                break;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
            const RolloutRequest req = read_request(&rr->slots[head & (REQUEST_RING_SIZE - 1)]);
            head++;
            sys_store_release(&rr->cons.head, head);
            if (req.request_id == ~0ull) {
                p.counters[2] = 1;
                break;
            }
            const uint32_t rid = (uint32_t)(req.request_id & 0xFFFFFFFFu);
            if (rid >= p.requests) {
                status = kBadRequest;
                break;
            }
            GpuRolloutSlot *rs = &p.state->slots[free_slot];
            rs->active = 1;
            rs->request_id = rid;
            rs->tokens_generated = 0;
            rs->max_tokens = req.max_tokens;
            rs->kv_blocks = req.kv_blocks;
            rs->rng_state[0] = req.rng_seed;
            rs->rng_state[1] = req.rng_seed ^ 0x9e3779b97f4a7c15ull;
            rs->rng_state[2] = (req.rng_seed << 17) ^ 0x3c6ef372fe94f82aull;
            rs->rng_state[3] = ~req.rng_seed;
            rs->temperature = req.temperature;
            rs->top_k = req.top_k;
            rs->top_p = req.top_p;
            p.state->bitmap[free_slot / 64] |= 1ull << (free_slot % 64);
            s_admit[free_slot] = rid;
            p.counters[1]++;
        }
        p.counters[3] = status;
    }
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
