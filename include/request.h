/*
 * request.h - v0.3 request/done rings for the GPU-resident rollout loop.
 *
 * Byte-compatible with the reference (include/request.h:12-150):
 *   RolloutRequest 34 B packed {request_id, max_tokens, kv_blocks,
 *     temperature, top_k, top_p, rng_seed};
 *   RolloutDone 24 B packed {request_id, rollout_id, tokens_generated,
 *     reward, status};
 *   RequestRing = head line @0, tail line @64, slots @128 (34,944 B);
 *   DoneRing = head @0, tail @64, overflow @128, slots @256 (24,832 B);
 *   GpuRolloutSlot 72 B / GpuRolloutState 18,464 B (natural alignment).
 * request_id == UINT64_MAX is the shutdown sentinel. Done push on a full
 * ring bumps `overflow` and returns -1. Empty tests are wrap-safe.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define REQUEST_RING_SIZE 1024
#define GPU_MAX_ROLLOUTS 256

#pragma pack(push, 1)
typedef struct {
    uint64_t request_id;
    uint32_t max_tokens;
    uint32_t kv_blocks;
    float temperature;
    uint16_t top_k;
    float top_p;
    uint64_t rng_seed;
} RolloutRequest;

RL_STATIC_ASSERT(sizeof(RolloutRequest) == 34, "RolloutRequest must be 34 bytes");

typedef struct {
    uint64_t request_id;
    uint32_t rollout_id;
    uint32_t tokens_generated;
    float reward;
    uint32_t status;
} RolloutDone;
#pragma pack(pop)

RL_STATIC_ASSERT(sizeof(RolloutDone) == 24, "RolloutDone must be 24 bytes");

typedef struct __attribute__((packed)) {
    volatile uint32_t head __attribute__((aligned(64)));
    uint8_t pad[60];
} ReqHead;

typedef struct __attribute__((packed)) {
    volatile uint32_t tail __attribute__((aligned(64)));
    uint8_t pad[60];
} ReqTail;

typedef struct __attribute__((packed)) {
    volatile uint32_t value __attribute__((aligned(64)));
    uint8_t pad[60];
} ReqCounter;

typedef struct {
    ReqHead cons __attribute__((aligned(64)));
    ReqTail prod __attribute__((aligned(64)));
    RolloutRequest slots[REQUEST_RING_SIZE] __attribute__((aligned(128)));
} RequestRing;

typedef struct {
    ReqHead cons __attribute__((aligned(64)));
    ReqTail prod __attribute__((aligned(64)));
    ReqCounter overflow __attribute__((aligned(64)));
    RolloutDone slots[REQUEST_RING_SIZE] __attribute__((aligned(128)));
} DoneRing;

RL_STATIC_ASSERT(sizeof(RequestRing) == 34944, "RequestRing size");
RL_STATIC_ASSERT(sizeof(DoneRing) == 24832, "DoneRing size");

typedef struct {
    uint32_t active;
    uint32_t request_id;
    uint32_t tokens_generated;
    uint32_t max_tokens;
    uint32_t kv_blocks;
    uint64_t rng_state[4];
    float temperature;
    uint16_t top_k;
    float top_p;
} GpuRolloutSlot;

typedef struct {
    GpuRolloutSlot slots[GPU_MAX_ROLLOUTS];
    uint64_t bitmap[(GPU_MAX_ROLLOUTS + 63) / 64];
} GpuRolloutState;

RL_STATIC_ASSERT(sizeof(GpuRolloutSlot) == 72, "GpuRolloutSlot size");
RL_STATIC_ASSERT(sizeof(GpuRolloutState) == 18464, "GpuRolloutState size");

/* Host producer: masked slot index, or UINT32_MAX when full. */
static inline uint32_t
req_ring_acquire(RequestRing *r)
{
    const uint32_t h = RL_LOAD_ACQ_U32(&r->cons.head);
    const uint32_t t = RL_LOAD_RLX_U32(&r->prod.tail);
    if ((uint32_t)REQUEST_RING_SIZE - (t - h) < 1u)
        return UINT32_MAX;
    return t & (REQUEST_RING_SIZE - 1);
}

static inline void
req_ring_commit(RequestRing *r)
{
    const uint32_t t = RL_LOAD_RLX_U32(&r->prod.tail);
    RL_STORE_REL_U32(&r->prod.tail, t + 1u);
}

static inline void
done_ring_record_overflow(volatile uint32_t *value)
{
    __atomic_add_fetch((uint32_t *)value, 1U, __ATOMIC_RELAXED);
}

/* Consumer of requests (host restatement of the device side). */
static inline int
req_ring_consume(RequestRing *r, RolloutRequest *out)
{
    const uint32_t h = RL_LOAD_RLX_U32(&r->cons.head);
    if (RL_LOAD_ACQ_U32(&r->prod.tail) == h)
        return 0;
    *out = r->slots[h & (REQUEST_RING_SIZE - 1)];
    RL_STORE_REL_U32(&r->cons.head, h + 1u);
    return 1;
}

/* Producer of dones (host restatement of the device side). */
static inline int
done_ring_push(DoneRing *r, const RolloutDone *d)
{
    const uint32_t t = RL_LOAD_RLX_U32(&r->prod.tail);
    if (t - RL_LOAD_ACQ_U32(&r->cons.head) >= (uint32_t)REQUEST_RING_SIZE) {
        done_ring_record_overflow(&r->overflow.value);
        return -1;
    }
    r->slots[t & (REQUEST_RING_SIZE - 1)] = *d;
    RL_STORE_REL_U32(&r->prod.tail, t + 1u);
    return 0;
}

/* Host consumer of dones: 1 with an item, 0 when empty. */
static inline int
done_ring_pop(DoneRing *r, RolloutDone *out)
{
    const uint32_t h = RL_LOAD_RLX_U32(&r->cons.head);
    if (RL_LOAD_ACQ_U32(&r->prod.tail) == h)
        return 0;
    *out = r->slots[h & (REQUEST_RING_SIZE - 1)];
    RL_STORE_REL_U32(&r->cons.head, h + 1u);
    return 1;
}

RL_EXTERN_C_BEGIN

/* Ring allocation in coherent host memory when a device is open (new; the
 * reference harness calls cudaHostAlloc(Mapped) inline,
 * bench/bench_gpu_scheduler.cu:43-44). Zero-initialised. */
RequestRing *req_ring_create(void);
void req_ring_destroy(RequestRing *r);
DoneRing *done_ring_create(void);
void done_ring_destroy(DoneRing *r);

RL_EXTERN_C_END
