/*
 * hw_ring.h - 65,536-slot SPSC ring of hw_desc_t.
 *
 * Layout and semantics follow the reference ring (include/hw_ring.h:7-69,
 * src/hw_ring.c:6-42): head on its own cache line at offset 0, tail on its
 * own cache line at offset 64, descriptors from offset 128; indices are
 * free-running u32 and wrap through HW_RING_MASK; push fails with -1 when
 * tail-head reaches HW_RING_SIZE, pop fails with -1 when head == tail.
 *
 * MI355X placement: hw_ring_create() allocates the ring in fine-grained
 * coherent host memory (hipHostMalloc, coherent|mapped) once rl_hip_open()
 * has bound a device, so the persistent worker can poll it with system-scope
 * atomics; without an open device it falls back to 64-byte aligned pageable
 * memory exactly like the reference (CPU-only use, hw_worker_sim).
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "hw_desc.h"

#define HW_RING_SIZE (1u << 16)
#define HW_RING_MASK (HW_RING_SIZE - 1u)

typedef struct {
    RL_ALIGNAS(64) volatile uint32_t head; /* consumer-owned */
    char pad0[60];

    RL_ALIGNAS(64) volatile uint32_t tail; /* producer-owned */
    char pad1[60];

    RL_ALIGNAS(64) hw_desc_t desc[HW_RING_SIZE];
} hw_ring_t;

RL_STATIC_ASSERT(RL_OFFSETOF(hw_ring_t, tail) == 64, "hw_ring_t.tail");
RL_STATIC_ASSERT(RL_OFFSETOF(hw_ring_t, desc) == 128, "hw_ring_t.desc");
RL_STATIC_ASSERT(sizeof(hw_ring_t) == 4194432, "hw_ring_t size");

RL_EXTERN_C_BEGIN

/* Exported (reference: src/hw_ring.c:6-16). */
uint32_t hw_ring_load_acquire(volatile uint32_t *p);
void hw_ring_store_release(volatile uint32_t *p, uint32_t value);

/* Exported (reference: src/hw_ring.c:18-42). */
hw_ring_t *hw_ring_create(void);
void hw_ring_reset(hw_ring_t *ring);
void hw_ring_destroy(hw_ring_t *ring);

RL_EXTERN_C_END

/* Occupancy as seen by either side: both indices acquire-loaded. */
static inline uint32_t
hw_ring_occupancy(hw_ring_t *ring)
{
    const uint32_t h = hw_ring_load_acquire(&ring->head);
    const uint32_t t = hw_ring_load_acquire(&ring->tail);
    return t - h;
}

static inline int
hw_ring_full(hw_ring_t *ring)
{
    return hw_ring_occupancy(ring) >= HW_RING_SIZE;
}

static inline int
hw_ring_empty(hw_ring_t *ring)
{
    return hw_ring_occupancy(ring) == 0u;
}

/* Producer: 0 on success, -1 when the ring holds HW_RING_SIZE entries. */
static inline int
hw_ring_push(hw_ring_t *ring, const hw_desc_t *desc)
{
    const uint32_t t = hw_ring_load_acquire(&ring->tail);
    if (t - hw_ring_load_acquire(&ring->head) >= HW_RING_SIZE)
        return -1;
    ring->desc[t & HW_RING_MASK] = *desc;
    hw_ring_store_release(&ring->tail, t + 1u);
    return 0;
}

/* Consumer: 0 on success, -1 when empty. */
static inline int
hw_ring_pop(hw_ring_t *ring, hw_desc_t *out)
{
    const uint32_t h = hw_ring_load_acquire(&ring->head);
    if (hw_ring_load_acquire(&ring->tail) == h)
        return -1;
    *out = ring->desc[h & HW_RING_MASK];
    hw_ring_store_release(&ring->head, h + 1u);
    return 0;
}
