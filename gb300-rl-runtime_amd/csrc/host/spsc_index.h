/*
 * spsc_index.h - slot accounting of a single-producer single-consumer queue
 * kept as two free-running 32-bit counters: `head` counts writes (stored
 * only by the producer), `tail` counts reads (stored only by the consumer).
 * Occupancy is head - tail modulo 2^32, so the queue is empty exactly when
 * head == tail and full when head - tail == capacity, for any number of
 * operations. Capacity is a power of two; a slot index is counter & (cap - 1).
 *
 * Used by the rollout-id queues (pipeline.h) and the reward ring (reward.h),
 * whose index lines both hold the producer's counter in prod.head and the
 * consumer's in cons.tail.
 */
#pragma once

#include <stdint.h>

/* Producer: 0 and the slot to fill, or -1 when the queue is full. The
 * acquire on `tail` orders the consumer's read of a recycled slot before our
 * overwrite of it. */
static inline int
spsc_reserve(const volatile uint32_t *head, const uint32_t *tail, uint32_t cap, uint32_t *slot)
{
    const uint32_t h = __atomic_load_n(head, __ATOMIC_RELAXED);
    const uint32_t t = __atomic_load_n(tail, __ATOMIC_ACQUIRE);
    if (h - t >= cap)
        return -1;
    *slot = h & (cap - 1u);
    return 0;
}

/* Producer: makes the reserved slot visible. */
static inline void
spsc_publish(volatile uint32_t *head)
{
    const uint32_t h = __atomic_load_n(head, __ATOMIC_RELAXED);
    __atomic_store_n(head, h + 1u, __ATOMIC_RELEASE);
}

/* Consumer: 0 and the slot to read, or -1 when the queue is empty. The
 * acquire on `head` orders the producer's write of the slot before our read. */
static inline int
spsc_peek(const volatile uint32_t *head, const uint32_t *tail, uint32_t cap, uint32_t *slot)
{
    const uint32_t t = __atomic_load_n(tail, __ATOMIC_RELAXED);
    if (__atomic_load_n(head, __ATOMIC_ACQUIRE) == t)
        return -1;
    *slot = t & (cap - 1u);
    return 0;
}

/* Consumer: releases the slot read after spsc_peek. */
static inline void
spsc_retire(uint32_t *tail)
{
    const uint32_t t = __atomic_load_n(tail, __ATOMIC_RELAXED);
    __atomic_store_n(tail, t + 1u, __ATOMIC_RELEASE);
}

/* Either side: queued items (a snapshot). */
static inline uint32_t
spsc_count(const volatile uint32_t *head, const uint32_t *tail)
{
    const uint32_t t = __atomic_load_n(tail, __ATOMIC_ACQUIRE);
    return __atomic_load_n(head, __ATOMIC_ACQUIRE) - t;
}
