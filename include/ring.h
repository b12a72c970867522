/*
 * ring.h - 4,096-slot command ring of 32-byte Descriptors (v0.2 contract).
 *
 * Byte-compatible with the reference (include/ring.h:7-75): consumer head
 * line @0, producer tail line @64, slots @128 (sizeof 131,200).
 *   ring_acquire(n): masked tail, or UINT32_MAX when fewer than n slots free;
 *   ring_commit(n):  release-store tail + n;
 *   ring_consume:    1 with a descriptor, 0 when empty.
 * The empty test is wrap-safe (see completion.h).
 *
 * ring_create/comp_ring_create place the rings in fine-grained coherent host
 * memory when a HIP device is open (the reference uses anonymous mmap, which
 * only a cache-coherent NVLink-C2C/ATS host can hand to a GPU).
 */
#pragma once

#include <stdint.h>
#include "completion.h"
#include "descriptor.h"

typedef struct __attribute__((packed)) {
    volatile uint32_t head __attribute__((aligned(64)));
    uint8_t pad[60];
} RingHead;

typedef struct __attribute__((packed)) {
    volatile uint32_t tail __attribute__((aligned(64)));
    uint8_t pad[60];
} RingTail;

typedef struct {
    RingHead cons __attribute__((aligned(64)));
    RingTail prod __attribute__((aligned(64)));
    Descriptor slots[RING_SIZE] __attribute__((aligned(DESCRIPTOR_ALIGN)));
} CommandRing;

RL_STATIC_ASSERT(RL_OFFSETOF(CommandRing, prod) == 64, "CommandRing.prod");
RL_STATIC_ASSERT(RL_OFFSETOF(CommandRing, slots) == 128, "CommandRing.slots");
RL_STATIC_ASSERT(sizeof(CommandRing) == 131200, "CommandRing size");

static inline uint32_t
ring_acquire(CommandRing *ring, uint32_t n)
{
    const uint32_t h = RL_LOAD_ACQ_U32(&ring->cons.head);
    const uint32_t t = RL_LOAD_RLX_U32(&ring->prod.tail);
    if ((uint32_t)RING_SIZE - (t - h) < n)
        return UINT32_MAX;
    return t & (RING_SIZE - 1);
}

static inline void
ring_commit(CommandRing *ring, uint32_t n)
{
    const uint32_t t = RL_LOAD_RLX_U32(&ring->prod.tail);
    RL_STORE_REL_U32(&ring->prod.tail, t + n);
}

static inline int
ring_consume(CommandRing *ring, Descriptor *desc)
{
    const uint32_t h = RL_LOAD_RLX_U32(&ring->cons.head);
    if (RL_LOAD_ACQ_U32(&ring->prod.tail) == h)
        return 0;
    *desc = ring->slots[h & (RING_SIZE - 1)];
    RL_STORE_REL_U32(&ring->cons.head, h + 1u);
    return 1;
}

RL_EXTERN_C_BEGIN

CommandRing *ring_create(void);
void ring_destroy(CommandRing *ring);
CompletionRing *comp_ring_create(void);
void comp_ring_destroy(CompletionRing *ring);

RL_EXTERN_C_END
