/*
 * completion.h - 32-byte completion record and its 4,096-slot ring.
 *
 * Byte-compatible with the reference (include/completion.h:8-87): packed
 * Completion {seq_id, token_id, kv_block_offset, reward_cookie,
 * cycles_taken}; CompletionRing = consumer head line @0, producer tail line
 * @64, overflow counter line @128, slots @256 (sizeof 131,328).
 *
 * Push on a full ring bumps the overflow counter and returns -1; poll returns
 * 1 with an item, 0 when empty. The empty test is written wrap-safe
 * (tail - head == 0); the reference's `head >= tail` gives the same answer
 * for every index pair reachable in fewer than 2^32 operations.
 */
#pragma once

#include <stdint.h>
#include "rl_abi.h"

#define COMP_RING_SIZE 4096

#pragma pack(push, 1)
typedef struct {
    uint64_t seq_id;
    uint32_t token_id;
    uint32_t kv_block_offset;
    uint64_t reward_cookie;
    uint64_t cycles_taken;
} Completion;
#pragma pack(pop)

RL_STATIC_ASSERT(sizeof(Completion) == 32, "Completion must be 32 bytes");

typedef struct __attribute__((packed)) {
    volatile uint32_t head __attribute__((aligned(64)));
    uint8_t pad[60];
} CompHead;

typedef struct __attribute__((packed)) {
    volatile uint32_t tail __attribute__((aligned(64)));
    uint8_t pad[60];
} CompTail;

typedef struct __attribute__((packed)) {
    volatile uint32_t value __attribute__((aligned(64)));
    uint8_t pad[60];
} CompCounter;

RL_STATIC_ASSERT(sizeof(CompHead) == 64, "CompHead is one cache line");
RL_STATIC_ASSERT(sizeof(CompTail) == 64, "CompTail is one cache line");
RL_STATIC_ASSERT(sizeof(CompCounter) == 64, "CompCounter is one cache line");

/* Status codes of the RTL completion record (unused by the C path). */
enum comp_status {
    COMP_STATUS_DONE = 0x01,
    COMP_STATUS_REWARD_NEEDED = 0x02,
    COMP_STATUS_STOPPED = 0xFF,
};

typedef struct {
    CompHead cons __attribute__((aligned(64)));
    CompTail prod __attribute__((aligned(64)));
    CompCounter overflow __attribute__((aligned(64)));
    Completion slots[COMP_RING_SIZE] __attribute__((aligned(128)));
} CompletionRing;

RL_STATIC_ASSERT(RL_OFFSETOF(CompletionRing, overflow) == 128, "CompletionRing.overflow");
RL_STATIC_ASSERT(RL_OFFSETOF(CompletionRing, slots) == 256, "CompletionRing.slots");
RL_STATIC_ASSERT(sizeof(CompletionRing) == 131328, "CompletionRing size");

static inline void
comp_ring_record_overflow(volatile uint32_t *value)
{
    __atomic_add_fetch((uint32_t *)value, 1U, __ATOMIC_RELAXED);
}

/* Producer side (host restatement; the gfx950 worker has its own
 * system-scope version in the HIP sources). */
static inline int
comp_ring_push(CompletionRing *cr, const Completion *c)
{
    const uint32_t t = RL_LOAD_RLX_U32(&cr->prod.tail);
    if (t - RL_LOAD_ACQ_U32(&cr->cons.head) >= (uint32_t)COMP_RING_SIZE) {
        comp_ring_record_overflow(&cr->overflow.value);
        return -1;
    }
    cr->slots[t & (COMP_RING_SIZE - 1)] = *c;
    RL_STORE_REL_U32(&cr->prod.tail, t + 1u);
    return 0;
}

/* Consumer side: 1 with an item, 0 when empty. */
static inline int
comp_ring_poll(CompletionRing *cr, Completion *out)
{
    const uint32_t h = RL_LOAD_RLX_U32(&cr->cons.head);
    if (RL_LOAD_ACQ_U32(&cr->prod.tail) == h)
        return 0;
    *out = cr->slots[h & (COMP_RING_SIZE - 1)];
    RL_STORE_REL_U32(&cr->cons.head, h + 1u);
    return 1;
}
