/*
 * arena.h - KV block arena.
 *
 * KVArena is byte-compatible with the reference (include/arena.h:5-35):
 * {base, capacity, block_size, bitmap[16384]} = 131,096 B, a 1 = used bitmap
 * over up to 1,048,576 blocks. arena_acquire returns the lowest clear bit
 * (or -1 when exhausted), arena_release clears it (negative idx ignored),
 * arena_block_ptr = base + idx * block_size, arena_init aborts on failure.
 *
 * MI355X placement: when rl_hip_open() has bound a device, arena_init takes
 * `base` from hipMalloc (HBM) and zero-fills it with hipMemset, so
 * arena_block_ptr() yields a DEVICE address that the decode kernels read;
 * the bitmap stays in host memory. Without an open device it maps anonymous
 * host memory as the reference does.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define BITMAP_WORDS ((1UL << 20) / 64)

typedef struct {
    uint8_t *base;
    size_t capacity;
    size_t block_size;
    uint64_t bitmap[BITMAP_WORDS];
} KVArena;

RL_STATIC_ASSERT(sizeof(KVArena) == 131096, "KVArena size");
RL_STATIC_ASSERT(RL_OFFSETOF(KVArena, bitmap) == 24, "KVArena.bitmap");

RL_EXTERN_C_BEGIN

void arena_init(KVArena *a, size_t capacity, size_t block_size);
int64_t arena_acquire(KVArena *a);
void arena_release(KVArena *a, int64_t idx);
void arena_destroy(KVArena *a);

/* 1 when a->base is device (HBM) memory, 0 for host memory. New. */
int arena_is_device(const KVArena *a);

RL_EXTERN_C_END

static inline uint8_t *
arena_block_ptr(KVArena *a, int64_t idx)
{
    return a->base + idx * (int64_t)a->block_size;
}
