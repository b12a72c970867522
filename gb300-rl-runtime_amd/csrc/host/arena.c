/*
 * arena.c - KV block arena (reference src/arena.c:7-58).
 *
 * With an open device the block storage is HBM (hipMalloc + zero fill): the
 * decode kernels read blocks straight from it and arena_block_ptr() returns
 * device addresses. Without one it is anonymous host memory, hugepages
 * first, zero-filled, as in the reference. The 1 = used bitmap and its
 * lowest-free-first policy are host-side and identical in both modes.
 */
#define _GNU_SOURCE
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#include "arena.h"
#include "rl_hip.h"

void
arena_init(KVArena *a, size_t capacity, size_t block_size)
{
    a->capacity = capacity;
    a->block_size = block_size;
    memset(a->bitmap, 0, sizeof(a->bitmap));

    if (rl_hip_is_open()) {
        a->base = (uint8_t *)rl_hip_dev_alloc(capacity);
        if (!a->base || rl_hip_memset_d(a->base, 0, capacity) != 0 || rl_hip_sync() != 0) {
            fprintf(stderr, "arena_init: device allocation of %zu bytes failed: %s\n",
                    capacity, rl_hip_last_error());
            abort();
        }
        return;
    }

    void *p = mmap(NULL, capacity, PROT_READ | PROT_WRITE,
                   MAP_ANONYMOUS | MAP_PRIVATE | MAP_HUGETLB, -1, 0);
    if (p == MAP_FAILED) {
        p = mmap(NULL, capacity, PROT_READ | PROT_WRITE, MAP_ANONYMOUS | MAP_PRIVATE, -1, 0);
        if (p == MAP_FAILED) {
            perror("arena_init: mmap");
            abort();
        }
    }
    memset(p, 0, capacity); /* prefault every page */
    a->base = (uint8_t *)p;
}

int
arena_is_device(const KVArena *a)
{
    return a && a->base && rl_hip_is_device_ptr(a->base);
}

int64_t
arena_acquire(KVArena *a)
{
    for (size_t w = 0; w < BITMAP_WORDS; w++) {
        const uint64_t free_bits = ~a->bitmap[w];
        if (free_bits != 0) {
            const unsigned b = (unsigned)__builtin_ctzll(free_bits);
            a->bitmap[w] |= 1ULL << b;
            return (int64_t)(w * 64u + b);
        }
    }
    return -1;
}

void
arena_release(KVArena *a, int64_t idx)
{
    if (idx < 0)
        return;
    a->bitmap[idx / 64] &= ~(1ULL << (idx % 64));
}

void
arena_destroy(KVArena *a)
{
    if (a->base) {
        if (rl_hip_is_device_ptr(a->base))
            rl_hip_dev_free(a->base);
        else
            munmap(a->base, a->capacity);
    }
    a->base = NULL;
}
