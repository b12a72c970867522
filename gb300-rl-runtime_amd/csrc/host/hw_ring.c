/*
 * hw_ring.c - exported half of the hw_desc ring (reference src/hw_ring.c:6-42).
 *
 * The ring is placed in fine-grained coherent host memory when a device is
 * open, so the persistent gfx950 worker can poll head/tail over the host
 * link with system-scope atomics; otherwise it is 64-byte aligned pageable
 * memory (the reference's posix_memalign) for CPU-only use.
 */
#include <stdlib.h>
#include <string.h>

#include "hw_ring.h"
#include "rl_host_mem.h"

uint32_t
hw_ring_load_acquire(volatile uint32_t *p)
{
    return __atomic_load_n(p, __ATOMIC_ACQUIRE);
}

void
hw_ring_store_release(volatile uint32_t *p, uint32_t value)
{
    __atomic_store_n(p, value, __ATOMIC_RELEASE);
}

hw_ring_t *
hw_ring_create(void)
{
    return (hw_ring_t *)rl_ring_mem_alloc(sizeof(hw_ring_t));
}

void
hw_ring_reset(hw_ring_t *ring)
{
    if (ring)
        memset((void *)ring, 0, sizeof(*ring));
}

void
hw_ring_destroy(hw_ring_t *ring)
{
    rl_ring_mem_free(ring);
}
