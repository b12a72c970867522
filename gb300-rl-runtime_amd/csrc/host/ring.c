/*
 * ring.c - allocation of the v0.2 command/completion rings and the v0.3
 * request/done rings (reference src/ring.c:10-58 for the first pair; the
 * reference allocates the second pair inline with cudaHostAlloc(Mapped),
 * bench/bench_gpu_scheduler.cu:43-44). All four come back zero-filled, in
 * coherent host memory when a device is open.
 */
#include "request.h"
#include "ring.h"
#include "rl_host_mem.h"

CommandRing *
ring_create(void)
{
    return (CommandRing *)rl_ring_mem_alloc(sizeof(CommandRing));
}

void
ring_destroy(CommandRing *ring)
{
    rl_ring_mem_free(ring);
}

CompletionRing *
comp_ring_create(void)
{
    return (CompletionRing *)rl_ring_mem_alloc(sizeof(CompletionRing));
}

void
comp_ring_destroy(CompletionRing *ring)
{
    rl_ring_mem_free(ring);
}

RequestRing *
req_ring_create(void)
{
    return (RequestRing *)rl_ring_mem_alloc(sizeof(RequestRing));
}

void
req_ring_destroy(RequestRing *r)
{
    rl_ring_mem_free(r);
}

DoneRing *
done_ring_create(void)
{
    return (DoneRing *)rl_ring_mem_alloc(sizeof(DoneRing));
}

void
done_ring_destroy(DoneRing *r)
{
    rl_ring_mem_free(r);
}
