#define _POSIX_C_SOURCE 200112L
#include <stdlib.h>
#include <string.h>

#include "rl_hip.h"
#include "rl_host_mem.h"

void *
rl_ring_mem_alloc(size_t bytes)
{
    void *p = NULL;
    if (rl_hip_is_open())
        return rl_hip_host_alloc_coherent(bytes); /* zero-filled */
    if (posix_memalign(&p, 64, bytes) != 0)
        return NULL;
    memset(p, 0, bytes);
    return p;
}

void
rl_ring_mem_free(void *p)
{
    if (!p)
        return;
    if (rl_hip_is_coherent_host(p)) {
        rl_hip_host_free(p);
        return;
    }
    free(p);
}
