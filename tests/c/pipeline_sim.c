/* A host thread standing in for the command-ring worker, for CPU tests of the
 * pipeline's command-ring driver: it consumes Descriptors and pushes one
 * Completion each, in order, passing seq_id, kv_block_offset and
 * reward_cookie through, token_id = low 32 bits of reward_cookie * 2654435761
 * and cycles_taken = batch_size | batch_index << 16 (the window stamps). */
#include <pthread.h>
#include <stdint.h>

#include "completion.h"
#include "ring.h"

static pthread_t sim_thread;
static volatile int sim_stop_flag;
static CommandRing *sim_cmd;
static CompletionRing *sim_comp;
static uint64_t sim_done;

static void *
sim_main(void *unused)
{
    Descriptor d;
    Completion c;
    (void)unused;
    for (;;) {
        if (!ring_consume(sim_cmd, &d)) {
            if (__atomic_load_n(&sim_stop_flag, __ATOMIC_ACQUIRE))
                return NULL;
            continue;
        }
        c.seq_id = d.seq_id;
        c.token_id = (uint32_t)(d.reward_cookie * 2654435761ull);
        c.kv_block_offset = d.kv_block_offset;
        c.reward_cookie = d.reward_cookie;
        c.cycles_taken = (uint64_t)d.batch_size | (uint64_t)d.batch_index << 16;
        while (comp_ring_push(sim_comp, &c) != 0)
            if (__atomic_load_n(&sim_stop_flag, __ATOMIC_ACQUIRE))
                return NULL;
        sim_done++;
    }
}

int
sim_start(CommandRing *cmd, CompletionRing *comp)
{
    sim_cmd = cmd;
    sim_comp = comp;
    sim_done = 0;
    sim_stop_flag = 0;
    return pthread_create(&sim_thread, NULL, sim_main, NULL);
}

uint64_t
sim_stop(void)
{
    __atomic_store_n(&sim_stop_flag, 1, __ATOMIC_RELEASE);
    pthread_join(sim_thread, NULL);
    return sim_done;
}
