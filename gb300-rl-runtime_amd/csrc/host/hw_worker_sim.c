/*
 * hw_worker_sim.c - CPU model of the device worker (reference
 * src/hw_worker_sim.c:5-59). The control rule lives in
 * hw_worker_apply_decode_rule so the GPU worker's tests can replay it.
 */
#include "hw_worker_sim.h"

static inline void
cpu_relax(void)
{
#if defined(__x86_64__)
    __asm__ volatile("pause" ::: "memory");
#elif defined(__aarch64__)
    __asm__ volatile("yield" ::: "memory");
#endif
}

uint32_t
hw_worker_apply_decode_rule(hw_desc_t *desc)
{
    uint32_t decoded = 0;
    while (desc->seq_len < desc->max_tokens) {
        desc->seq_len++;
        decoded++;
        if (desc->seq_len >= desc->max_tokens) {
            desc->flags |= (uint16_t)DESC_FLAG_DONE;
            break;
        }
        if ((desc->seq_len & 31u) == 0u) {
            desc->flags |= (uint16_t)DESC_FLAG_NEEDS_REWARD;
            break;
        }
    }
    return decoded;
}

void
hw_worker_sim_run(hw_worker_sim_t *worker)
{
    for (;;) {
        if (__atomic_load_n(worker->stop, __ATOMIC_ACQUIRE))
            return;
        hw_desc_t desc;
        if (hw_ring_pop(worker->cmdq, &desc) != 0) {
            cpu_relax();
            continue;
        }
        if (desc.opcode == DESC_OP_STOP)
            return;
        if (desc.opcode != DESC_OP_DECODE)
            continue;
        worker->decoded_tokens += hw_worker_apply_decode_rule(&desc);
        while (hw_ring_push(worker->doneq, &desc) != 0)
            cpu_relax();
        worker->completions++;
    }
}
