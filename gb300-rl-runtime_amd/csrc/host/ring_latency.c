/* ring_latency.c - unloaded ring latency drivers (specification:
 * ring_latency.h). One descriptor in flight at a time; the host stamps sit
 * right next to the release store that publishes the descriptor and right
 * after the acquire load that sees the completion. */
#define _POSIX_C_SOURCE 200809L
#include "ring_latency.h"

#include <time.h>

static uint64_t now_ns(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

uint32_t ring_lockstep_hw(hw_ring_t *const *cmdq, hw_ring_t *const *doneq, uint32_t pairs, const hw_desc_t *desc,
                          uint32_t n, const volatile uint64_t *stamps, uint64_t timeout_ns,
                          ring_lockstep_sample_t *out)
{
    if (!cmdq || !doneq || !pairs || !desc || !stamps || !out)
        return 0;
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t g = i % pairs;
        hw_ring_t *cq = cmdq[g], *dq = doneq[g];
        const uint32_t t = hw_ring_load_acquire(&cq->tail);
        if (t != hw_ring_load_acquire(&cq->head))
            return i;  /* not idle */
        hw_desc_t d = *desc;
        d.user_data = i;
        cq->desc[t & HW_RING_MASK] = d;
        const uint32_t h = hw_ring_load_acquire(&dq->head);
        out[i].submit_ns = now_ns();
        hw_ring_store_release(&cq->tail, t + 1u);
        for (;;) {
            if (hw_ring_load_acquire(&dq->tail) != h) {
                out[i].poll_ns = now_ns();
                break;
            }
            if (now_ns() - out[i].submit_ns > timeout_ns)
                return i;
        }
        const uint64_t tag = dq->desc[h & HW_RING_MASK].user_data;
        hw_ring_store_release(&dq->head, h + 1u);
        if (tag != i)
            return i;
        out[i].consume_tick = stamps[2 * (size_t)g];
        out[i].complete_tick = stamps[2 * (size_t)g + 1];
    }
    return n;
}

uint32_t ring_lockstep_cmd(CommandRing *const *rings, CompletionRing *const *comps, uint32_t pairs,
                           const Descriptor *desc, uint64_t seq0, uint32_t n, const volatile uint64_t *stamps,
                           uint64_t timeout_ns, ring_lockstep_sample_t *out)
{
    if (!rings || !comps || !pairs || !desc || !stamps || !out)
        return 0;
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t g = i % pairs;
        CommandRing *r = rings[g];
        CompletionRing *cr = comps[g];
        const uint32_t t = RL_LOAD_RLX_U32(&r->prod.tail);
        if (t != RL_LOAD_ACQ_U32(&r->cons.head))
            return i;  /* not idle */
        Descriptor d = *desc;
        d.seq_id = seq0 + i;
        d.batch_size = 1;
        d.batch_index = 0;
        r->slots[t & (RING_SIZE - 1)] = d;
        const uint32_t h = RL_LOAD_RLX_U32(&cr->cons.head);
        out[i].submit_ns = now_ns();
        RL_STORE_REL_U32(&r->prod.tail, t + 1u);
        for (;;) {
            if (RL_LOAD_ACQ_U32(&cr->prod.tail) != h) {
                out[i].poll_ns = now_ns();
                break;
            }
            if (now_ns() - out[i].submit_ns > timeout_ns)
                return i;
        }
        const uint64_t seq = cr->slots[h & (COMP_RING_SIZE - 1)].seq_id;
        RL_STORE_REL_U32(&cr->cons.head, h + 1u);
        if (seq != seq0 + i)
            return i;
        out[i].consume_tick = stamps[2 * (size_t)g];
        out[i].complete_tick = stamps[2 * (size_t)g + 1];
    }
    return n;
}
