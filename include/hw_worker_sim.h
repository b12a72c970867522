/*
 * hw_worker_sim.h - CPU model of the device worker on the hw_desc rings.
 *
 * Same struct (40 bytes) and entry point as the reference
 * (include/hw_worker_sim.h:6-14). The control rule it applies to each DECODE
 * descriptor (src/hw_worker_sim.c:23-59) is also the rule the gfx950
 * persistent worker applies after its real decode math, so the doneq
 * descriptors produced by both are byte-identical:
 *   while seq_len < max_tokens: seq_len++, decoded_tokens++;
 *     if seq_len >= max_tokens: flags |= DONE, stop;
 *     if (seq_len & 31) == 0:   flags |= NEEDS_REWARD, stop;
 *   push the updated descriptor to doneq (spin while full), completions++.
 * STOP exits without a completion; other opcodes are dropped.
 */
#pragma once

#include <stdint.h>
#include "hw_ring.h"

typedef struct {
    hw_ring_t *cmdq;
    hw_ring_t *doneq;
    volatile uint32_t *stop;
    uint64_t decoded_tokens;
    uint64_t completions;
} hw_worker_sim_t;

RL_STATIC_ASSERT(sizeof(hw_worker_sim_t) == 40, "hw_worker_sim_t size");

RL_EXTERN_C_BEGIN

void hw_worker_sim_run(hw_worker_sim_t *worker);

/* Applies the control rule above to one descriptor in place and returns the
 * number of tokens it decoded. Shared by hw_worker_sim_run and by the GPU
 * worker's host-side tests. */
uint32_t hw_worker_apply_decode_rule(hw_desc_t *desc);

RL_EXTERN_C_END
