/*
 * decode_batch.c - descriptor windows (reference src/decode_batch.c:3-51).
 */
#include "decode_batch.h"

void
decode_batch_reset(DecodeDispatchBatch *batch)
{
    if (batch)
        batch->count = 0;
}

int
decode_batch_push(DecodeDispatchBatch *batch, const Descriptor *desc)
{
    if (!batch || !desc || batch->count >= DECODE_DESCRIPTOR_BATCH_LIMIT)
        return -1;
    batch->descs[batch->count] = *desc;
    batch->count++;
    return 0;
}

int
decode_batch_submit(CommandRing *ring, const DecodeDispatchBatch *batch)
{
    if (!ring || !batch || batch->count == 0)
        return -1;
    const uint32_t n = batch->count;
    const uint32_t pos = ring_acquire(ring, n);
    if (pos == UINT32_MAX)
        return -1;
    for (uint32_t i = 0; i < n; i++) {
        Descriptor *slot = &ring->slots[(pos + i) & (RING_SIZE - 1u)];
        *slot = batch->descs[i];
        slot->batch_size = (uint16_t)n;
        slot->batch_index = (uint16_t)i;
    }
    ring_commit(ring, n);
    return 0;
}

DecodeBatchContract
decode_batch_contract(const Descriptor *desc)
{
    DecodeBatchContract c = {0u, 0u};
    if (desc) {
        c.batch_size = desc->batch_size;
        c.batch_index = desc->batch_index;
    }
    return c;
}
