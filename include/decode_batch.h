/*
 * decode_batch.h - windows of up to 32 descriptors committed at once.
 *
 * Same types and functions as the reference (include/decode_batch.h:7-22,
 * src/decode_batch.c:3-51): push appends to the window (-1 when NULL or
 * full); submit acquires `count` slots, writes each descriptor with
 * batch_size = count and batch_index = i, then commits once (-1 on NULL,
 * empty window or full ring); contract reads the two stamps (0,0 for NULL).
 */
#pragma once

#include <stdint.h>
#include "descriptor.h"
#include "ring.h"

#define DECODE_DESCRIPTOR_BATCH_LIMIT 32U

typedef struct {
    uint32_t count;
    Descriptor descs[DECODE_DESCRIPTOR_BATCH_LIMIT];
} DecodeDispatchBatch;

typedef struct {
    uint16_t batch_size;
    uint16_t batch_index;
} DecodeBatchContract;

RL_EXTERN_C_BEGIN

void decode_batch_reset(DecodeDispatchBatch *batch);
int decode_batch_push(DecodeDispatchBatch *batch, const Descriptor *desc);
int decode_batch_submit(CommandRing *ring, const DecodeDispatchBatch *batch);
DecodeBatchContract decode_batch_contract(const Descriptor *desc);

RL_EXTERN_C_END
