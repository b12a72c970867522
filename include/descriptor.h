/*
 * descriptor.h - 32-byte per-step command descriptor (v0.2 ring contract).
 *
 * Byte-compatible with the reference (include/descriptor.h:5-23): packed,
 * seq_id@0, kv_block_offset@8, num_kv_blocks@12, attention_flags@14, pad@15,
 * output_token_offset@16, reward_cookie@20, batch_size@28, batch_index@30.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define RING_SIZE 4096
#define MAX_KV_BLOCKS_PER_STEP 64
#define DESCRIPTOR_ALIGN 128

#pragma pack(push, 1)
typedef struct {
    uint64_t seq_id;              /* trajectory id; UINT64_MAX = shutdown sentinel */
    uint32_t kv_block_offset;     /* arena block index */
    uint16_t num_kv_blocks;
    uint8_t attention_flags;
    uint8_t pad;
    uint32_t output_token_offset; /* io slot of the q/o buffers */
    uint64_t reward_cookie;
    uint16_t batch_size;          /* stamped by decode_batch_submit */
    uint16_t batch_index;
} Descriptor;
#pragma pack(pop)

RL_STATIC_ASSERT(sizeof(Descriptor) == 32, "Descriptor must be 32 bytes");
RL_STATIC_ASSERT(RL_OFFSETOF(Descriptor, output_token_offset) == 16, "Descriptor.oto");
RL_STATIC_ASSERT(RL_OFFSETOF(Descriptor, batch_index) == 30, "Descriptor.batch_index");
