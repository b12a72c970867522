/*
 * kv_prefix.h - copy-on-write prefix refcounts and per-rollout branches.
 *
 * Same field order and packing as the reference (include/kv_prefix.h:6-56).
 * The reference asserts sizeof(KVPrefix) == 24 and sizeof(KVBranch) == 28,
 * which contradicts its own packed field lists; the packed sizes are 28 and
 * 36 and those are asserted here. Table layout: prefixes[512]@0,
 * prefix_bitmap[8]@14,336, branches[16384]@14,400, branch_bitmap[256]
 * @604,224, next_branch_id@606,272; sizeof 606,280. Bitmaps use 1 = free.
 *
 * Rules (src/kv_prefix.c:5-149):
 *  register: lowest free id; refcnt 1, offset/len/count set, flags 0.
 *  acquire:  -1 if id >= 512 or refcnt == 0, else refcnt++.
 *  release:  -1 if id >= 512 or refcnt == 0; else refcnt--, and at 0 set
 *            kv_block_offset = -1, token_len = 0 and free the id
 *            (kv_block_count and flags are kept).
 *  branch_alloc: lowest free branch id, fields set, state = flags = 0,
 *            then kv_prefix_acquire (its failure ignored).
 *  branch_free: -1 if id >= 16384; release the prefix (ignored),
 *            rollout_id = UINT32_MAX, free the id.
 *  total_offset: -1 if id >= 16384; the prefix's kv_block_offset when
 *            prefix_id < 512, else the branch's delta offset.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#ifndef MAX_ROLLOUTS
#define MAX_ROLLOUTS 8192
#endif
#define MAX_PREFIXES 512
#define MAX_BRANCHES (MAX_ROLLOUTS * 2)

typedef struct __attribute__((packed)) {
    uint32_t prefix_id;
    uint32_t refcnt;
    int64_t kv_block_offset;
    uint32_t token_len;
    uint32_t kv_block_count;
    uint32_t flags;
} KVPrefix;

RL_STATIC_ASSERT(sizeof(KVPrefix) == 28, "KVPrefix packed size");

typedef struct __attribute__((packed)) {
    uint32_t branch_id;
    uint32_t rollout_id;
    uint32_t prefix_id;
    int64_t delta_kv_offset;
    uint32_t delta_len;
    uint32_t delta_block_count;
    uint32_t state;
    uint32_t flags;
} KVBranch;

RL_STATIC_ASSERT(sizeof(KVBranch) == 36, "KVBranch packed size");

typedef struct {
    KVPrefix prefixes[MAX_PREFIXES];
    uint64_t prefix_bitmap[(MAX_PREFIXES + 63) / 64];
    KVBranch branches[MAX_BRANCHES];
    uint64_t branch_bitmap[(MAX_BRANCHES + 63) / 64];
    uint32_t next_branch_id;
} KVPrefixTable;

RL_STATIC_ASSERT(RL_OFFSETOF(KVPrefixTable, prefix_bitmap) == 14336, "prefix_bitmap");
RL_STATIC_ASSERT(RL_OFFSETOF(KVPrefixTable, branches) == 14400, "branches");
RL_STATIC_ASSERT(RL_OFFSETOF(KVPrefixTable, branch_bitmap) == 604224, "branch_bitmap");
RL_STATIC_ASSERT(RL_OFFSETOF(KVPrefixTable, next_branch_id) == 606272, "next_branch_id");
RL_STATIC_ASSERT(sizeof(KVPrefixTable) == 606280, "KVPrefixTable size");

RL_EXTERN_C_BEGIN

void kv_prefix_table_init(KVPrefixTable *t);
int kv_prefix_register(KVPrefixTable *t, int64_t kv_offset, uint32_t token_len,
                       uint32_t nblocks, uint32_t *out_id);
int kv_prefix_acquire(KVPrefixTable *t, uint32_t prefix_id);
int kv_prefix_release(KVPrefixTable *t, uint32_t prefix_id);
KVPrefix *kv_prefix_get(KVPrefixTable *t, uint32_t prefix_id);

int kv_branch_alloc(KVPrefixTable *t, uint32_t rollout_id, uint32_t prefix_id,
                    int64_t delta_kv_offset, uint32_t delta_len, uint32_t delta_blocks,
                    uint32_t *out_branch_id);
int kv_branch_free(KVPrefixTable *t, uint32_t branch_id);
KVBranch *kv_branch_get(KVPrefixTable *t, uint32_t branch_id);
int64_t kv_branch_total_offset(KVPrefixTable *t, uint32_t branch_id);

RL_EXTERN_C_END
