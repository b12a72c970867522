/*
 * kv_prefix.c - copy-on-write prefix refcounts (reference
 * src/kv_prefix.c:5-149; rules restated in kv_prefix.h).
 */
#include <string.h>

#include "kv_prefix.h"

#define PREFIX_WORDS ((MAX_PREFIXES + 63) / 64)
#define BRANCH_WORDS ((MAX_BRANCHES + 63) / 64)

static void
bitmap_fill_free(uint64_t *words, unsigned n_words, unsigned n_ids)
{
    for (unsigned w = 0; w < n_words; w++)
        words[w] = ~0ULL;
    if (n_ids % 64u)
        words[n_ids / 64u] &= (1ULL << (n_ids % 64u)) - 1ULL;
}

/* Lowest free (set) bit, cleared; -1 when none. */
static int
bitmap_take_lowest(uint64_t *words, unsigned n_words, uint32_t *out_id)
{
    for (unsigned w = 0; w < n_words; w++) {
        if (words[w]) {
            const unsigned b = (unsigned)__builtin_ctzll(words[w]);
            words[w] &= ~(1ULL << b);
            *out_id = w * 64u + b;
            return 0;
        }
    }
    return -1;
}

static void
bitmap_give_back(uint64_t *words, uint32_t id)
{
    words[id / 64u] |= 1ULL << (id % 64u);
}

void
kv_prefix_table_init(KVPrefixTable *t)
{
    memset(t, 0, sizeof(*t));
    bitmap_fill_free(t->prefix_bitmap, PREFIX_WORDS, MAX_PREFIXES);
    bitmap_fill_free(t->branch_bitmap, BRANCH_WORDS, MAX_BRANCHES);
}

int
kv_prefix_register(KVPrefixTable *t, int64_t kv_offset, uint32_t token_len, uint32_t nblocks,
                   uint32_t *out_id)
{
    uint32_t id;
    if (bitmap_take_lowest(t->prefix_bitmap, PREFIX_WORDS, &id) != 0)
        return -1;
    KVPrefix *p = &t->prefixes[id];
    p->prefix_id = id;
    p->refcnt = 1;
    p->kv_block_offset = kv_offset;
    p->token_len = token_len;
    p->kv_block_count = nblocks;
    p->flags = 0;
    *out_id = id;
    return 0;
}

int
kv_prefix_acquire(KVPrefixTable *t, uint32_t prefix_id)
{
    if (prefix_id >= MAX_PREFIXES || t->prefixes[prefix_id].refcnt == 0)
        return -1;
    t->prefixes[prefix_id].refcnt++;
    return 0;
}

int
kv_prefix_release(KVPrefixTable *t, uint32_t prefix_id)
{
    if (prefix_id >= MAX_PREFIXES)
        return -1;
    KVPrefix *p = &t->prefixes[prefix_id];
    if (p->refcnt == 0)
        return -1;
    if (--p->refcnt == 0) {
        p->kv_block_offset = -1;
        p->token_len = 0;
        bitmap_give_back(t->prefix_bitmap, prefix_id);
    }
    return 0;
}

KVPrefix *
kv_prefix_get(KVPrefixTable *t, uint32_t prefix_id)
{
    return prefix_id < MAX_PREFIXES ? &t->prefixes[prefix_id] : NULL;
}

int
kv_branch_alloc(KVPrefixTable *t, uint32_t rollout_id, uint32_t prefix_id, int64_t delta_kv_offset,
                uint32_t delta_len, uint32_t delta_blocks, uint32_t *out_branch_id)
{
    uint32_t id;
    if (bitmap_take_lowest(t->branch_bitmap, BRANCH_WORDS, &id) != 0)
        return -1;
    KVBranch *b = &t->branches[id];
    b->branch_id = id;
    b->rollout_id = rollout_id;
    b->prefix_id = prefix_id;
    b->delta_kv_offset = delta_kv_offset;
    b->delta_len = delta_len;
    b->delta_block_count = delta_blocks;
    b->state = 0;
    b->flags = 0;
    (void)kv_prefix_acquire(t, prefix_id);
    *out_branch_id = id;
    return 0;
}

int
kv_branch_free(KVPrefixTable *t, uint32_t branch_id)
{
    if (branch_id >= MAX_BRANCHES)
        return -1;
    KVBranch *b = &t->branches[branch_id];
    (void)kv_prefix_release(t, b->prefix_id);
    b->rollout_id = UINT32_MAX;
    bitmap_give_back(t->branch_bitmap, branch_id);
    return 0;
}

KVBranch *
kv_branch_get(KVPrefixTable *t, uint32_t branch_id)
{
    return branch_id < MAX_BRANCHES ? &t->branches[branch_id] : NULL;
}

int64_t
kv_branch_total_offset(KVPrefixTable *t, uint32_t branch_id)
{
    if (branch_id >= MAX_BRANCHES)
        return -1;
    const KVBranch *b = &t->branches[branch_id];
    const KVPrefix *p = kv_prefix_get(t, b->prefix_id);
    return p ? p->kv_block_offset : b->delta_kv_offset;
}
