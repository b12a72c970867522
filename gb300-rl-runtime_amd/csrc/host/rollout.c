/*
 * rollout.c - the rollout slab and its state machine (reference
 * src/rollout.c:4-67, behaviour restated in include/rollout.h).
 *
 * Allocation takes the lowest free id: the first non-zero free-bitmap word,
 * its lowest set bit. The record is wiped to {rollout_id = id, FREE} so a
 * recycled slot never carries a previous rollout's fields.
 */
#include <string.h>

#include "rollout.h"

void
rollout_slab_init(rollout_slab_t *slab)
{
    if (!slab)
        return;
    memset(slab, 0, sizeof(*slab));
    for (uint32_t id = 0; id < MAX_ROLLOUTS; id++)
        slab->slots[id].rollout_id = id;   /* state 0 == ROLL_FREE */
    for (uint32_t w = 0; w < ROLLOUT_BITMAP_WORDS; w++) {
        const uint32_t first = w * 64u;
        const uint32_t live = MAX_ROLLOUTS - first < 64u ? MAX_ROLLOUTS - first : 64u;
        slab->free_bitmap[w] = live == 64u ? ~0ull : (1ull << live) - 1ull;
    }
}

int
rollout_alloc(rollout_slab_t *slab, uint32_t *out_id)
{
    if (!slab || !out_id)
        return -1;
    for (uint32_t w = 0; w < ROLLOUT_BITMAP_WORDS; w++) {
        const uint64_t free_bits = slab->free_bitmap[w];
        if (!free_bits)
            continue;
        const uint32_t bit = (uint32_t)__builtin_ctzll(free_bits);
        const uint32_t id = w * 64u + bit;
        slab->free_bitmap[w] = free_bits & (free_bits - 1ull);   /* clear the lowest set bit */
        rollout_t *r = &slab->slots[id];
        memset(r, 0, sizeof(*r));
        r->rollout_id = id;
        *out_id = id;
        return 0;
    }
    return -1;
}

void
rollout_free(rollout_slab_t *slab, uint32_t id)
{
    if (!slab || id >= MAX_ROLLOUTS)
        return;
    slab->slots[id].state = ROLL_FREE;
    slab->free_bitmap[id >> 6] |= 1ull << (id & 63u);
}

rollout_t *
rollout_get(rollout_slab_t *slab, uint32_t id)
{
    return slab && id < MAX_ROLLOUTS ? &slab->slots[id] : NULL;
}

int
rollout_transition(rollout_t *r, rollout_state_t from, rollout_state_t to)
{
    if (!r || !rollout_is_valid_transition(from, to))
        return -1;
    uint32_t seen = (uint32_t)from;
    return __atomic_compare_exchange_n(&r->state, &seen, (uint32_t)to, 0, __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE)
               ? 0 : -1;
}
