/*
 * rollout.h - per-rollout record and the 8,192-slot rollout slab.
 *
 * Byte-compatible with the reference (include/rollout.h:5-53): rollout_t is
 * 48 bytes packed, rollout_slab_t is the slot array followed by a 128-word
 * free bitmap (bit set = slot free), 394,240 bytes.
 *
 * Lifecycle (include/rollout.h:40-51):
 *   FREE -> PREFILL_READY -> DECODING -> REWARD_PENDING -> TRAJECTORY_READY
 *        -> DONE -> FREE, plus DECODING -> DONE (aborted decode) and
 *   REWARD_PENDING -> DECODING (another decode turn after a partial reward).
 * rollout_transition is a compare-and-swap on `state`: it fails (-1) for a
 * pair outside that table and when the record is not in `from`, and leaves
 * the record unchanged in both cases.
 *
 * The slab hands out the lowest free id (src/rollout.c:19-37) and wipes the
 * record on allocation; rollout_free ignores ids >= MAX_ROLLOUTS.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define MAX_ROLLOUTS 8192

typedef enum {
    ROLL_FREE = 0,
    ROLL_PREFILL_READY,
    ROLL_DECODING,
    ROLL_REWARD_PENDING,
    ROLL_TRAJECTORY_READY,
    ROLL_DONE
} rollout_state_t;

typedef struct __attribute__((packed)) {
    uint32_t rollout_id;
    uint32_t state;          /* rollout_state_t, updated by CAS only */
    uint32_t kv_arena_id;
    int64_t kv_block_idx;
    uint32_t seq_len;
    uint32_t max_tokens;
    uint32_t reward_id;
    uint32_t flags;
    uint64_t rng_seed;
    uint32_t pad;
} rollout_t;

RL_STATIC_ASSERT(sizeof(rollout_t) == 48, "rollout_t must be 48 bytes");
RL_STATIC_ASSERT(RL_OFFSETOF(rollout_t, kv_block_idx) == 12, "rollout_t.kv_block_idx");
RL_STATIC_ASSERT(RL_OFFSETOF(rollout_t, rng_seed) == 36, "rollout_t.rng_seed");

#define ROLLOUT_BITMAP_WORDS ((MAX_ROLLOUTS + 63) / 64)

typedef struct {
    rollout_t slots[MAX_ROLLOUTS];
    uint64_t free_bitmap[ROLLOUT_BITMAP_WORDS];
} rollout_slab_t;

RL_STATIC_ASSERT(sizeof(rollout_slab_t) == 394240, "rollout_slab_t size");

RL_EXTERN_C_BEGIN

/* src/rollout.c:4-18: every record {id = slot, state FREE}, every bit free. */
void rollout_slab_init(rollout_slab_t *slab);
/* src/rollout.c:19-37: lowest free id, record wiped to {id, FREE}; -1 when full. */
int rollout_alloc(rollout_slab_t *slab, uint32_t *out_id);
/* src/rollout.c:39-48: state FREE and the bit set again; ids out of range ignored. */
void rollout_free(rollout_slab_t *slab, uint32_t id);
/* src/rollout.c:50-55: NULL for ids out of range. */
rollout_t *rollout_get(rollout_slab_t *slab, uint32_t id);
/* src/rollout.c:57-67: table check, then CAS from -> to (acq_rel). 0 or -1. */
int rollout_transition(rollout_t *r, rollout_state_t from, rollout_state_t to);

RL_EXTERN_C_END

/* The transition table (include/rollout.h:40-51). */
static inline int
rollout_is_valid_transition(rollout_state_t from, rollout_state_t to)
{
    /* row f (in enum order), bit t set when f -> t is allowed */
    static const uint8_t allowed[6] = {
        1u << ROLL_PREFILL_READY,                            /* FREE */
        1u << ROLL_DECODING,                                 /* PREFILL_READY */
        (1u << ROLL_REWARD_PENDING) | (1u << ROLL_DONE),     /* DECODING */
        (1u << ROLL_TRAJECTORY_READY) | (1u << ROLL_DECODING), /* REWARD_PENDING */
        1u << ROLL_DONE,                                     /* TRAJECTORY_READY */
        1u << ROLL_FREE,                                     /* DONE */
    };
    if ((unsigned)from > ROLL_DONE || (unsigned)to > ROLL_DONE)
        return 0;
    return (allowed[from] >> to) & 1u;
}

static inline const char *
rollout_state_name(rollout_state_t s)
{
    static const char *const names[6] = {"FREE", "PREFILL_READY", "DECODING", "REWARD_PENDING",
                                         "TRAJECTORY_READY", "DONE"};
    return (unsigned)s <= ROLL_DONE ? names[s] : "?";
}
