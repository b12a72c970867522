/*
 * reward.h - rollout reward rule and GRPO group advantage.
 *
 * RewardDesc is byte-compatible with the reference (include/reward.h:6-15,
 * 24 B packed). The scoring rule is the reference's
 * (src/reward.c:36-41, cu/reward.cu:11): score = (count & 0xFF) / 255.0f.
 *
 * The rollout loop applies that rule to a target sequence: `count` is the
 * number of positions i < n where tokens[i] == target[i]
 * (reward_match_count). The group advantage over each group of `group_size`
 * consecutive rewards is A_i = (r_i - mean) / std with the population std
 * (divide by group_size), mean and std accumulated in double in index order;
 * a group whose std is 0 gets A = 0 for every member.
 *
 * RewardRing is the reference's 1,024-entry SPSC handoff of RewardDescs from
 * the rollout pipeline to the reward stage (include/reward.h:17-31,
 * src/reward.c:6-34): producer line @0, consumer line @64, slots @128
 * (24,704 B). push fails (-1) when 1,024 are queued, pop when none is; the
 * empty test is head == tail (wrap-safe, like the id queues of pipeline.h).
 */
#pragma once

#include <stdint.h>
#include "rl_abi.h"

typedef struct __attribute__((packed)) {
    uint32_t rollout_id;
    uint32_t token_start;
    uint32_t token_count;
    uint32_t reward_model_id;
    float reward;
    uint32_t flags;
} RewardDesc;

RL_STATIC_ASSERT(sizeof(RewardDesc) == 24, "RewardDesc must be 24 bytes");

#define REWARD_RING_SIZE 1024

typedef struct __attribute__((packed)) {
    volatile uint32_t head __attribute__((aligned(64)));
    uint32_t tail;
    uint8_t pad[56];
} RewardIndex;

typedef struct {
    RewardIndex prod __attribute__((aligned(64)));  /* prod.head: next write */
    RewardIndex cons __attribute__((aligned(64)));  /* cons.tail: next read */
    RewardDesc slots[REWARD_RING_SIZE] __attribute__((aligned(128)));
} RewardRing;

RL_STATIC_ASSERT(RL_OFFSETOF(RewardRing, slots) == 128, "RewardRing.slots");
RL_STATIC_ASSERT(sizeof(RewardRing) == 24704, "RewardRing size");

RL_EXTERN_C_BEGIN

/* src/reward.c:5-34 */
void reward_ring_init(RewardRing *r);
int reward_push(RewardRing *r, const RewardDesc *d);
int reward_pop(RewardRing *r, RewardDesc *d);

/* Reference export: tokens is ignored, n is the token count. */
float reward_score_mock(const void *tokens, uint32_t n);

/* Number of i < n with tokens[i] == target[i]. */
uint32_t reward_match_count(const uint32_t *tokens, const uint32_t *target, uint32_t n);

/* A_i = (r_i - mean_g) / std_g over consecutive groups; returns -1 on NULL
 * pointers or group_size == 0. */
int reward_group_advantage(const float *rewards, uint32_t n_groups, uint32_t group_size,
                           float *advantage);

RL_EXTERN_C_END

static inline float
reward_score_count(uint32_t count)
{
    return (float)(count & 0xFFu) / 255.0f;
}
