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
 * (The reference's RewardRing handoff is not part of this runtime.)
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

RL_EXTERN_C_BEGIN

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
