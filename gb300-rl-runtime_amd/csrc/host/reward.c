/*
 * reward.c - the reward handoff ring (reference src/reward.c:5-34), the
 * reward rule (src/reward.c:36-41) and the group advantage.
 */
#include <math.h>
#include <stddef.h>
#include <string.h>

#include "reward.h"
#include "spsc_index.h"

void
reward_ring_init(RewardRing *r)
{
    if (r)
        memset(r, 0, sizeof(*r));
}

int
reward_push(RewardRing *r, const RewardDesc *d)
{
    uint32_t slot;
    if (!r || !d || spsc_reserve(&r->prod.head, &r->cons.tail, REWARD_RING_SIZE, &slot) != 0)
        return -1;
    r->slots[slot] = *d;
    spsc_publish(&r->prod.head);
    return 0;
}

int
reward_pop(RewardRing *r, RewardDesc *d)
{
    uint32_t slot;
    if (!r || !d || spsc_peek(&r->prod.head, &r->cons.tail, REWARD_RING_SIZE, &slot) != 0)
        return -1;
    *d = r->slots[slot];
    spsc_retire(&r->cons.tail);
    return 0;
}

float
reward_score_mock(const void *tokens, uint32_t n)
{
    (void)tokens;
    return reward_score_count(n);
}

uint32_t
reward_match_count(const uint32_t *tokens, const uint32_t *target, uint32_t n)
{
    uint32_t c = 0;
    if (!tokens || !target)
        return 0;
    for (uint32_t i = 0; i < n; i++)
        c += tokens[i] == target[i];
    return c;
}

int
reward_group_advantage(const float *rewards, uint32_t n_groups, uint32_t group_size,
                       float *advantage)
{
    if (!rewards || !advantage || group_size == 0)
        return -1;
    for (uint32_t g = 0; g < n_groups; g++) {
        const float *r = rewards + (size_t)g * group_size;
        float *a = advantage + (size_t)g * group_size;
        double sum = 0.0;
        for (uint32_t i = 0; i < group_size; i++)
            sum += (double)r[i];
        const double mean = sum / (double)group_size;
        double ss = 0.0;
        for (uint32_t i = 0; i < group_size; i++) {
            const double d = (double)r[i] - mean;
            ss += d * d;
        }
        const double sd = sqrt(ss / (double)group_size);
        for (uint32_t i = 0; i < group_size; i++)
            a[i] = sd > 0.0 ? (float)(((double)r[i] - mean) / sd) : 0.0f;
    }
    return 0;
}
