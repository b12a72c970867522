// reward.hip - per-rollout reward and GRPO group advantage on the device.
//
// Replaces reward_score_kernel (cu/reward.cu:4-15) and adds the group
// advantage (no reference function). One workgroup per group of rollouts:
//  count   matches of each member's generated tokens against the group's
//          target sequence at positions i < min(n, target_len, token_stride) (all
//          256 threads stride the tokens; LDS atomics per member);
//  reward  (count & 0xFF) / 255.0f, the reference rule (src/reward.c:36-41);
//  advantage A_i = (r_i - mean) / std, population std, accumulated in double
//          in member order by one thread, 0 when std is 0 - the same
//          operations as reward_group_advantage on the host, so the floats
//          agree bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "reward.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMaxGroup = 64;

struct RewardParams {
    const uint32_t *tokens;
    const uint32_t *n_tokens;
    const uint32_t *targets;
    uint32_t group_size, token_stride, target_stride, target_len;
    RewardDesc *descs;
    float *reward;
    float *advantage;
};

__global__ __launch_bounds__(kThreads) void reward_advantage_kernel(RewardParams p)
{
    __shared__ uint32_t s_count[kMaxGroup];
    const uint32_t g = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    if (tid < p.group_size)
        s_count[tid] = 0;
    __syncthreads();
    const uint32_t *target = p.targets + (size_t)g * p.target_stride;
    for (uint32_t m = 0; m < p.group_size; m++) {
        const uint32_t r = g * p.group_size + m;
        // positions past the target never match; n never exceeds the token row
        const uint32_t n = min(min(p.n_tokens[r], p.target_len), p.token_stride);
        const uint32_t *tok = p.tokens + (size_t)r * p.token_stride;
        uint32_t c = 0;
        for (uint32_t j = tid; j < n; j += kThreads)
            c += tok[j] == target[j] ? 1u : 0u;
        if (c)
            atomicAdd(&s_count[m], c);
    }
    __syncthreads();
    if (tid != 0)
        return;
    double sum = 0.0;
    for (uint32_t m = 0; m < p.group_size; m++) {
        const float rw = (float)(s_count[m] & 0xFFu) / 255.0f;
        const uint32_t r = g * p.group_size + m;
        p.reward[r] = rw;
        if (p.descs) {
            RewardDesc d;
            d.rollout_id = r;
            d.token_start = 0;
            d.token_count = s_count[m];
            d.reward_model_id = 0;
            d.reward = rw;
            d.flags = 0;
            p.descs[r] = d;
        }
        sum += (double)rw;
    }
    const double mean = sum / (double)p.group_size;
    double ss = 0.0;
    for (uint32_t m = 0; m < p.group_size; m++) {
        const double d = (double)p.reward[g * p.group_size + m] - mean;
        ss += d * d;
    }
    const double sd = sqrt(ss / (double)p.group_size);
    for (uint32_t m = 0; m < p.group_size; m++) {
        const uint32_t r = g * p.group_size + m;
        p.advantage[r] = sd > 0.0 ? (float)(((double)p.reward[r] - mean) / sd) : 0.0f;
    }
}

}  // namespace

extern "C" int rl_hip_reward_advantage(const rl_reward_args_t *a)
{
    if (rl_require_open("rl_hip_reward_advantage"))
        return -1;
    if (!a || !a->tokens || !a->n_tokens || !a->targets || !a->reward || !a->advantage) {
        rl_set_error("rl_hip_reward_advantage: NULL argument");
        return -1;
    }
    if (a->group_size == 0 || a->group_size > kMaxGroup || a->rollouts % a->group_size != 0 ||
        a->rollouts == 0) {
        rl_set_error("rl_hip_reward_advantage: %u rollouts in groups of %u (1..%u, dividing the rollouts)",
                     a->rollouts, a->group_size, kMaxGroup);
        return -1;
    }
    if (a->target_len > a->target_stride) {
        rl_set_error("rl_hip_reward_advantage: target_len %u exceeds target_stride %u", a->target_len,
                     a->target_stride);
        return -1;
    }
    RewardParams p;
    p.tokens = a->tokens;
    p.n_tokens = a->n_tokens;
    p.targets = a->targets;
    p.group_size = a->group_size;
    p.token_stride = a->token_stride;
    p.target_stride = a->target_stride;
    p.target_len = a->target_len;
    p.descs = a->descs;
    p.reward = a->reward;
    p.advantage = a->advantage;
    hipLaunchKernelGGL(reward_advantage_kernel, dim3(a->rollouts / a->group_size), dim3(kThreads), 0, rl_stream(),
                       p);
    return rl_check_launch("reward_advantage_kernel launch");
}
