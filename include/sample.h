/*
 * sample.h - per-trajectory sampling state (ABI type) and the sampling
 * specification of this runtime.
 *
 * SampleState keeps the reference's 48-byte layout (include/sample.h:14-20;
 * the reference comment calls it 64 bytes, the struct is 48). Its rng_state
 * field is not used by this runtime: draws come from a counter-based
 * Philox4x32-10 stream keyed by the request seed instead of xoshiro256**.
 *
 * Sampling of one row of logits l[0..V) (reference cu/sample.cu:41-123
 * restated, with the nucleus made real):
 *  1. greedy (temperature <= 0): token = argmax l, lowest index on ties;
 *     logprob = l[tok] - logsumexp(l).
 *  2. x_i = l_i * inv_t, inv_t = 1.0f / temperature (fp32, round-to-nearest).
 *  3. top-k (0 < k < V): k_eff = min(k, 256); cutoff = k_eff-th largest x
 *     counted with multiplicity; keep K = {i : x_i >= cutoff} (ties at the
 *     cutoff all survive, as in the reference). Otherwise K = all.
 *  4. weights: m = max_i x_i; w_i = floor(rl_expf_cw(x_i - m) * 2^24) as an
 *     integer (rl_sample_math.h), so every sum below is exact and
 *     independent of summation order.
 *  5. top-p (0 < p < 1): order K by (x desc, index asc); keep the shortest
 *     prefix P whose weight sum reaches ceil(p * W_K) (computed in double),
 *     at least one element. Otherwise P = K.
 *  6. draw: (r0, r1, r2, r3) = Philox4x32-10(key = (seed lo, seed hi),
 *     ctr = (step lo, step hi, id, 0)), id the row's draw id (the row
 *     index unless the caller names the stream, e.g. by its rollout id);
 *     r64 = r0 | r1 << 32;
 *     u = floor(r64 * W_P / 2^64). The token is the smallest index i in P
 *     whose ascending-index prefix weight sum exceeds u.
 *  7. logprob = x_tok - logsumexp(x) over the whole vocabulary (the
 *     temperature-scaled policy distribution before truncation).
 */
#pragma once

#include <stdint.h>
#include "rl_abi.h"

#define MAX_VOCAB_SIZE 131072
#define RL_SAMPLE_TOPK_MAX 256u
#define RL_SAMPLE_WEIGHT_BITS 24

typedef struct {
    uint64_t rng_state[4];
    float temperature;
    uint16_t top_k;
    float top_p;
    uint32_t vocab_size;
} SampleState;

RL_STATIC_ASSERT(sizeof(SampleState) == 48, "SampleState size");
RL_STATIC_ASSERT(RL_OFFSETOF(SampleState, top_p) == 40, "SampleState.top_p");
