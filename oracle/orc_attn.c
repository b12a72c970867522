/*
 * orc_attn.c - oracle: paged GQA single-query decode attention
 * (test infrastructure only).
 *
 * Generalises the reference computation (cu/attention_decode.cu:60-204 and
 * its host reference test/test_bench.cu:109-155: scores q.k * scale, softmax,
 * weighted sum of V) to a block table over a paged arena, GQA groups and
 * batches. orc_attn_decode_f64 is the fp64 truth; orc_attn_decode_f32 is the
 * fp32 online-softmax CPU baseline (16-token tiles, OpenMP over rollout x
 * KV head), the same math the device kernel performs.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

double
orc_bf16_to_f64(uint16_t v)
{
    const uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

double
orc_f16_to_f64(uint16_t v)
{
    const int s = (v >> 15) & 1, e = (v >> 10) & 31, m = v & 1023;
    double r;
    if (e == 0)
        r = ldexp((double)m, -24);
    else if (e == 31)
        r = m ? NAN : INFINITY;
    else
        r = ldexp((double)(m | 1024), e - 25);
    return s ? -r : r;
}

/* fp16 -> fp32 by fields (exact): zero / subnormal m * 2^-24, inf / NaN, or
 * the rebiased exponent with the mantissa shifted into place. */
static inline float
f16_to_f32(uint16_t v)
{
    const uint32_t s = (uint32_t)(v & 0x8000u) << 16, e = (v >> 10) & 31u, m = v & 1023u;
    uint32_t u;
    if (e == 0) {
        const float r = (float)m * 5.9604644775390625e-8f; /* 2^-24 */
        memcpy(&u, &r, 4);
        u |= s;
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float
to_f32(uint16_t v, uint32_t dtype)
{
    if (dtype == 0) {
        const uint32_t u = (uint32_t)v << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
    return f16_to_f32(v);
}

/* Address of token t's K (plane 0) or V (plane 1) row for (b, g). */
static const uint16_t *
kv_row(const orc_attn_t *a, uint32_t b, uint32_t g, uint32_t t, int plane)
{
    const uint32_t row_bytes = a->head_dim * 2u;
    const uint32_t blk = a->table[((size_t)b * a->kv_heads + g) * a->table_stride + t / a->token_count];
    const uint8_t *base = a->arena + (uint64_t)blk * a->block_bytes;
    return (const uint16_t *)(base + (size_t)plane * a->token_count * row_bytes +
                              (size_t)(t % a->token_count) * row_bytes);
}

void
orc_attn_decode_f64(const orc_attn_t *a, double *out)
{
    const uint32_t G = a->q_heads / a->kv_heads, D = a->head_dim;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (uint32_t b = 0; b < a->batch; b++) {
        for (uint32_t h = 0; h < a->q_heads; h++) {
            const uint32_t g = h / G, ctx = a->ctx[b];
            double *o = out + ((size_t)b * a->q_heads + h) * D;
            memset(o, 0, D * sizeof(double));
            if (ctx == 0)
                continue;
            const uint16_t *q = a->q + ((size_t)b * a->q_heads + h) * D;
            double *s = (double *)malloc(ctx * sizeof(double));
            double m = -INFINITY;
            for (uint32_t t = 0; t < ctx; t++) {
                const uint16_t *k = kv_row(a, b, g, t, 0);
                double dot = 0.0;
                for (uint32_t d = 0; d < D; d++)
                    dot += (a->dtype == 0 ? orc_bf16_to_f64(q[d]) * orc_bf16_to_f64(k[d])
                                          : orc_f16_to_f64(q[d]) * orc_f16_to_f64(k[d]));
                s[t] = dot * a->scale;
                if (s[t] > m)
                    m = s[t];
            }
            double l = 0.0;
            for (uint32_t t = 0; t < ctx; t++) {
                const double pw = exp(s[t] - m);
                l += pw;
                const uint16_t *v = kv_row(a, b, g, t, 1);
                for (uint32_t d = 0; d < D; d++)
                    o[d] += pw * (a->dtype == 0 ? orc_bf16_to_f64(v[d]) : orc_f16_to_f64(v[d]));
            }
            for (uint32_t d = 0; d < D; d++)
                o[d] /= l;
            free(s);
        }
    }
}

void
orc_attn_decode_f32(const orc_attn_t *a, float *out)
{
    const uint32_t G = a->q_heads / a->kv_heads, D = a->head_dim;
    const float scale = (float)a->scale;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (uint32_t b = 0; b < a->batch; b++) {
        for (uint32_t g = 0; g < a->kv_heads; g++) {
            const uint32_t ctx = a->ctx[b];
            float q[8][128], acc[8][128], mrun[8], lrun[8];
            for (uint32_t i = 0; i < G; i++) {
                const uint16_t *qs = a->q + ((size_t)b * a->q_heads + g * G + i) * D;
                for (uint32_t d = 0; d < D; d++) {
                    q[i][d] = to_f32(qs[d], a->dtype);
                    acc[i][d] = 0.f;
                }
                mrun[i] = -INFINITY;
                lrun[i] = 0.f;
            }
            float krow[128], vrow[128];
            for (uint32_t t0 = 0; t0 < ctx; t0 += 16) {
                const uint32_t nt = ctx - t0 < 16 ? ctx - t0 : 16;
                float s[8][16];
                for (uint32_t j = 0; j < nt; j++) {
                    const uint16_t *k = kv_row(a, b, g, t0 + j, 0);
                    for (uint32_t d = 0; d < D; d++)
                        krow[d] = to_f32(k[d], a->dtype);
                    for (uint32_t i = 0; i < G; i++) {
                        float dot = 0.f;
                        for (uint32_t d = 0; d < D; d++)
                            dot += q[i][d] * krow[d];
                        s[i][j] = dot * scale;
                    }
                }
                for (uint32_t i = 0; i < G; i++) {
                    float mx = mrun[i];
                    for (uint32_t j = 0; j < nt; j++)
                        mx = s[i][j] > mx ? s[i][j] : mx;
                    const float alpha = expf(mrun[i] - mx);
                    lrun[i] *= alpha;
                    for (uint32_t d = 0; d < D; d++)
                        acc[i][d] *= alpha;
                    for (uint32_t j = 0; j < nt; j++) {
                        s[i][j] = expf(s[i][j] - mx);
                        lrun[i] += s[i][j];
                    }
                    mrun[i] = mx;
                }
                for (uint32_t j = 0; j < nt; j++) {
                    const uint16_t *v = kv_row(a, b, g, t0 + j, 1);
                    for (uint32_t d = 0; d < D; d++)
                        vrow[d] = to_f32(v[d], a->dtype);
                    for (uint32_t i = 0; i < G; i++)
                        for (uint32_t d = 0; d < D; d++)
                            acc[i][d] += s[i][j] * vrow[d];
                }
            }
            for (uint32_t i = 0; i < G; i++) {
                float *o = out + ((size_t)b * a->q_heads + g * G + i) * D;
                for (uint32_t d = 0; d < D; d++)
                    o[d] = lrun[i] > 0.f ? acc[i][d] / lrun[i] : 0.f;
            }
        }
    }
}

/* The fixed128 step's query when no q buffer is given
 * (decode_synth_query_component, cu/attention_decode.cu:16-28):
 * seed = seq_id ^ reward_cookie ^ (idx + 1) * 0x9e3779b97f4a7c15
 * [^ rng_state[idx & 3]]; bits = low 32 of seed ^ (seed >> 32);
 * q = ((bits & 0xFF) - 127) / 127. */
float
orc_synth_query(uint64_t seq_id, uint64_t reward_cookie, const uint64_t *rng_state, uint32_t idx)
{
    uint64_t seed = seq_id ^ reward_cookie ^ ((uint64_t)(idx + 1u) * 0x9e3779b97f4a7c15ULL);
    if (rng_state)
        seed ^= rng_state[idx & 3u];
    const uint32_t bits = (uint32_t)(seed ^ (seed >> 32));
    const int centered = (int)(bits & 0xFFu) - 127;
    return (float)centered / 127.0f;
}
