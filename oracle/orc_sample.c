/*
 * orc_sample.c - oracle: sampling by the specification in include/sample.h
 * (test infrastructure only).
 *
 * Restates cu/sample.cu:41-123 (temperature multiply by 1/T; top-k cutoff
 * taken as the k-th largest value with multiplicity and ties kept; inverse
 * CDF walk) with a real nucleus, a Philox4x32-10 draw and 24-bit integer
 * weights. Written with a min-heap for top-k and qsort for ordering, i.e. by
 * a different route than the device kernels; the weight function
 * rl_sample_weight and nucleus threshold rl_topp_threshold are part of the
 * specification and are shared (they are pinned against libm in tests/).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "rl_sample_math.h"

/* cu/sample.cu:55: the insertion buffer holds at most 256 entries. */
#define ORC_TOPK_CAP 256u

typedef struct {
    float x;
    uint32_t idx;
    uint64_t w;
} cand_t;

/* sorted by x descending, then index ascending */
static int
cmp_desc(const void *pa, const void *pb)
{
    const cand_t *a = pa, *b = pb;
    if (a->x != b->x)
        return a->x > b->x ? -1 : 1;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

static int
cmp_idx(const void *pa, const void *pb)
{
    const cand_t *a = pa, *b = pb;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

/* k-th largest value counted with multiplicity: min-heap of the k largest. */
static float
kth_largest(const float *x, uint32_t n, uint32_t k)
{
    float *heap = (float *)malloc(k * sizeof(float));
    uint32_t size = 0;
    for (uint32_t i = 0; i < n; i++) {
        const float v = x[i];
        if (size < k) {
            uint32_t c = size++;
            heap[c] = v;
            while (c > 0 && heap[(c - 1) / 2] > heap[c]) {
                const float t = heap[c];
                heap[c] = heap[(c - 1) / 2];
                heap[(c - 1) / 2] = t;
                c = (c - 1) / 2;
            }
        } else if (v > heap[0]) {
            heap[0] = v;
            uint32_t c = 0;
            for (;;) {
                uint32_t l = 2 * c + 1, r = l + 1, m = c;
                if (l < size && heap[l] < heap[m])
                    m = l;
                if (r < size && heap[r] < heap[m])
                    m = r;
                if (m == c)
                    break;
                const float t = heap[c];
                heap[c] = heap[m];
                heap[m] = t;
                c = m;
            }
        }
    }
    const float r = heap[0];
    free(heap);
    return r;
}

static double
logsumexp_f64(const float *x, uint32_t n)
{
    double m = -INFINITY;
    for (uint32_t i = 0; i < n; i++)
        if ((double)x[i] > m)
            m = x[i];
    if (m == -INFINITY)
        return -INFINITY;
    double s = 0.0;
    for (uint32_t i = 0; i < n; i++)
        s += exp((double)x[i] - m);
    return m + log(s);
}

uint32_t
orc_sample_row(const float *l, uint32_t vocab, int greedy, float temperature, uint32_t top_k, float top_p,
               uint64_t seed, uint64_t step, uint32_t row, double *logprob)
{
    if (greedy || !(temperature > 0.f)) {
        uint32_t best = 0;
        for (uint32_t i = 1; i < vocab; i++)
            if (l[i] > l[best])
                best = i;
        *logprob = (double)l[best] - logsumexp_f64(l, vocab);
        return best;
    }

    const float inv_t = 1.0f / temperature;
    float *x = (float *)malloc(vocab * sizeof(float));
    float m = -INFINITY;
    for (uint32_t i = 0; i < vocab; i++) {
        x[i] = l[i] * inv_t;
        if (x[i] > m)
            m = x[i];
    }

    uint32_t k_eff = 0;
    if (top_k > 0 && top_k < vocab)
        k_eff = top_k < ORC_TOPK_CAP ? top_k : ORC_TOPK_CAP;
    const float cutoff = k_eff ? kth_largest(x, vocab, k_eff) : -INFINITY;

    cand_t *kept = (cand_t *)malloc(vocab * sizeof(cand_t));
    uint32_t nk = 0;
    for (uint32_t i = 0; i < vocab; i++)
        if (x[i] >= cutoff && x[i] != -INFINITY)
            kept[nk++] = (cand_t){x[i], i, 0};
    qsort(kept, nk, sizeof(cand_t), cmp_desc);

    uint64_t wk = 0;
    for (uint32_t i = 0; i < nk; i++) {
        kept[i].w = rl_sample_weight(kept[i].x - m);
        wk += kept[i].w;
    }
    uint32_t np = nk;
    if (top_p > 0.f && top_p < 1.f) {
        const uint64_t thr = rl_topp_threshold(top_p, wk);
        uint64_t c = 0;
        np = 0;
        while (np < nk) {
            c += kept[np++].w;
            if (c >= thr)
                break;
        }
        if (np == 0 && nk > 0) /* at least one element of a non-empty kept set */
            np = 1;
    }
    uint64_t wp = 0;
    for (uint32_t i = 0; i < np; i++)
        wp += kept[i].w;

    /* Philox draw: key = seed, counter = (step, row) */
    uint32_t ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), row, 0};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    orc_philox4x32_10(ctr, key, out);
    const uint64_t r64 = (uint64_t)out[0] | ((uint64_t)out[1] << 32);
    const uint64_t u = (uint64_t)(((unsigned __int128)r64 * (unsigned __int128)wp) >> 64);

    /* ascending-index walk over P (weights travel with their elements) */
    qsort(kept, np, sizeof(cand_t), cmp_idx);
    uint32_t tok = np ? kept[0].idx : 0;
    uint64_t c = 0;
    for (uint32_t i = 0; i < np; i++) {
        c += kept[i].w;
        if (c > u) {
            tok = kept[i].idx;
            break;
        }
    }
    *logprob = (double)x[tok] - logsumexp_f64(x, vocab);
    free(kept);
    free(x);
    return tok;
}

void
orc_sample_rows(const float *logits, uint32_t rows, uint32_t vocab, uint32_t stride, int greedy,
                float temperature, uint32_t top_k, float top_p, const uint64_t *seeds, uint64_t step,
                uint32_t *tokens, double *logprobs)
{
#pragma omp parallel for schedule(dynamic)
    for (uint32_t r = 0; r < rows; r++)
        tokens[r] = orc_sample_row(logits + (size_t)r * stride, vocab, greedy, temperature, top_k, top_p, seeds[r],
                                   step, r, &logprobs[r]);
}

/* orc_sample_rows with per-row parameters (any of the arrays may be NULL: the
 * scalar then serves every row) and per-row draw ids (NULL: the row index),
 * OpenMP over rows. */
void
orc_sample_rows_v(const float *logits, uint32_t rows, uint32_t vocab, uint32_t stride, const float *temperature,
                  const uint32_t *top_k, const float *top_p, const uint64_t *seeds, const uint64_t *steps,
                  const uint32_t *draw_ids, float temperature_all, uint32_t top_k_all, float top_p_all,
                  uint64_t step_all, uint32_t *tokens, double *logprobs)
{
#pragma omp parallel for schedule(dynamic)
    for (uint32_t r = 0; r < rows; r++) {
        const float t = temperature ? temperature[r] : temperature_all;
        tokens[r] = orc_sample_row(logits + (size_t)r * stride, vocab, !(t > 0.f), t, top_k ? top_k[r] : top_k_all,
                                   top_p ? top_p[r] : top_p_all, seeds ? seeds[r] : 0u, steps ? steps[r] : step_all,
                                   draw_ids ? draw_ids[r] : r, &logprobs[r]);
    }
}
