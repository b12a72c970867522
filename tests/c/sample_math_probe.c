/* Exports the specification functions of include/rl_sample_math.h (the
 * header-inline code shared by the host and the gfx950 sampler). */
#include "rl_sample_math.h"

void probe_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) { rl_philox4x32_10(ctr, key, out); }
uint64_t probe_draw64(uint64_t seed, uint64_t step, uint32_t row) { return rl_sample_draw64(seed, step, row); }
uint64_t probe_mulhi(uint64_t a, uint64_t b) { return rl_mulhi_u64(a, b); }
float probe_expf_cw(float x) { return rl_expf_cw(x); }
uint32_t probe_weight(float d) { return rl_sample_weight(d); }
uint32_t probe_weight_nb(float d) { return rl_sample_weight_nb(d); }
void probe_weight_pair_many(const float *d, uint32_t *a, uint32_t *b, uint32_t n)
{
    for (uint32_t i = 0; i < n; i++) {
        a[i] = rl_sample_weight(d[i]);
        b[i] = rl_sample_weight_nb(d[i]);
    }
}
/* rl_sample_weight_f next to rl_sample_weight: weights a, b and b's float f */
void probe_weight_f_many(const float *d, uint32_t *a, uint32_t *b, float *f, uint32_t n)
{
    for (uint32_t i = 0; i < n; i++) {
        a[i] = rl_sample_weight(d[i]);
        b[i] = rl_sample_weight_f(d[i], &f[i]);
    }
}
uint32_t probe_key(float x) { return rl_float_key(x); }
float probe_key_float(uint32_t k) { return rl_key_float(k); }
uint64_t probe_topp(float p, uint64_t w) { return rl_topp_threshold(p, w); }
void probe_expf_many(const float *x, float *y, uint32_t n) { for (uint32_t i = 0; i < n; i++) y[i] = rl_expf_cw(x[i]); }
