/*
 * orc_kv.c - oracle: one-token KV append with copy-on-write of a partially
 * filled shared block (test infrastructure only). The reference only
 * refcounts prefixes (src/kv_prefix.c:66-149); the copy restated here is the
 * behaviour of rl_hip_kv_append.
 */
#include <string.h>

#include "oracle.h"

#ifdef _OPENMP
#include <omp.h>
#endif

void
orc_kv_append(uint8_t *arena, uint64_t block_bytes, uint32_t token_count, uint32_t row_bytes,
              const uint32_t *table, uint32_t stride, uint32_t batch, uint32_t kv_heads,
              const uint32_t *positions, const int32_t *cow_src, const uint8_t *k_new, const uint8_t *v_new)
{
    for (uint32_t b = 0; b < batch; b++) {
        for (uint32_t g = 0; g < kv_heads; g++) {
            const uint32_t row = b * kv_heads + g, pos = positions[b];
            const uint32_t slot = pos % token_count;
            if (pos / token_count >= stride)
                continue;
            uint8_t *dst = arena + (uint64_t)table[(size_t)row * stride + pos / token_count] * block_bytes;
            if (cow_src && cow_src[row] >= 0 && slot > 0) {
                const uint8_t *src = arena + (uint64_t)(uint32_t)cow_src[row] * block_bytes;
                memcpy(dst, src, (size_t)slot * row_bytes);                           /* K rows */
                memcpy(dst + (size_t)token_count * row_bytes, src + (size_t)token_count * row_bytes,
                       (size_t)slot * row_bytes);                                    /* V rows */
            }
            memcpy(dst + (size_t)slot * row_bytes, k_new + (size_t)row * row_bytes, row_bytes);
            memcpy(dst + (size_t)token_count * row_bytes + (size_t)slot * row_bytes,
                   v_new + (size_t)row * row_bytes, row_bytes);
        }
    }
}

void
orc_set_num_threads(int n)
{
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int
orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
