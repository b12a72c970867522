/*
 * orc_tables.c - oracle: arena bitmap and kv_prefix table on raw images;
 * reward rule; group advantage; Philox4x32-10 (test infrastructure only).
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* src/arena.c:31-51: lowest clear bit of 16,384 words (1 = used). */
int64_t
orc_arena_acquire(uint64_t *bitmap)
{
    for (int64_t i = 0; i < 16384 * 64; i++) {
        if (!((bitmap[i / 64] >> (i % 64)) & 1u)) {
            bitmap[i / 64] |= 1ull << (i % 64);
            return i;
        }
    }
    return -1;
}

void
orc_arena_release(uint64_t *bitmap, int64_t idx)
{
    if (idx >= 0)
        bitmap[idx / 64] &= ~(1ull << (idx % 64));
}

/* KVPrefixTable byte offsets (packed KVPrefix 28 B, KVBranch 36 B). */
#define P_BASE(id) ((size_t)(id) * 28u)
#define P_BITMAP 14336u
#define B_BASE(id) (14400u + (size_t)(id) * 36u)
#define B_BITMAP 604224u
#define N_PREFIX 512u
#define N_BRANCH 16384u

static uint32_t g32(const uint8_t *t, size_t off) { uint32_t v; memcpy(&v, t + off, 4); return v; }
static void s32(uint8_t *t, size_t off, uint32_t v) { memcpy(t + off, &v, 4); }
static int64_t g64(const uint8_t *t, size_t off) { int64_t v; memcpy(&v, t + off, 8); return v; }
static void s64(uint8_t *t, size_t off, int64_t v) { memcpy(t + off, &v, 8); }
static int bit_get(const uint8_t *t, size_t bm, uint32_t id)
{
    uint64_t w;
    memcpy(&w, t + bm + (id / 64u) * 8u, 8);
    return (int)((w >> (id % 64u)) & 1u);
}
static void bit_put(uint8_t *t, size_t bm, uint32_t id, int v)
{
    uint64_t w;
    memcpy(&w, t + bm + (id / 64u) * 8u, 8);
    w = v ? (w | (1ull << (id % 64u))) : (w & ~(1ull << (id % 64u)));
    memcpy(t + bm + (id / 64u) * 8u, &w, 8);
}

/* src/kv_prefix.c:5-19: zero, then every id free (1). */
void
orc_kvp_init(uint8_t *t)
{
    memset(t, 0, ORC_PREFIX_TABLE_BYTES);
    for (uint32_t i = 0; i < N_PREFIX; i++)
        bit_put(t, P_BITMAP, i, 1);
    for (uint32_t i = 0; i < N_BRANCH; i++)
        bit_put(t, B_BITMAP, i, 1);
}

static int
take_lowest(uint8_t *t, size_t bm, uint32_t n, uint32_t *out)
{
    for (uint32_t i = 0; i < n; i++)
        if (bit_get(t, bm, i)) {
            bit_put(t, bm, i, 0);
            *out = i;
            return 0;
        }
    return -1;
}

/* src/kv_prefix.c:45-64 */
int
orc_kvp_register(uint8_t *t, int64_t off, uint32_t len, uint32_t nblocks, uint32_t *out_id)
{
    uint32_t id;
    if (take_lowest(t, P_BITMAP, N_PREFIX, &id) != 0)
        return -1;
    s32(t, P_BASE(id) + 0, id);
    s32(t, P_BASE(id) + 4, 1);
    s64(t, P_BASE(id) + 8, off);
    s32(t, P_BASE(id) + 16, len);
    s32(t, P_BASE(id) + 20, nblocks);
    s32(t, P_BASE(id) + 24, 0);
    *out_id = id;
    return 0;
}

/* src/kv_prefix.c:66-74 */
int
orc_kvp_acquire(uint8_t *t, uint32_t id)
{
    if (id >= N_PREFIX || g32(t, P_BASE(id) + 4) == 0)
        return -1;
    s32(t, P_BASE(id) + 4, g32(t, P_BASE(id) + 4) + 1);
    return 0;
}

/* src/kv_prefix.c:76-89 */
int
orc_kvp_release(uint8_t *t, uint32_t id)
{
    if (id >= N_PREFIX)
        return -1;
    const uint32_t rc = g32(t, P_BASE(id) + 4);
    if (rc == 0)
        return -1;
    s32(t, P_BASE(id) + 4, rc - 1);
    if (rc - 1 == 0) {
        s64(t, P_BASE(id) + 8, -1);
        s32(t, P_BASE(id) + 16, 0);
        bit_put(t, P_BITMAP, id, 1);
    }
    return 0;
}

/* src/kv_prefix.c:98-121 */
int
orc_kvb_alloc(uint8_t *t, uint32_t rollout, uint32_t prefix, int64_t delta, uint32_t dlen, uint32_t dblocks,
              uint32_t *out_id)
{
    uint32_t id;
    if (take_lowest(t, B_BITMAP, N_BRANCH, &id) != 0)
        return -1;
    s32(t, B_BASE(id) + 0, id);
    s32(t, B_BASE(id) + 4, rollout);
    s32(t, B_BASE(id) + 8, prefix);
    s64(t, B_BASE(id) + 12, delta);
    s32(t, B_BASE(id) + 20, dlen);
    s32(t, B_BASE(id) + 24, dblocks);
    s32(t, B_BASE(id) + 28, 0);
    s32(t, B_BASE(id) + 32, 0);
    (void)orc_kvp_acquire(t, prefix);
    *out_id = id;
    return 0;
}

/* src/kv_prefix.c:123-132 */
int
orc_kvb_free(uint8_t *t, uint32_t id)
{
    if (id >= N_BRANCH)
        return -1;
    (void)orc_kvp_release(t, g32(t, B_BASE(id) + 8));
    s32(t, B_BASE(id) + 4, UINT32_MAX);
    bit_put(t, B_BITMAP, id, 1);
    return 0;
}

/* src/kv_prefix.c:141-149 */
int64_t
orc_kvb_total_offset(const uint8_t *t, uint32_t id)
{
    if (id >= N_BRANCH)
        return -1;
    const uint32_t prefix = g32(t, B_BASE(id) + 8);
    if (prefix >= N_PREFIX)
        return g64(t, B_BASE(id) + 12);
    return g64(t, P_BASE(prefix) + 8);
}

/* cu/kv_prefix.cu:4-15 */
int64_t
orc_kvb_resolve(const uint8_t *t, uint32_t id)
{
    if (id >= N_BRANCH)
        return -1;
    const uint32_t prefix = g32(t, B_BASE(id) + 8);
    if (prefix >= N_PREFIX || g32(t, P_BASE(prefix) + 4) == 0)
        return g64(t, B_BASE(id) + 12);
    return g64(t, P_BASE(prefix) + 8);
}

int64_t
orc_kvb_cow_source(const uint8_t *t, uint32_t branch, uint32_t position, uint32_t tpb, uint32_t kv_heads,
                   uint32_t head)
{
    if (branch >= N_BRANCH)
        return -1;
    const uint32_t prefix = g32(t, B_BASE(branch) + 8);
    if (prefix >= N_PREFIX || g32(t, P_BASE(prefix) + 4) == 0)
        return -1;
    const int64_t off = g64(t, P_BASE(prefix) + 8);
    const uint32_t len = g32(t, P_BASE(prefix) + 16);
    const uint32_t per_head = g32(t, P_BASE(prefix) + 20) / kv_heads;
    if (len % tpb == 0 || position != len || len / tpb >= per_head || off < 0)
        return -1;
    return off + (int64_t)head * per_head + len / tpb;
}

/* src/reward.c:36-41 and cu/reward.cu:11 */
float
orc_reward_score(uint32_t count)
{
    return (float)(count & 0xFFu) / 255.0f;
}

uint32_t
orc_match_count(const uint32_t *tokens, const uint32_t *target, uint32_t n)
{
    uint32_t c = 0;
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] == target[i])
            c++;
    return c;
}

/* A = (r - mean) / std, population std, 0 when std == 0; double, index order. */
void
orc_group_advantage(const float *r, uint32_t n_groups, uint32_t group, float *adv)
{
    for (uint32_t g = 0; g < n_groups; g++) {
        double mean = 0.0, var = 0.0;
        for (uint32_t i = 0; i < group; i++)
            mean += (double)r[g * group + i];
        mean /= (double)group;
        for (uint32_t i = 0; i < group; i++) {
            const double d = (double)r[g * group + i] - mean;
            var += d * d;
        }
        const double sd = sqrt(var / (double)group);
        for (uint32_t i = 0; i < group; i++)
            adv[g * group + i] = sd > 0.0 ? (float)(((double)r[g * group + i] - mean) / sd) : 0.0f;
    }
}

/* Philox4x32-10: ten rounds of (hi0, lo0) = M0 * c0, (hi1, lo1) = M1 * c2,
 * c' = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0), key += Weyl constants. */
void
orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
    uint32_t k[2] = {key[0], key[1]};
    for (int r = 0; r < 10; r++) {
        if (r) {
            k[0] += 0x9E3779B9u;
            k[1] += 0xBB67AE85u;
        }
        const uint64_t a = (uint64_t)0xD2511F53u * c[0];
        const uint64_t b = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(b >> 32) ^ c[1] ^ k[0];
        const uint32_t n2 = (uint32_t)(a >> 32) ^ c[3] ^ k[1];
        c[0] = n0;
        c[1] = (uint32_t)b;
        c[2] = n2;
        c[3] = (uint32_t)a;
    }
    memcpy(out, c, sizeof(c));
}
