/*
 * orc_rings.c - oracle: rings, submit, worker rule, descriptor windows, on raw
 * byte images at the reference structs' byte offsets (test infrastructure only).
 */
#include <string.h>

#include "oracle.h"

static uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static void wr32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
static uint16_t rd16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }
static void wr16(uint8_t *p, uint16_t v) { memcpy(p, &v, 2); }
static void wr64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); }

/* include/hw_ring.h:43-55: full when tail - head >= 65536. */
int
orc_hw_ring_push(uint8_t *ring, const uint8_t desc[64])
{
    const uint32_t h = rd32(ring + 0), t = rd32(ring + 64);
    if (t - h >= ORC_HW_RING_SLOTS)
        return -1;
    memcpy(ring + 128 + (size_t)(t % ORC_HW_RING_SLOTS) * 64, desc, 64);
    wr32(ring + 64, t + 1);
    return 0;
}

/* include/hw_ring.h:57-69: empty when head == tail. */
int
orc_hw_ring_pop(uint8_t *ring, uint8_t out[64])
{
    const uint32_t h = rd32(ring + 0), t = rd32(ring + 64);
    if (h == t)
        return -1;
    memcpy(out, ring + 128 + (size_t)(h % ORC_HW_RING_SLOTS) * 64, 64);
    wr32(ring + 0, h + 1);
    return 0;
}

/* src/infer_submit.c:12-32 (the descriptor infer_submit_decode builds) */
void
orc_decode_desc(uint8_t d[64], uint32_t group, uint32_t arena_id, uint32_t rollout, uint64_t kv_off,
                uint64_t delta_off, uint32_t prefix, uint32_t seq, uint32_t max_tokens)
{
    memset(d, 0, 64);
    wr16(d + 0, 1);                       /* DESC_OP_DECODE */
    wr16(d + 2, prefix ? 4 : 0);          /* DESC_FLAG_COW_PREFIX */
    wr32(d + 4, rollout);
    wr32(d + 8, arena_id);
    wr32(d + 12, prefix);
    wr64(d + 16, kv_off);
    wr64(d + 24, delta_off);
    wr32(d + 32, seq);
    wr32(d + 36, max_tokens);
    wr32(d + 40, 0);
    wr32(d + 44, group);
    wr64(d + 48, rollout);
    wr64(d + 56, kv_off ^ delta_off ^ ((uint64_t)rollout << 32));
}

/* src/infer_submit.c:12-36 */
int64_t
orc_submit_decode(uint8_t *cmdq, uint32_t group, uint32_t arena_id, uint32_t rollout, uint64_t kv_off,
                  uint64_t delta_off, uint32_t prefix, uint32_t seq, uint32_t max_tokens)
{
    uint8_t d[64];
    orc_decode_desc(d, group, arena_id, rollout, kv_off, delta_off, prefix, seq, max_tokens);
    if (orc_hw_ring_push(cmdq, d) != 0)
        return -1;
    return rd32(cmdq + 64);
}

/* src/hw_worker_sim.c:23-59 (one pass over what is queued). */
uint64_t
orc_worker_sim_drain(uint8_t *cmdq, uint8_t *doneq, uint64_t *decoded, int *stopped)
{
    uint64_t completions = 0;
    uint8_t d[64];
    *stopped = 0;
    while (orc_hw_ring_pop(cmdq, d) == 0) {
        const uint16_t op = rd16(d);
        if (op == 255) {
            *stopped = 1;
            break;
        }
        if (op != 1)
            continue;
        uint32_t seq = rd32(d + 32);
        const uint32_t max_tokens = rd32(d + 36);
        uint16_t flags = rd16(d + 2);
        while (seq < max_tokens) {
            seq++;
            (*decoded)++;
            if (seq >= max_tokens) {
                flags |= 2; /* DONE */
                break;
            }
            if ((seq % 32u) == 0) {
                flags |= 1; /* NEEDS_REWARD */
                break;
            }
        }
        wr32(d + 32, seq);
        wr16(d + 2, flags);
        if (orc_hw_ring_push(doneq, d) != 0)
            break; /* the simulator would spin; callers keep doneq drained */
        completions++;
    }
    return completions;
}

/* include/ring.h:38-45, include/request.h:85-93 */
uint32_t
orc_ring_acquire(uint8_t *ring, const orc_ring_shape_t *s, uint32_t n)
{
    const uint32_t h = rd32(ring + 0), t = rd32(ring + 64);
    if (s->n_slots - (t - h) < n)
        return UINT32_MAX;
    return t % s->n_slots;
}

/* include/ring.h:49-53 */
void
orc_ring_commit(uint8_t *ring, uint32_t n)
{
    wr32(ring + 64, rd32(ring + 64) + n);
}

/* include/ring.h:60-69 (and the completion/request/done pops) */
int
orc_ring_consume(uint8_t *ring, const orc_ring_shape_t *s, uint8_t *out)
{
    const uint32_t h = rd32(ring + 0), t = rd32(ring + 64);
    if (t - h == 0)
        return 0;
    memcpy(out, ring + s->slot_off + (size_t)(h % s->n_slots) * s->slot_size, s->slot_size);
    wr32(ring + 0, h + 1);
    return 1;
}

/* include/completion.h:63-75, include/request.h:125-138 */
int
orc_ring_push_or_overflow(uint8_t *ring, const orc_ring_shape_t *s, const uint8_t *item)
{
    const uint32_t h = rd32(ring + 0), t = rd32(ring + 64);
    if (s->n_slots - (t - h) < 1) {
        if (s->overflow_off >= 0)
            wr32(ring + s->overflow_off, rd32(ring + s->overflow_off) + 1);
        return -1;
    }
    memcpy(ring + s->slot_off + (size_t)(t % s->n_slots) * s->slot_size, item, s->slot_size);
    wr32(ring + 64, t + 1);
    return 0;
}

/* src/decode_batch.c:20-42 on the 4,096 x 32-byte CommandRing */
int
orc_decode_batch_submit(uint8_t *ring, const uint8_t *descs, uint32_t count)
{
    const orc_ring_shape_t s = {32, 4096, 128, -1};
    if (count == 0 || count > 32)
        return -1;
    const uint32_t pos = orc_ring_acquire(ring, &s, count);
    if (pos == UINT32_MAX)
        return -1;
    for (uint32_t i = 0; i < count; i++) {
        uint8_t *slot = ring + 128 + (size_t)((pos + i) % 4096u) * 32;
        memcpy(slot, descs + (size_t)i * 32, 32);
        wr16(slot + 28, (uint16_t)count);
        wr16(slot + 30, (uint16_t)i);
    }
    orc_ring_commit(ring, count);
    return 0;
}
