/*
 * trace.c - the 20-byte trace ring and its latency report (reference
 * src/trace.c:1-149; contract in include/trace.h), plus the clock map and
 * merge that let device-stamped rings join the report.
 */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "trace.h"

uint64_t
trace_now_ns(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

void
trace_init(TraceRing *r)
{
    if (r)
        memset(r, 0, sizeof(*r));
}

void
trace_push_ts(TraceRing *r, uint64_t tsc, trace_event_t type, uint32_t rollout_id, uint32_t seq)
{
    if (!r)
        return;
    const uint64_t h = __atomic_load_n(&r->head, __ATOMIC_RELAXED);   /* single producer */
    trace_entry_t *e = &r->entries[h & (TRACE_CAPACITY - 1)];
    e->tsc = tsc;
    e->type = (uint32_t)type;
    e->rollout_id = rollout_id;
    e->seq = seq;
    __atomic_store_n(&r->head, h + 1, __ATOMIC_RELEASE);
}

void
trace_push(TraceRing *r, trace_event_t type, uint32_t rollout_id, uint32_t seq)
{
    trace_push_ts(r, trace_now_ns(), type, rollout_id, seq);
}

static uint64_t
ring_count(const TraceRing *r)
{
    const uint64_t h = __atomic_load_n(&r->head, __ATOMIC_ACQUIRE);
    return h < TRACE_CAPACITY ? h : TRACE_CAPACITY;
}

/* Latencies of the (start, end) pairs. Two cursors walk the entries in index
 * order: the start cursor stops only at start events, the end cursor only at
 * end events; when both stand on one, the pair counts if the keys
 * (rollout_id, seq) agree and the end is not earlier, and both cursors move
 * on either way (the reference's rule, src/trace.c:65-96). */
static uint64_t
pair_latencies(const trace_entry_t *e, uint64_t count, uint32_t start, uint32_t end, uint64_t *lat)
{
    uint64_t n = 0, s = 0, t = 0;
    while (s < count && t < count) {
        const trace_entry_t *a = &e[s], *b = &e[t];
        if (a->type != start) {
            s++;
            continue;
        }
        if (b->type != end) {
            t++;
            continue;
        }
        if (a->rollout_id == b->rollout_id && a->seq == b->seq && b->tsc >= a->tsc)
            lat[n++] = b->tsc - a->tsc;
        s++;
        t++;
    }
    return n;
}

static int
u64_order(const void *x, const void *y)
{
    const uint64_t a = *(const uint64_t *)x, b = *(const uint64_t *)y;
    return (a > b) - (a < b);
}

int
trace_pair_stats(const TraceRing *r, trace_event_t start, trace_event_t end, trace_pair_stats_t *out)
{
    if (!r || !out)
        return -1;
    memset(out, 0, sizeof(*out));
    const uint64_t count = ring_count(r);
    if (count == 0)
        return 0;
    uint64_t *lat = (uint64_t *)malloc(count * sizeof(uint64_t));
    if (!lat)
        return -1;
    const uint64_t n = pair_latencies(r->entries, count, (uint32_t)start, (uint32_t)end, lat);
    if (n) {
        qsort(lat, n, sizeof(uint64_t), u64_order);
        uint64_t sum = 0;
        for (uint64_t i = 0; i < n; i++)
            sum += lat[i];
        out->n = n;
        out->avg_ns = sum / n;
        out->p50_ns = lat[n / 2];
        out->p90_ns = lat[n * 9 / 10];
        out->p99_ns = lat[n * 99 / 100];
    }
    free(lat);
    return 0;
}

/* The report's pairs and labels (src/trace.c:130-146). */
static const struct {
    trace_event_t start, end;
    const char *label;
} report_pairs[] = {
    {TRACE_DESC_POSTED, TRACE_DESC_COMMITTED, "descriptor post -> commit"},
    {TRACE_DESC_POSTED, TRACE_DESC_CONSUMED, "descriptor post -> GPU dequeue"},
    {TRACE_DESC_POSTED, TRACE_COMPLETION_POLLED, "descriptor post -> completion polled"},
    {TRACE_DESC_CONSUMED, TRACE_COMPLETION_POLLED, "GPU dequeue -> completion polled"},
    {TRACE_ROLLOUT_ALLOC, TRACE_REWARD_POSTED, "rollout alloc -> reward posted"},
    {TRACE_ROLLOUT_ALLOC, TRACE_TRAJECTORY_DONE, "rollout alloc -> trajectory done"},
    {TRACE_REWARD_POSTED, TRACE_REWARD_SCORED, "reward posted -> scored"},
    {TRACE_REWARD_POSTED, TRACE_TRAJECTORY_DONE, "reward posted -> trajectory done"},
};

int
trace_report_from(const TraceRing *r, uint64_t wall_ns, uint64_t n_tokens, uint64_t n_rollouts,
                  const char *prefix)
{
    (void)n_tokens;
    (void)n_rollouts;
    if (!r)
        return 0;
    printf("\n%sTrace Latency Report (%lu events, %.3f s wall)\n", prefix ? prefix : "",
           (unsigned long)ring_count(r), (double)wall_ns / 1.0e9);
    for (size_t i = 0; i < sizeof(report_pairs) / sizeof(report_pairs[0]); i++) {
        trace_pair_stats_t s;
        if (trace_pair_stats(r, report_pairs[i].start, report_pairs[i].end, &s) != 0)
            continue;
        if (s.n == 0)
            printf("  %-40s  no samples\n", report_pairs[i].label);
        else
            printf("  %-40s  n=%-6lu  avg=%-5lu  p50=%-5lu  p90=%-5lu  p99=%-5lu ns\n", report_pairs[i].label,
                   (unsigned long)s.n, (unsigned long)s.avg_ns, (unsigned long)s.p50_ns, (unsigned long)s.p90_ns,
                   (unsigned long)s.p99_ns);
    }
    fflush(stdout);
    return 0;
}

int
trace_clock_fit(uint64_t ticks0, double host_ns0, uint64_t ticks1, double host_ns1, trace_clock_map_t *out)
{
    if (!out)
        return -1;
    const double dt = (double)(int64_t)(ticks1 - ticks0);
    out->ns_per_tick = dt != 0.0 ? (host_ns1 - host_ns0) / dt : 10.0;
    out->offset_ns = host_ns0 - (double)ticks0 * out->ns_per_tick;
    return 0;
}

void
trace_rebase(TraceRing *r, const trace_clock_map_t *map)
{
    if (!r || !map)
        return;
    const uint64_t count = ring_count(r);
    for (uint64_t i = 0; i < count; i++) {
        const double ns = map->offset_ns + (double)r->entries[i].tsc * map->ns_per_tick;
        r->entries[i].tsc = ns > 0.0 ? (uint64_t)llround(ns) : 0u;
    }
}

uint64_t
trace_merge(TraceRing *dst, const TraceRing *const *src, uint32_t n_src)
{
    enum { kMaxSrc = 16 };
    uint64_t pos[kMaxSrc] = {0}, cnt[kMaxSrc] = {0}, out = 0;
    if (!dst || !src || n_src > kMaxSrc)
        return 0;
    for (uint32_t i = 0; i < n_src; i++)
        cnt[i] = src[i] ? ring_count(src[i]) : 0;
    while (out < TRACE_CAPACITY) {
        int pick = -1;
        for (uint32_t i = 0; i < n_src; i++)
            if (pos[i] < cnt[i] &&
                (pick < 0 || src[i]->entries[pos[i]].tsc < src[pick]->entries[pos[pick]].tsc))
                pick = (int)i;
        if (pick < 0)
            break;
        dst->entries[out++] = src[pick]->entries[pos[pick]++];
    }
    __atomic_store_n(&dst->head, out, __ATOMIC_RELEASE);
    return out;
}
