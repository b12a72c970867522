/*
 * trace.h - latency tracing on both sides of the ring boundary.
 *
 * Byte-compatible with the reference (include/trace.h:5-37): 20-byte packed
 * records {tsc, type, rollout_id, seq} in a TraceRing of 2^20 entries
 * followed by the 64-bit head (sizeof 20,971,528). trace_push stamps
 * CLOCK_MONOTONIC ns; the ring overwrites its oldest entries once head
 * passes the capacity. trace_report_from prints the reference's eight
 * latency pairs (src/trace.c:119-149) with its pairing rule and its
 * percentile picks (p50 = lats[n / 2], p90 = lats[n * 9 / 10], p99 =
 * lats[n * 99 / 100], avg = integer mean), in the same format.
 *
 * Added here:
 *   trace_pair_stats  one pair's {n, avg, p50, p90, p99} as numbers.
 *   device stamps     a producer on the GPU (the command-ring worker) writes
 *                     the same records into its own TraceRing in coherent
 *                     host memory, with tsc = the GPU's constant 100 MHz
 *                     clock (s_memrealtime). trace_clock_fit turns two
 *                     host/GPU clock samples into a linear map and
 *                     trace_rebase applies it, so device records read in
 *                     host CLOCK_MONOTONIC ns; trace_merge then interleaves
 *                     several rings by timestamp into one, which the report
 *                     walks like a single host ring.
 *
 * Event keys used by this runtime's producers: descriptor events carry
 * rollout_id = low 32 bits of seq_id and seq = output_token_offset (the
 * decode step); rollout events (alloc, reward, trajectory, free) carry
 * seq = 0, so every pair of the report can match.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>
#include "rl_abi.h"

#define TRACE_CAPACITY (1UL << 20)

typedef enum {
    TRACE_ROLLOUT_ALLOC,
    TRACE_ROLLOUT_FREE,
    TRACE_DESC_POSTED,
    TRACE_DESC_COMMITTED,
    TRACE_DESC_CONSUMED,
    TRACE_COMPLETION_POSTED,
    TRACE_COMPLETION_POLLED,
    TRACE_DECODE_BATCH,
    TRACE_REWARD_POSTED,
    TRACE_REWARD_SCORED,
    TRACE_TRAJECTORY_DONE,
    TRACE_EVENT_COUNT,
} trace_event_t;

typedef struct __attribute__((packed)) {
    uint64_t tsc;
    uint32_t type;
    uint32_t rollout_id;
    uint32_t seq;
} trace_entry_t;

RL_STATIC_ASSERT(sizeof(trace_entry_t) == 20, "trace_entry_t must be 20 bytes");

typedef struct {
    trace_entry_t entries[TRACE_CAPACITY];
    volatile uint64_t head;
} TraceRing;

RL_STATIC_ASSERT(RL_OFFSETOF(TraceRing, head) == 20971520, "TraceRing.head");
RL_STATIC_ASSERT(sizeof(TraceRing) == 20971528, "TraceRing size");

typedef struct {
    uint64_t n;
    uint64_t avg_ns;
    uint64_t p50_ns;
    uint64_t p90_ns;
    uint64_t p99_ns;
} trace_pair_stats_t;

/* host_ns = offset_ns + ticks * ns_per_tick */
typedef struct {
    double ns_per_tick;
    double offset_ns;
} trace_clock_map_t;

RL_EXTERN_C_BEGIN

/* src/trace.c:14-37 */
void trace_init(TraceRing *r);
void trace_push(TraceRing *r, trace_event_t type, uint32_t rollout_id, uint32_t seq);
void trace_push_ts(TraceRing *r, uint64_t tsc, trace_event_t type, uint32_t rollout_id, uint32_t seq);
/* src/trace.c:119-149; returns 0. */
int trace_report_from(const TraceRing *r, uint64_t wall_ns, uint64_t n_tokens, uint64_t n_rollouts,
                      const char *prefix);

/* The pair (start, end) over the ring's first min(head, capacity) entries
 * (src/trace.c:65-117). 0, or -1 when r or out is NULL or no memory. */
int trace_pair_stats(const TraceRing *r, trace_event_t start, trace_event_t end, trace_pair_stats_t *out);
/* CLOCK_MONOTONIC in ns (the clock trace_push stamps). */
uint64_t trace_now_ns(void);
/* Linear map from two samples (ticks_i, host_ns_i), each taken at the
 * midpoint of a host round trip; with one usable sample (ticks equal) the
 * rate is the nominal 10 ns per tick of the 100 MHz clock. -1 on NULL. */
int trace_clock_fit(uint64_t ticks0, double host_ns0, uint64_t ticks1, double host_ns1, trace_clock_map_t *out);
/* Rewrites tsc of the ring's entries through the map (rounded to ns). */
void trace_rebase(TraceRing *r, const trace_clock_map_t *map);
/* dst = the entries of src[0..n_src) (each in its index order, which must
 * be timestamp order), merged by tsc, ties to the lower ring index; returns
 * the entries written (at most TRACE_CAPACITY, the earliest kept). */
uint64_t trace_merge(TraceRing *dst, const TraceRing *const *src, uint32_t n_src);

RL_EXTERN_C_END
