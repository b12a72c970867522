/*
 * ring_latency.h - unloaded latency across the ring boundary, from device
 * stamps.
 *
 * No counterpart in the reference's code: its latency targets (docs/
 * metrics.md:70-72) are "worker poll latency", the time from the CPU's
 * enqueue to the GPU's consume, and "completion notification", the time
 * from the GPU's completion write to the CPU's poll seeing it, measured on
 * its trace pairs DESC_POSTED -> DESC_CONSUMED and COMPLETION_POSTED ->
 * COMPLETION_POLLED (src/trace.c:119-149). These drivers measure both with
 * nothing else in flight: persistent workers run on `pairs` ring pairs with
 * their stamps array set (rl_hw_worker_args_t / rl_cmd_worker_args_t), and
 * descriptor i goes to pair i % pairs only after descriptor i - 1's
 * completion was polled, so every ring holds at most one descriptor while
 * the other workers poll empty rings.
 *
 * Sample i: submit_ns = CLOCK_MONOTONIC just before the tail release of the
 * command ring; consume_tick / complete_tick = the worker's s_memrealtime
 * stamps (100 MHz) when its poll saw the descriptor and just before it
 * released the completion; poll_ns = CLOCK_MONOTONIC when the host's poll
 * saw the completion tail. A clock map (trace_clock_fit) turns the ticks
 * into host ns. Returns the number of samples taken: n, or fewer when a
 * command ring was not empty or a completion took longer than timeout_ns
 * (the driver stops there).
 */
#pragma once

#include <stdint.h>
#include "hw_ring.h"
#include "ring.h"
#include "rl_abi.h"

typedef struct {
    uint64_t submit_ns;
    uint64_t consume_tick;
    uint64_t complete_tick;
    uint64_t poll_ns;
} ring_lockstep_sample_t;

RL_STATIC_ASSERT(sizeof(ring_lockstep_sample_t) == 32, "ring_lockstep_sample_t size");

RL_EXTERN_C_BEGIN

/* hw_desc rings: each sample sends a copy of *desc (user_data = i). */
uint32_t ring_lockstep_hw(hw_ring_t *const *cmdq, hw_ring_t *const *doneq, uint32_t pairs, const hw_desc_t *desc,
                          uint32_t n, const volatile uint64_t *stamps, uint64_t timeout_ns,
                          ring_lockstep_sample_t *out);

/* v0.2 command / completion rings: each sample sends a copy of *desc
 * (seq_id = seq0 + i) as a window of one. */
uint32_t ring_lockstep_cmd(CommandRing *const *rings, CompletionRing *const *comps, uint32_t pairs,
                           const Descriptor *desc, uint64_t seq0, uint32_t n, const volatile uint64_t *stamps,
                           uint64_t timeout_ns, ring_lockstep_sample_t *out);

RL_EXTERN_C_END
