// rl_hip_internal.h - helpers shared by the HIP translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_hip.h"

void rl_set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int rl_check_hip(hipError_t e, const char *what);
int rl_require_open(const char *what);
hipStream_t rl_stream(void);
// Lane `lane`'s stream, or nullptr (error set) when no device is open or the
// lane is out of range.
hipStream_t rl_lane_stream(int lane, const char *what);
// Compute units of the open device (0 when no device is open).
uint32_t rl_cu_count(void);
// The open device's ordinal (-1 when no device is open).
int rl_device(void);
// Takes the device address of the decode step's scratch array on `device`,
// which must be current (attn_decode.hip). Called by rl_hip_open.
int rl_attn_scratch_setup(int device);

// rl_hip_decode_step with the block table indexed through row_map: batch row
// b reads the table row of rollout row_map[b] (device [batch]); queries,
// outputs, contexts, positions and new K/V rows stay batch-ordered
// (attn_decode.hip; the ring-driven step uses it).
int rl_decode_step_mapped(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                          const uint32_t *row_map);
// rl_hip_attn_decode with the same row map (attn_decode.hip).
int rl_attn_mapped(const rl_attn_decode_args_t *attn, const uint32_t *row_map);
// rl_hip_decode_sample_step with the same row map for the attention and the
// append (decode_fused.hip; errors name `who`).
int rl_decode_sample_step_mapped(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                                 const rl_sample_args_t *samp, const uint32_t *row_map, void *workspace,
                                 size_t workspace_bytes, const char *who);

// Argument checks of the attention, the decode step and the sampler (0, or
// -1 with the error set), for entry points that combine them.
int rl_attn_check(const rl_attn_decode_args_t *a);
int rl_decode_step_check(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append, const char *who);
int rl_sample_check(const rl_sample_args_t *a);
// For a greedy batch (a->greedy set) that rl_hip_sample runs as split +
// merge: 1, with the slices per row and the offset of the candidate lists in
// its workspace (the slice records start at 0); 0 when the batch takes
// another path; -1 (error set) for invalid arguments or a short workspace.
int rl_sample_greedy_split(const rl_sample_args_t *a, uint32_t *splits, size_t *cand_off);
// rl_hip_decode_step (rl_hip_attn_decode when append is NULL) with the greedy
// sampling of `samp` riding in its launches: the slices as extra workgroups
// after the attention's, the row merges as extra workgroups of the attention
// merge. Results equal the two calls'. 1 when samp is not such a batch
// (nothing launched), 0 on success, -1 on error (attn_decode.hip).
int rl_decode_step_greedy_side(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                               const rl_sample_args_t *samp);

// Reports a launch error (or a fault of an earlier asynchronous call).
static inline int rl_check_launch(const char *what)
{
    return rl_check_hip(hipGetLastError(), what);
}
