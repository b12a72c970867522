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

// Reports a launch error (or a fault of an earlier asynchronous call).
static inline int rl_check_launch(const char *what)
{
    return rl_check_hip(hipGetLastError(), what);
}
