// kv_append.hip - one-token KV append into the paged arena, with
// copy-on-write of a partially filled shared (prefix) block.
//
// The reference keeps copy-on-write as refcounting only (src/kv_prefix.c:
// 66-149; nothing is ever copied). Here the copy is real: when a rollout's
// next token falls into a block it shares with its prefix, the filled slots
// of the shared block are copied into the rollout's private block before the
// new K/V rows are written. One 64-lane wave per (rollout, kv head); every
// access is a 16-byte vector load/store.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_hip_internal.h"
#include "kv_append_core.h"

namespace {

__global__ __launch_bounds__(64) void kv_append_kernel(AppendParams p)
{
    append_row(p, blockIdx.y, blockIdx.x, threadIdx.x, 64);
}

}  // namespace

extern "C" int rl_hip_kv_append(const rl_kv_append_args_t *a)
{
    if (rl_require_open("rl_hip_kv_append") || append_validate(a, "rl_hip_kv_append"))
        return -1;
    const AppendParams p = append_params(a);
    hipLaunchKernelGGL(kv_append_kernel, dim3(a->kv_heads, a->batch), dim3(64), 0, rl_stream(), p);
    return rl_check_launch("kv_append_kernel launch");
}
