// kv_prefix.hip - the device side of the copy-on-write prefix table.
//
// The reference resolves a rollout branch to its KV offset on the device
// with kv_branch_resolve (cu/kv_prefix.cu:4-23): the branch's delta offset
// when its prefix id is out of range or the prefix's refcount is 0, else the
// prefix's kv_block_offset. Its refcounts (src/kv_prefix.c:46-133) decide
// which blocks are shared, but nothing is ever copied. Here both run on the
// byte-compatible KVPrefixTable image (include/kv_prefix.h) in device memory:
//
//  resolve  one thread per branch id, the reference's rule.
//  cow      the first token a branch writes into the partially filled last
//           block of its (live) prefix: the prefix's filled slots of that
//           block are copied into the branch's private block before the
//           step's attention reads it, so the attention and the append of
//           that step both see one table that maps the private block. One
//           wave per (row, kv head); rows not at that position do nothing.
//
// Prefix block layout: a live prefix's kv_block_count blocks start at block
// index kv_block_offset of the arena, head-major: kv head g's logical block j
// is block kv_block_offset + g * (kv_block_count / kv_heads) + j.
//
// The table's records are packed at 28- and 36-byte strides, so every field
// is read as aligned 32-bit words (all field offsets are multiples of 4).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_layout.h"
#include "kv_prefix.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr uint32_t kPrefixBytes = sizeof(KVPrefix);
constexpr uint32_t kBranchBytes = sizeof(KVBranch);
constexpr uint32_t kBranchesOff = offsetof(KVPrefixTable, branches);

__device__ __forceinline__ uint32_t tab32(const uint8_t *t, uint32_t off)
{
    return *(const uint32_t *)(t + off);
}

__device__ __forceinline__ int64_t tab64(const uint8_t *t, uint32_t off)
{
    return (int64_t)(((uint64_t)tab32(t, off + 4) << 32) | tab32(t, off));
}

// kv_branch_resolve's rule for one branch id; *live tells whether the result
// is the prefix's offset (prefix id in range and refcount nonzero).
__device__ int64_t resolve(const uint8_t *t, uint32_t id, bool *live, uint32_t *prefix)
{
    *live = false;
    if (id >= MAX_BRANCHES)
        return -1;
    const uint32_t b = kBranchesOff + id * kBranchBytes;
    const uint32_t pid = tab32(t, b + 8);
    const int64_t delta = tab64(t, b + 12);
    if (pid >= MAX_PREFIXES)
        return delta;
    const uint32_t p = pid * kPrefixBytes;
    if (tab32(t, p + 4) == 0)  // refcnt
        return delta;
    *live = true;
    *prefix = pid;
    return tab64(t, p + 8);   // kv_block_offset
}

__global__ __launch_bounds__(256) void kv_branch_resolve_kernel(const uint8_t *t, const uint32_t *ids,
                                                                int64_t *out, uint32_t n)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n)
        return;
    bool live;
    uint32_t pid;
    out[i] = resolve(t, ids[i], &live, &pid);
}

struct CowParams {
    uint8_t *arena;
    uint64_t arena_blocks;
    uint64_t block_bytes;
    uint32_t token_count;
    uint32_t row_bytes;
    const uint8_t *table;       // KVPrefixTable image
    const uint32_t *row_key;
    const uint32_t *branch_of_key;
    uint32_t keys;
    const uint32_t *block_table;
    uint32_t table_stride;
    uint32_t kv_heads;
    const uint32_t *positions;
    uint32_t *row_status;  // [batch][kv_heads] or nullptr
};

__global__ __launch_bounds__(64) void kv_cow_kernel(CowParams p)
{
    const uint32_t g = blockIdx.x, b = blockIdx.y;
    const uint32_t key = p.row_key[b];
    uint32_t br = key;
    if (p.branch_of_key)
        br = key < p.keys ? p.branch_of_key[key] : 0xFFFFFFFFu;
    uint32_t *status = p.row_status ? p.row_status + (size_t)b * p.kv_heads + g : nullptr;
    auto report = [&](uint32_t v) {
        if (status && threadIdx.x == 0)
            *status = v;
    };
    bool live;
    uint32_t pid = 0;
    const int64_t off = resolve(p.table, br, &live, &pid);
    if (!live) {
        report(RL_COW_NONE);  // no shared prefix: nothing to copy
        return;
    }
    const uint32_t pbase = pid * kPrefixBytes;
    const uint32_t len = tab32(p.table, pbase + 16);    // token_len
    const uint32_t count = tab32(p.table, pbase + 20);  // kv_block_count
    const uint32_t slot = len % p.token_count, j = len / p.token_count;
    if (slot == 0 || p.positions[b] != len) {
        report(RL_COW_NONE);  // the prefix ends on a block boundary, or this is not the branch's first own token
        return;
    }
    const uint32_t per_head = count / p.kv_heads;
    if (j >= per_head || j >= p.table_stride || off < 0) {
        report(RL_COW_OUT_OF_RANGE);
        return;
    }
    const uint64_t src = (uint64_t)off + (uint64_t)g * per_head + j;
    const uint32_t dst = p.block_table[((size_t)b * p.kv_heads + g) * p.table_stride + j];
    if (src >= p.arena_blocks || dst >= p.arena_blocks) {
        report(RL_COW_OUT_OF_RANGE);
        return;
    }
    if (src == dst) {
        report(RL_COW_SHARED);  // the row maps the prefix block itself: no private copy to make
        return;
    }
    report(RL_COW_COPIED);
    const uint8_t *s = p.arena + src * p.block_bytes;
    uint8_t *d = p.arena + (uint64_t)dst * p.block_bytes;
    const uint32_t chunks = slot * p.row_bytes / 16;  // 16-byte chunks of the filled rows of one plane
    const uint32_t v_plane = p.token_count * p.row_bytes;
    for (uint32_t i = threadIdx.x; i < 2 * chunks; i += 64) {
        const uint32_t off_b = (i >= chunks ? v_plane : 0u) + (i % chunks) * 16;
        *(rl_u32x4 *)(d + off_b) = *(const rl_u32x4 *)(s + off_b);
    }
}

}  // namespace

extern "C" int rl_hip_kv_branch_resolve(const KVPrefixTable *table, const uint32_t *branch_ids,
                                        int64_t *out_offsets, uint32_t n)
{
    if (rl_require_open("rl_hip_kv_branch_resolve"))
        return -1;
    if (!table || !branch_ids || !out_offsets) {
        rl_set_error("rl_hip_kv_branch_resolve: NULL argument");
        return -1;
    }
    if (n == 0)
        return 0;
    hipLaunchKernelGGL(kv_branch_resolve_kernel, dim3((n + 255) / 256), dim3(256), 0, rl_stream(),
                       (const uint8_t *)table, branch_ids, out_offsets, n);
    return rl_check_launch("kv_branch_resolve_kernel launch");
}

extern "C" int rl_hip_kv_cow(const rl_kv_cow_args_t *a)
{
    if (rl_require_open("rl_hip_kv_cow"))
        return -1;
    if (!a || !a->arena_base || !a->prefixes || !a->row_key || !a->block_table || !a->positions) {
        rl_set_error("rl_hip_kv_cow: NULL argument");
        return -1;
    }
    if (kv_layout_check_paged(&a->layout) != 0) {
        rl_set_error("rl_hip_kv_cow: unsupported KV layout");
        return -1;
    }
    if (a->batch == 0 || a->kv_heads == 0 || a->batch > 65535 || a->kv_heads > 65535 || a->table_stride == 0) {
        rl_set_error("rl_hip_kv_cow: batch %u kv_heads %u table_stride %u out of range", a->batch, a->kv_heads,
                     a->table_stride);
        return -1;
    }
    if (a->branch_of_key && a->keys == 0) {
        rl_set_error("rl_hip_kv_cow: branch_of_key given with keys 0");
        return -1;
    }
    CowParams p;
    p.arena = (uint8_t *)a->arena_base;
    p.block_bytes = a->layout.block_bytes;
    p.arena_blocks = a->arena_bytes / a->layout.block_bytes;
    p.token_count = a->layout.token_count;
    p.row_bytes = a->layout.k_stride_bytes;
    p.table = (const uint8_t *)a->prefixes;
    p.row_key = a->row_key;
    p.branch_of_key = a->branch_of_key;
    p.keys = a->keys;
    p.block_table = a->block_table;
    p.table_stride = a->table_stride;
    p.kv_heads = a->kv_heads;
    p.positions = a->positions;
    p.row_status = a->row_status;
    hipLaunchKernelGGL(kv_cow_kernel, dim3(a->kv_heads, a->batch), dim3(64), 0, rl_stream(), p);
    return rl_check_launch("kv_cow_kernel launch");
}
