// ring_step.hip - the batched decode step driven through the hw_desc rings.
//
// The reference's device worker takes one descriptor at a time on one SM
// (cu/worker.cu:66-131) and its CPU model applies the hw_worker_sim rule per
// descriptor (src/hw_worker_sim.c:23-59). Here up to `batch` DECODE
// descriptors share one decode step that spreads over every compute unit,
// in a stream-ordered pipeline the host enqueues ahead of time. Per step:
//
//  turn     one wave (ring_turn_kernel). First the publish of the step just
//           decoded: the hw_worker_sim rule for its token on every active
//           row (seq_len++, DONE at max_tokens, NEEDS_REWARD at a multiple of
//           32, else the row stays for the next step), the finished
//           descriptors pushed to the completion ring in row order (bounded
//           wait for room) and their rows freed. Then the admission: the
//           command ring (coherent host memory, system-scope loads) drained
//           into the free rows, lowest row first, in ring order: DECODE
//           descriptors with seq_len < max_tokens decode, those at
//           max_tokens pass through unchanged, other opcodes are dropped,
//           STOP ends admission. It waits (bounded) only while no row is
//           active; once rows are active it takes what the ring holds and
//           goes. Last, every row's step arguments: its rollout (the
//           block-table row the step reads), context (= seq_len), append
//           position, Philox seed and counter. The three ring indexes and
//           the stop flag it needs are read in one round trip, and both
//           ring releases share one fence.
//  step     rl_hip_decode_sample_step over the batch rows with the
//           rollout-ordered block table read through the row map: one launch
//           streams the paged GQA attention's tiles beside the sampling of
//           the step's logits (an input of the step, not the attention's
//           output), a second merges the split rows and appends the K/V
//           token. Shapes outside the fused kernel take rl_hip_decode_step
//           and rl_hip_sample.
//
// A call of `steps` steps launches steps + 1 turns: the last one only
// publishes. Each kernel boundary makes the previous kernel's writes visible
// on every XCD, which an in-kernel hand-off between workgroups would have to
// buy with L2 write-backs and invalidations. Waits are bounded: the
// admission gives up after max_idle_polls empty polls (status 1), the publish
// after as many polls of a full completion ring (status 3); a STOP, the host
// stop flag, an idle limit or a bad rollout id end admission while active
// rows finish.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hw_desc.h"
#include "hw_ring.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

#include "ring_core.h"

namespace {

__global__ __launch_bounds__(64) void ring_turn_kernel(RingParams p, uint32_t do_publish, uint32_t do_poll)
{
    __shared__ uint16_t s_free[kMaxBatch];  // free rows, ascending
    (void)ring_turn(p, do_publish, do_poll, s_free);
}

}  // namespace


extern "C" size_t rl_hip_ring_step_workspace(const rl_ring_step_args_t *a)
{
    if (rl_require_open("rl_hip_ring_step_workspace") || ring_validate(a, "rl_hip_ring_step_workspace"))
        return 0;
    RingWs w;
    if (ring_layout(a, w))
        return 0;
    return w.total;
}

extern "C" int rl_hip_ring_step_enqueue(const rl_ring_step_args_t *a, uint32_t steps, uint64_t first_step)
{
    if (rl_require_open("rl_hip_ring_step_enqueue") || ring_validate(a, "rl_hip_ring_step_enqueue"))
        return -1;
    RingWs w;
    if (ring_layout(a, w))
        return -1;
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_ring_step_enqueue: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    uint8_t *ws = (uint8_t *)a->workspace;
    RingParams p = ring_params_of(a, ws, w);

    const size_t B = a->batch;
    const size_t qrow = (size_t)a->q_heads * a->layout.head_dim * 2;
    const size_t kvrow = (size_t)a->kv_heads * a->layout.head_dim * 2;
    if (steps == 0)
        return 0;
    for (uint32_t n = 0; n < steps; n++) {
        const uint64_t k = first_step + n;
        const size_t si = k % a->input_slots, so = k % a->output_slots;
        p.row_rollout = a->row_rollout_out ? a->row_rollout_out + so * B : nullptr;
        // publish the previous step of this call (if any), admit for this one
        hipLaunchKernelGGL(ring_turn_kernel, dim3(1), dim3(64), 0, rl_stream(), p, n > 0 ? 1u : 0u, 1u);
        if (rl_check_launch("ring_turn_kernel launch"))
            return -1;
        rl_attn_decode_args_t t = attn_of(a, nullptr, 0);
        t.block_table = a->block_table;
        t.ctx_lens = p.ctx;
        t.q = (const uint8_t *)a->q + si * B * qrow;
        t.out = (uint8_t *)a->attn_out + so * B * qrow;
        t.out_f32 = a->attn_out_f32 ? a->attn_out_f32 + so * B * (qrow / 2) : nullptr;
        rl_kv_append_args_t ap = {};
        ap.arena_base = a->arena_base;
        ap.arena_bytes = a->arena_bytes;
        ap.layout = a->layout;
        ap.block_table = a->block_table;
        ap.table_stride = a->table_stride;
        ap.batch = a->batch;
        ap.kv_heads = a->kv_heads;
        ap.positions = p.pos;
        ap.cow_src = nullptr;
        ap.k_new = (const uint8_t *)a->k_new + si * B * kvrow;
        ap.v_new = (const uint8_t *)a->v_new + si * B * kvrow;
        rl_sample_args_t s = samp_of(a);
        s.logits = a->logits + si * B * a->vocab;
        s.seed = p.rseed;
        s.steps = p.rstep;
        s.draw_ids = p.rmap;  // the draw follows the rollout, not the row it was admitted into
        s.token_out = a->token_out + so * B;
        s.logprob_out = a->logprob_out + so * B;
        // batch row i reads the block-table row of the rollout it holds
        if (rl_decode_sample_step_mapped(&t, &ap, &s, p.rmap, ws + w.step, w.step_bytes,
                                         "rl_hip_ring_step_enqueue"))
            return -1;
    }
    // publish the last step
    p.row_rollout = nullptr;
    hipLaunchKernelGGL(ring_turn_kernel, dim3(1), dim3(64), 0, rl_stream(), p, 1u, 0u);
    if (rl_check_launch("ring_turn_kernel launch"))
        return -1;
    return 0;
}
