"""ctypes binding of librlrt_amd.so (the C ABI declared in include/*.h).

The product is the C library: the reference's host C API (rings, submit,
worker model, descriptor windows, arena, prefix table, reward) plus the thin
HIP layer (rl_hip_*) in front of the gfx950 kernels. This module only mirrors
those entry points for tests and benchmarks, with numpy arrays as host
buffers. Every call checks the C return code and raises RlrtError with
rl_hip_last_error() on failure; there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# RLRT_LIB points the binding at another build of the same library (used to
# compare builds); by default the in-tree build is loaded.
LIB_PATH = os.environ.get("RLRT_LIB", os.path.join(_HERE, "lib", "librlrt_amd.so"))


class RlrtError(RuntimeError):
    pass


# ---------------------------------------------------------------- ABI types
class KvLayoutDesc(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("token_count", "head_dim", "scalar_bytes", "vec_bytes",
                                          "k_stride_bytes", "v_stride_bytes", "block_bytes", "alignment")]

    @classmethod
    def paged(cls, token_count: int, head_dim: int, scalar_bytes: int = 2) -> "KvLayoutDesc":
        row = head_dim * scalar_bytes
        return cls(token_count, head_dim, scalar_bytes, 16, row, row, 2 * token_count * row, 128)


class HwDesc(C.Structure):
    _pack_ = 1
    _fields_ = [("opcode", C.c_uint16), ("flags", C.c_uint16), ("rollout_id", C.c_uint32),
                ("kv_arena_id", C.c_uint32), ("prefix_id", C.c_uint32), ("kv_offset", C.c_uint64),
                ("delta_offset", C.c_uint64), ("seq_len", C.c_uint32), ("max_tokens", C.c_uint32),
                ("reward_model_id", C.c_uint32), ("reserved0", C.c_uint32), ("user_data", C.c_uint64),
                ("checksum_or_cookie", C.c_uint64)]


class InferHwCtx(C.Structure):
    _fields_ = [("cmdq", C.c_void_p), ("doneq", C.c_void_p), ("doorbell", C.c_void_p),
                ("gpu_group_id", C.c_uint32), ("kv_arena_id", C.c_uint32)]


class HwWorkerSim(C.Structure):
    _fields_ = [("cmdq", C.c_void_p), ("doneq", C.c_void_p), ("stop", C.c_void_p),
                ("decoded_tokens", C.c_uint64), ("completions", C.c_uint64)]


class Descriptor(C.Structure):
    _pack_ = 1
    _fields_ = [("seq_id", C.c_uint64), ("kv_block_offset", C.c_uint32), ("num_kv_blocks", C.c_uint16),
                ("attention_flags", C.c_uint8), ("pad", C.c_uint8), ("output_token_offset", C.c_uint32),
                ("reward_cookie", C.c_uint64), ("batch_size", C.c_uint16), ("batch_index", C.c_uint16)]


class DecodeDispatchBatch(C.Structure):
    _fields_ = [("count", C.c_uint32), ("descs", Descriptor * 32)]


class DecodeBatchContract(C.Structure):
    _fields_ = [("batch_size", C.c_uint16), ("batch_index", C.c_uint16)]


class Completion(C.Structure):
    _pack_ = 1
    _fields_ = [("seq_id", C.c_uint64), ("token_id", C.c_uint32), ("kv_block_offset", C.c_uint32),
                ("reward_cookie", C.c_uint64), ("cycles_taken", C.c_uint64)]


class RolloutRequest(C.Structure):
    _pack_ = 1
    _fields_ = [("request_id", C.c_uint64), ("max_tokens", C.c_uint32), ("kv_blocks", C.c_uint32),
                ("temperature", C.c_float), ("top_k", C.c_uint16), ("top_p", C.c_float),
                ("rng_seed", C.c_uint64)]


class RolloutDone(C.Structure):
    _pack_ = 1
    _fields_ = [("request_id", C.c_uint64), ("rollout_id", C.c_uint32), ("tokens_generated", C.c_uint32),
                ("reward", C.c_float), ("status", C.c_uint32)]


class PipelineCredits(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("max_decode_credits", "max_reward_credits", "max_trajectory_credits",
                                          "kv_block_limit", "decode_used", "reward_used", "trajectory_used",
                                          "kv_blocks_used")]


class PipelineSnapshot(C.Structure):
    _fields_ = [("queue_occupancy", C.c_uint32 * 6), ("stage_credit_headroom", C.c_uint32 * 6),
                ("credits", PipelineCredits), ("policy", C.c_int)]


PIPELINE_BYTES = 493376       # sizeof(RolloutPipeline)
PIPELINE_SLAB_OFF = 99072     # offsetof(RolloutPipeline, slab)
PIPELINE_CREDITS_OFF = 493312
PIPELINE_POLICY_OFF = 493344
REWARD_RING_BYTES = 24704     # sizeof(RewardRing)
Q_FREE, Q_PREFILL, Q_DECODE, Q_REWARD, Q_TRAJECTORY, Q_DONE = range(6)
ROLL_FREE, ROLL_PREFILL_READY, ROLL_DECODING, ROLL_REWARD_PENDING, ROLL_TRAJECTORY_READY, ROLL_DONE = range(6)


class RewardDesc(C.Structure):
    _pack_ = 1
    _fields_ = [("rollout_id", C.c_uint32), ("token_start", C.c_uint32), ("token_count", C.c_uint32),
                ("reward_model_id", C.c_uint32), ("reward", C.c_float), ("flags", C.c_uint32)]


class FeedParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("block_tokens", C.c_uint32)]


class FeedStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("registered", "admitted", "sent", "retired", "reward_handoffs",
                                          "reward_ring_full", "bad_dones", "req_ring_full")]


class PipelineFeeder(C.Structure):
    _fields_ = [("pipeline", C.c_void_p), ("requests", C.c_void_p), ("dones", C.c_void_p),
                ("rewards", C.c_void_p), ("rid_of_request", C.c_void_p), ("n_requests", C.c_uint32),
                ("end_sent", C.c_uint32), ("params", FeedParams), ("stats", FeedStats)]


class CmdPipelineCfg(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_rollouts", "tokens_per_rollout", "batch_max", "kv_blocks",
                                          "max_decode_credits", "max_reward_credits", "max_trajectory_credits",
                                          "kv_block_limit")] + \
               [(n, C.c_uint64) for n in ("seed_base", "full_wait_ns", "drain_wait_ns")]


class CmdPipelineStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "rollouts_started", "rollouts_completed", "rollouts_dropped", "descriptors_posted",
        "descriptors_consumed", "decode_batches", "decode_rollouts_scheduled", "decode_batch_peak",
        "ring_full_spins", "pipeline_overflow", "reward_handoffs", "reward_ring_full", "wall_ns",
        "rollouts_failed")]


TRACE_RING_BYTES = 20971528  # sizeof(TraceRing)
TRACE_CAPACITY = 1 << 20
TRACE_EVENTS = ("ROLLOUT_ALLOC", "ROLLOUT_FREE", "DESC_POSTED", "DESC_COMMITTED", "DESC_CONSUMED",
                "COMPLETION_POSTED", "COMPLETION_POLLED", "DECODE_BATCH", "REWARD_POSTED", "REWARD_SCORED",
                "TRAJECTORY_DONE")
TRACE = {n: i for i, n in enumerate(TRACE_EVENTS)}
TRACE_ENTRY = np.dtype([("tsc", "<u8"), ("type", "<u4"), ("rollout_id", "<u4"), ("seq", "<u4")])


class TracePairStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("n", "avg_ns", "p50_ns", "p90_ns", "p99_ns")]


class TraceClockMap(C.Structure):
    _fields_ = [("ns_per_tick", C.c_double), ("offset_ns", C.c_double)]


class RingLockstepSample(C.Structure):
    _fields_ = [("submit_ns", C.c_uint64), ("consume_tick", C.c_uint64), ("complete_tick", C.c_uint64),
                ("poll_ns", C.c_uint64)]


class KVPrefix(C.Structure):
    _pack_ = 1
    _fields_ = [("prefix_id", C.c_uint32), ("refcnt", C.c_uint32), ("kv_block_offset", C.c_int64),
                ("token_len", C.c_uint32), ("kv_block_count", C.c_uint32), ("flags", C.c_uint32)]


class KVBranch(C.Structure):
    _pack_ = 1
    _fields_ = [("branch_id", C.c_uint32), ("rollout_id", C.c_uint32), ("prefix_id", C.c_uint32),
                ("delta_kv_offset", C.c_int64), ("delta_len", C.c_uint32), ("delta_block_count", C.c_uint32),
                ("state", C.c_uint32), ("flags", C.c_uint32)]


class KVArenaHead(C.Structure):
    """First 24 bytes of KVArena; the 131,072-byte bitmap follows."""
    _fields_ = [("base", C.c_void_p), ("capacity", C.c_size_t), ("block_size", C.c_size_t)]


class DecodeMicrokernelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("head_dim", "tokens_per_block", "tile_tokens", "prefetch_stages",
                                          "shared_bytes")]


class DecodeStepResult(C.Structure):
    _fields_ = [("path_kind", C.c_uint32), ("token_id", C.c_uint32), ("bytes_touched", C.c_uint32),
                ("tile_count", C.c_uint32), ("cycle_estimate", C.c_uint64)]


class DeviceInfo(C.Structure):
    _fields_ = [("device", C.c_int32), ("cu_count", C.c_uint32), ("wave_size", C.c_uint32),
                ("lds_bytes_per_block", C.c_uint32), ("clock_khz", C.c_uint32), ("mem_clock_khz", C.c_uint32),
                ("mem_bus_width_bits", C.c_uint32), ("l2_bytes", C.c_uint32), ("hbm_bytes", C.c_uint64),
                ("arch", C.c_char * 64)]


class AttnArgs(C.Structure):
    _fields_ = [("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64), ("layout", KvLayoutDesc),
                ("block_table", C.c_void_p), ("table_stride", C.c_uint32), ("batch", C.c_uint32),
                ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("dtype", C.c_uint32),
                ("ctx_lens", C.c_void_p), ("max_ctx", C.c_uint32), ("grid_waves", C.c_uint32),
                ("scale", C.c_float), ("q", C.c_void_p), ("out", C.c_void_p), ("out_f32", C.c_void_p),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t)]


class SampleArgs(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("rows", C.c_uint32), ("vocab", C.c_uint32), ("row_stride", C.c_uint32),
                ("greedy", C.c_uint32), ("temperature", C.c_void_p), ("top_k", C.c_void_p),
                ("top_p", C.c_void_p), ("seed", C.c_void_p), ("temperature_all", C.c_float),
                ("top_k_all", C.c_uint32), ("top_p_all", C.c_float), ("seed_all", C.c_uint64),
                ("step", C.c_uint64), ("steps", C.c_void_p), ("token_out", C.c_void_p), ("logprob_out", C.c_void_p),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t), ("draw_ids", C.c_void_p)]


class AppendArgs(C.Structure):
    _fields_ = [("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64), ("layout", KvLayoutDesc),
                ("block_table", C.c_void_p), ("table_stride", C.c_uint32), ("batch", C.c_uint32),
                ("kv_heads", C.c_uint32), ("positions", C.c_void_p), ("cow_src", C.c_void_p),
                ("k_new", C.c_void_p), ("v_new", C.c_void_p)]


class ProjArgs(C.Structure):
    _fields_ = [("x", C.c_void_p), ("w", C.c_void_p), ("logits", C.c_void_p), ("rows", C.c_uint32),
                ("vocab", C.c_uint32), ("hidden", C.c_uint32), ("x_stride", C.c_uint32),
                ("w_stride", C.c_uint32), ("logits_stride", C.c_uint32)]


class RewardArgs(C.Structure):
    _fields_ = [("tokens", C.c_void_p), ("n_tokens", C.c_void_p), ("targets", C.c_void_p),
                ("rollouts", C.c_uint32), ("group_size", C.c_uint32), ("token_stride", C.c_uint32),
                ("target_stride", C.c_uint32), ("target_len", C.c_uint32), ("descs", C.c_void_p),
                ("reward", C.c_void_p), ("advantage", C.c_void_p)]


class SchedArgs(C.Structure):
    _fields_ = [("req_ring", C.c_void_p), ("done_ring", C.c_void_p), ("state", C.c_void_p),
                ("requests", C.c_uint32), ("prompt_len", C.c_void_p), ("req_table", C.c_void_p),
                ("kv_heads", C.c_uint32), ("table_stride", C.c_uint32), ("gen_tokens", C.c_void_p),
                ("gen_stride", C.c_uint32), ("targets", C.c_void_p), ("group_size", C.c_uint32),
                ("target_len", C.c_uint32), ("rewards", C.c_void_p), ("slot_table", C.c_void_p),
                ("slot_ctx", C.c_void_p), ("slot_pos", C.c_void_p), ("slot_temp", C.c_void_p),
                ("slot_topk", C.c_void_p), ("slot_topp", C.c_void_p), ("slot_seed", C.c_void_p),
                ("slot_step", C.c_void_p), ("sampled", C.c_void_p), ("counters", C.c_void_p),
                ("max_spin", C.c_uint64), ("slot_request", C.c_void_p)]


class CowArgs(C.Structure):
    _fields_ = [("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64), ("layout", KvLayoutDesc),
                ("prefixes", C.c_void_p), ("row_key", C.c_void_p), ("branch_of_key", C.c_void_p),
                ("keys", C.c_uint32), ("block_table", C.c_void_p), ("table_stride", C.c_uint32),
                ("batch", C.c_uint32), ("kv_heads", C.c_uint32), ("positions", C.c_void_p),
                ("row_status", C.c_void_p)]

COW_NONE, COW_COPIED, COW_SHARED, COW_OUT_OF_RANGE = 0, 1, 2, 3


class HwWorkerArgs(C.Structure):
    _fields_ = [("cmdq", C.c_void_p), ("doneq", C.c_void_p), ("groups", C.c_uint32), ("stop", C.c_void_p),
                ("max_idle_polls", C.c_uint64), ("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64),
                ("layout", KvLayoutDesc), ("block_table", C.c_void_p), ("table_stride", C.c_uint32),
                ("rollouts", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("dtype", C.c_uint32), ("scale", C.c_float), ("max_steps", C.c_uint32), ("q", C.c_void_p),
                ("k_new", C.c_void_p), ("v_new", C.c_void_p), ("logits", C.c_void_p), ("vocab", C.c_uint32),
                ("attn_out", C.c_void_p), ("token_out", C.c_void_p), ("logprob_out", C.c_void_p),
                ("stats", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
                ("stamps", C.c_void_p)]


class RingStepArgs(C.Structure):
    _fields_ = [("cmdq", C.c_void_p), ("doneq", C.c_void_p), ("stop", C.c_void_p), ("max_idle_polls", C.c_uint64),
                ("batch", C.c_uint32), ("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64),
                ("layout", KvLayoutDesc), ("block_table", C.c_void_p), ("table_stride", C.c_uint32),
                ("rollouts", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("dtype", C.c_uint32),
                ("scale", C.c_float), ("max_ctx", C.c_uint32), ("input_slots", C.c_uint32), ("q", C.c_void_p),
                ("k_new", C.c_void_p), ("v_new", C.c_void_p), ("logits", C.c_void_p), ("vocab", C.c_uint32),
                ("greedy", C.c_uint32), ("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("seeds", C.c_void_p), ("output_slots", C.c_uint32), ("attn_out", C.c_void_p),
                ("attn_out_f32", C.c_void_p), ("token_out", C.c_void_p), ("logprob_out", C.c_void_p),
                ("row_rollout_out", C.c_void_p), ("stats", C.c_void_p), ("workspace", C.c_void_p),
                ("workspace_bytes", C.c_size_t)]


class CmdWorkerArgs(C.Structure):
    _fields_ = [("rings", C.c_void_p), ("comp_rings", C.c_void_p), ("groups", C.c_uint32), ("stop", C.c_void_p),
                ("max_idle_polls", C.c_uint64), ("arena_base", C.c_void_p), ("arena_bytes", C.c_uint64),
                ("sample_state", C.c_void_p), ("q_buffer", C.c_void_p), ("o_buffer", C.c_void_p),
                ("io_slots", C.c_uint32), ("stats", C.c_void_p), ("trace", C.c_void_p), ("stamps", C.c_void_p)]


DTYPE_BF16 = 0
DTYPE_FP16 = 1


# ---------------------------------------------------------------- library
def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise RlrtError(f"{path} is not built: run __graft_entry__.build()")
    lib = C.CDLL(path)
    vp, sz, u32, u64, i64, i32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_int64, C.c_int
    sigs = {
        "rl_hip_open": (i32, [i32]), "rl_hip_close": (i32, []), "rl_hip_is_open": (i32, []),
        "rl_hip_device_info": (i32, [C.POINTER(DeviceInfo)]), "rl_hip_last_error": (C.c_char_p, []),
        "rl_hip_host_alloc_coherent": (vp, [sz]), "rl_hip_host_free": (i32, [vp]),
        "rl_hip_is_coherent_host": (i32, [vp]), "rl_hip_dev_alloc": (vp, [sz]),
        "rl_hip_is_device_ptr": (i32, [vp]), "rl_hip_dev_free": (i32, [vp]),
        "rl_hip_memcpy_h2d": (i32, [vp, vp, sz]), "rl_hip_memcpy_d2h": (i32, [vp, vp, sz]),
        "rl_hip_memcpy_d2d": (i32, [vp, vp, sz]), "rl_hip_memset_d": (i32, [vp, i32, sz]),
        "rl_hip_sync": (i32, []), "rl_hip_timer_begin": (i32, []),
        "rl_hip_capture_begin": (i32, []), "rl_hip_capture_end": (i32, [C.POINTER(vp)]),
        "rl_hip_graph_launch": (i32, [vp]), "rl_hip_graph_destroy": (i32, [vp]),
        "rl_hip_timer_end": (i32, [C.POINTER(C.c_float)]),
        "rl_hip_attn_decode_workspace": (sz, [C.POINTER(AttnArgs)]),
        "rl_hip_attn_decode": (i32, [C.POINTER(AttnArgs)]),
        "rl_hip_sample_workspace": (sz, [C.POINTER(SampleArgs)]),
        "rl_hip_sample": (i32, [C.POINTER(SampleArgs)]),
        "rl_hip_kv_append": (i32, [C.POINTER(AppendArgs)]),
        "rl_hip_kv_branch_resolve": (i32, [vp, vp, vp, u32]),
        "rl_hip_kv_cow": (i32, [C.POINTER(CowArgs)]),
        "rl_hip_decode_step": (i32, [C.POINTER(AttnArgs), C.POINTER(AppendArgs)]),
        "rl_hip_decode_step_noalloc": (i32, [C.POINTER(AttnArgs), C.POINTER(AppendArgs)]),
        "rl_hip_decode_sample_step_workspace": (C.c_size_t, [C.POINTER(AttnArgs), C.POINTER(SampleArgs)]),
        "rl_hip_decode_sample_step": (i32, [C.POINTER(AttnArgs), C.POINTER(AppendArgs), C.POINTER(SampleArgs),
                                             C.c_void_p, C.c_size_t]),
        "rl_hip_decode_pipeline_step": (i32, [C.POINTER(AttnArgs), C.POINTER(SampleArgs), C.POINTER(AttnArgs),
                                               C.POINTER(AppendArgs), C.c_void_p, C.c_void_p, C.c_size_t]),
        "rl_hip_decode_pipeline_flush": (i32, [C.POINTER(AttnArgs), C.POINTER(AppendArgs), C.c_void_p,
                                                C.c_size_t]),
        "rl_hip_lanes_fork": (i32, []), "rl_hip_lanes_join": (i32, []),
        "rl_hip_decode_lane_step": (i32, [i32, C.POINTER(AttnArgs), C.POINTER(SampleArgs), C.POINTER(AttnArgs),
                                           C.POINTER(AppendArgs), C.c_void_p, C.c_void_p, C.c_size_t]),
        "rl_hip_decode_lane_flush": (i32, [i32, C.POINTER(AttnArgs), C.POINTER(AppendArgs), C.c_void_p,
                                            C.c_size_t]),
        "rl_hip_logits_proj": (i32, [C.POINTER(ProjArgs)]),
        "rl_hip_reward_advantage": (i32, [C.POINTER(RewardArgs)]),
        "rl_hip_rollout_schedule": (i32, [C.POINTER(SchedArgs)]),
        "rl_hip_hw_worker_workspace": (sz, [C.POINTER(HwWorkerArgs)]),
        "rl_hip_hw_worker_launch": (i32, [C.POINTER(HwWorkerArgs)]),
        "rl_hip_cmd_worker_launch": (i32, [C.POINTER(CmdWorkerArgs)]),
        "rl_hip_ring_step_workspace": (sz, [C.POINTER(RingStepArgs)]),
        "rl_hip_ring_step_enqueue": (i32, [C.POINTER(RingStepArgs), u32, u64]),
        "rl_hip_ring_loop_launch": (i32, [C.POINTER(RingStepArgs), u32, u64, vp]),
        # reference host API
        "hw_ring_create": (vp, []), "hw_ring_reset": (None, [vp]), "hw_ring_destroy": (None, [vp]),
        "hw_ring_load_acquire": (u32, [vp]), "hw_ring_store_release": (None, [vp, u32]),
        "infer_submit_decode": (i32, [C.POINTER(InferHwCtx), u32, u64, u64, u32, u32, u32]),
        "hw_worker_sim_run": (None, [C.POINTER(HwWorkerSim)]),
        "hw_worker_apply_decode_rule": (u32, [C.POINTER(HwDesc)]),
        "rtl_desc_pack": (C.c_int, [C.POINTER(HwDesc), C.POINTER(C.c_uint32)]),
        "rtl_desc_unpack": (C.c_int, [C.POINTER(C.c_uint32), C.POINTER(HwDesc)]),
        "rtl_comp_pack": (C.c_int, [C.POINTER(HwDesc), C.POINTER(C.c_uint32)]),
        "rtl_comp_unpack": (C.c_int, [C.POINTER(C.c_uint32)] + [C.POINTER(C.c_uint32)] * 4),
        "ring_create": (vp, []), "ring_destroy": (None, [vp]),
        "comp_ring_create": (vp, []), "comp_ring_destroy": (None, [vp]),
        "req_ring_create": (vp, []), "req_ring_destroy": (None, [vp]),
        "done_ring_create": (vp, []), "done_ring_destroy": (None, [vp]),
        "decode_batch_reset": (None, [C.POINTER(DecodeDispatchBatch)]),
        "decode_batch_push": (i32, [C.POINTER(DecodeDispatchBatch), C.POINTER(Descriptor)]),
        "decode_batch_submit": (i32, [vp, C.POINTER(DecodeDispatchBatch)]),
        "decode_batch_contract": (DecodeBatchContract, [C.POINTER(Descriptor)]),
        "arena_init": (None, [vp, sz, sz]), "arena_acquire": (i64, [vp]), "arena_release": (None, [vp, i64]),
        "arena_destroy": (None, [vp]), "arena_is_device": (i32, [vp]),
        "kv_prefix_table_init": (None, [vp]),
        "kv_prefix_register": (i32, [vp, i64, u32, u32, C.POINTER(u32)]),
        "kv_prefix_acquire": (i32, [vp, u32]), "kv_prefix_release": (i32, [vp, u32]),
        "kv_prefix_get": (C.POINTER(KVPrefix), [vp, u32]),
        "kv_branch_alloc": (i32, [vp, u32, u32, i64, u32, u32, C.POINTER(u32)]),
        "kv_branch_free": (i32, [vp, u32]), "kv_branch_get": (C.POINTER(KVBranch), [vp, u32]),
        "kv_branch_total_offset": (i64, [vp, u32]),
        "rollout_slab_init": (None, [vp]), "rollout_alloc": (i32, [vp, C.POINTER(u32)]),
        "rollout_free": (None, [vp, u32]), "rollout_get": (vp, [vp, u32]),
        "rollout_transition": (i32, [vp, i32, i32]),
        "pipeline_init": (i32, [vp]), "pipeline_push": (i32, [vp, i32, u32]),
        "pipeline_pop": (i32, [vp, i32, C.POINTER(u32)]), "pipeline_transition": (i32, [vp, u32, i32, i32]),
        "pipeline_credits_set": (None, [vp, u32, u32, u32, u32]), "pipeline_try_push": (i32, [vp, i32, u32]),
        "pipeline_release": (None, [vp, i32, u32]), "pipeline_set_schedule_policy": (i32, [vp, i32]),
        "pipeline_schedule": (i32, [vp, i32, C.POINTER(u32)]), "pipeline_occupancy": (u32, [vp, i32]),
        "pipeline_stage_available_credits": (u32, [vp, i32]),
        "pipeline_stage_target_batch": (u32, [vp, i32, u32]),
        "pipeline_snapshot": (None, [vp, C.POINTER(PipelineSnapshot)]),
        "reward_ring_init": (None, [vp]), "reward_push": (i32, [vp, C.POINTER(RewardDesc)]),
        "reward_pop": (i32, [vp, C.POINTER(RewardDesc)]),
        "rl_feed_init": (i32, [C.POINTER(PipelineFeeder), vp, vp, vp, vp, vp, u32, C.POINTER(FeedParams)]),
        "rl_feed_register": (i64, [C.POINTER(PipelineFeeder), u32, u32, u32, u64]),
        "rl_feed_admit": (u32, [C.POINTER(PipelineFeeder), u32]),
        "rl_feed_send": (u32, [C.POINTER(PipelineFeeder), u32]),
        "rl_feed_retire": (u32, [C.POINTER(PipelineFeeder)]), "rl_feed_end": (i32, [C.POINTER(PipelineFeeder)]),
        "rl_feed_pump": (u32, [C.POINTER(PipelineFeeder)]),
        "rl_pipeline_cmd_run": (i32, [vp, vp, vp, vp, C.POINTER(CmdPipelineCfg), C.POINTER(CmdPipelineStats),
                                      vp, u64, vp]),
        "trace_init": (None, [vp]), "trace_push": (None, [vp, i32, u32, u32]),
        "trace_push_ts": (None, [vp, u64, i32, u32, u32]),
        "trace_report_from": (i32, [vp, u64, u64, u64, C.c_char_p]),
        "trace_pair_stats": (i32, [vp, i32, i32, C.POINTER(TracePairStats)]), "trace_now_ns": (u64, []),
        "trace_clock_fit": (i32, [u64, C.c_double, u64, C.c_double, C.POINTER(TraceClockMap)]),
        "trace_rebase": (None, [vp, C.POINTER(TraceClockMap)]), "trace_merge": (u64, [vp, vp, u32]),
        "rl_hip_trace_clock_sample": (i32, [u32, C.POINTER(u64), C.POINTER(C.c_double), C.POINTER(u64)]),
        "ring_lockstep_hw": (u32, [vp, vp, u32, vp, u32, vp, u64, vp]),
        "ring_lockstep_cmd": (u32, [vp, vp, u32, vp, u64, u32, vp, u64, vp]),
        "rl_hip_wave_broadcast_selftest": (i32, [vp, vp, vp]),
        "reward_score_mock": (C.c_float, [vp, u32]),
        "reward_match_count": (u32, [vp, vp, u32]),
        "reward_group_advantage": (i32, [vp, u32, u32, vp]),
        "attention_decode_config_fixed128": (DecodeMicrokernelConfig, []),
        "attention_decode_result_fixed128": (DecodeStepResult, [u32]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def _err() -> str:
    return lib().rl_hip_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RlrtError(f"{what} failed: {_err()}")


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- device
class DeviceBuffer:
    """Device allocation owned by Python; freed on close()/GC."""

    def __init__(self, nbytes: int, zero: bool = False):
        self.nbytes = int(nbytes)
        p = lib().rl_hip_dev_alloc(max(self.nbytes, 1))
        if not p:
            raise RlrtError(f"rl_hip_dev_alloc({nbytes}) failed: {_err()}")
        self.ptr = p
        if zero:
            check(lib().rl_hip_memset_d(p, 0, max(self.nbytes, 1)), "rl_hip_memset_d")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().rl_hip_memcpy_h2d(self.ptr + offset, ptr(a), a.nbytes), "rl_hip_memcpy_h2d")

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().rl_hip_memcpy_d2h(ptr(out), self.ptr + offset, out.nbytes), "rl_hip_memcpy_d2h")
        return out

    def close(self) -> None:
        if self.ptr:
            lib().rl_hip_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


KV_ARENA_BYTES = 131096  # sizeof(KVArena)


class Arena(DeviceBuffer):
    """The byte-compatible KVArena (arena.h) after rl_hip_open: arena_init
    takes its base from HBM (zero-filled), arena_acquire hands out block ids
    lowest-first from the host bitmap, arena_destroy frees the HBM. ptr / nbytes
    are base / capacity, so the arena passes wherever a DeviceBuffer does."""

    def __init__(self, capacity: int, block_size: int):
        L = lib()
        self.struct = np.zeros(KV_ARENA_BYTES, np.uint8)
        self.nbytes = int(capacity)
        L.arena_init(self.struct.ctypes.data, self.nbytes, int(block_size))
        head = KVArenaHead.from_address(self.struct.ctypes.data)
        self.ptr, self.block_size = head.base, int(block_size)
        if not L.arena_is_device(self.struct.ctypes.data):
            raise RlrtError("arena_init did not place the arena in device memory (no device open?)")

    def acquire(self) -> int:
        return int(lib().arena_acquire(self.struct.ctypes.data))

    def acquire_n(self, n: int) -> np.ndarray:
        ids = np.array([self.acquire() for _ in range(n)], np.int64)
        if (ids < 0).any():
            raise RlrtError(f"arena exhausted after {int((ids >= 0).sum())} of {n} blocks")
        return ids

    def release(self, idx: int) -> None:
        lib().arena_release(self.struct.ctypes.data, int(idx))

    def close(self) -> None:
        if self.ptr:
            lib().arena_destroy(self.struct.ctypes.data)
            self.ptr = None


def open_device(device: int = 0) -> DeviceInfo:
    check(lib().rl_hip_open(device), "rl_hip_open")
    info = DeviceInfo()
    check(lib().rl_hip_device_info(C.byref(info)), "rl_hip_device_info")
    return info


def sync() -> None:
    check(lib().rl_hip_sync(), "rl_hip_sync")


class CmdWorker:
    """One persistent command-ring worker (rl_hip_cmd_worker_launch) on a
    fresh CommandRing / CompletionRing pair in coherent host memory. q is the
    query buffer (None: the synthesized query from seq_id, reward_cookie and
    the sample state's rng words); the o buffer has io_slots rows of 128
    floats; trace, a TraceRing in coherent host memory, receives the worker's
    device-stamped records. stop() raises the stop flag and waits for the
    worker to exit."""

    def __init__(self, arena: DeviceBuffer, io_slots: int, q: DeviceBuffer | None = None,
                 sample_state: DeviceBuffer | None = None, max_idle_polls: int = 1 << 24, trace: int | None = None):
        L = lib()
        self.ring, self.comp = L.ring_create(), L.comp_ring_create()
        self.pairs = L.rl_hip_host_alloc_coherent(16)
        self.stop_flag = L.rl_hip_host_alloc_coherent(64)
        if not (self.ring and self.comp and self.pairs and self.stop_flag):
            raise RlrtError(f"command-ring worker rings: {_err()}")
        C.memset(self.stop_flag, 0, 64)
        C.cast(self.pairs, C.POINTER(C.c_void_p))[0] = self.ring
        C.cast(self.pairs, C.POINTER(C.c_void_p))[1] = self.comp
        self.o = DeviceBuffer(io_slots * 128 * 4, zero=True)
        self.stats = DeviceBuffer(32, zero=True)
        self.args = CmdWorkerArgs(rings=self.pairs, comp_rings=self.pairs + 8, groups=1, stop=self.stop_flag,
                                  max_idle_polls=max_idle_polls, arena_base=arena.ptr, arena_bytes=arena.nbytes,
                                  sample_state=sample_state.ptr if sample_state is not None else None,
                                  q_buffer=q.ptr if q is not None else None, o_buffer=self.o.ptr,
                                  io_slots=io_slots, stats=self.stats.ptr, trace=trace)
        self.running = False
        check(L.rl_hip_cmd_worker_launch(C.byref(self.args)), "rl_hip_cmd_worker_launch")
        self.running = True

    def stop(self) -> np.ndarray:
        """Stops the worker; returns its counters {descriptors, completions,
        windows, status}."""
        if self.running:
            C.cast(self.stop_flag, C.POINTER(C.c_uint32))[0] = 1
            sync()
            self.running = False
        return self.stats.download(np.uint64, 4)

    def close(self) -> None:
        L = lib()
        self.stop()
        self.o.close()
        self.stats.close()
        if self.ring:
            L.ring_destroy(self.ring)
            L.comp_ring_destroy(self.comp)
            L.rl_hip_host_free(self.pairs)
            L.rl_hip_host_free(self.stop_flag)
            self.ring = self.comp = None


class Graph:
    """What fn() launches on the library stream, captured once into a HIP
    graph and replayed by launch()."""

    def __init__(self, fn):
        check(lib().rl_hip_capture_begin(), "rl_hip_capture_begin")
        try:
            fn()
        finally:
            h = C.c_void_p()
            rc = lib().rl_hip_capture_end(C.byref(h))
        check(rc, "rl_hip_capture_end")
        self.handle = h.value

    def launch(self) -> None:
        check(lib().rl_hip_graph_launch(self.handle), "rl_hip_graph_launch")

    def close(self) -> None:
        if self.handle:
            lib().rl_hip_graph_destroy(self.handle)
            self.handle = None


class Timer:
    """HIP events on the library stream."""

    def begin(self) -> None:
        check(lib().rl_hip_timer_begin(), "rl_hip_timer_begin")

    def end(self) -> float:
        ms = C.c_float()
        check(lib().rl_hip_timer_end(C.byref(ms)), "rl_hip_timer_end")
        return float(ms.value)


# ---------------------------------------------------------------- kernels
def attn_args(arena: DeviceBuffer, layout: KvLayoutDesc, table: DeviceBuffer, table_stride: int, batch: int,
              q_heads: int, kv_heads: int, dtype: int, ctx: DeviceBuffer, max_ctx: int, q: DeviceBuffer,
              out: DeviceBuffer, out_f32: DeviceBuffer | None = None, grid_waves: int = 0,
              scale: float = 0.0) -> AttnArgs:
    a = AttnArgs()
    a.arena_base, a.arena_bytes, a.layout = arena.ptr, arena.nbytes, layout
    a.block_table, a.table_stride = table.ptr, table_stride
    a.batch, a.q_heads, a.kv_heads, a.dtype = batch, q_heads, kv_heads, dtype
    a.ctx_lens, a.max_ctx, a.grid_waves, a.scale = ctx.ptr, max_ctx, grid_waves, scale
    a.q, a.out, a.out_f32 = q.ptr, out.ptr, (out_f32.ptr if out_f32 is not None else None)
    return a


def attn_workspace(args: AttnArgs) -> DeviceBuffer:
    n = lib().rl_hip_attn_decode_workspace(C.byref(args))
    if n == 0:
        raise RlrtError(f"rl_hip_attn_decode_workspace: {_err()}")
    ws = DeviceBuffer(n)
    args.workspace, args.workspace_bytes = ws.ptr, n
    return ws


def attn_decode(args: AttnArgs) -> None:
    check(lib().rl_hip_attn_decode(C.byref(args)), "rl_hip_attn_decode")


def sample_args(logits: DeviceBuffer, rows: int, vocab: int, row_stride: int, tokens: DeviceBuffer,
                logprobs: DeviceBuffer, greedy: bool = False, temperature: float = 1.0, top_k: int = 0,
                top_p: float = 1.0, seed: int = 0, step: int = 0,
                seeds: DeviceBuffer | None = None, draw_ids: DeviceBuffer | None = None) -> SampleArgs:
    """Scalar parameters for every row; `seeds` (device u64[rows]) overrides `seed`,
    `draw_ids` (device u32[rows]) replaces the row index in the Philox counter."""
    s = SampleArgs()
    s.logits, s.rows, s.vocab, s.row_stride, s.greedy = logits.ptr, rows, vocab, row_stride, int(greedy)
    s.temperature = s.top_k = s.top_p = None
    s.seed = seeds.ptr if seeds is not None else None
    s.temperature_all, s.top_k_all, s.top_p_all, s.seed_all, s.step = temperature, top_k, top_p, seed, step
    s.token_out, s.logprob_out = tokens.ptr, logprobs.ptr
    s.draw_ids = draw_ids.ptr if draw_ids is not None else None
    return s


def sample_workspace(args: SampleArgs) -> DeviceBuffer:
    n = lib().rl_hip_sample_workspace(C.byref(args))
    if n == 0:
        raise RlrtError(f"rl_hip_sample_workspace: {_err()}")
    ws = DeviceBuffer(n)
    args.workspace, args.workspace_bytes = ws.ptr, n
    return ws


def sample(args: SampleArgs) -> None:
    check(lib().rl_hip_sample(C.byref(args)), "rl_hip_sample")


def kv_append(args: AppendArgs) -> None:
    check(lib().rl_hip_kv_append(C.byref(args)), "rl_hip_kv_append")


def kv_cow(args: CowArgs) -> None:
    check(lib().rl_hip_kv_cow(C.byref(args)), "rl_hip_kv_cow")


def decode_step(attn: AttnArgs, append: AppendArgs) -> None:
    """Attention, then the KV append, in one call (the append rides in the merge kernel)."""
    check(lib().rl_hip_decode_step(C.byref(attn), C.byref(append)), "rl_hip_decode_step")


DECODE_STEP_NOALLOC_SCRATCH_BYTES = 16 << 20


def decode_sample_step_workspace_bytes(attn: AttnArgs, samp: SampleArgs) -> int:
    n = lib().rl_hip_decode_sample_step_workspace(C.byref(attn), C.byref(samp))
    if n == 0:
        raise RlrtError(f"rl_hip_decode_sample_step_workspace: {_err()}")
    return int(n)


def decode_sample_step_workspace(attn: AttnArgs, samp: SampleArgs) -> DeviceBuffer:
    """The workspace of rl_hip_decode_sample_step (and of one micro-batch of its pipelined form)."""
    return DeviceBuffer(decode_sample_step_workspace_bytes(attn, samp), zero=True)


def decode_sample_step(attn: AttnArgs, append: AppendArgs | None, samp: SampleArgs, ws: DeviceBuffer) -> None:
    """The decode step of one micro-batch (attention + KV append, or no append
    when append is None) and the sampling of another micro-batch's logits in
    one launch (plus the merge), or the two calls for shapes outside the
    fused kernel."""
    check(lib().rl_hip_decode_sample_step(C.byref(attn), C.byref(append) if append is not None else None,
                                          C.byref(samp), ws.ptr, ws.nbytes), "rl_hip_decode_sample_step")


def decode_pipeline_step(attn: AttnArgs, samp: SampleArgs, ws: DeviceBuffer, prev_attn: AttnArgs | None = None,
                         prev_append: AppendArgs | None = None, prev_ws: DeviceBuffer | None = None) -> None:
    """One step of the two-micro-batch pipeline: attn's partials into ws, the
    sampling of samp, and the merge + append of the previous step."""
    check(lib().rl_hip_decode_pipeline_step(
        C.byref(attn), C.byref(samp), C.byref(prev_attn) if prev_attn is not None else None,
        C.byref(prev_append) if prev_append is not None else None, ws.ptr,
        prev_ws.ptr if prev_ws is not None else None, ws.nbytes), "rl_hip_decode_pipeline_step")


def decode_pipeline_flush(prev_attn: AttnArgs, prev_append: AppendArgs, prev_ws: DeviceBuffer) -> None:
    check(lib().rl_hip_decode_pipeline_flush(C.byref(prev_attn), C.byref(prev_append), prev_ws.ptr, prev_ws.nbytes),
          "rl_hip_decode_pipeline_flush")


LANES = 2


def lanes_fork() -> None:
    """Every lane waits for the work queued so far on the library stream."""
    check(lib().rl_hip_lanes_fork(), "rl_hip_lanes_fork")


def lanes_join() -> None:
    """The library stream waits for the work queued so far on every lane."""
    check(lib().rl_hip_lanes_join(), "rl_hip_lanes_join")


def decode_lane_step(lane: int, attn: AttnArgs, samp: SampleArgs, ws: DeviceBuffer, prev_attn: AttnArgs | None = None,
                     prev_append: AppendArgs | None = None, prev_ws: DeviceBuffer | None = None) -> None:
    """decode_pipeline_step on lane `lane` (0 or 1): steps on the two lanes may
    run at the same time, so each lane carries its own micro-batches."""
    check(lib().rl_hip_decode_lane_step(
        lane, C.byref(attn), C.byref(samp), C.byref(prev_attn) if prev_attn is not None else None,
        C.byref(prev_append) if prev_append is not None else None, ws.ptr,
        prev_ws.ptr if prev_ws is not None else None, ws.nbytes), "rl_hip_decode_lane_step")


def decode_lane_flush(lane: int, prev_attn: AttnArgs, prev_append: AppendArgs, prev_ws: DeviceBuffer) -> None:
    check(lib().rl_hip_decode_lane_flush(lane, C.byref(prev_attn), C.byref(prev_append), prev_ws.ptr,
                                         prev_ws.nbytes), "rl_hip_decode_lane_flush")


def decode_step_noalloc(attn: AttnArgs, append: AppendArgs) -> None:
    """rl_hip_decode_step on the library's fixed scratch: attn.workspace is ignored."""
    check(lib().rl_hip_decode_step_noalloc(C.byref(attn), C.byref(append)), "rl_hip_decode_step_noalloc")


# ---------------------------------------------------------------- hw_desc rings
HW_RING_SIZE = 1 << 16


def hw_ring_push(ring: int, d: HwDesc) -> int:
    """Producer side of hw_ring.h's push on a ring at address `ring`."""
    L = lib()
    tail = L.hw_ring_load_acquire(ring + 64)
    head = L.hw_ring_load_acquire(ring)
    if (tail - head) & 0xFFFFFFFF >= HW_RING_SIZE:
        return -1
    C.memmove(ring + 128 + (tail & (HW_RING_SIZE - 1)) * 64, C.byref(d), 64)
    L.hw_ring_store_release(ring + 64, (tail + 1) & 0xFFFFFFFF)
    return 0


def hw_ring_pop(ring: int) -> HwDesc | None:
    """Consumer side of hw_ring.h's pop; None when empty."""
    L = lib()
    head = L.hw_ring_load_acquire(ring)
    if head == L.hw_ring_load_acquire(ring + 64):
        return None
    d = HwDesc.from_buffer_copy((C.c_char * 64).from_address(ring + 128 + (head & (HW_RING_SIZE - 1)) * 64))
    L.hw_ring_store_release(ring, (head + 1) & 0xFFFFFFFF)
    return d


def hw_ring_indices(ring: int) -> tuple[int, int]:
    L = lib()
    return L.hw_ring_load_acquire(ring), L.hw_ring_load_acquire(ring + 64)


def hw_worker_workspace(args: HwWorkerArgs) -> DeviceBuffer:
    n = lib().rl_hip_hw_worker_workspace(C.byref(args))
    if n == 0:
        raise RlrtError(f"rl_hip_hw_worker_workspace: {_err()}")
    ws = DeviceBuffer(n)
    args.workspace, args.workspace_bytes = ws.ptr, n
    return ws


def hw_worker_launch(args: HwWorkerArgs) -> None:
    check(lib().rl_hip_hw_worker_launch(C.byref(args)), "rl_hip_hw_worker_launch")


def logits_proj(x: DeviceBuffer, w: DeviceBuffer, logits: DeviceBuffer, rows: int, vocab: int, hidden: int) -> None:
    a = ProjArgs(x=x.ptr, w=w.ptr, logits=logits.ptr, rows=rows, vocab=vocab, hidden=hidden, x_stride=hidden,
                 w_stride=hidden, logits_stride=vocab)
    check(lib().rl_hip_logits_proj(C.byref(a)), "rl_hip_logits_proj")
