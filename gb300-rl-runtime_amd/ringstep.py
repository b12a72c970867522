"""Host driver of the ring-driven batched decode step (rl_hip_ring_step_*).

The host side of the reference's hw path (infer_submit_decode into the
command ring, the completion ring polled back, include/infer_submit.h:7-21)
around rl_hip_ring_step_enqueue: the rings in coherent host memory, the
slotted per-step inputs and outputs in device memory, and the zeroed
workspace that carries the row table between calls.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import rlrt


class RingStepRun:
    """One run of the pipeline: rings, buffers and launch arguments.

    arena: a DeviceBuffer (or rlrt.Arena) holding the paged KV; table:
    [rollouts][kv_heads][stride] uint32 block ids; seeds: [rollouts] uint64."""

    def __init__(self, arena, layout: rlrt.KvLayoutDesc, table: np.ndarray, q_heads: int, max_ctx: int,
                 batch: int, vocab: int, input_slots: int = 1, output_slots: int = 1, dtype: int = rlrt.DTYPE_BF16,
                 greedy: bool = False, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
                 seeds: np.ndarray | None = None, max_idle_polls: int = 1 << 22, f32_out: bool = True):
        L = rlrt.lib()
        rollouts, kv_heads, stride = table.shape
        d = layout.head_dim
        self.batch, self.vocab, self.q_heads, self.kv_heads, self.head_dim = batch, vocab, q_heads, kv_heads, d
        self.input_slots, self.output_slots = input_slots, output_slots
        self.cq, self.dq = L.hw_ring_create(), L.hw_ring_create()
        self.stop_flag = L.rl_hip_host_alloc_coherent(64)
        self.doorbell = L.rl_hip_host_alloc_coherent(64)
        if not (self.cq and self.dq and self.stop_flag and self.doorbell):
            raise rlrt.RlrtError(f"ring step rings: {rlrt._err()}")
        if not (L.rl_hip_is_coherent_host(self.cq) and L.rl_hip_is_coherent_host(self.dq)):
            raise rlrt.RlrtError("hw rings are not in coherent host memory (no device open?)")
        C.memset(self.stop_flag, 0, 64)
        self.ctx = rlrt.InferHwCtx(cmdq=self.cq, doneq=self.dq, doorbell=self.doorbell, gpu_group_id=0,
                                   kv_arena_id=0)
        B, S, O = batch, input_slots, output_slots
        self.dev = dev = {
            "table": rlrt.DeviceBuffer.from_array(np.ascontiguousarray(table, np.uint32)),
            "q": rlrt.DeviceBuffer(S * B * q_heads * d * 2, zero=True),
            "k": rlrt.DeviceBuffer(S * B * kv_heads * d * 2, zero=True),
            "v": rlrt.DeviceBuffer(S * B * kv_heads * d * 2, zero=True),
            "logits": rlrt.DeviceBuffer(S * B * vocab * 4, zero=True),
            "out": rlrt.DeviceBuffer(O * B * q_heads * d * 2, zero=True),
            "tok": rlrt.DeviceBuffer(O * B * 4, zero=True),
            "lp": rlrt.DeviceBuffer(O * B * 4, zero=True),
            "rows": rlrt.DeviceBuffer(O * B * 4, zero=True),
            "stats": rlrt.DeviceBuffer(32, zero=True),
        }
        if f32_out:
            dev["out32"] = rlrt.DeviceBuffer(O * B * q_heads * d * 4, zero=True)
        if seeds is not None:
            dev["seeds"] = rlrt.DeviceBuffer.from_array(np.ascontiguousarray(seeds, np.uint64))
        a = rlrt.RingStepArgs(
            cmdq=self.cq, doneq=self.dq, stop=self.stop_flag, max_idle_polls=max_idle_polls, batch=B,
            arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=layout, block_table=dev["table"].ptr,
            table_stride=stride, rollouts=rollouts, q_heads=q_heads, kv_heads=kv_heads, dtype=dtype, scale=0.0,
            max_ctx=max_ctx, input_slots=S, q=dev["q"].ptr, k_new=dev["k"].ptr, v_new=dev["v"].ptr,
            logits=dev["logits"].ptr, vocab=vocab, greedy=int(greedy), temperature=temperature, top_k=top_k,
            top_p=top_p, seeds=dev["seeds"].ptr if seeds is not None else None, output_slots=O,
            attn_out=dev["out"].ptr, attn_out_f32=dev["out32"].ptr if f32_out else None, token_out=dev["tok"].ptr,
            logprob_out=dev["lp"].ptr, row_rollout_out=dev["rows"].ptr, stats=dev["stats"].ptr)
        n = L.rl_hip_ring_step_workspace(C.byref(a))
        if n == 0:
            raise rlrt.RlrtError(f"rl_hip_ring_step_workspace: {rlrt._err()}")
        dev["ws"] = rlrt.DeviceBuffer(n, zero=True)
        a.workspace, a.workspace_bytes = dev["ws"].ptr, n
        self.args = a
        self.next_step = 0

    # ---- inputs of a slot (row i = the i-th row of the step that reads it)
    def set_inputs(self, slot: int, q=None, k_new=None, v_new=None, logits=None) -> None:
        B, dv = self.batch, self.dev
        for name, arr, row in (("q", q, self.q_heads * self.head_dim * 2), ("k", k_new, self.kv_heads * self.head_dim * 2),
                               ("v", v_new, self.kv_heads * self.head_dim * 2), ("logits", logits, self.vocab * 4)):
            if arr is not None:
                a = np.ascontiguousarray(arr)
                assert a.nbytes == B * row, (name, a.nbytes, B * row)
                dv[name].upload(a, offset=slot * B * row)

    def submit_decode(self, rollout: int, seq_len: int, max_tokens: int, kv_offset: int = 0, delta: int = 0,
                      prefix: int = 0) -> None:
        if rlrt.lib().infer_submit_decode(C.byref(self.ctx), rollout, kv_offset, delta, prefix, seq_len,
                                          max_tokens) != 0:
            raise rlrt.RlrtError("infer_submit_decode: command ring full")

    def push(self, d: rlrt.HwDesc) -> None:
        if rlrt.hw_ring_push(self.cq, d) != 0:
            raise rlrt.RlrtError("command ring full")

    def enqueue(self, steps: int) -> None:
        rlrt.check(rlrt.lib().rl_hip_ring_step_enqueue(C.byref(self.args), steps, self.next_step),
                   "rl_hip_ring_step_enqueue")
        self.next_step += steps

    def loop_launch(self, max_steps: int) -> None:
        """rl_hip_ring_loop_launch: up to max_steps steps in one persistent
        launch, queued on the library stream (loop_done collects it)."""
        if "steps_run" not in self.dev:
            self.dev["steps_run"] = rlrt.DeviceBuffer(256, zero=True)
        rlrt.check(rlrt.lib().rl_hip_ring_loop_launch(C.byref(self.args), max_steps, self.next_step,
                                                      self.dev["steps_run"].ptr), "rl_hip_ring_loop_launch")

    def loop_done(self) -> int:
        """Waits for the loop; returns the steps it ran (the next call starts after them)."""
        rlrt.sync()
        n = int(self.dev["steps_run"].download(np.uint32, 1)[0])
        self.next_step += n
        return n

    def loop(self, max_steps: int) -> int:
        self.loop_launch(max_steps)
        return self.loop_done()

    def completions(self) -> list[bytes]:
        out = []
        while (d := rlrt.hw_ring_pop(self.dq)) is not None:
            out.append(bytes(d))
        return out

    def stop(self) -> None:
        C.cast(self.stop_flag, C.POINTER(C.c_uint32))[0] = 1

    def outputs(self, slot: int) -> dict:
        B, dv = self.batch, self.dev
        qd = self.q_heads * self.head_dim
        r = {"tok": dv["tok"].download(np.uint32, B, offset=slot * B * 4),
             "lp": dv["lp"].download(np.float32, B, offset=slot * B * 4),
             "rows": dv["rows"].download(np.uint32, B, offset=slot * B * 4),
             "out": dv["out"].download(np.uint16, (B, self.q_heads, self.head_dim), offset=slot * B * qd * 2)}
        if "out32" in dv:
            r["out32"] = dv["out32"].download(np.float32, (B, self.q_heads, self.head_dim), offset=slot * B * qd * 4)
        return r

    def stats(self) -> list[int]:
        return self.dev["stats"].download(np.uint64, 4).tolist()

    def close(self) -> None:
        L = rlrt.lib()
        for b in self.dev.values():
            b.close()
        if self.cq:
            L.hw_ring_destroy(self.cq)
            L.hw_ring_destroy(self.dq)
            L.rl_hip_host_free(self.stop_flag)
            L.rl_hip_host_free(self.doorbell)
            self.cq = self.dq = None
