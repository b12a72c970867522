#!/usr/bin/env python3
"""Decode-step benchmark of the GPU-resident rollout hot path on one MI355X.

One step = the batched decode work of 64 rollouts with inputs resident in HBM:
  1. paged GQA decode attention: 32 q / 8 kv heads, head_dim 128, bf16 K/V and
     queries ~N(0,1), ragged ctx ~U[512, 4096] (seeded), 16-token blocks at a
     seeded random permutation of the arena;
  2. sampling of 64 rows x 128,256 fp32 logits ~N(0,1) with 5 spike tokens per
     row at +8.0: temperature 0.8, top-k 50, top-p 0.9, Philox per-row seed,
     step counter = step index;
  3. KV append of one token per rollout and KV head.
value = tokens/s = 64 x steps/s (whole job, one GPU). The dominant kernel's
roofline (attention, HBM-bound) is measured over its own launches with HIP
events on the library stream. The CPU baseline is the oracle's OpenMP
restatement of the same step, timed on this host.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--only step|attn|sample|append]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gb300-rl-runtime_amd"))

import rlrt  # noqa: E402
import synth  # noqa: E402

METRIC = "decode steps/s + tokens/s at B=64 ctx≤4K; achieved HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0
B, QH, KVH, D, TPB = 64, 32, 8, 128, 16
CTX_LO, CTX_HI, MAX_CTX = 512, 4096, 4096
VOCAB, SPIKES, TEMP, TOPK, TOPP = 128256, 5, 0.8, 50, 0.9
LOGIT_COPIES = 4
SEED_KV, SEED_LOGITS = 2, 3


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Step:
    """Device-resident inputs and launch arguments of one decode step."""

    def __init__(self):
        t0 = time.time()
        self.w = synth.make_decode(SEED_KV, B, QH, KVH, D, CTX_LO, CTX_HI, dtype="bf16", max_ctx=MAX_CTX)
        logits = synth.make_logits(SEED_LOGITS, B, VOCAB, spikes=SPIKES)
        log(f"[bench] inputs generated in {time.time() - t0:.1f}s (arena {self.w.arena.nbytes / 1e6:.0f} MB)")
        w = self.w
        self.layout = rlrt.KvLayoutDesc.paged(TPB, D)
        self.arena = rlrt.DeviceBuffer.from_array(w.arena)
        self.table = rlrt.DeviceBuffer.from_array(w.table)
        self.ctx = rlrt.DeviceBuffer.from_array(w.ctx)
        self.q = rlrt.DeviceBuffer.from_array(w.q)
        self.out = rlrt.DeviceBuffer(B * QH * D * 2)
        self.attn = rlrt.attn_args(self.arena, self.layout, self.table, w.table_stride, B, QH, KVH, rlrt.DTYPE_BF16,
                                   self.ctx, MAX_CTX, self.q, self.out)
        self.attn_ws = rlrt.attn_workspace(self.attn)
        # sampling: rotate copies of the logits
        self.logits = [rlrt.DeviceBuffer.from_array(logits) for _ in range(LOGIT_COPIES)]
        self.seeds = rlrt.DeviceBuffer.from_array(
            np.random.default_rng(33).integers(0, 2**63, B, dtype=np.uint64))
        self.tok = rlrt.DeviceBuffer(B * 4)
        self.lp = rlrt.DeviceBuffer(B * 4)
        self.samp = [rlrt.sample_args(lg, B, VOCAB, VOCAB, self.tok, self.lp, temperature=TEMP, top_k=TOPK,
                                      top_p=TOPP, seeds=self.seeds) for lg in self.logits]
        self.samp_ws = rlrt.sample_workspace(self.samp[0])
        for s in self.samp[1:]:
            s.workspace, s.workspace_bytes = self.samp[0].workspace, self.samp[0].workspace_bytes
        # append: the slot right after each rollout's context
        rng = np.random.default_rng(44)
        self.pos = rlrt.DeviceBuffer.from_array(w.ctx.copy())
        self.knew = rlrt.DeviceBuffer.from_array(synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32)))
        self.vnew = rlrt.DeviceBuffer.from_array(synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32)))
        a = rlrt.AppendArgs()
        a.arena_base, a.arena_bytes, a.layout = self.arena.ptr, self.arena.nbytes, self.layout
        a.block_table, a.table_stride, a.batch, a.kv_heads = self.table.ptr, w.table_stride, B, KVH
        a.positions, a.cow_src, a.k_new, a.v_new = self.pos.ptr, None, self.knew.ptr, self.vnew.ptr
        self.app = a
        rlrt.sync()

    # algorithmic bytes per launch (compulsory HBM traffic)
    def attn_bytes(self):
        w = self.w
        table = int((-(-w.ctx.astype(np.int64) // TPB)).sum()) * KVH * 4
        return w.kv_bytes() + B * QH * D * 2 * 2 + table + B * 4

    @staticmethod
    def sample_bytes():
        return B * VOCAB * 4 + B * 8

    @staticmethod
    def append_bytes():
        return B * KVH * D * 2 * 2 * 2  # read new K/V rows, write them into the arena

    def run(self, i, only="step"):
        if only in ("step", "attn"):
            rlrt.attn_decode(self.attn)
        if only in ("step", "sample"):
            s = self.samp[i % LOGIT_COPIES]
            s.step = i
            rlrt.sample(s)
        if only in ("step", "append"):
            rlrt.kv_append(self.app)


def time_loop(step, k, only):
    timer = rlrt.Timer()
    rlrt.sync()
    t0 = time.perf_counter()
    timer.begin()
    for i in range(k):
        step.run(i, only)
    ms = timer.end()
    rlrt.sync()
    wall = (time.perf_counter() - t0) * 1e3
    return ms, wall


def stream_copy_gbps():
    n = 1 << 30
    a, b = rlrt.DeviceBuffer(n), rlrt.DeviceBuffer(n)
    rlrt.check(rlrt.lib().rl_hip_memset_d(a.ptr, 1, n), "memset")
    rlrt.check(rlrt.lib().rl_hip_memcpy_d2d(b.ptr, a.ptr, n), "d2d")
    timer = rlrt.Timer()
    rlrt.sync()
    timer.begin()
    for _ in range(5):
        rlrt.check(rlrt.lib().rl_hip_memcpy_d2d(b.ptr, a.ptr, n), "d2d")
    ms = timer.end()
    a.close()
    b.close()
    return 2 * n * 5 / (ms * 1e-3) / 1e9


def cpu_baseline(step, budget_s):
    """The oracle's OpenMP restatement of the same step on this host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes as C

    import orc

    olib = orc.load_oracle()
    w = step.w
    logits = synth.make_logits(SEED_LOGITS, B, VOCAB, spikes=SPIKES)
    seeds = np.random.default_rng(33).integers(0, 2**63, B, dtype=np.uint64)
    arena = w.arena.copy()
    rng = np.random.default_rng(44)
    knew = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32))
    vnew = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32))
    a = orc.attn_struct(w, 0)
    out = np.zeros((B, QH, D), np.float32)
    tok = np.zeros(B, np.uint32)
    lp = np.zeros(B, np.float64)

    def one(i):
        olib.orc_attn_decode_f32(C.byref(a), out.ctypes.data)
        olib.orc_sample_rows(logits.ctypes.data, B, VOCAB, VOCAB, 0, TEMP, TOPK, TOPP, seeds.ctypes.data, i,
                             tok.ctypes.data, lp.ctypes.data)
        olib.orc_kv_append(arena.ctypes.data, w.block_bytes, TPB, D * 2, w.table.ctypes.data, w.table_stride, B, KVH,
                           w.ctx.ctypes.data, None, knew.ctypes.data, vnew.ctypes.data)

    one(0)
    times = []
    t_start = time.perf_counter()
    i = 1
    while (time.perf_counter() - t_start < budget_s or len(times) < 3) and len(times) < 200:
        t0 = time.perf_counter()
        one(i)
        times.append(time.perf_counter() - t0)
        i += 1
    med = float(np.median(times))
    return {"value": B / med, "unit": "tokens/s", "cores": int(olib.orc_num_threads()), "kind": "port",
            "sample": f"the full 64-rollout step (fp32 online-softmax attention over the same arena, sampling "
                      f"of the same 64 x {VOCAB} logits, KV append), median of {len(times)} steps "
                      f"({sum(times):.1f} s of CPU work) after one warm-up, OpenMP over rollout x kv-head / rows",
            "steps_per_s": 1.0 / med, "ms_per_step": med * 1e3,
            "cpu_model": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="step", choices=["step", "attn", "sample", "append", "copy"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--grid-waves", type=int, default=0,
                    help="attention: persistent waves sharing the KV stream (0: library default, a full device)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs the decode hot path on one GPU only; multi-GPU runs are not part of it "
              "(DESIGN.md describes how the path would shard).", file=sys.stderr)
        sys.exit(2)

    info = rlrt.open_device(0)
    log(f"[bench] device {info.arch.decode()} cu={info.cu_count} clock={info.clock_khz / 1e3:.0f} MHz")
    if args.only == "copy":
        # calibration for the PMC byte counters: device copies of a known size
        n = 256 << 20
        a, b = rlrt.DeviceBuffer(n), rlrt.DeviceBuffer(n)
        rlrt.check(rlrt.lib().rl_hip_memset_d(a.ptr, 1, n), "memset")
        rlrt.sync()
        timer = rlrt.Timer()
        timer.begin()
        for _ in range(args.steps):
            rlrt.check(rlrt.lib().rl_hip_memcpy_d2d(b.ptr, a.ptr, n), "d2d")
        ms = timer.end()
        print(json.dumps({"only": "copy", "bytes_per_copy": n, "avg_launch_us": ms / args.steps * 1e3,
                          "gbps_read_plus_write": 2 * n / (ms / args.steps * 1e-3) / 1e9}), flush=True)
        return
    step = Step()
    step.attn.grid_waves = args.grid_waves
    if args.grid_waves:
        step.attn_ws = rlrt.attn_workspace(step.attn)

    for i in range(args.warmup):
        step.run(i, args.only)
    rlrt.sync()

    ms, wall = time_loop(step, args.steps, args.only)
    ms_step = ms / args.steps
    log(f"[bench] {args.only}: {args.steps} steps in {ms:.2f} ms (events), {wall:.2f} ms (host wall)")

    if args.only != "step":
        per = {"attn": step.attn_bytes(), "sample": step.sample_bytes(), "append": step.append_bytes()}[args.only]
        print(json.dumps({"only": args.only, "avg_launch_us": ms_step * 1e3,
                          "alg_gbps": per / (ms_step * 1e-3) / 1e9, "alg_bytes": per}), flush=True)
        return

    # per-kernel averages (each over its own back-to-back launches, HIP events)
    kern = {}
    for k in ("attn", "sample", "append"):
        kms, _ = time_loop(step, args.steps, k)
        kern[k] = kms / args.steps * 1e3
    attn_bytes = step.attn_bytes()
    achieved = attn_bytes / (kern["attn"] * 1e-6) / 1e9
    step_bytes = attn_bytes + step.sample_bytes() + step.append_bytes()
    step_gbps = step_bytes / (ms_step * 1e-3) / 1e9
    copy_gbps = stream_copy_gbps()
    log(f"[bench] attn {kern['attn']:.1f} us ({achieved:.0f} GB/s), sample {kern['sample']:.1f} us, "
        f"append {kern['append']:.1f} us, stream copy {copy_gbps:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(step, args.cpu_seconds)
        log(f"[bench] cpu baseline {cpu['ms_per_step']:.1f} ms/step on {cpu['cores']} threads")

    ctx = step.w.ctx
    result = {
        "metric": METRIC,
        "value": B / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded numpy N(0,1) bf16 K/V and queries, fp32 logits N(0,1) with 5 spikes/row",
        "config": {"workload": "gqa_decode_b64_q32kv8_d128_ctx512-4096 + sample_b64_v128256_t0.8_k50_p0.9 + "
                               "kv_append_b64",
                   "batch": B, "q_heads": QH, "kv_heads": KVH, "head_dim": D, "block_tokens": TPB,
                   "ctx": f"U[{CTX_LO},{CTX_HI}] seed {SEED_KV}: mean {ctx.mean():.0f}, sum {int(ctx.sum())}",
                   "vocab": VOCAB, "temperature": TEMP, "top_k": TOPK, "top_p": TOPP},
        "steps_per_s": 1e3 / ms_step,
        "step_alg_bytes": step_bytes,
        "step_hbm_gbps": step_gbps,
        "step_hbm_frac": step_gbps / PEAK_HBM_GBPS,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS, "traffic": None,
                     "kernel": "attn_decode_kernel<128,4,bf16,16,4>", "alg_bytes_per_launch": attn_bytes,
                     "avg_launch_us": kern["attn"]},
        "kernels_us": kern,
        "stream_copy_gbps": copy_gbps,
        "device": {"arch": info.arch.decode(), "cu": info.cu_count, "clock_mhz": info.clock_khz / 1e3},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
