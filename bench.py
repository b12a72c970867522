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
Four such micro-batches (256 rollouts in flight, each with its own copy of
the arena in HBM) take turns: step t is one launch of decode_fused_kernel
that streams micro-batch t % 4's attention tiles and samples its logits,
while its sampling waves first merge step t - 2's split rows and append that
step's K/V token; steps alternate between the library's two lanes (streams),
so one launch fills the compute units the other leaves idle as it drains.
value = tokens/s = 64 x steps/s (whole job, one GPU). The dominant (only)
kernel's roofline is measured over the same launches back to back on one
stream with HIP events. Beside it: the same pipeline on one stream and the
unfused step (rl_hip_decode_step + rl_hip_sample). The CPU baseline is the
oracle's OpenMP restatement of the step, timed on this host.

Before the timed run, two rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE)
in child processes measure the fused kernel's HBM traffic per step,
calibrated on a 256 MiB device copy in the same pass (--no-traffic skips
them).

  python bench.py [--gpus 1] [--steps K] [--warmup W]
                  [--only step|pipeline|unfused|attn|sample|append|copy]
  python bench.py --workload sample256|longctx|proj|plumbing|rollout|rollout_pipeline|cmdring|pipeline|
                            pipeline_trace
      the other synthetic workloads (sampling at 256 rows, long-context
      split-KV decode, the vocabulary projection, the hw_desc ring plumbing
      decode, the GRPO rollout loop with its requests sent at once or fed by
      the host rollout pipeline, the v0.2 command/completion rings, the host
      pipeline driving them, and that run traced on both sides), one JSON
      line each
"""
import argparse
import json
import os
import sys
import time

import numpy as np

# the CPU baseline's OpenMP threads: one per core, packed (read when the
# oracle's library loads libgomp)
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
# the CPUs this process may run on, read before OpenMP binds the main thread
try:
    NPROC = len(os.sched_getaffinity(0))
except OSError:
    NPROC = os.cpu_count()

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gb300-rl-runtime_amd")
sys.path.insert(0, PKG)

# The library is loaded only after the counter passes (child processes) ran:
# nothing in this process touches the GPU before them.
rlrt = synth = None


def _load():
    global rlrt, synth
    import rlrt as _rlrt
    import synth as _synth
    rlrt, synth = _rlrt, _synth


METRIC = "decode steps/s + tokens/s at B=64 ctx≤4K; achieved HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0
B, QH, KVH, D, TPB = 64, 32, 8, 128, 16
CTX_LO, CTX_HI, MAX_CTX = 512, 4096, 4096
VOCAB, SPIKES, TEMP, TOPK, TOPP = 128256, 5, 0.8, 50, 0.9
LOGIT_COPIES = 4
MICRO_BATCHES = 4
SEED_KV, SEED_LOGITS = 2, 3
PMC_CALLS, PMC_COPY_BYTES = 4, 256 << 20


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
        # the KV arena through arena.h (HBM base from arena_init); the
        # workload's permuted block ids are the ids arena_acquire hands out
        n_blocks = w.arena.nbytes // w.block_bytes
        self.arena = rlrt.Arena(w.arena.nbytes, w.block_bytes)
        if not np.array_equal(self.arena.acquire_n(n_blocks), np.arange(n_blocks)):
            raise rlrt.RlrtError("arena_acquire did not hand out the lowest free blocks in order")
        self.arena.upload(w.arena)
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

    def run(self, i, only):
        """One launch of `only`: the unfused step (rl_hip_decode_step, then
        rl_hip_sample), or one of its entry points alone."""
        if only == "unfused":
            # attention, then the KV append inside the attention's merge kernel
            rlrt.decode_step(self.attn, self.app)
        elif only == "attn":
            rlrt.attn_decode(self.attn)
        elif only == "append":
            rlrt.kv_append(self.app)
        if only in ("unfused", "sample"):
            s = self.samp[i % LOGIT_COPIES]
            s.step = i
            rlrt.sample(s)


class Pipeline:
    """The headline step: four micro-batches of 64 rollouts (256 in flight),
    each with its own arena, table, queries, outputs, logits and workspace
    (the arena and contexts are copies of the same seeded draw, so every step
    streams the same bytes from its own HBM). Step t runs micro-batch t % 4:
    its attention's tiles and the sampling of its logits in one launch whose
    sampling waves first merge step t - 2's split rows and append its K/V
    token, on lane t % 2 (or all on the library stream). The sampled logits
    are not the step's own attention's output: in an engine they come from
    the forward pass of a micro-batch whose attention an earlier step ran."""

    def __init__(self, step):
        w = step.w
        self.step = step
        self.attn, self.app, self.keep = [step.attn], [step.app], []
        for m in range(1, MICRO_BATCHES):
            arena = rlrt.DeviceBuffer.from_array(w.arena)
            table = rlrt.DeviceBuffer.from_array(w.table)
            ctx = rlrt.DeviceBuffer.from_array(w.ctx)
            q = rlrt.DeviceBuffer.from_array(w.q)
            out = rlrt.DeviceBuffer(B * QH * D * 2)
            pos = rlrt.DeviceBuffer.from_array(w.ctx.copy())
            self.keep += [arena, table, ctx, q, out, pos]
            self.attn.append(rlrt.attn_args(arena, step.layout, table, w.table_stride, B, QH, KVH, rlrt.DTYPE_BF16,
                                            ctx, MAX_CTX, q, out))
            self.app.append(rlrt.AppendArgs(arena_base=arena.ptr, arena_bytes=arena.nbytes, layout=step.layout,
                                            block_table=table.ptr, table_stride=w.table_stride, batch=B,
                                            kv_heads=KVH, positions=pos.ptr, cow_src=None, k_new=step.knew.ptr,
                                            v_new=step.vnew.ptr))
        self.tok = [rlrt.DeviceBuffer(B * 4) for _ in range(MICRO_BATCHES)]
        self.lp = [rlrt.DeviceBuffer(B * 4) for _ in range(MICRO_BATCHES)]
        self.samp = [rlrt.sample_args(step.logits[m], B, VOCAB, VOCAB, self.tok[m], self.lp[m], temperature=TEMP,
                                      top_k=TOPK, top_p=TOPP, seeds=step.seeds) for m in range(MICRO_BATCHES)]
        self.ws = [rlrt.decode_sample_step_workspace(self.attn[m], self.samp[m]) for m in range(MICRO_BATCHES)]
        self.t = 0
        rlrt.sync()

    def launch(self, n, on_lanes):
        """Steps self.t .. self.t + n - 1, each merging step t - 2."""
        for _ in range(n):
            t, m = self.t, self.t % MICRO_BATCHES
            s = self.samp[m]
            s.step = t
            prev = ()
            if t >= 2:
                pm = (t - 2) % MICRO_BATCHES
                prev = (self.attn[pm], self.app[pm], self.ws[pm])
            if on_lanes:
                rlrt.decode_lane_step(t % 2, self.attn[m], s, self.ws[m], *prev)
            else:
                rlrt.decode_pipeline_step(self.attn[m], s, self.ws[m], *prev)
            self.t += 1

    def flush(self, on_lanes):
        """Merges and appends the last two steps; the next step starts a new pipeline."""
        for t in range(max(self.t - 2, 0), self.t):
            m = t % MICRO_BATCHES
            if on_lanes:
                rlrt.decode_lane_flush(t % 2, self.attn[m], self.app[m], self.ws[m])
            else:
                rlrt.decode_pipeline_flush(self.attn[m], self.app[m], self.ws[m])
        if on_lanes:
            rlrt.lanes_join()
        rlrt.sync()
        self.t = 0

    def timed(self, k, warmup, on_lanes):
        """ms for k steps after `warmup` steps of the same pipeline: the timed
        steps merge the two steps before them, the flush after is not timed."""
        timer = rlrt.Timer()
        if on_lanes:
            rlrt.lanes_fork()
        self.launch(warmup, on_lanes)
        if on_lanes:
            rlrt.lanes_join()
        timer.begin()
        if on_lanes:
            rlrt.lanes_fork()
        t0 = time.perf_counter()
        self.launch(k, on_lanes)
        if on_lanes:
            rlrt.lanes_join()
        ms = timer.end()
        wall = (time.perf_counter() - t0) * 1e3
        self.flush(on_lanes)
        return ms, wall


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

    threads = int(olib.orc_num_threads())

    def timed(n_warm, n_min, budget, cap):
        for i in range(n_warm):
            one(i)
        times = []
        t_start = time.perf_counter()
        i = n_warm
        while (time.perf_counter() - t_start < budget or len(times) < n_min) and len(times) < cap:
            t0 = time.perf_counter()
            one(i)
            times.append(time.perf_counter() - t0)
            i += 1
        return times

    times = timed(2, 10, budget_s, 200)
    med = float(np.median(times))
    # the same step on one thread: 2 warm-ups, median of 5
    olib.orc_set_num_threads(1)
    t1 = timed(2, 5, 0.0, 5)
    olib.orc_set_num_threads(threads)
    med1 = float(np.median(t1))
    return {"value": B / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the full 64-rollout step (fp32 online-softmax attention over the same arena, sampling "
                      f"of the same 64 x {VOCAB} logits, KV append), median of {len(times)} steps "
                      f"({sum(times):.1f} s of CPU work) after 2 warm-ups, OpenMP over rollout x kv-head / rows "
                      f"on {threads} threads; one thread: median of {len(t1)} after 2 warm-ups",
            "steps_per_s": 1.0 / med, "ms_per_step": med * 1e3,
            "one_thread": {"value": B / med1, "ms_per_step": med1 * 1e3},
            **_host_info(threads)}


def _cpu_model():
    """The CPU model as lscpu and /proc/cpuinfo print it (family / model numbers too)."""
    import subprocess

    name, fam, mod = None, None, None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() == "Model name" and v.strip():
                name = v.strip()
    except Exception:
        pass
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k == "model name" and not name:
                name = v.strip()
            elif k == "cpu family" and fam is None:
                fam = v.strip()
            elif k == "model" and mod is None:
                mod = v.strip()
    except OSError:
        pass
    return f"{name or 'unknown'} (family {fam}, model {mod})"


def _host_info(threads):
    """nproc, OpenMP threads, CPU model and NUMA nodes of this host."""
    import glob

    return {"nproc": NPROC, "omp_threads": threads, "cpu_model": _cpu_model(),
            "numa_nodes": len(glob.glob("/sys/devices/system/node/node[0-9]*")) or 1,
            "omp_env": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES")}}


# ---------------------------------------------------------------- HBM traffic (rocprofv3 counters)
def _pmc_pass(counter, tmp):
    """One rocprofv3 --pmc pass over `bench.py --only pmc` (a child process);
    returns {kernel name: counter summed over its dispatches}."""
    import csv
    import glob
    import subprocess

    out = os.path.join(tmp, counter)
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "pmc", "--",
           sys.executable, os.path.abspath(__file__), "--only", "pmc"]
    subprocess.run(cmd, check=True, timeout=120, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise RuntimeError(f"no counter_collection.csv under {out}")
    acc = {}
    with open(files[0], newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            k = row["Kernel_Name"]
            acc[k] = acc.get(k, 0.0) + float(row["Counter_Value"])
    return acc


def measure_traffic():
    """HBM bytes per pipeline step from FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by what the counter reads for a device copy of
    256 MiB (read 256 MiB, write 256 MiB) run in the same pass. The runtime
    may split one copy into several blit dispatches, so both the calls and
    the copies are counted by what the target ran (PMC_CALLS of each)."""
    import shutil
    import tempfile

    if not shutil.which("rocprofv3"):
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="rlrt_pmc_")
    try:
        fetch = _pmc_pass("FETCH_SIZE", tmp)
        write = _pmc_pass("WRITE_SIZE", tmp)
    except Exception as e:  # the counters are reported as null, the bench goes on
        return None, f"counter pass failed: {e}"
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    def pick(d, key):
        v = [x for k, x in d.items() if key in k]
        return sum(v) if v else None

    copy_kib = PMC_COPY_BYTES / 1024.0
    cf, cw = pick(fetch, "copyBuffer"), pick(write, "copyBuffer")
    af, aw = pick(fetch, "decode_fused_kernel"), pick(write, "decode_fused_kernel")
    mf, mw = pick(fetch, "merge_pieces_kernel") or 0.0, pick(write, "merge_pieces_kernel") or 0.0
    if not (cf and cw and af is not None and aw is not None):
        return None, f"kernels missing from the counter output: {sorted(fetch)}"
    cf, cw = cf / PMC_CALLS, cw / PMC_CALLS                     # per 256 MiB copy
    af, aw = (af + mf) / PMC_CALLS, (aw + mw) / PMC_CALLS       # per pipeline step
    kf, kw = copy_kib / cf, copy_kib / cw
    total = (af * kf + aw * kw) * 1024.0
    return {"bytes": total, "fetch_kib": af, "write_kib": aw, "fetch_scale": kf, "write_scale": kw,
            "copy_fetch_kib": cf, "copy_write_kib": cw}, None


def pmc_target():
    """What the counter passes profile: PMC_CALLS steps of the pipeline on
    the library stream and its flush (the merges of the first two steps run
    in the flush's kernels instead of a later step's), then PMC_CALLS device
    copies of 256 MiB (the calibration kernel)."""
    rlrt.open_device(0)
    pipe = Pipeline(Step())
    pipe.launch(PMC_CALLS, False)
    pipe.flush(False)
    n = PMC_COPY_BYTES
    a, b = rlrt.DeviceBuffer(n), rlrt.DeviceBuffer(n)
    rlrt.check(rlrt.lib().rl_hip_memset_d(a.ptr, 1, n), "memset")
    for _ in range(PMC_CALLS):
        rlrt.check(rlrt.lib().rl_hip_memcpy_d2d(b.ptr, a.ptr, n), "d2d")
    rlrt.sync()


# ---------------------------------------------------------------- the other workloads
def _event_us(fn, k, warmup=3):
    for i in range(warmup):
        fn(i)
    rlrt.sync()
    timer = rlrt.Timer()
    timer.begin()
    for i in range(k):
        fn(i)
    ms = timer.end()
    return ms / k * 1e3


def wl_sample256(args):
    """256 rows x 128,256 fp32 logits ~N(0,1), 5 spikes per row at +8.0;
    T 0.8, top-k 50, top-p 0.9, Philox per-row seed; greedy on the same rows.
    Three copies of the logits (394 MB) rotate past the 256 MB Infinity Cache."""
    rows, copies = 256, 3
    x = synth.make_logits(3, rows, VOCAB, spikes=SPIKES)
    lg = [rlrt.DeviceBuffer.from_array(x) for _ in range(copies)]
    seeds = rlrt.DeviceBuffer.from_array(np.random.default_rng(34).integers(0, 2**63, rows, dtype=np.uint64))
    tok, lp = rlrt.DeviceBuffer(rows * 4), rlrt.DeviceBuffer(rows * 4)
    res = {}
    for name, greedy in (("topk_topp", False), ("greedy", True)):
        ss = [rlrt.sample_args(b, rows, VOCAB, VOCAB, tok, lp, greedy=greedy, temperature=TEMP, top_k=TOPK,
                               top_p=TOPP, seeds=seeds) for b in lg]
        ws = rlrt.sample_workspace(ss[0])
        for s in ss[1:]:
            s.workspace, s.workspace_bytes = ws.ptr, ws.nbytes

        def run(i, ss=ss):
            s = ss[i % copies]
            s.step = i
            rlrt.sample(s)

        us = _event_us(run, args.steps)
        nbytes = rows * VOCAB * 4 + rows * 8
        res[name] = {"us_per_call": us, "rows_per_s": rows / (us * 1e-6), "alg_bytes": nbytes,
                     "alg_gbps": nbytes / (us * 1e-6) / 1e9, "frac": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS}
        ws.close()
    return {"workload": "sample_r256_v128256_t0.8_k50_p0.9 (+ greedy)", **res}


def wl_sample32k(args):
    """The rollout loop's sampler shape: 256 rows x 32,000 fp32 logits
    ~N(0, 0.3); top-p 0.9 over the whole vocabulary (T 1, no top-k), then
    top-k 50 + top-p 0.9, then greedy. Nine copies of the logits (295 MB)
    rotate past the 256 MB Infinity Cache, so every call reads HBM."""
    rows, vocab, copies = 256, 32000, 9
    rng = np.random.default_rng(35)
    x = rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(0.3)
    lg = [rlrt.DeviceBuffer.from_array(x) for _ in range(copies)]
    seeds = rlrt.DeviceBuffer.from_array(rng.integers(0, 2**63, rows, dtype=np.uint64))
    tok, lp = rlrt.DeviceBuffer(rows * 4), rlrt.DeviceBuffer(rows * 4)
    res = {}
    for name, greedy, k in (("topp", False, 0), ("topk_topp", False, TOPK), ("greedy", True, 0)):
        ss = [rlrt.sample_args(b, rows, vocab, vocab, tok, lp, greedy=greedy, temperature=1.0, top_k=k,
                               top_p=TOPP, seeds=seeds) for b in lg]
        ws = rlrt.sample_workspace(ss[0])
        for s in ss[1:]:
            s.workspace, s.workspace_bytes = ws.ptr, ws.nbytes

        def run(i, ss=ss):
            s = ss[i % copies]
            s.step = i
            rlrt.sample(s)

        us = _event_us(run, args.steps)
        nbytes = rows * vocab * 4 + rows * 8
        res[name] = {"us_per_call": us, "alg_bytes": nbytes, "alg_gbps": nbytes / (us * 1e-6) / 1e9,
                     "frac": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS}
        ws.close()
    for b in lg + [seeds, tok, lp]:
        b.close()
    return {"workload": "sample_r256_v32000_p0.9 (+ top-k 50, greedy)", **res}


def wl_longctx(args):
    """B=8, ctx 32,768, 64 q / 8 kv heads, d128, bf16 K/V ~N(0,1), permuted
    16-token blocks, split-KV over the whole device with the fp32 LSE merge;
    then greedy over 8 x 128,256 fp32 logits ~N(0,1). The step is
    rl_hip_decode_sample_step without an append: GQA 64/8 is outside the fused
    kernel, so the greedy sampler's slices ride in the attention's launch (as
    workgroups after the attention's) and its row merges in the attention
    merge's; the logits are an input, not the attention's output. The same
    two calls one after the other are timed beside it."""
    bb, qh = 8, 64
    w = synth.make_decode(5, bb, qh, KVH, D, 32768, 32768, dtype="bf16")
    layout = rlrt.KvLayoutDesc.paged(TPB, D)
    bufs = [rlrt.DeviceBuffer.from_array(a) for a in (w.arena, w.table, w.ctx, w.q)]
    out = rlrt.DeviceBuffer(bb * qh * D * 2)
    a = rlrt.attn_args(bufs[0], layout, bufs[1], w.table_stride, bb, qh, KVH, rlrt.DTYPE_BF16, bufs[2], w.max_ctx,
                       bufs[3], out)
    ws = rlrt.attn_workspace(a)
    x = synth.make_logits(6, bb, VOCAB)
    lg = rlrt.DeviceBuffer.from_array(x)
    tok, lp = rlrt.DeviceBuffer(bb * 4), rlrt.DeviceBuffer(bb * 4)
    s = rlrt.sample_args(lg, bb, VOCAB, VOCAB, tok, lp, greedy=True)
    sws = rlrt.sample_workspace(s)
    attn_bytes = w.kv_bytes() + bb * qh * D * 2 * 2 + int((-(-w.ctx.astype(np.int64) // TPB)).sum()) * KVH * 4
    us_attn = _event_us(lambda i: rlrt.attn_decode(a), args.steps)
    us_seq = _event_us(lambda i: (rlrt.attn_decode(a), rlrt.sample(s)), args.steps)
    fws = rlrt.decode_sample_step_workspace(a, s)
    us_step = _event_us(lambda i: rlrt.decode_sample_step(a, None, s, fws), args.steps)
    step_bytes = attn_bytes + bb * VOCAB * 4
    return {"workload": "gqa_decode_b8_q64kv8_d128_ctx32768 + greedy_b8_v128256",
            "attn_us": us_attn, "attn_alg_bytes": attn_bytes, "attn_gbps": attn_bytes / (us_attn * 1e-6) / 1e9,
            "attn_frac": attn_bytes / (us_attn * 1e-6) / 1e9 / PEAK_HBM_GBPS,
            "step_us": us_step, "steps_per_s": 1e6 / us_step, "tokens_per_s": bb * 1e6 / us_step,
            "step_gbps": step_bytes / (us_step * 1e-6) / 1e9, "step_two_calls_us": us_seq,
            "step": "rl_hip_decode_sample_step(attn, NULL append, greedy): the sampler's slices ride in the "
                    "attention launch, its row merges in the attention merge launch"}


def wl_proj(args):
    """logits[rows, 32,000] = X[rows, 4,096] . W^T, bf16 in, fp32 out, at the
    rollout loop's 256 slots and at 512 rows; W bf16 ~N(0, 0.02^2)."""
    vocab, hid = 32000, 4096
    rng = np.random.default_rng(7)
    w = rlrt.DeviceBuffer.from_array(synth.f32_to_bf16(rng.standard_normal((vocab, hid), np.float32) * 0.02))
    res = {}
    for rows in (256, 512):
        x = rlrt.DeviceBuffer.from_array(synth.f32_to_bf16(rng.standard_normal((rows, hid), np.float32)))
        out = rlrt.DeviceBuffer(rows * vocab * 4)
        us = _event_us(lambda i: rlrt.logits_proj(x, w, out, rows, vocab, hid), args.steps)
        flop = 2.0 * rows * vocab * hid
        nbytes = vocab * hid * 2 + rows * hid * 2 + rows * vocab * 4
        res[f"rows{rows}"] = {"us": us, "tflops": flop / (us * 1e-6) / 1e12,
                              "mfma_frac_bf16_dense": flop / (us * 1e-6) / 2.5e15,
                              "alg_bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9,
                              "hbm_frac": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
                              "ideal_us": max(flop / 2.5e15, nbytes / 8e12) * 1e6}
        x.close()
        out.close()
    return {"workload": "logits_proj_h4096_v32000", **res}


def wl_plumbing(args):
    """One rollout, MHA 8 heads x d64 fp16 K/V ~N(0, 0.5^2), 16-token blocks,
    KV length 256 at the start. 100 descriptors through infer_submit_decode
    into the hw_desc command ring; the persistent worker runs each (attention,
    greedy over 32,000 fp32 logits ~N(0, 2^2), KV append) and publishes on the
    completion ring. Measured twice: pipelined (all submitted back to back)
    and lock-step (submit one, wait for its completion)."""
    import ctypes as C

    L = rlrt.lib()
    steps, ctx0, vocab = 100, 256, 32000
    rng = np.random.default_rng(1001)
    w = synth.make_decode(1000, 1, 8, 8, 64, ctx0, ctx0, dtype="fp16", kv_std=0.5, reserve_tokens=ctx0 + 2 * steps + 1)
    q = synth.f32_to_f16(rng.standard_normal((2 * steps, 8, 64), dtype=np.float32))
    kv = synth.f32_to_f16(rng.standard_normal((2 * steps, 8, 64), dtype=np.float32) * np.float32(0.5))
    logits = rng.standard_normal((2 * steps, vocab), dtype=np.float32) * np.float32(2.0)
    bufs = {n: rlrt.DeviceBuffer.from_array(a) for n, a in
            (("arena", w.arena), ("table", w.table), ("q", q), ("kv", kv), ("logits", logits))}
    outs = [rlrt.DeviceBuffer(n, zero=True) for n in (2 * steps * 8 * 64 * 4, 2 * steps * 4, 2 * steps * 4, 32)]

    def coherent(n):
        p = L.rl_hip_host_alloc_coherent(n)
        if not p:
            raise rlrt.RlrtError("coherent host allocation failed")
        return p

    cq, dq = L.hw_ring_create(), L.hw_ring_create()
    rings, stop, doorbell = coherent(16), coherent(64), coherent(64)
    C.cast(rings, C.POINTER(C.c_void_p))[0] = cq
    C.cast(rings, C.POINTER(C.c_void_p))[1] = dq
    a = rlrt.HwWorkerArgs(cmdq=rings, doneq=rings + 8, groups=1, stop=stop, max_idle_polls=1 << 24,
                          arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes,
                          layout=rlrt.KvLayoutDesc.paged(16, 64), block_table=bufs["table"].ptr,
                          table_stride=w.table_stride, rollouts=1, q_heads=8, kv_heads=8, dtype=rlrt.DTYPE_FP16,
                          scale=0.0, max_steps=2 * steps, q=bufs["q"].ptr, k_new=bufs["kv"].ptr, v_new=bufs["kv"].ptr,
                          logits=bufs["logits"].ptr, vocab=vocab, attn_out=outs[0].ptr, token_out=outs[1].ptr,
                          logprob_out=outs[2].ptr, stats=outs[3].ptr)
    ws = rlrt.hw_worker_workspace(a)
    ctx = rlrt.InferHwCtx(cmdq=cq, doneq=dq, doorbell=doorbell, gpu_group_id=7, kv_arena_id=42)
    rlrt.hw_worker_launch(a)
    lat = []
    try:
        t0 = time.perf_counter()
        for i in range(steps):
            if L.infer_submit_decode(C.byref(ctx), 0, 0x1000 * i, 0x40 * i, 0, ctx0 + i, ctx0 + i + 1) != 0:
                raise rlrt.RlrtError("submit failed")
        got, deadline = 0, time.perf_counter() + 30
        while got < steps and time.perf_counter() < deadline:
            if rlrt.hw_ring_pop(dq) is not None:
                got += 1
        pipelined = time.perf_counter() - t0
        if got != steps:
            raise rlrt.RlrtError(f"pipelined: {got} of {steps} completions")
        for i in range(steps, 2 * steps):
            t1 = time.perf_counter()
            if L.infer_submit_decode(C.byref(ctx), 0, 0x1000 * i, 0x40 * i, 0, ctx0 + i, ctx0 + i + 1) != 0:
                raise rlrt.RlrtError("submit failed")
            deadline = t1 + 5
            while rlrt.hw_ring_pop(dq) is None:
                if time.perf_counter() > deadline:
                    raise rlrt.RlrtError("lock-step completion timed out")
            lat.append(time.perf_counter() - t1)
        rlrt.hw_ring_push(cq, rlrt.HwDesc(opcode=255))
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rlrt.sync()
    st = outs[3].download(np.uint64, 4)
    lat_us = np.array(lat) * 1e6
    for b in list(bufs.values()) + outs + [ws]:
        b.close()
    L.hw_ring_destroy(cq)
    L.hw_ring_destroy(dq)
    for p in (rings, stop, doorbell):
        L.rl_hip_host_free(p)
    cpu = None
    if not args.no_cpu:
        cpu = _plumbing_cpu(w, q, kv, logits, steps, ctx0, vocab)
    return {"workload": "plumbing_mha8_d64_fp16_ctx256_v32000_100steps",
            "pipelined_steps_per_s": steps / pipelined, "pipelined_ms": pipelined * 1e3, "cpu_baseline": cpu,
            "lockstep_latency_us": {"p50": float(np.percentile(lat_us, 50)), "p90": float(np.percentile(lat_us, 90)),
                                    "p99": float(np.percentile(lat_us, 99)), "mean": float(lat_us.mean())},
            "lockstep_steps_per_s": 1e6 / float(lat_us.mean()), "worker_stats": st.tolist(),
            "note": "host side polls the completion ring from Python (ctypes)"}


def _plumbing_cpu(w, q, kv, logits, steps, ctx0, vocab):
    """The CPU path of the plumbing decode: the hw_worker_sim loop on a pthread
    with a real decode step per token (the oracle's fp32 attention, greedy,
    KV append), fed through ring images, on the same inputs: 100 descriptors
    back to back, then 100 one at a time."""
    import ctypes as C

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc

    olib = orc.load_oracle()
    arena = w.arena.copy()
    out = np.zeros((2 * steps, 8, 64), np.float32)
    tok = np.zeros(2 * steps, np.uint32)
    p = orc.OrcPlumbing(arena=arena.ctypes.data, block_bytes=w.block_bytes, token_count=16, head_dim=64, dtype=1,
                        table=w.table.ctypes.data, table_stride=w.table_stride, q_heads=8, kv_heads=8,
                        scale=1.0 / 8.0, q=q.ctypes.data, k_new=kv.ctypes.data, v_new=kv.ctypes.data,
                        logits=logits.ctypes.data, vocab=vocab, steps=2 * steps, attn_out=out.ctypes.data,
                        tokens=tok.ctypes.data)
    pipe = C.c_double()
    lat = np.zeros(steps, np.float64)
    if olib.orc_plumbing_run(C.byref(p), ctx0, steps, C.byref(pipe), lat.ctypes.data) != 0:
        return None
    threads = int(olib.orc_num_threads())
    lat_us = lat * 1e6
    return {"value": steps / pipe.value, "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"{steps} descriptors pipelined then {steps} lock-step through hw_desc ring images: the "
                      f"hw_worker_sim loop on a pthread, per token fp32 attention (OpenMP over the 8 heads), "
                      f"greedy over {vocab} logits and the KV append",
            "lockstep_latency_us": {"p50": float(np.percentile(lat_us, 50)), "p99": float(np.percentile(lat_us, 99))},
            **_host_info(threads)}


def wl_plumbing256(args):
    """One persistent hw_desc worker per compute unit, each with its own ring
    pair and rollout (MHA 8 heads x d64 fp16 K/V ~N(0, 0.5^2), 16-token
    blocks, KV length 256 at the start, greedy over 32,000 fp32 logits).
    Pipelined: 32 one-token descriptors per ring queued through
    infer_submit_decode before the launch, then STOP; the kernel's duration
    (HIP events) over all 256 x 32 steps is the aggregate rate. Lock-step:
    one descriptor per ring per round, the round ends when every ring has its
    completion (Python polls the 256 completion rings)."""
    import ctypes as C

    L = rlrt.lib()
    info = rlrt.DeviceInfo()
    rlrt.check(L.rl_hip_device_info(C.byref(info)), "rl_hip_device_info")
    G, S, R, ctx0, vocab = int(info.cu_count), 32, 20, 256, 32000
    rng = np.random.default_rng(1010)
    n_steps = S + R
    w = synth.make_decode(1011, G, 8, 8, 64, ctx0, ctx0, dtype="fp16", kv_std=0.5, reserve_tokens=ctx0 + n_steps + 1)
    q = synth.f32_to_f16(rng.standard_normal((G, n_steps, 8, 64), dtype=np.float32))
    kv = synth.f32_to_f16(rng.standard_normal((G, n_steps, 8, 64), dtype=np.float32) * np.float32(0.5))
    logits = rng.standard_normal((G, n_steps, vocab), dtype=np.float32) * np.float32(2.0)
    bufs = {n: rlrt.DeviceBuffer.from_array(a) for n, a in
            (("arena", w.arena), ("table", w.table), ("q", q), ("kv", kv), ("logits", logits))}
    outs = [rlrt.DeviceBuffer(n, zero=True) for n in (G * n_steps * 8 * 64 * 4, G * n_steps * 4, G * n_steps * 4,
                                                       G * 32)]

    def coherent(n):
        p = L.rl_hip_host_alloc_coherent(n)
        if not p:
            raise rlrt.RlrtError("coherent host allocation failed")
        return p

    cqs = [L.hw_ring_create() for _ in range(G)]
    dqs = [L.hw_ring_create() for _ in range(G)]
    rings, stop, bells = coherent(16 * G), coherent(64), coherent(64 * G)
    for g in range(G):
        C.cast(rings, C.POINTER(C.c_void_p))[g] = cqs[g]
        C.cast(rings, C.POINTER(C.c_void_p))[G + g] = dqs[g]
    ctxs = [rlrt.InferHwCtx(cmdq=cqs[g], doneq=dqs[g], doorbell=bells + 64 * g, gpu_group_id=g, kv_arena_id=0)
            for g in range(G)]

    def make_args():
        return rlrt.HwWorkerArgs(cmdq=rings, doneq=rings + 8 * G, groups=G, stop=stop, max_idle_polls=1 << 24,
                                 arena_base=bufs["arena"].ptr, arena_bytes=bufs["arena"].nbytes,
                                 layout=rlrt.KvLayoutDesc.paged(16, 64), block_table=bufs["table"].ptr,
                                 table_stride=w.table_stride, rollouts=G, q_heads=8, kv_heads=8,
                                 dtype=rlrt.DTYPE_FP16, scale=0.0, max_steps=n_steps, q=bufs["q"].ptr,
                                 k_new=bufs["kv"].ptr, v_new=bufs["kv"].ptr, logits=bufs["logits"].ptr, vocab=vocab,
                                 attn_out=outs[0].ptr, token_out=outs[1].ptr, logprob_out=outs[2].ptr,
                                 stats=outs[3].ptr)

    # pipelined: everything queued first, the kernel runs until STOP
    for i in range(S):
        for g in range(G):
            if L.infer_submit_decode(C.byref(ctxs[g]), g, 0, 0, 0, ctx0 + i, ctx0 + i + 1) != 0:
                raise rlrt.RlrtError("submit failed")
    for g in range(G):
        rlrt.hw_ring_push(cqs[g], rlrt.HwDesc(opcode=255))
    a = make_args()
    ws = rlrt.hw_worker_workspace(a)
    timer = rlrt.Timer()
    rlrt.sync()
    timer.begin()
    rlrt.hw_worker_launch(a)
    ms = timer.end()
    st = outs[3].download(np.uint64, (G, 4))
    if not (st[:, 1] == S).all():
        raise rlrt.RlrtError(f"pipelined: completions per pair {np.unique(st[:, 1]).tolist()}")
    for g in range(G):
        while rlrt.hw_ring_pop(dqs[g]) is not None:
            pass
    # lock-step rounds on a fresh launch (each worker continues its rollout at step S)
    for o in outs[3:]:
        rlrt.check(L.rl_hip_memset_d(o.ptr, 0, o.nbytes), "memset")
    a2 = make_args()  # a fresh launch counts its steps from 0 again: input rows are reused
    a2.workspace, a2.workspace_bytes = a.workspace, a.workspace_bytes
    rlrt.hw_worker_launch(a2)
    rounds = []
    try:
        for i in range(S, S + R):
            t1 = time.perf_counter()
            for g in range(G):
                if L.infer_submit_decode(C.byref(ctxs[g]), g, 0, 0, 0, ctx0 + i, ctx0 + i + 1) != 0:
                    raise rlrt.RlrtError("submit failed")
            pending = set(range(G))
            deadline = t1 + 10
            while pending:
                for g in list(pending):
                    if rlrt.hw_ring_pop(dqs[g]) is not None:
                        pending.discard(g)
                if time.perf_counter() > deadline:
                    raise rlrt.RlrtError(f"lock-step round: {len(pending)} rings without a completion")
            rounds.append(time.perf_counter() - t1)
        for g in range(G):
            rlrt.hw_ring_push(cqs[g], rlrt.HwDesc(opcode=255))
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rlrt.sync()
    for b in list(bufs.values()) + outs + [ws]:
        b.close()
    for r in cqs + dqs:
        L.hw_ring_destroy(r)
    for p in (rings, stop, bells):
        L.rl_hip_host_free(p)
    r_us = np.array(rounds) * 1e6
    return {"workload": f"plumbing_{G}pairs_mha8_d64_fp16_ctx256_v32000",
            "pairs": G, "pipelined_steps": G * S, "pipelined_kernel_ms": ms,
            "pipelined_steps_per_s": G * S / (ms * 1e-3),
            "lockstep_round_us": {"p50": float(np.percentile(r_us, 50)), "p99": float(np.percentile(r_us, 99))},
            "lockstep_steps_per_s": G / (float(np.median(r_us)) * 1e-6),
            "note": "pipelined: rings filled before the launch, HIP events around the persistent kernel; lock-step: "
                    "one descriptor per ring per round, submitted and polled from Python"}


def wl_ringstep(args):
    """The headline step (64 rollouts, GQA 32/8, d128, bf16 K/V, ctx
    U[512,4096] or the --ctx range, sampling of 64 x 128,256 logits with T 0.8 / top-k 50 /
    top-p 0.9, KV append) driven through the hw_desc rings
    (rl_hip_ring_step_enqueue): per step 64 one-token descriptors drained by
    the poll kernel, the batched step over every compute unit, 64 completions
    published. The descriptors of every step are queued before the timed
    region; logits rotate over 4 input slots. Then the same pipeline as one
    persistent launch of K steps (rl_hip_ring_loop_launch). Beside them, on
    the same inputs: the launched fused step (rl_hip_decode_sample_step: the same two kernels
    without the rings) and the unfused one (rl_hip_decode_step +
    rl_hip_sample)."""
    import ringstep

    K, W = args.steps, args.warmup
    if B * (K + W) > 65536:
        raise SystemExit("ringstep: every step's descriptors and completions are queued up front; "
                         f"{B} x (steps + warmup) must fit the 65,536-slot rings")
    st = Step()
    w = st.w
    seeds = np.random.default_rng(33).integers(0, 2**63, B, dtype=np.uint64)
    run = ringstep.RingStepRun(st.arena, st.layout, w.table, QH, MAX_CTX, B, VOCAB, input_slots=LOGIT_COPIES,
                               output_slots=1, temperature=TEMP, top_k=TOPK, top_p=TOPP, seeds=seeds, f32_out=False)
    logits = synth.make_logits(SEED_LOGITS, B, VOCAB, spikes=SPIKES)
    rng = np.random.default_rng(44)
    kn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32))
    vn = synth.f32_to_bf16(rng.standard_normal((B, KVH, D), np.float32))
    for sl in range(LOGIT_COPIES):
        run.set_inputs(sl, w.q, kn, vn, logits)
    for _ in range(K + W):
        for r in range(B):
            run.submit_decode(r, int(w.ctx[r]), int(w.ctx[r]) + 1)
    run.enqueue(W)
    rlrt.sync()
    timer = rlrt.Timer()
    timer.begin()
    run.enqueue(K)
    ms = timer.end()
    stats = run.stats()
    n_comp = len(run.completions())
    run.stop()
    run.close()
    if stats[:3] != [B * (K + W), B * (K + W), K + W] or n_comp != B * (K + W):
        raise rlrt.RlrtError(f"ring step stats {stats}, {n_comp} completions")
    # the same pipeline as one persistent launch per call (rl_hip_ring_loop_launch;
    # three consecutive steps write their own output slots)
    run = ringstep.RingStepRun(st.arena, st.layout, w.table, QH, MAX_CTX, B, VOCAB, input_slots=LOGIT_COPIES,
                               output_slots=3, temperature=TEMP, top_k=TOPK, top_p=TOPP, seeds=seeds, f32_out=False)
    for sl in range(LOGIT_COPIES):
        run.set_inputs(sl, w.q, kn, vn, logits)
    for _ in range(K + W):
        for r in range(B):
            run.submit_decode(r, int(w.ctx[r]), int(w.ctx[r]) + 1)
    if run.loop(W) != W:
        raise rlrt.RlrtError("ring loop warm-up ended early")
    timer.begin()
    run.loop_launch(K)
    loop_ms = timer.end()
    loop_ran = run.loop_done()
    loop_stats = run.stats()
    n_comp = len(run.completions())
    run.stop()
    run.close()
    if loop_ran != K or loop_stats[:3] != [B * (K + W), B * (K + W), K + W] or n_comp != B * (K + W):
        raise rlrt.RlrtError(f"ring loop ran {loop_ran}, stats {loop_stats}, {n_comp} completions")
    # the launched steps on the same inputs
    fws = rlrt.decode_sample_step_workspace(st.attn, st.samp[0])

    def fused(i):
        s = st.samp[i % LOGIT_COPIES]
        s.step = i
        rlrt.decode_sample_step(st.attn, st.app, s, fws)

    fused_us = _event_us(fused, K, W)
    for i in range(W):
        st.run(i, "unfused")
    lms, _ = time_loop(st, K, "unfused")
    ring_us, launched_us, loop_us = ms / K * 1e3, lms / K * 1e3, loop_ms / K * 1e3
    step_bytes = st.attn_bytes() + st.sample_bytes() + st.append_bytes()
    return {"workload": f"ringstep_b64_q32kv8_d128_ctx{CTX_LO}-{CTX_HI}_v128256_t0.8_k50_p0.9",
            "ctx_sum": int(w.ctx.astype(np.int64).sum()), "step_alg_bytes": int(step_bytes),
            "steps": K, "ring_step_us": ring_us, "ring_steps_per_s": 1e6 / ring_us,
            "ring_tokens_per_s": B * 1e6 / ring_us, "ring_step_hbm_frac": step_bytes / (ring_us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
            "loop_step_us": loop_us, "loop_tokens_per_s": B * 1e6 / loop_us,
            "loop_step_hbm_frac": step_bytes / (loop_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, "loop_over_ring": loop_us / ring_us,
            "launched_fused_step_us": fused_us, "ring_over_launched_fused": ring_us / fused_us,
            "launched_step_us": launched_us, "launched_tokens_per_s": B * 1e6 / launched_us,
            "stats": stats,
            "note": "per step: the turn kernel (one wave: the previous step's 64 completions published and 64 "
                    "descriptors admitted over PCIe), the fused attention + sampling launch and its merge + append "
                    "kernel; loop_step_us: the same turns and steps in one persistent launch of K steps "
                    "(rl_hip_ring_loop_launch: the turn on its own wave beside the steps, a step released once every "
                    "workgroup has finished the one before, a step's split rows merged by the next step's sampling "
                    "waves); launched_fused_step_us: "
                    "the same two kernels called directly; launched_step_us: rl_hip_decode_step + rl_hip_sample; "
                    "HIP events on the library stream"}


def wl_cmdring(args):
    """The v0.2 path: Descriptors in decode_batch windows of 32 through a
    CommandRing to the persistent worker (fixed128 decode step per
    descriptor: one head, d128, fp16 K/V ~N(0,1) in 16 KiB arena blocks,
    seq_len 32, q from the q buffer) and Completions back. Prefilled: 127
    windows and the shutdown sentinel committed before the launch, the
    persistent kernel timed with HIP events (the worker's own rate, no host in
    the loop); pipelined: 4,096 descriptors submitted from Python as fast as
    the ring takes them; lock-step: one descriptor at a time, submit to
    completion."""
    import ctypes as C

    L = rlrt.lib()
    nblk, io, total = 256, 64, 4096
    rng = np.random.default_rng(71)
    arena = synth.f32_to_f16(rng.standard_normal(nblk * 8192, dtype=np.float32))
    qf = synth.f32_to_f16(rng.standard_normal((io, 128), dtype=np.float32))
    darena, dq = rlrt.DeviceBuffer.from_array(arena), rlrt.DeviceBuffer.from_array(qf)
    do, stats = rlrt.DeviceBuffer(io * 128 * 4), rlrt.DeviceBuffer(32, zero=True)
    ring, cr = L.ring_create(), L.comp_ring_create()

    def coherent(n):
        p = L.rl_hip_host_alloc_coherent(n)
        if not p:
            raise rlrt.RlrtError("coherent host allocation failed")
        return p

    pairs, stop = coherent(16), coherent(64)
    C.cast(pairs, C.POINTER(C.c_void_p))[0] = ring
    C.cast(pairs, C.POINTER(C.c_void_p))[1] = cr
    a = rlrt.CmdWorkerArgs(rings=pairs, comp_rings=pairs + 8, groups=1, stop=stop, max_idle_polls=1 << 24,
                           arena_base=darena.ptr, arena_bytes=darena.nbytes, sample_state=None, q_buffer=dq.ptr,
                           o_buffer=do.ptr, io_slots=io, stats=stats.ptr)
    batch = rlrt.DecodeDispatchBatch()

    def submit(first, n):
        L.decode_batch_reset(C.byref(batch))
        for k in range(first, first + n):
            d = rlrt.Descriptor(seq_id=k, kv_block_offset=k % nblk, num_kv_blocks=32, output_token_offset=k,
                                reward_cookie=k)
            L.decode_batch_push(C.byref(batch), C.byref(d))
        return L.decode_batch_submit(ring, C.byref(batch)) == 0

    def drain():
        n = 0
        while True:
            head, tail = L.hw_ring_load_acquire(cr), L.hw_ring_load_acquire(cr + 64)
            if head == tail:
                return n
            n += (tail - head) & 0xFFFFFFFF
            L.hw_ring_store_release(cr, tail)

    # prefilled: the worker drains a full ring on its own (twice; the second
    # pass is reported)
    pre_windows = 127
    timer = rlrt.Timer()
    for _ in range(2):
        for w in range(pre_windows):
            if not submit(w * 32, 32):
                raise rlrt.RlrtError("prefill: command ring full")
        L.decode_batch_reset(C.byref(batch))
        L.decode_batch_push(C.byref(batch), C.byref(rlrt.Descriptor(seq_id=2**64 - 1)))
        L.decode_batch_submit(ring, C.byref(batch))
        timer.begin()
        rlrt.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
        pre_ms = timer.end()
        rlrt.sync()
        if drain() != pre_windows * 32:
            raise rlrt.RlrtError("prefill: completions missing")
        pre_st = stats.download(np.uint64, 4)

    rlrt.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
    lat = []
    try:
        t0 = time.perf_counter()
        sent = done = 0
        while done < total and time.perf_counter() - t0 < 30:
            if sent < total and submit(sent, 32):
                sent += 32
            done += drain()
        pipelined = time.perf_counter() - t0
        for k in range(200):
            t1 = time.perf_counter()
            submit(total + k, 1)
            while drain() == 0:
                if time.perf_counter() - t1 > 5:
                    raise rlrt.RlrtError("lock-step completion timed out")
            lat.append(time.perf_counter() - t1)
        submit_sentinel = rlrt.Descriptor(seq_id=2**64 - 1)
        L.decode_batch_reset(C.byref(batch))
        L.decode_batch_push(C.byref(batch), C.byref(submit_sentinel))
        L.decode_batch_submit(ring, C.byref(batch))
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rlrt.sync()
    st = stats.download(np.uint64, 4)
    for b in (darena, dq, do, stats):
        b.close()
    L.ring_destroy(ring)
    L.comp_ring_destroy(cr)
    L.rl_hip_host_free(pairs)
    L.rl_hip_host_free(stop)
    lat_us = np.array(lat) * 1e6
    return {"workload": "cmdring_fixed128_d128_fp16_seq32_windows32", "descriptors": total,
            "prefilled_descriptors_per_s": pre_windows * 32 / (pre_ms * 1e-3), "prefilled_ms": pre_ms,
            "prefilled_us_per_window": pre_ms * 1e3 / pre_windows, "prefilled_worker_stats": pre_st.tolist(),
            "pipelined_descriptors_per_s": total / pipelined, "pipelined_ms": pipelined * 1e3,
            "lockstep_latency_us": {"p50": float(np.percentile(lat_us, 50)), "p90": float(np.percentile(lat_us, 90)),
                                    "p99": float(np.percentile(lat_us, 99))},
            "worker_stats": st.tolist(),
            "note": "prefilled: kernel time of one worker draining 127 committed windows; pipelined and lock-step: "
                    "host side in Python (ctypes) on both ends of the rings"}


def wl_rollout(args):
    """512 GRPO requests (64 groups of 8, shared 512-token prefix, U[0,512]
    private prompt tokens, 256 generated tokens each) through the request
    ring, the device scheduler, batched decode (attention, projection, top-p
    sampling, KV append) over 256 slots and the done ring."""
    import grpo

    cfg = grpo.build_workload(404)
    loop = grpo.RolloutLoop(cfg)
    loop.submit_requests()
    res = loop.run()
    dones = len(loop.dones)
    loop.close()
    gen_tokens = grpo.REQ * grpo.GEN
    return {"workload": "grpo_512req_64x8_prefix512_gen256_q32kv8_d128_v32000", "steps": res["steps"],
            "wall_s": res["wall_s"], "generated_tokens_per_s": gen_tokens / res["wall_s"], "dones": dones,
            "steady_us_per_step": res["window_us_per_step"],
            "steady_tokens_per_s": grpo.SLOTS / res["window_us_per_step"] * 1e6}


def wl_rollout_pipeline(args):
    """The GRPO run of the rollout workload with its request ring fed by the
    host rollout pipeline (384 decode credits; retire, admit and send at each
    done poll) instead of one upfront burst."""
    import grpo

    cfg = grpo.build_workload(404)
    loop = grpo.RolloutLoop(cfg)
    loop.attach_pipeline(decode_credits=384)
    res = loop.run()
    st = loop.feeder.stats
    stats = {k: getattr(st, k) for k, _ in st._fields_}
    loop.close()
    gen_tokens = grpo.REQ * grpo.GEN
    return {"workload": "grpo_512req_pipeline_fed_credits384", "steps": res["steps"], "wall_s": res["wall_s"],
            "generated_tokens_per_s": gen_tokens / res["wall_s"], "steady_us_per_step": res["window_us_per_step"],
            "feeder": stats}


def wl_pipeline(args):
    """bench/bench_pipeline.cu's run: 1,000 rollouts x 128 decode tokens
    through the host rollout pipeline (credits 256/128/128/1024, decode
    batches of 32 rollouts, decode_batch windows of 32 descriptors) into the
    command ring, natively (rl_pipeline_cmd_run); the persistent worker runs
    the fixed128 step of each descriptor (one KV token of one of 128 arena
    blocks, fp16, synthesized query) and the same host thread drains the
    completions. Tokens/s = descriptors completed / wall time."""
    import ctypes as C

    L = rlrt.lib()
    n, tokens, nblk, io = 1000, 128, 128, 4096
    rng = np.random.default_rng(81)
    arena = synth.f32_to_f16(rng.standard_normal(nblk * 8192, dtype=np.float32))
    import struct

    seed, m64 = 42, 2**64 - 1                   # SampleState as bench/bench_pipeline.cu:108-117 fills it
    st = np.frombuffer(struct.pack("<4QfH2xfI", seed, seed ^ 0x9E3779B97F4A7C15,
                                   ((seed << 17) ^ 0x3C6EF372FE94F82A) & m64, ~seed & m64, 1.0, 50, 0.9, 128256),
                       np.uint8).copy()
    darena, dst = rlrt.DeviceBuffer.from_array(arena), rlrt.DeviceBuffer.from_array(st)
    pipe = np.zeros(rlrt.PIPELINE_BYTES, np.uint8)
    rew = np.zeros(rlrt.REWARD_RING_BYTES, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    L.reward_ring_init(rew.ctypes.data)
    cfg = rlrt.CmdPipelineCfg(n_rollouts=n, tokens_per_rollout=tokens, batch_max=32, kv_blocks=nblk,
                              max_decode_credits=256, max_reward_credits=128, max_trajectory_credits=128,
                              kv_block_limit=1024, seed_base=42, full_wait_ns=10**10, drain_wait_ns=10**10)
    stats = rlrt.CmdPipelineStats()
    w = rlrt.CmdWorker(darena, io, sample_state=dst)
    try:
        rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, w.ring, w.comp, rew.ctypes.data, C.byref(cfg),
                                   C.byref(stats), None, 0, None)
    finally:
        wst = w.stop()
        w.close()
    darena.close()
    dst.close()
    if rc != 0:
        raise rlrt.RlrtError(f"rl_pipeline_cmd_run: {stats.descriptors_consumed} of {stats.descriptors_posted}")
    sd = {k: getattr(stats, k) for k, _ in stats._fields_}
    return {"workload": "pipeline_1000rollouts_x128tok_fixed128_cmdring", "rc": rc,
            "tokens_per_s": stats.descriptors_consumed / (stats.wall_ns * 1e-9),
            "rollouts_per_s": stats.rollouts_completed / (stats.wall_ns * 1e-9), "wall_ms": stats.wall_ns * 1e-6,
            "stats": sd, "worker_stats": wst.tolist(),
            "note": "host loop native (C); one persistent worker workgroup"}


def wl_pipeline_trace(args):
    """The pipeline run with tracing on both sides of the rings: the driver's
    host records (CLOCK_MONOTONIC) and the worker's device records
    (s_memrealtime, mapped onto the host clock by ping-pong clock samples
    before and after the run), merged and paired as the reference's trace
    report does. Latencies in ns."""
    import ctypes as C

    L = rlrt.lib()
    n, tokens, nblk, io = 1000, 128, 128, 4096
    rng = np.random.default_rng(81)
    arena = synth.f32_to_f16(rng.standard_normal(nblk * 8192, dtype=np.float32))
    darena = rlrt.DeviceBuffer.from_array(arena)
    host = np.zeros(rlrt.TRACE_RING_BYTES, np.uint8)
    L.trace_init(host.ctypes.data)
    dev_ring = L.rl_hip_host_alloc_coherent(rlrt.TRACE_RING_BYTES)
    if not dev_ring:
        raise rlrt.RlrtError("coherent trace ring allocation failed")
    C.memset(dev_ring, 0, rlrt.TRACE_RING_BYTES)

    def clock():
        t, h, r = C.c_uint64(), C.c_double(), C.c_uint64()
        rlrt.check(L.rl_hip_trace_clock_sample(64, C.byref(t), C.byref(h), C.byref(r)), "clock sample")
        return t.value, h.value, r.value

    pipe = np.zeros(rlrt.PIPELINE_BYTES, np.uint8)
    rew = np.zeros(rlrt.REWARD_RING_BYTES, np.uint8)
    L.pipeline_init(pipe.ctypes.data)
    L.reward_ring_init(rew.ctypes.data)
    cfg = rlrt.CmdPipelineCfg(n_rollouts=n, tokens_per_rollout=tokens, batch_max=32, kv_blocks=nblk,
                              max_decode_credits=256, max_reward_credits=128, max_trajectory_credits=128,
                              kv_block_limit=1024, seed_base=42, full_wait_ns=10**10, drain_wait_ns=10**10)
    stats = rlrt.CmdPipelineStats()
    c0 = clock()
    w = rlrt.CmdWorker(darena, io, trace=dev_ring)
    try:
        rc = L.rl_pipeline_cmd_run(pipe.ctypes.data, w.ring, w.comp, rew.ctypes.data, C.byref(cfg),
                                   C.byref(stats), None, 0, host.ctypes.data)
    finally:
        w.stop()
        w.close()
        darena.close()
    c1 = clock()
    if rc != 0:
        L.rl_hip_host_free(dev_ring)
        raise rlrt.RlrtError("rl_pipeline_cmd_run did not complete")
    m = rlrt.TraceClockMap()
    L.trace_clock_fit(c0[0], c0[1], c1[0], c1[1], C.byref(m))
    L.trace_rebase(dev_ring, C.byref(m))
    merged = np.zeros(rlrt.TRACE_RING_BYTES, np.uint8)
    events = L.trace_merge(merged.ctypes.data, (C.c_void_p * 2)(host.ctypes.data, dev_ring), 2)
    L.rl_hip_host_free(dev_ring)
    T = rlrt.TRACE
    pairs = {}
    s = rlrt.TracePairStats()
    for a, b in (("DESC_POSTED", "DESC_COMMITTED"), ("DESC_POSTED", "DESC_CONSUMED"),
                 ("DESC_CONSUMED", "COMPLETION_POSTED"), ("COMPLETION_POSTED", "COMPLETION_POLLED"),
                 ("DESC_POSTED", "COMPLETION_POLLED"), ("DESC_CONSUMED", "COMPLETION_POLLED"),
                 ("ROLLOUT_ALLOC", "REWARD_POSTED"), ("ROLLOUT_ALLOC", "TRAJECTORY_DONE"),
                 ("REWARD_POSTED", "REWARD_SCORED"), ("REWARD_POSTED", "TRAJECTORY_DONE")):
        L.trace_pair_stats(merged.ctypes.data, T[a], T[b], C.byref(s))
        pairs[f"{a.lower()}->{b.lower()}"] = {"n": s.n, "avg": s.avg_ns, "p50": s.p50_ns, "p90": s.p90_ns,
                                             "p99": s.p99_ns}
    return {"workload": "pipeline_trace_1000rollouts_x128tok", "events": events,
            "tokens_per_s_traced": stats.descriptors_consumed / (stats.wall_ns * 1e-9),
            "clock": {"ns_per_tick": m.ns_per_tick, "rtt_ns": [c0[2], c1[2]]}, "latency_ns": pairs}


def _lat_stats(samples, m, n):
    """Latencies in ns of the first n lock-step samples under clock map m."""
    sub = np.array([s.submit_ns for s in samples[:n]], np.float64)
    con = np.array([s.consume_tick for s in samples[:n]], np.float64)
    com = np.array([s.complete_tick for s in samples[:n]], np.float64)
    pol = np.array([s.poll_ns for s in samples[:n]], np.float64)
    to_ns = lambda t: m.offset_ns + t * m.ns_per_tick

    def pct(x):
        return {"p50": float(np.percentile(x, 50)), "p99": float(np.percentile(x, 99)), "min": float(x.min()),
                "mean": float(x.mean())}

    return {"n": int(n), "submit_to_consume_ns": pct(to_ns(con) - sub), "complete_to_poll_ns": pct(pol - to_ns(com)),
            "round_trip_ns": pct(pol - sub), "device_consume_to_complete_ns": pct((com - con) * m.ns_per_tick)}


def _lat_run(L, launch, drive, pairs, n):
    """Clock samples, workers launched, a warm-up of 2 descriptors per pair,
    n lock-step samples, workers stopped, clock samples again."""
    import ctypes as C

    def clock():
        t, h, r = C.c_uint64(), C.c_double(), C.c_uint64()
        rlrt.check(L.rl_hip_trace_clock_sample(64, C.byref(t), C.byref(h), C.byref(r)), "clock sample")
        return t.value, h.value, r.value

    c0 = clock()
    stop = launch()
    try:
        warm = (rlrt.RingLockstepSample * (2 * pairs))()
        if drive(2 * pairs, warm, 0, 10**10) != 2 * pairs:
            raise rlrt.RlrtError("latency warm-up: a completion did not arrive")
        out = (rlrt.RingLockstepSample * n)()
        got = drive(n, out, 2 * pairs, 10**9)
    finally:
        C.cast(stop, C.POINTER(C.c_uint32))[0] = 1
        rlrt.sync()
    c1 = clock()
    if got != n:
        raise rlrt.RlrtError(f"latency: {got} of {n} lock-step samples")
    m = rlrt.TraceClockMap()
    L.trace_clock_fit(c0[0], c0[1], c1[0], c1[1], C.byref(m))
    res = _lat_stats(out, m, n)
    res["clock"] = {"ns_per_tick": m.ns_per_tick, "rtt_ns": [c0[2], c1[2]],
                    "split_error_ns_at_most": max(c0[2], c1[2]) / 2}
    return res


def wl_latency(args):
    """Unloaded latency across the ring boundary from device stamps, for the
    hw_desc worker and the command-ring worker at 1 pair and at one pair per
    compute unit: descriptor i goes to pair i % pairs only after the previous
    one's completion was polled (native lock-step driver, ring_latency.h), so
    every ring holds at most one descriptor while the other workers poll
    empty rings. submit -> consume: host CLOCK_MONOTONIC just before the
    command tail's release to the worker's s_memrealtime when its poll saw
    it; complete -> poll: the worker's stamp just before the completion
    tail's release to the host's poll seeing it. GPU ticks map to host ns by
    ping-pong clock samples before and after (the split between the two
    halves is good to half the best sample's round trip; their sum, the round
    trip, needs no map). hw_desc descriptors have seq_len = max_tokens (no
    decode step: a pure ring round trip); command-ring descriptors run the
    fixed128 step (one head, 32 tokens). The reference's targets (H100,
    docs/metrics.md:70-72): worker poll latency < 100 ns, completion
    notification < 200 ns."""
    import ctypes as C

    L = rlrt.lib()
    info = rlrt.DeviceInfo()
    rlrt.check(L.rl_hip_device_info(C.byref(info)), "rl_hip_device_info")
    G = int(info.cu_count)

    def coherent(n):
        p = L.rl_hip_host_alloc_coherent(n)
        if not p:
            raise rlrt.RlrtError("coherent host allocation failed")
        return p

    res = {"workload": "ring_latency_unloaded", "pairs": [1, G]}
    # ---- hw_desc worker: one rollout, MHA 8 x d64 fp16 (no step is run)
    w = synth.make_decode(1201, 1, 8, 8, 64, 16, 16, dtype="fp16", kv_std=0.5, reserve_tokens=32)
    bufs = [rlrt.DeviceBuffer.from_array(x) for x in (w.arena, w.table)]
    small = [rlrt.DeviceBuffer(1 << 16, zero=True) for _ in range(6)]
    for pairs in (1, G):
        cqs = [L.hw_ring_create() for _ in range(pairs)]
        dqs = [L.hw_ring_create() for _ in range(pairs)]
        rings, stop, stamps = coherent(16 * pairs), coherent(64), coherent(16 * pairs)
        for g in range(pairs):
            C.cast(rings, C.POINTER(C.c_void_p))[g] = cqs[g]
            C.cast(rings, C.POINTER(C.c_void_p))[pairs + g] = dqs[g]
        stats = rlrt.DeviceBuffer(pairs * 32, zero=True)
        a = rlrt.HwWorkerArgs(cmdq=rings, doneq=rings + 8 * pairs, groups=pairs, stop=stop, max_idle_polls=1 << 26,
                              arena_base=bufs[0].ptr, arena_bytes=bufs[0].nbytes,
                              layout=rlrt.KvLayoutDesc.paged(16, 64), block_table=bufs[1].ptr,
                              table_stride=w.table_stride, rollouts=1, q_heads=8, kv_heads=8, dtype=rlrt.DTYPE_FP16,
                              scale=0.0, max_steps=1, q=small[0].ptr, k_new=small[1].ptr, v_new=small[2].ptr,
                              logits=small[3].ptr, vocab=16, attn_out=small[4].ptr, token_out=small[5].ptr,
                              logprob_out=small[5].ptr, stats=stats.ptr, stamps=stamps)
        ws = rlrt.hw_worker_workspace(a)
        desc = rlrt.HwDesc(opcode=1, rollout_id=0, seq_len=16, max_tokens=16)

        def launch(a=a, stop=stop):
            C.cast(stop, C.POINTER(C.c_uint32))[0] = 0
            rlrt.hw_worker_launch(a)
            return stop

        def drive(n, out, first, timeout, rings=rings, pairs=pairs, stamps=stamps, desc=desc):
            return L.ring_lockstep_hw(rings, rings + 8 * pairs, pairs, C.byref(desc), n, stamps, timeout, out)

        log(f"[bench] latency: hw_desc worker, {pairs} pair(s)")
        res[f"hw_desc_{pairs}pairs"] = _lat_run(L, launch, drive, pairs, max(2000, 8 * pairs))
        st = stats.download(np.uint64, (pairs, 4))
        res[f"hw_desc_{pairs}pairs"]["worker_status"] = np.unique(st[:, 3]).tolist()
        for r in cqs + dqs:
            L.hw_ring_destroy(r)
        for p in (rings, stop, stamps):
            L.rl_hip_host_free(p)
        stats.close()
        ws.close()
    for b in bufs + small:
        b.close()
    # ---- command-ring worker: fixed128 step per descriptor
    nblk, io = 64, 64
    rng = np.random.default_rng(1202)
    darena = rlrt.DeviceBuffer.from_array(synth.f32_to_f16(rng.standard_normal(nblk * 8192, dtype=np.float32)))
    dq = rlrt.DeviceBuffer.from_array(synth.f32_to_f16(rng.standard_normal((io, 128), dtype=np.float32)))
    do = rlrt.DeviceBuffer(io * 128 * 4)
    for pairs in (1, G):
        rs = [L.ring_create() for _ in range(pairs)]
        crs = [L.comp_ring_create() for _ in range(pairs)]
        tab, stop, stamps = coherent(16 * pairs), coherent(64), coherent(16 * pairs)
        for g in range(pairs):
            C.cast(tab, C.POINTER(C.c_void_p))[g] = rs[g]
            C.cast(tab, C.POINTER(C.c_void_p))[pairs + g] = crs[g]
        stats = rlrt.DeviceBuffer(pairs * 32, zero=True)
        a = rlrt.CmdWorkerArgs(rings=tab, comp_rings=tab + 8 * pairs, groups=pairs, stop=stop,
                               max_idle_polls=1 << 26, arena_base=darena.ptr, arena_bytes=darena.nbytes,
                               sample_state=None, q_buffer=dq.ptr, o_buffer=do.ptr, io_slots=io, stats=stats.ptr,
                               stamps=stamps)
        desc = rlrt.Descriptor(seq_id=0, kv_block_offset=0, num_kv_blocks=32, output_token_offset=0,
                               reward_cookie=0)

        def launch(a=a, stop=stop):
            C.cast(stop, C.POINTER(C.c_uint32))[0] = 0
            rlrt.check(L.rl_hip_cmd_worker_launch(C.byref(a)), "rl_hip_cmd_worker_launch")
            return stop

        def drive(n, out, first, timeout, tab=tab, pairs=pairs, stamps=stamps, desc=desc):
            return L.ring_lockstep_cmd(tab, tab + 8 * pairs, pairs, C.byref(desc), first, n, stamps, timeout, out)

        log(f"[bench] latency: command-ring worker, {pairs} pair(s)")
        res[f"cmd_{pairs}pairs"] = _lat_run(L, launch, drive, pairs, max(2000, 8 * pairs))
        st = stats.download(np.uint64, (pairs, 4))
        res[f"cmd_{pairs}pairs"]["worker_status"] = np.unique(st[:, 3]).tolist()
        for r in rs:
            L.ring_destroy(r)
        for r in crs:
            L.comp_ring_destroy(r)
        for p in (tab, stop, stamps):
            L.rl_hip_host_free(p)
        stats.close()
    for b in (darena, dq, do):
        b.close()
    res["reference_targets_ns"] = {"worker_poll_latency": 100, "completion_notification": 200,
                                   "source": "docs/metrics.md:70-72 (H100 targets; context only)"}
    return res


WORKLOADS = {"sample256": wl_sample256, "sample32k": wl_sample32k, "longctx": wl_longctx, "proj": wl_proj,
             "plumbing": wl_plumbing, "plumbing256": wl_plumbing256, "ringstep": wl_ringstep,
             "rollout": wl_rollout, "cmdring": wl_cmdring, "rollout_pipeline": wl_rollout_pipeline,
             "pipeline": wl_pipeline, "pipeline_trace": wl_pipeline_trace, "latency": wl_latency}


def main():
    global CTX_LO, CTX_HI
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="step",
                    choices=["step", "pipeline", "unfused", "attn", "sample", "append", "copy", "pmc"],
                    help="step: the headline JSON line; pipeline: only the lane and one-stream pipeline passes; "
                         "unfused: rl_hip_decode_step + rl_hip_sample; attn/sample/append: one entry point alone")
    ap.add_argument("--workload", default="step", choices=["step"] + sorted(WORKLOADS),
                    help="step: the headline decode step; the others print one JSON line of their own")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--ctx", default=None, metavar="LO,HI",
                    help=f"ringstep only: contexts uniform in [LO, HI] (1 <= LO <= HI <= {MAX_CTX}; default "
                         f"{CTX_LO},{CTX_HI})")
    ap.add_argument("--grid-waves", type=int, default=0,
                    help="attention: persistent waves sharing the KV stream (0: library default, a full device)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: the decode hot path runs on one GPU here; multi-GPU runs are not part of it; "
              "the path shards by rollout, with no exchange inside a decode step.", file=sys.stderr)
        sys.exit(2)
    if args.ctx is not None:
        try:
            lo, hi = (int(v) for v in args.ctx.split(","))
        except ValueError:
            raise SystemExit(f"bench.py: --ctx takes LO,HI, not {args.ctx!r}")
        if args.workload != "ringstep" or not 1 <= lo <= hi <= MAX_CTX:
            raise SystemExit(f"bench.py: --ctx LO,HI applies to --workload ringstep, with 1 <= LO <= HI <= {MAX_CTX}")
        CTX_LO, CTX_HI = lo, hi

    traffic, traffic_note = None, "not measured (--no-traffic)"
    headline = args.workload == "step" and args.only == "step"
    if headline and not args.no_traffic:
        t0 = time.time()
        traffic, traffic_note = measure_traffic()
        log(f"[bench] counter passes in {time.time() - t0:.1f}s: {traffic if traffic else traffic_note}")

    _load()
    info = rlrt.open_device(0)
    log(f"[bench] device {info.arch.decode()} cu={info.cu_count} clock={info.clock_khz / 1e3:.0f} MHz")
    if args.only == "pmc":
        pmc_target()
        return
    if args.workload != "step":
        res = WORKLOADS[args.workload](args)
        res["device"] = info.arch.decode()
        print(json.dumps(res), flush=True)
        return
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
    attn_bytes = step.attn_bytes()
    step_bytes = attn_bytes + step.sample_bytes() + step.append_bytes()

    if args.only not in ("step", "pipeline"):
        for i in range(args.warmup):
            step.run(i, args.only)
        rlrt.sync()
        ms, wall = time_loop(step, args.steps, args.only)
        ms_step = ms / args.steps
        log(f"[bench] {args.only}: {args.steps} steps in {ms:.2f} ms (events), {wall:.2f} ms (host wall)")
        per = {"attn": attn_bytes, "sample": step.sample_bytes(), "append": step.append_bytes(),
               "unfused": step_bytes}[args.only]
        print(json.dumps({"only": args.only, "avg_launch_us": ms_step * 1e3,
                          "alg_gbps": per / (ms_step * 1e-3) / 1e9, "alg_bytes": per}), flush=True)
        return

    # the headline: the pipeline on the two lanes, then the same launches on
    # the library stream alone (back to back: the fused kernel's own rate)
    pipe = Pipeline(step)
    ms, wall = pipe.timed(args.steps, args.warmup, True)
    ms_one, _ = pipe.timed(args.steps, args.warmup, False)
    ms_step, one_us = ms / args.steps, ms_one / args.steps * 1e3
    step_gbps = step_bytes / (ms_step * 1e-3) / 1e9
    achieved = step_bytes / (one_us * 1e-6) / 1e9
    log(f"[bench] lanes: {args.steps} steps in {ms:.2f} ms (events), {wall:.2f} ms (host wall): "
        f"{ms_step * 1e3:.1f} us/step ({step_gbps:.0f} GB/s); one stream {one_us:.1f} us/step ({achieved:.0f} GB/s)")
    if args.only == "pipeline":
        print(json.dumps({"only": "pipeline", "lanes_us_per_step": ms_step * 1e3, "one_stream_us_per_step": one_us,
                          "alg_bytes": step_bytes}), flush=True)
        return

    # the unfused step of the same micro-batch and its kernels, each over its
    # own back-to-back launches (HIP events on the library stream)
    kern = {}
    for k in ("unfused", "attn", "sample", "append"):
        for i in range(args.warmup):
            step.run(i, k)
        kms, _ = time_loop(step, args.steps, k)
        kern[k] = kms / args.steps * 1e3
    copy_gbps = stream_copy_gbps()
    log(f"[bench] unfused step {kern['unfused']:.1f} us: attn {kern['attn']:.1f} us, sample {kern['sample']:.1f} us, "
        f"append {kern['append']:.1f} us; stream copy {copy_gbps:.0f} GB/s")

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
                               "kv_append_b64, 4 micro-batches on 2 lanes",
                   "batch": B, "q_heads": QH, "kv_heads": KVH, "head_dim": D, "block_tokens": TPB,
                   "ctx": f"U[{CTX_LO},{CTX_HI}] seed {SEED_KV}: mean {ctx.mean():.0f}, sum {int(ctx.sum())}",
                   "vocab": VOCAB, "temperature": TEMP, "top_k": TOPK, "top_p": TOPP,
                   "micro_batches": MICRO_BATCHES, "rollouts_in_flight": MICRO_BATCHES * B, "lanes": 2,
                   "step": "one launch per step: micro-batch t % 4's attention tiles and the sampling of its "
                           "logits; its sampling waves first merge step t - 2's split rows and append that "
                           "step's K/V token; steps alternate between two streams"},
        "steps_per_s": 1e3 / ms_step,
        "step_alg_bytes": step_bytes,
        "step_hbm_gbps": step_gbps,
        "step_hbm_frac": step_gbps / PEAK_HBM_GBPS,
        "one_stream_us_per_step": one_us,
        "unfused_us_per_step": kern["unfused"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS,
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_detail": traffic if traffic else traffic_note,
                     "kernel": "decode_fused_kernel<128,4,bf16,16> (one launch per step, with the merge of "
                               "step t - 2)",
                     "alg_bytes_per_launch": step_bytes, "avg_launch_us": one_us,
                     "avg_launch_note": "launches back to back on one stream (HIP events over the timed "
                                        "steps / steps); on the two lanes launches overlap, so their rate is "
                                        "the headline step_hbm_gbps instead"},
        "kernels_us": kern,
        "stream_copy_gbps": copy_gbps,
        "device": {"arch": info.arch.decode(), "cu": info.cu_count, "clock_mhz": info.clock_khz / 1e3},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
