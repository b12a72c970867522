"""The GRPO rollout loop on one GPU, driven through the C ABI.

Host-side driver of the device rollout path, in the shape of the reference's
bench/bench_gpu_scheduler.cu (request ring in, done ring out) with the real
decode step of cu/worker.cu in between:

  request ring -> rl_hip_rollout_schedule (commit / retire / admit / prepare)
               -> rl_hip_decode_step (GQA over the block-paged arena, with the
                  step's KV append inside the attention's merge kernel)
               -> rl_hip_logits_proj (attn_out . W_vocab on MFMA)
               -> rl_hip_sample (top-p, per-slot Philox seed and step)
               -> done ring, then rl_hip_reward_advantage per group.

Workload: 512 requests in 64 groups of 8. A group shares a 512-token prompt
prefix (32 full 16-token blocks per kv head: the same physical blocks in every
member's table; a kv_prefix with one branch per member, whose table image the
device reads) plus U[0, 512] private prompt tokens; each request generates
256 tokens. GQA 32 q / 8 kv heads, d128, bf16 K/V ~N(0,1); queries and new K/V
rows come from a pool of 8 seeded steps; W_vocab bf16 [32,000 x 4,096]
~N(0, 0.02^2); top-p 0.9 at temperature 1. 256 rollout slots.
"""
from __future__ import annotations

import ctypes as C
import time

import numpy as np

import rlrt
import synth

GROUPS, GS = 64, 8
REQ = GROUPS * GS
PREFIX, PRIV_MAX, GEN = 512, 512, 256
QH, KVH, D, TPB = 32, 8, 128, 16
HID, VOCAB = QH * D, 32000
SLOTS = 256
TEMPERATURE, TOP_K, TOP_P = 1.0, 0, 0.9  # every request's sampling parameters
POOL = 8
REQ_RING_SLOTS = 1024
STATE_BYTES = 18464        # sizeof(GpuRolloutState)
PREFIX_TABLE_BYTES = 606280  # sizeof(KVPrefixTable)


def req_ring_push(ring: int, req: rlrt.RolloutRequest) -> int:
    """Producer side of request.h's RequestRing (34-byte packed slots)."""
    L = rlrt.lib()
    head, tail = L.hw_ring_load_acquire(ring), L.hw_ring_load_acquire(ring + 64)
    if (tail - head) & 0xFFFFFFFF >= REQ_RING_SLOTS:
        return -1
    C.memmove(ring + 128 + (tail & (REQ_RING_SLOTS - 1)) * 34, C.byref(req), 34)
    L.hw_ring_store_release(ring + 64, (tail + 1) & 0xFFFFFFFF)
    return 0


def done_ring_pop(ring: int) -> rlrt.RolloutDone | None:
    """Consumer side of request.h's DoneRing (24-byte packed slots)."""
    L = rlrt.lib()
    head = L.hw_ring_load_acquire(ring)
    if head == L.hw_ring_load_acquire(ring + 64):
        return None
    d = rlrt.RolloutDone.from_buffer_copy(
        (C.c_char * 24).from_address(ring + 256 + (head & (REQ_RING_SLOTS - 1)) * 24))
    L.hw_ring_store_release(ring, (head + 1) & 0xFFFFFFFF)
    return d


def build_workload(seed: int, prefix: int = PREFIX, priv_zero_every: int = 0) -> dict:
    """Seeded host inputs: prompts, block tables (shared prefix blocks), arena,
    W_vocab, query / K / V pools, per-group targets and per-request seeds.

    Group g's prefix occupies KVH * ceil(prefix / TPB) consecutive arena
    blocks from prefix_base[g], head-major (the layout a KVPrefix's
    kv_block_offset / kv_block_count describe); the groups' ranges and the
    private blocks sit at seeded random places. Full prefix blocks are shared
    by the group's members. When prefix is not a multiple of TPB, its last
    block is partly filled: each member writes its own tokens into a private
    block instead (copy-on-write). Members with private prompt tokens hold the
    prefix's slots of that block already (their prompt was prefilled); those
    without (every priv_zero_every-th request, when set) still hold random
    bytes there, and the loop's copy-on-write fills them before their first
    step."""
    rng = np.random.default_rng(seed)
    priv = rng.integers(0, PRIV_MAX + 1, REQ)
    if priv_zero_every:
        priv[::priv_zero_every] = 0
    prompt = (prefix + priv).astype(np.uint32)
    n_shared = prefix // TPB                    # full prefix blocks, shared
    n_pb = -(-prefix // TPB)                    # prefix blocks per head (the last maybe partial)
    first_own = prefix - prefix % TPB           # first position in a private block
    n_priv = -(-(prompt.astype(np.int64) + GEN + 1 - first_own) // TPB)
    stride = -(-(prefix + PRIV_MAX + GEN + 1) // TPB)  # covers the largest context
    n_private = int(n_priv.sum()) * KVH
    # place the 64 prefix ranges and the private blocks in one seeded shuffle of units
    units = np.concatenate([np.full(GROUPS, KVH * n_pb), np.ones(n_private, np.int64)])
    order = rng.permutation(len(units))
    start = np.zeros(len(units), np.int64)
    start[order] = np.concatenate([[0], np.cumsum(units[order])[:-1]])
    total = int(units.sum())
    prefix_base = start[:GROUPS].astype(np.uint32)
    private = start[GROUPS:].astype(np.uint32)
    prefix_blocks = (prefix_base[:, None, None] + np.arange(KVH)[None, :, None] * n_pb
                     + np.arange(n_pb)[None, None, :]).astype(np.uint32)
    table = np.zeros((REQ, KVH, stride), np.uint32)
    k = 0
    for r in range(REQ):
        for h in range(KVH):
            table[r, h, :n_shared] = prefix_blocks[r // GS, h, :n_shared]
            m = int(n_priv[r])
            table[r, h, n_shared:n_shared + m] = private[k:k + m]
            k += m
    arena = np.empty(total * 2 * TPB * D, np.uint16)
    synth._fill_normal(rng, arena.size, 1.0, "bf16", arena)
    if prefix % TPB:
        # prefill of the members with private prompt tokens: the prefix's slots
        # of the partly filled block copied into their private block (K and V planes)
        blk = arena.reshape(total, 2, TPB, D)
        slot = prefix % TPB
        for r in np.nonzero(priv > 0)[0]:
            for h in range(KVH):
                src, dst = prefix_blocks[r // GS, h, n_shared], table[r, h, n_shared]
                blk[dst, :, :slot] = blk[src, :, :slot]
    w = synth.f32_to_bf16(rng.standard_normal((VOCAB, HID), dtype=np.float32) * np.float32(0.02))
    qpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, QH, D), dtype=np.float32))
    kpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, KVH, D), dtype=np.float32))
    vpool = synth.f32_to_bf16(rng.standard_normal((POOL, SLOTS, KVH, D), dtype=np.float32))
    targets = rng.integers(0, VOCAB, (GROUPS, GEN), dtype=np.uint32)
    seeds = rng.integers(0, 2**63, REQ, dtype=np.uint64)
    return dict(prompt=prompt, table=table, stride=stride, arena=arena.view(np.uint8), w=w, qpool=qpool,
                kpool=kpool, vpool=vpool, targets=targets, seeds=seeds, prefix_blocks=prefix_blocks,
                prefix_base=prefix_base, prefix=prefix, priv=priv, n_blocks=n_shared + n_priv)


def build_prefix_table(cfg: dict) -> tuple[np.ndarray, np.ndarray]:
    """The host KVPrefixTable of a workload (src/kv_prefix.c rules through the
    library): group g's prefix registered as id g at block offset
    prefix_base[g] with KVH * ceil(prefix / TPB) blocks, and one branch per
    request (rollout id = request id) on its group's prefix, whose delta is the
    request's first private block. Returns (table image, branch id of each request)."""
    L = rlrt.lib()
    ptab = np.zeros(PREFIX_TABLE_BYTES, np.uint8)
    L.kv_prefix_table_init(ptab.ctypes.data)
    prefix = cfg["prefix"]
    n_shared, n_pb = prefix // TPB, -(-prefix // TPB)
    pid, bid = C.c_uint32(), C.c_uint32()
    branch = np.zeros(REQ, np.uint32)
    for g in range(GROUPS):
        if L.kv_prefix_register(ptab.ctypes.data, int(cfg["prefix_base"][g]), prefix, KVH * n_pb,
                                C.byref(pid)) != 0 or pid.value != g:
            raise rlrt.RlrtError(f"kv_prefix_register for group {g} failed")
    for r in range(REQ):
        if L.kv_branch_alloc(ptab.ctypes.data, r, r // GS, int(cfg["table"][r, 0, n_shared]), int(cfg["priv"][r]),
                             int(cfg["n_blocks"][r]) - n_shared, C.byref(bid)) != 0:
            raise rlrt.RlrtError(f"kv_branch_alloc for request {r} failed")
        branch[r] = bid.value
    return ptab, branch


class RolloutLoop:
    """Device buffers, rings and launch arguments of one GRPO run."""

    def __init__(self, cfg: dict):
        L = rlrt.lib()
        self.cfg = cfg
        self.dev = dev = {}
        # the KV arena through arena.h: HBM base from arena_init, one arena_acquire
        # per block (lowest id first, so the workload's block ids are arena ids)
        block_bytes = 2 * TPB * D * 2
        n_blocks = cfg["arena"].nbytes // block_bytes
        arena = rlrt.Arena(n_blocks * block_bytes, block_bytes)
        ids = arena.acquire_n(n_blocks)
        if not np.array_equal(ids, np.arange(n_blocks)):
            raise rlrt.RlrtError("arena_acquire did not hand out the lowest free blocks in order")
        arena.upload(cfg["arena"])
        dev["arena"] = arena
        for k in ("w", "qpool", "kpool", "vpool", "prompt", "targets"):
            dev[k] = rlrt.DeviceBuffer.from_array(cfg[k])
        dev["rtab"] = rlrt.DeviceBuffer.from_array(cfg["table"])
        stride = self.stride = cfg["stride"]
        self.ptab, self.branch = build_prefix_table(cfg)
        dev["ptab"] = rlrt.DeviceBuffer.from_array(self.ptab)
        dev["branch"] = rlrt.DeviceBuffer.from_array(self.branch)
        for k, n in (("state", STATE_BYTES), ("counters", 16), ("gen", REQ * GEN * 4), ("rewards", REQ * 4),
                     ("stab", SLOTS * KVH * stride * 4), ("ctx", SLOTS * 4), ("temp", SLOTS * 4),
                     ("topk", SLOTS * 4), ("topp", SLOTS * 4), ("seed", SLOTS * 8), ("step", SLOTS * 8),
                     ("out", SLOTS * HID * 2), ("out32", SLOTS * HID * 4), ("logits", SLOTS * VOCAB * 4),
                     ("tok", SLOTS * 4), ("lp", SLOTS * 4), ("sreq", SLOTS * 4)):
            dev[k] = rlrt.DeviceBuffer(n, zero=True)
        dev["pos"] = rlrt.DeviceBuffer.from_array(np.full(SLOTS, 0xFFFFFFFF, np.uint32))

        self.rr, self.dr = L.req_ring_create(), L.done_ring_create()
        if not (self.rr and self.dr):
            raise rlrt.RlrtError("request/done ring allocation failed")
        self.sched = rlrt.SchedArgs(
            req_ring=self.rr, done_ring=self.dr, state=dev["state"].ptr, requests=REQ, prompt_len=dev["prompt"].ptr,
            req_table=dev["rtab"].ptr, kv_heads=KVH, table_stride=stride, gen_tokens=dev["gen"].ptr,
            gen_stride=GEN, targets=dev["targets"].ptr, group_size=GS, target_len=GEN,
            rewards=dev["rewards"].ptr, slot_table=dev["stab"].ptr, slot_ctx=dev["ctx"].ptr,
            slot_pos=dev["pos"].ptr, slot_temp=dev["temp"].ptr, slot_topk=dev["topk"].ptr,
            slot_topp=dev["topp"].ptr, slot_seed=dev["seed"].ptr, slot_step=dev["step"].ptr, sampled=None,
            counters=dev["counters"].ptr, slot_request=dev["sreq"].ptr)
        self.layout = rlrt.KvLayoutDesc.paged(TPB, D)
        max_ctx = cfg["prefix"] + PRIV_MAX + GEN + 1
        # copy-on-write of the prefix's partly filled block before a member's
        # first own token: needed only when the prefix ends inside a block
        self.cow = None
        if cfg["prefix"] % TPB:
            self.cow = rlrt.CowArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=self.layout,
                                    prefixes=dev["ptab"].ptr, row_key=dev["sreq"].ptr,
                                    branch_of_key=dev["branch"].ptr, keys=REQ, block_table=dev["stab"].ptr,
                                    table_stride=stride, batch=SLOTS, kv_heads=KVH, positions=dev["pos"].ptr)
        self.attn = rlrt.attn_args(dev["arena"], self.layout, dev["stab"], stride, SLOTS, QH, KVH,
                                   rlrt.DTYPE_BF16, dev["ctx"], max_ctx, dev["qpool"], dev["out"], dev["out32"])
        self.attn_ws = rlrt.attn_workspace(self.attn)
        s = rlrt.sample_args(dev["logits"], SLOTS, VOCAB, VOCAB, dev["tok"], dev["lp"])
        s.temperature, s.top_k, s.top_p = dev["temp"].ptr, dev["topk"].ptr, dev["topp"].ptr
        if TOP_K == 0:  # no request uses top-k: the sampler's whole-row path takes every slot
            s.top_k, s.top_k_all = None, 0
        s.seed, s.steps = dev["seed"].ptr, dev["step"].ptr
        self.samp = s
        self.samp_ws = rlrt.sample_workspace(s)
        self.app = rlrt.AppendArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=self.layout,
                                   block_table=dev["stab"].ptr, table_stride=stride, batch=SLOTS, kv_heads=KVH,
                                   positions=dev["pos"].ptr, cow_src=None)
        self.proj = rlrt.ProjArgs(x=dev["out"].ptr, w=dev["w"].ptr, logits=dev["logits"].ptr, rows=SLOTS,
                                  vocab=VOCAB, hidden=HID, x_stride=HID, w_stride=HID, logits_stride=VOCAB)
        self.q_row = SLOTS * QH * D * 2
        self.kv_row = SLOTS * KVH * D * 2
        self.dones: list[tuple] = []
        self.t = 0
        self.feeder = None

    def submit_requests(self) -> None:
        """512 requests (temperature 1, top-p 0.9, per-request seed) and the end marker."""
        cfg = self.cfg
        for r in range(REQ):
            req = rlrt.RolloutRequest(request_id=r, max_tokens=GEN, kv_blocks=int(cfg["n_blocks"][r]),
                                      temperature=TEMPERATURE, top_k=TOP_K, top_p=TOP_P,
                                      rng_seed=int(cfg["seeds"][r]))
            if req_ring_push(self.rr, req) != 0:
                raise rlrt.RlrtError("request ring full")
        if req_ring_push(self.rr, rlrt.RolloutRequest(request_id=2**64 - 1)) != 0:
            raise rlrt.RlrtError("request ring full")

    def attach_pipeline(self, decode_credits: int = 384) -> None:
        """Feed the request ring from the host rollout pipeline (pipeline.h /
        pipeline_feed.h) instead of one upfront burst: every request is
        registered as a rollout (FREE -> PREFILL_READY, Q_PREFILL); each done
        poll retires the dones (reward handoff on the RewardRing, the rollout
        freed, its decode credit returned), admits rollouts to Q_DECODE while
        decode credits last and sends them FIFO. decode_credits bounds the
        rollouts queued on or running in the device (256 slots)."""
        L = rlrt.lib()
        cfg = self.cfg
        self.pipe = np.zeros(rlrt.PIPELINE_BYTES, np.uint8)
        self.reward_ring = np.zeros(rlrt.REWARD_RING_BYTES, np.uint8)
        self.rid_map = np.zeros(REQ, np.uint32)
        if L.pipeline_init(self.pipe.ctypes.data) != 0:
            raise rlrt.RlrtError("pipeline_init failed")
        L.pipeline_credits_set(self.pipe.ctypes.data, decode_credits, 0, 0, 0)
        L.reward_ring_init(self.reward_ring.ctypes.data)
        self.feeder = rlrt.PipelineFeeder()
        fp = rlrt.FeedParams(temperature=TEMPERATURE, top_k=TOP_K, top_p=TOP_P, block_tokens=TPB)
        if L.rl_feed_init(C.byref(self.feeder), self.pipe.ctypes.data, self.rr, self.dr,
                          self.reward_ring.ctypes.data, self.rid_map.ctypes.data, REQ, C.byref(fp)) != 0:
            raise rlrt.RlrtError("rl_feed_init failed")
        self.request_of_rid = {}
        for r in range(REQ):
            rid = L.rl_feed_register(C.byref(self.feeder), r, int(cfg["prompt"][r]), GEN, int(cfg["seeds"][r]))
            if rid < 0:
                raise rlrt.RlrtError(f"rl_feed_register({r}) failed")
            self.request_of_rid[rid] = r
        self._pump()

    def _pump(self) -> None:
        L = rlrt.lib()
        L.rl_feed_pump(C.byref(self.feeder))
        if self.feeder.stats.sent == REQ:
            L.rl_feed_end(C.byref(self.feeder))
        rd = rlrt.RewardDesc()
        while L.reward_pop(self.reward_ring.ctypes.data, C.byref(rd)) == 0:
            self.dones.append((self.request_of_rid[rd.rollout_id], None, rd.token_count, rd.reward, rd.flags))

    def schedule(self) -> None:
        self.sched.sampled = self.dev["tok"].ptr if self.t > 0 else None
        rlrt.check(rlrt.lib().rl_hip_rollout_schedule(C.byref(self.sched)), "rl_hip_rollout_schedule")

    def step(self) -> None:
        """Schedule, the copy-on-write of members at their first own token when
        the prefix ends inside a block (rl_hip_kv_cow: the device resolves each
        slot's branch in the prefix table image), then one batched decode step over the 256 slots: attention
        with the step's KV append run inside its merge kernel
        (rl_hip_decode_step; the append writes position ctx, which the
        attention does not read), projection, sampling."""
        dev, t = self.dev, self.t
        self.schedule()
        if self.cow is not None:
            rlrt.kv_cow(self.cow)
        self.attn.q = dev["qpool"].ptr + (t % POOL) * self.q_row
        self.app.k_new = dev["kpool"].ptr + (t % POOL) * self.kv_row
        self.app.v_new = dev["vpool"].ptr + (t % POOL) * self.kv_row
        rlrt.decode_step(self.attn, self.app)
        rlrt.check(rlrt.lib().rl_hip_logits_proj(C.byref(self.proj)), "rl_hip_logits_proj")
        rlrt.sample(self.samp)
        self.t += 1

    def drain_dones(self) -> np.ndarray:
        """Pops every published RolloutDone; returns the scheduler counters
        {dones, admitted, end seen, status}."""
        if self.feeder is not None:
            self._pump()
        else:
            while (d := done_ring_pop(self.dr)) is not None:
                self.dones.append((d.request_id, d.rollout_id, d.tokens_generated, d.reward, d.status))
        return self.dev["counters"].download(np.uint32, 4)

    def finish(self) -> None:
        """The commit of the last step and the final retirements."""
        self.schedule()
        rlrt.sync()
        self.drain_dones()

    def run(self, check_steps=(), on_check=None, window=(20, 120), poll_every: int = 32,
            max_steps: int = 700) -> dict:
        """Runs until every request is done. After each step in check_steps the
        stream is synchronised and on_check(t) runs. Done polling (one sync
        every poll_every steps) pauses inside `window`, whose steps are timed
        on the host clock with the stream drained at both ends."""
        t0 = time.perf_counter()
        tw = None
        while len(self.dones) < REQ:
            if self.t >= max_steps:
                raise rlrt.RlrtError(f"rollout loop did not finish: {len(self.dones)} dones, "
                                     f"counters {self.dev['counters'].download(np.uint32, 4)}")
            t = self.t
            self.step()
            if t in check_steps and on_check is not None:
                rlrt.sync()
                on_check(t)
            if t in window:
                rlrt.sync()
                if t == window[0]:
                    tw = time.perf_counter()
                else:
                    tw = time.perf_counter() - tw
            if self.t % poll_every == 0 and not window[0] <= t <= window[1]:
                rlrt.sync()
                st = self.drain_dones()
                if st[3] != 0:
                    raise rlrt.RlrtError(f"scheduler status {st[3]}")
        self.finish()
        wall = time.perf_counter() - t0
        return {"steps": self.t, "wall_s": wall, "window_steps": window[1] - window[0],
                "window_us_per_step": tw / (window[1] - window[0]) * 1e6 if tw is not None else None}

    def close(self) -> None:
        L = rlrt.lib()
        for b in list(self.dev.values()) + [self.attn_ws, self.samp_ws]:
            b.close()
        if self.rr:
            L.req_ring_destroy(self.rr)
            L.done_ring_destroy(self.dr)
            self.rr = self.dr = None
