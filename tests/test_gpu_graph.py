"""A decode step captured into a HIP graph (rl_hip_capture_begin / _end) and
replayed (rl_hip_graph_launch) gives, at every replay, the bytes the same
calls give when launched directly: attention outputs (bf16 and fp32), the
KV arena after the fused append, sampled tokens and logprobs. The replays
are interleaved with direct launches and synchronisations."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def test_captured_decode_step_replays_exactly(rl, gpu):
    B, QH, KVH, D, TPB, V = 16, 32, 8, 128, 16, 32000
    w = synth.make_decode(51, B, QH, KVH, D, 300, 900, dtype="bf16", spare_blocks=8)
    logits = synth.make_logits(52, B, V, spikes=3)
    rng = np.random.default_rng(53)
    dev = {k: rl.DeviceBuffer.from_array(v) for k, v in
           (("arena", w.arena), ("table", w.table), ("ctx", w.ctx), ("q", w.q), ("pos", w.ctx.copy()),
            ("kn", rng.integers(0, 256, (B, KVH, D * 2), dtype=np.uint8)),
            ("vn", rng.integers(0, 256, (B, KVH, D * 2), dtype=np.uint8)), ("logits", logits),
            ("seeds", rng.integers(0, 2**63, B, dtype=np.uint64)))}
    n = B * QH * D
    out, out32, tok, lp = rl.DeviceBuffer(n * 2), rl.DeviceBuffer(n * 4), rl.DeviceBuffer(B * 4), rl.DeviceBuffer(B * 4)
    layout = rl.KvLayoutDesc.paged(TPB, D)
    a = rl.attn_args(dev["arena"], layout, dev["table"], w.table_stride, B, QH, KVH, rl.DTYPE_BF16, dev["ctx"],
                     w.max_ctx, dev["q"], out, out32)
    ws = rl.attn_workspace(a)
    ap = rl.AppendArgs(arena_base=dev["arena"].ptr, arena_bytes=dev["arena"].nbytes, layout=layout,
                       block_table=dev["table"].ptr, table_stride=w.table_stride, batch=B, kv_heads=KVH,
                       positions=dev["pos"].ptr, cow_src=None, k_new=dev["kn"].ptr, v_new=dev["vn"].ptr)
    s = rl.sample_args(dev["logits"], B, V, V, tok, lp, temperature=0.8, top_k=50, top_p=0.9, seeds=dev["seeds"])
    s.step = 7
    sws = rl.sample_workspace(s)

    def step():
        rl.decode_step(a, ap)
        rl.sample(s)

    def state():
        return (out.download(np.uint16, n), out32.download(np.float32, n), dev["arena"].download(np.uint8, w.arena.size),
                tok.download(np.uint32, B), lp.download(np.float32, B))

    step()
    rl.sync()
    want = state()
    g = rl.Graph(step)
    try:
        for r in range(3):
            print(f"[graph] replay {r}", flush=True)
            for b in (out, out32, tok, lp):
                rl.check(rl.lib().rl_hip_memset_d(b.ptr, 0xFF, b.nbytes), "memset")   # eager, between replays
            rl.sync()
            g.launch()
            rl.sync()
            got = state()
            for x, y in zip(got, want):
                assert np.array_equal(x, y), r
            step()          # a direct launch between the replays
            rl.sync()
    finally:
        g.close()
    for b in list(dev.values()) + [out, out32, tok, lp, ws, sws]:
        b.close()
