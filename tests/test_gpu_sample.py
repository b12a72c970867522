"""On-device sampling vs the oracle: token ids bit-exact, logprobs within 1e-4."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _run(rl, logits, vocab=None, greedy=False, temperature=1.0, top_k=0, top_p=1.0, seeds=None, step=0):
    rows, stride = logits.shape
    vocab = stride if vocab is None else vocab
    lg = rl.DeviceBuffer.from_array(np.ascontiguousarray(logits, dtype=np.float32))
    tok = rl.DeviceBuffer(rows * 4)
    lp = rl.DeviceBuffer(rows * 4)
    sd = rl.DeviceBuffer.from_array(np.asarray(seeds, dtype=np.uint64)) if seeds is not None else None
    args = rl.sample_args(lg, rows, vocab, stride, tok, lp, greedy=greedy, temperature=temperature, top_k=top_k,
                          top_p=top_p, step=step, seeds=sd)
    ws = rl.sample_workspace(args)
    rl.sample(args)
    rl.sync()
    out = tok.download(np.uint32, rows), lp.download(np.float32, rows)
    for b in (lg, tok, lp, ws) + ((sd,) if sd is not None else ()):
        b.close()
    return out


def _check(rl, orc, olib, logits, vocab=None, **kw):
    rows, stride = logits.shape
    print(f"[sample] rows={rows} vocab={vocab or stride} {kw.get('greedy')} T={kw.get('temperature')} "
          f"k={kw.get('top_k')} p={kw.get('top_p')} step={kw.get('step', 0)}", flush=True)
    gt, gl = _run(rl, logits, vocab=vocab, **kw)
    seeds = kw.get("seeds")
    ot, ol = orc.sample_rows(olib, logits, kw.get("greedy", False), kw.get("temperature", 1.0), kw.get("top_k", 0),
                             kw.get("top_p", 1.0), seeds if seeds is not None else 0, kw.get("step", 0), vocab=vocab)
    bad = np.nonzero(gt != ot)[0]
    assert bad.size == 0, (bad[:10], gt[bad[:10]], ot[bad[:10]])
    np.testing.assert_allclose(gl.astype(np.float64), ol, rtol=0, atol=1e-4, equal_nan=True)
    return gt


def test_greedy_config3_shape_with_spike_ties(rl, gpu, orc, olib):
    """256 rows x 128,256 fp32 ~N(0,1) with 5 spike tokens per row SET to 8.0
    (5-way ties: the lowest index must win)."""
    x = synth.make_logits(3, 256, 128256, spikes=5)
    tok = _check(rl, orc, olib, x, greedy=True)
    for r in range(0, 256, 37):
        assert tok[r] == np.flatnonzero(x[r] == np.float32(8.0)).min()


def test_topk_topp_config3(rl, gpu, orc, olib):
    """Temperature 0.8, top-k 50, top-p 0.9, Philox per-row seed, several steps."""
    x = synth.make_logits(3, 256, 128256, spikes=5)
    seeds = np.random.default_rng(33).integers(0, 2**63, 256, dtype=np.uint64)
    prev = None
    for step in (0, 1, 12345):
        tok = _check(rl, orc, olib, x, temperature=0.8, top_k=50, top_p=0.9, seeds=seeds, step=step)
        if prev is not None:
            assert (tok != prev).any()
        prev = tok


@pytest.mark.parametrize("vocab,stride", [(32000, 32000), (50257, 50260), (1000, 1000), (16384, 16384),
                                          (16385, 16388)])
@pytest.mark.parametrize("k,p,T", [(1, 1.0, 1.0), (50, 0.9, 0.8), (256, 0.95, 1.3), (300, 0.5, 1.0),
                                   (7, 0.05, 0.6)])
def test_vocab_and_parameter_grid(rl, gpu, orc, olib, vocab, stride, k, p, T):
    rng = np.random.default_rng(vocab + k)
    x = np.full((24, stride), -1e30, dtype=np.float32)
    x[:, :vocab] = rng.standard_normal((24, vocab), dtype=np.float32) * 2
    x[3, :vocab] = np.round(x[3, :vocab])                    # heavy ties, also at the cutoff
    x[5, :vocab] = 0.0                                       # all equal
    x[7, :vocab] = -np.inf
    x[7, vocab // 2] = 1.0                                   # one finite logit
    _check(rl, orc, olib, x, vocab=vocab, temperature=T, top_k=k, top_p=p,
           seeds=np.arange(24, dtype=np.uint64) * 7919 + 1, step=3)
    _check(rl, orc, olib, x, vocab=vocab, greedy=True)


def test_whole_vocab_nucleus_rollout_shape(rl, gpu, orc, olib):
    """Top-p 0.9 with no top-k over 32,000 logits (the rollout-loop sampler):
    the exact full-row path, 512 rows."""
    rng = np.random.default_rng(77)
    x = rng.standard_normal((512, 32000), dtype=np.float32) * np.float32(0.3)
    seeds = rng.integers(0, 2**63, 512, dtype=np.uint64)
    _check(rl, orc, olib, x, temperature=1.0, top_k=0, top_p=0.9, seeds=seeds, step=5)


@pytest.mark.parametrize("vocab,std,p,T", [(128256, 1.0, 0.9, 1.0), (50257, 2.0, 0.99, 0.7), (1000, 3.0, 0.5, 1.0),
                                           (32000, 6.0, 0.95, 1.0), (4099, 0.05, 0.3, 2.0)])
def test_whole_vocab_nucleus_spreads(rl, gpu, orc, olib, vocab, std, p, T):
    """Whole-vocabulary nucleus over several spreads: the boundary lands in
    dense bins (small std), in the sparse tail (large std, p near 1) and near
    the zero-weight limit; rows with spike ties and a few -inf entries."""
    rng = np.random.default_rng(vocab)
    stride = -(-vocab // 4) * 4
    x = np.full((40, stride), 5.0, dtype=np.float32)          # the padding is never read
    x[:, :vocab] = rng.standard_normal((40, vocab), dtype=np.float32) * np.float32(std)
    x[1, rng.choice(vocab, 7, replace=False)] = np.float32(3.0 * std)
    x[2, rng.choice(vocab, vocab // 3, replace=False)] = -np.inf
    seeds = rng.integers(0, 2**63, 40, dtype=np.uint64)
    _check(rl, orc, olib, x, vocab=vocab, temperature=T, top_k=0, top_p=p, seeds=seeds, step=11)


@pytest.mark.parametrize("k", [0, 3])
def test_exact_path_edge_rows(rl, gpu, orc, olib, k):
    """Rows forcing the exact path: every logit equal, heavy ties, all -inf."""
    x = np.zeros((6, 20000), dtype=np.float32)
    x[1] = np.round(np.random.default_rng(1).standard_normal(20000) * 2)
    x[2, :] = -np.inf
    x[3, :] = -np.inf
    x[3, 12345] = 0.5
    x[4, ::2] = 1.0
    x[5] = np.random.default_rng(2).standard_normal(20000)
    for p in (1.0, 0.9, 0.3):
        _check(rl, orc, olib, x, temperature=0.7, top_k=k, top_p=p, seeds=np.arange(6, dtype=np.uint64) + 9, step=2)


@pytest.mark.parametrize("vocab,stride", [(32768, 32768), (32769, 32772), (32001, 32004), (5, 8)])
def test_row_kernel_vocab_edges(rl, gpu, orc, olib, vocab, stride):
    """Whole-vocabulary nucleus at the row kernel's limits: 32,768 logits (the
    largest row one workgroup holds), 32,769 (the split and merge path), a
    row ending inside a quad, and a five-logit row; p from 0.05 to 0.999 over
    the rows, ~N(0, 1) logits with spike ties and -inf entries."""
    rng = np.random.default_rng(vocab)
    rows = 24
    x = np.full((rows, stride), np.float32(7.0))           # padding past vocab never read
    x[:, :vocab] = rng.standard_normal((rows, vocab), dtype=np.float32)
    x[1, :vocab:97] = np.float32(3.5)
    x[2, rng.choice(vocab, max(1, vocab // 4), replace=False)] = -np.inf
    seeds = rng.integers(0, 2**63, rows, dtype=np.uint64)
    for p in (0.05, 0.5, 0.9, 0.999):
        _check(rl, orc, olib, x, vocab=vocab, temperature=0.9, top_k=0, top_p=p, seeds=seeds, step=int(p * 1000))
    _check(rl, orc, olib, x, vocab=vocab, greedy=True)


def test_row_kernel_per_row_parameters(rl, gpu, orc, olib):
    """Per-row temperature / top-p / seed / step arrays over 32,000 logits with
    no top-k: greedy rows (temperature 0) next to nucleus rows and rows with
    top-p 1 in one launch, every row against the oracle with its own
    parameters."""
    rows, V = 48, 32000
    rng = np.random.default_rng(4242)
    x = rng.standard_normal((rows, V), dtype=np.float32) * np.float32(0.5)
    temp = rng.choice(np.float32([0.0, 0.6, 1.0, 1.7]), rows).astype(np.float32)
    topp = rng.choice(np.float32([1.0, 0.95, 0.9, 0.3]), rows).astype(np.float32)
    seeds = rng.integers(0, 2**63, rows, dtype=np.uint64)
    steps = rng.integers(0, 2**40, rows, dtype=np.uint64)
    bufs = [rl.DeviceBuffer.from_array(a) for a in (x, temp, topp, seeds, steps)]
    tok, lp = rl.DeviceBuffer(rows * 4), rl.DeviceBuffer(rows * 4)
    args = rl.sample_args(bufs[0], rows, V, V, tok, lp)
    args.temperature, args.top_p, args.seed, args.steps = bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, bufs[4].ptr
    ws = rl.sample_workspace(args)
    print("[sample] per-row parameters, 48 x 32000", flush=True)
    rl.sample(args)
    rl.sync()
    gt, gl = tok.download(np.uint32, rows), lp.download(np.float32, rows)
    import ctypes as C
    lpv = C.c_double()
    for r in range(rows):
        want = olib.orc_sample_row(x[r].ctypes.data, V, 0, float(temp[r]), 0, float(topp[r]), int(seeds[r]),
                                   int(steps[r]), r, C.byref(lpv))
        assert gt[r] == want, (r, temp[r], topp[r], gt[r], want)
        assert abs(gl[r] - lpv.value) < 1e-4, r
    for b in bufs + [tok, lp, ws]:
        b.close()


@pytest.mark.parametrize("rows,vocab,stride", [(160, 50257, 50260), (144, 128256, 128256), (40, 128256, 128256),
                                                (24, 70001, 70004), (150, 32769, 32772), (144, 65537, 65540)])
def test_stream_kernel_mixed_rows(rl, gpu, orc, olib, rows, vocab, stride):
    """Per-row arrays over long rows: 144 or more rows take the
    one-workgroup-per-row stream kernel, fewer the split and merge kernels.
    32,769 and 65,537 logits end one logit into the stream kernel's second
    and third 32,768-logit chunk (an odd chunk count, the pipeline's tail).
    Greedy rows (temperature 0) next to top-k 1 / 7 / 50 / 256 / 300 rows and
    rows without top-k (the exact whole-row path); rows of heavy ties, all
    equal (candidate lists overflow), all -inf, one finite logit, spike ties
    and a row ending in -inf. Every row against the oracle with its own
    parameters."""
    rng = np.random.default_rng(rows + vocab)
    x = np.full((rows, stride), np.float32(9.0))          # padding past vocab never read
    x[:, :vocab] = rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(1.5)
    x[1, :vocab] = np.round(x[1, :vocab])
    x[2, :vocab] = 0.25
    x[3, :vocab] = -np.inf
    x[4, :vocab] = -np.inf
    x[4, vocab - 3] = 2.0
    x[5, rng.choice(vocab, 6, replace=False)] = np.float32(7.0)
    x[6, vocab // 2:vocab] = -np.inf
    temp = rng.choice(np.float32([0.0, 0.7, 1.0, 1.3]), rows).astype(np.float32)
    temp[1:7] = np.float32(0.9)
    topk = rng.choice(np.uint32([0, 1, 7, 50, 50, 256, 300]), rows).astype(np.uint32)
    topk[1:7] = np.uint32(50)
    topk[8] = 0
    temp[8] = np.float32(1.0)
    topp = rng.choice(np.float32([1.0, 0.95, 0.9, 0.3]), rows).astype(np.float32)
    seeds = rng.integers(0, 2**63, rows, dtype=np.uint64)
    steps = rng.integers(0, 2**40, rows, dtype=np.uint64)
    bufs = [rl.DeviceBuffer.from_array(a) for a in (x, temp, topk, topp, seeds, steps)]
    tok, lp = rl.DeviceBuffer(rows * 4), rl.DeviceBuffer(rows * 4)
    args = rl.sample_args(bufs[0], rows, vocab, stride, tok, lp)
    args.temperature, args.top_k, args.top_p = bufs[1].ptr, bufs[2].ptr, bufs[3].ptr
    args.seed, args.steps = bufs[4].ptr, bufs[5].ptr
    ws = rl.sample_workspace(args)
    print(f"[sample] stream kernel, mixed rows, {rows} x {vocab}", flush=True)
    rl.sample(args)
    rl.sync()
    gt, gl = tok.download(np.uint32, rows), lp.download(np.float32, rows)
    import ctypes as C
    lpv = C.c_double()
    for r in range(rows):
        want = olib.orc_sample_row(x[r].ctypes.data, vocab, int(not temp[r] > 0), float(temp[r]), int(topk[r]),
                                   float(topp[r]), int(seeds[r]), int(steps[r]), r, C.byref(lpv))
        assert gt[r] == want, (r, temp[r], topk[r], topp[r], gt[r], want)
        assert gl[r] == pytest.approx(lpv.value, abs=1e-4, nan_ok=True), (r, gl[r], lpv.value)
    for b in bufs + [tok, lp, ws]:
        b.close()


def test_greedy_long_rows_repeated_calls(rl, gpu, orc, olib):
    """Greedy batches of rows above 32,768 logits take the split kernel (each
    slice's argmax into the workspace) and the merge kernel (the row's argmax
    over its slices): calls of different shapes back to back (more and fewer
    rows and slices than the call before) must each match the oracle, ties
    to the lowest index and all -inf rows included."""
    rng = np.random.default_rng(515)
    for it, (rows, vocab, stride) in enumerate([(8, 128256, 128256), (3, 50001, 50004), (40, 40000, 40000),
                                                (8, 128256, 128256), (1, 524288, 524288), (40, 40000, 40000)]):
        x = np.full((rows, stride), np.float32(50.0))          # padding past vocab never read
        x[:, :vocab] = rng.standard_normal((rows, vocab), dtype=np.float32)
        x[0, rng.choice(vocab, 4, replace=False)] = np.float32(6.0)   # a 4-way tie: lowest index
        if rows > 2:
            x[2, :vocab] = -np.inf
        print(f"[sample] greedy call {it}: {rows} x {vocab}", flush=True)
        tok = _check(rl, orc, olib, x, vocab=vocab, greedy=True)
        assert tok[0] == np.flatnonzero(x[0, :vocab] == np.float32(6.0)).min()
