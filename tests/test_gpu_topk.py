"""GPU parity of the sampling pre-work (softcap -> repetition penalty -> top-k) and the fused LM head,
through the C ABI, against the numpy oracle.

The first case is the reference's own validation (``kernels.ts:2828-2870``): vocab 152064, K 64,
penalty 1.15, cap 30, logits U(-8, 8), 40 recent ids deduplicated; its acceptance rule (values within
1e-4 (1 + |v|) of the reference ranking, ids checked through their reference logit) is applied, and on
top of it the ids must equal the oracle's exact ranking (the values are well separated).
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_EINVAL
from helpers import Gpu, PLANES

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def run_topk(gpu, logits, recent, penalty, softcap, k):
    n = logits.size
    lb = gpu.up(np.asarray(logits, np.float32))
    rb = gpu.up(np.asarray(recent, np.int32)) if len(recent) else None
    ob = gpu.up(np.zeros(2 * k, np.int32))
    gpu.ctx.logits_topk(lb, n, rb, len(recent), penalty, softcap, k, ob, ob.offset(4 * k))
    ids = gpu.ctx.download(ob, np.int32, k)
    vals = gpu.ctx.download(ob, np.float32, k, src_offset=4 * k)
    after = gpu.ctx.download(lb, np.float32, n)
    return ids, vals, after


def oracle_passes(logits, recent, penalty, softcap, k):
    ref = np.asarray(logits, np.float32)
    if softcap > 0:
        ref = O.softcap_logits(ref, softcap)
    if penalty and penalty != 1 and len(recent):
        ref = O.penalize_logits(ref, recent, penalty)
    ids, vals = O.top_k(ref, k)
    return ref, ids, vals


def reference_rule(ids, vals, ref, order):
    """kernels.ts:2862-2866."""
    for r in range(len(order)):
        okv = abs(vals[r] - ref[order[r]]) <= 1e-4 * (1 + abs(ref[order[r]]))
        oki = abs(ref[ids[r]] - vals[r]) <= 1e-4 * (1 + abs(vals[r]))
        assert okv and oki, f"rank {r}"


def test_reference_validation_case(gpu):
    vocab, K, penalty, cap = 152064, 64, 1.15, 30.0
    logits = (synth.uniform(2024, vocab) * 2 - 1) * 8
    recent = list(dict.fromkeys((synth.uniform(2025, 40) * vocab).astype(np.int64).tolist()))
    ids, vals, after = run_topk(gpu, logits, recent, penalty, cap, K)
    ref, rids, rvals = oracle_passes(logits, recent, penalty, cap, K)
    reference_rule(ids, vals, ref, rids)
    assert np.array_equal(ids, rids.astype(np.int32))
    np.testing.assert_allclose(vals, rvals, rtol=2e-6, atol=2e-6)
    # the passes left the softcapped, penalised logits in place, as the reference's do
    np.testing.assert_allclose(after, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("k,cap,penalty", [(1, 0.0, 1.0), (64, 0.0, 1.0), (40, 30.0, 1.0), (17, 0.0, 1.3),
                                           (64, 0.0, 0.0), (8, 50.0, 0.7)])
def test_topk_options(gpu, k, cap, penalty):
    n = 151936
    logits = synth.normal(300 + k, n) * 4
    recent = list(dict.fromkeys((synth.uniform(301 + k, 64) * n).astype(np.int64).tolist()))
    # put some recent ids at the top so the penalty changes the ranking
    top = np.argsort(-logits)[:5]
    recent = list(dict.fromkeys(recent + top.tolist()))
    ids, vals, _ = run_topk(gpu, logits, recent, penalty, cap, k)
    ref, rids, rvals = oracle_passes(logits, recent, penalty, cap, k)
    assert np.array_equal(ids, rids.astype(np.int32))
    np.testing.assert_allclose(vals, rvals, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("n,k", [(1, 1), (5, 5), (64, 64), (100, 64), (1025, 33), (4097, 64), (70000, 3)])
def test_topk_sizes(gpu, n, k):
    logits = synth.normal(400 + n, n)
    ids, vals, _ = run_topk(gpu, logits, [], 1.0, 0.0, k)
    _, rids, rvals = oracle_passes(logits, [], 1.0, 0.0, k)
    assert np.array_equal(ids, rids.astype(np.int32))
    assert np.array_equal(vals, rvals)


def test_topk_ties_nan_inf(gpu):
    n = 20000
    v = np.round(synth.normal(501, n) * 2).astype(np.float32)     # heavy ties
    v[::997] = np.nan
    v[123] = np.inf
    v[4567] = -np.inf
    ids, vals, _ = run_topk(gpu, v, [], 1.0, 0.0, 64)
    _, rids, rvals = oracle_passes(v, [], 1.0, 0.0, 64)
    assert np.array_equal(ids, rids.astype(np.int32))
    assert np.array_equal(vals, rvals)


def test_topk_all_equal_overflow_path(gpu):
    # every value equal: the candidate list overflows and the exact scan path answers
    n = 50000
    ids, vals, _ = run_topk(gpu, np.full(n, 1.5, np.float32), [], 1.0, 0.0, 64)
    assert np.array_equal(ids, np.arange(64, dtype=np.int32))
    assert np.all(vals == 1.5)


def test_topk_out_of_range_recent_ids_skipped(gpu):
    n = 3000
    logits = synth.normal(601, n)
    recent = [-5, n, n + 100, 7]
    ids, vals, after = run_topk(gpu, logits, recent, 2.0, 0.0, 10)
    ref, rids, _ = oracle_passes(logits, recent, 2.0, 0.0, 10)
    assert np.array_equal(ids, rids.astype(np.int32))
    np.testing.assert_allclose(after, ref, rtol=1e-7)


def test_topk_rejects_bad_k(gpu):
    lb = gpu.up(np.zeros(100, np.float32))
    ob = gpu.up(np.zeros(200, np.int32))
    for k in (0, 65, 101):
        with pytest.raises(BrikError) as e:
            gpu.ctx.logits_topk(lb, 100, None, 0, 1.0, 0.0, k, ob, ob.offset(400))
        assert e.value.code == BRIK_EINVAL


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_lm_head_topk(gpu, fmt):
    K, vocab, k = 512, 6000, 64
    t = synth.tensor(fmt, 700, vocab, K)
    x = synth.normal(701, K)
    planes = gpu.planes(fmt, t)
    recent = [3, 17, 5999, 1234]
    xb = gpu.up(x)
    rb = gpu.up(np.asarray(recent, np.int32))
    ob = gpu.up(np.zeros(2 * k, np.int32))
    gpu.ctx.lm_head_topk(fmt, xb, planes, K, vocab, rb, len(recent), 1.2, 25.0, k, ob, ob.offset(4 * k))
    ids = gpu.ctx.download(ob, np.int32, k)
    vals = gpu.ctx.download(ob, np.float32, k, src_offset=4 * k)
    logits = getattr(O, f"matmul_t_{fmt}")(x, *[t[p] for p in PLANES[fmt]], 1, K, vocab).ravel()
    ref, rids, rvals = oracle_passes(logits, recent, 1.2, 25.0, k)
    # the GPU logits agree with the oracle's to ~1e-6, so near-ties may swap: the reference's own rule
    reference_rule(ids, vals, ref, rids)
    assert len(set(ids.tolist())) == k


@pytest.mark.parametrize("fmt", ["q4", "q3"])
@pytest.mark.parametrize("vocab,cap,penalty", [(151936, 30.0, 1.15), (24583, 0.0, 1.3), (32768, 25.0, 1.0)])
def test_lm_head_topk_fused_epilogue(gpu, fmt, vocab, cap, penalty):
    """A q4 / q3 head of at least 24576 rows runs the softcap, the penalty and the 16-logit maxima in
    its GEMV epilogue (brik_gemvh_*): its ids and values must be bit-identical to the same head's
    logits (brik_matmul_t_*, the same GEMV variant) passed through brik_logits_topk."""
    K, k = 256, 64
    t = synth.tensor(fmt, 710, vocab, K)
    x = synth.normal(711, K)
    planes = gpu.planes(fmt, t)
    recent = sorted({0, 15, 16, 31, 32, 777, vocab // 2, vocab - 17, vocab - 16, vocab - 1}
                    | set((synth.uniform(712, 40) * vocab).astype(np.int64).tolist()))
    xb, rb = gpu.up(x), gpu.up(np.asarray(recent, np.int32))
    ob = gpu.up(np.zeros(2 * k, np.int32))
    print(f"fused head: fmt={fmt} vocab={vocab} cap={cap} penalty={penalty}", flush=True)
    gpu.ctx.lm_head_topk(fmt, xb, planes, K, vocab, rb, len(recent), penalty, cap, k, ob, ob.offset(4 * k))
    ids = gpu.ctx.download(ob, np.int32, k)
    vals = gpu.ctx.download(ob, np.float32, k, src_offset=4 * k)
    yb = gpu.up(np.zeros(vocab, np.float32))
    getattr(gpu.ctx, f"matmul_t_{fmt}")(xb, *planes, yb, 1, K, vocab)
    gpu.ctx.sync()
    plain = gpu.ctx.download(yb, np.float32, vocab)
    pids, pvals, _ = run_topk(gpu, plain, recent, penalty, cap, k)
    assert np.array_equal(ids, pids)
    assert np.array_equal(vals.view(np.uint32), pvals.view(np.uint32))
    ref, rids, _ = oracle_passes(plain, recent, penalty, cap, k)
    reference_rule(ids, vals, ref, rids)


@pytest.mark.parametrize("fmt", ["q4", "q3"])
def test_lm_head_topk_fused_non_finite_input(gpu, fmt):
    """An Inf in x sends the fused head through its exact path; the epilogue then reads the rows back:
    the same ids and values as the unfused form."""
    K, vocab, k = 128, 24576, 8
    t = synth.tensor(fmt, 720, vocab, K)
    x = synth.normal(721, K)
    x[3] = np.inf
    planes = gpu.planes(fmt, t)
    recent = [1, 2, 24575]
    xb, rb = gpu.up(x), gpu.up(np.asarray(recent, np.int32))
    ob = gpu.up(np.zeros(2 * k, np.int32))
    gpu.ctx.lm_head_topk(fmt, xb, planes, K, vocab, rb, len(recent), 1.2, 20.0, k, ob, ob.offset(4 * k))
    ids = gpu.ctx.download(ob, np.int32, k)
    vals = gpu.ctx.download(ob, np.float32, k, src_offset=4 * k)
    yb = gpu.up(np.zeros(vocab, np.float32))
    getattr(gpu.ctx, f"matmul_t_{fmt}")(xb, *planes, yb, 1, K, vocab)
    gpu.ctx.sync()
    plain = gpu.ctx.download(yb, np.float32, vocab)
    pids, pvals, _ = run_topk(gpu, plain, recent, 1.2, 20.0, k)
    assert np.array_equal(ids, pids)
    assert np.array_equal(vals.view(np.uint32), pvals.view(np.uint32))
