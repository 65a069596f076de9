"""The lightning indexer (DeepSeek-V3.2's producer of the sparse indices the
decode consumes; no counterpart in the reference, whose tests draw indices at
random, tests/test_dsa.cu:73-85).

CPU: the oracle's scores against a direct float64 evaluation of the
published formula, and its top-k against numpy's lexicographic sort (score
descending, position ascending).  GPU (through the C ABI): on inputs whose
scores are exact in fp32 (small-integer e4m3 codes, power-of-two scales) the
scores and the selected positions are bit-identical to the oracle, ties
included; on random data the scores agree to 1e-4 of max |score| (fp32
MFMA and head sums against float64; the measured gap is 1.6e-5) and the
selected sets agree except where the oracle's score lies within that
tolerance of the threshold; ragged and short sequences; the selected
positions drive the paged decode end to end."""
import numpy as np
import pytest

ONE, TWO, MONE, MTWO = 0x38, 0x40, 0xB8, 0xC0  # e4m3 codes of 1, 2, -1, -2


def exact_inputs(Q, Hi, ctx, page, seed):
    rng = np.random.default_rng(seed)
    codes = np.array([0, ONE, TWO, MONE, MTWO], np.uint8)
    qc = codes[rng.integers(0, 5, (Q, Hi, 128))]
    kc = codes[rng.integers(0, 5, (Q * ctx, 128))]
    qs = np.exp2(rng.integers(-3, 2, (Q, Hi))).astype(np.float32)
    ks = np.exp2(rng.integers(-3, 2, Q * ctx)).astype(np.float32)
    hw = (rng.integers(-2, 3, (Q, Hi)) * 0.25).astype(np.float32)
    pps = ctx // page
    pt = rng.permutation(Q * pps).astype(np.int32).reshape(Q, pps)
    return qc, qs, hw, kc, ks, pt


def direct_scores(qc, qs, hw, kc, ks, pt, seq_len, page, max_seq, orc):
    """The formula evaluated with numpy in float64 (a second restatement)."""
    qf = orc.e4m3_to_f32(qc).astype(np.float64)
    kf = orc.e4m3_to_f32(kc).astype(np.float64)
    Q = qc.shape[0]
    out = np.full((Q, max_seq), -np.inf)
    for q in range(Q):
        s = np.arange(seq_len[q])
        rows = pt[q][s // page] * page + s % page
        dots = kf[rows] @ qf[q].T                                  # [S, Hi]
        w = hw[q].astype(np.float64) * qs[q].astype(np.float64)
        out[q, :seq_len[q]] = (np.maximum(dots, 0.0) @ w) * ks[rows]
    return out.astype(np.float32)


def test_oracle_scores_match_direct_formula(orc):
    Q, Hi, ctx, page = 3, 16, 256, 16
    rng = np.random.default_rng(1)
    qc = rng.integers(0, 256, (Q, Hi, 128)).astype(np.uint8)
    qc[(qc & 0x7F) == 0x7F] = 0                                    # no NaN codes
    kc = rng.integers(0, 256, (Q * ctx, 128)).astype(np.uint8)
    kc[(kc & 0x7F) == 0x7F] = 0
    qs = rng.uniform(0.01, 1, (Q, Hi)).astype(np.float32)
    ks = rng.uniform(0.01, 1, Q * ctx).astype(np.float32)
    hw = rng.standard_normal((Q, Hi)).astype(np.float32)
    pt = rng.permutation(Q * ctx // page).astype(np.int32).reshape(Q, -1)
    sl = np.array([256, 200, 17], np.int32)
    got = orc.dsa_indexer_scores(qc, qs, hw, kc, ks, pt, sl, page, ctx)
    ref = direct_scores(qc, qs, hw, kc, ks, pt, sl, page, ctx, orc)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=0)
    assert np.isneginf(got[2, 17:]).all()


def test_oracle_topk_tie_rule(orc):
    rng = np.random.default_rng(2)
    sc = rng.integers(-3, 4, (6, 300)).astype(np.float32)
    sc[0] = 0.0
    sc[0, ::7] = -0.0                                              # -0 ties +0
    sl = np.array([300, 300, 40, 5, 299, 1], np.int32)
    out = orc.dsa_indexer_topk(sc, sl, 32)
    for q in range(6):
        n = int(sl[q])
        order = np.lexsort((np.arange(n), -sc[q, :n].astype(np.float64)))
        ref = np.sort(order[:32])
        ref = np.concatenate([ref, -np.ones(32 - len(ref), np.int64)])
        np.testing.assert_array_equal(out[q], ref)


@pytest.mark.gpu
@pytest.mark.parametrize("Q,Hi,ctx,page,topk", [(3, 64, 4096, 64, 512), (2, 16, 1024, 16, 100),
                                                (2, 128, 2048, 64, 2048), (4, 32, 640, 32, 64),
                                                (2, 32, 8192, 64, 2048), (2, 16, 16384, 64, 1000),
                                                (2, 16, 960, 48, 100)])
def test_gpu_indexer_bit_exact_on_exact_scores(amd, orc, Q, Hi, ctx, page, topk):
    import torch
    print(f"indexer exact Q={Q} Hi={Hi} ctx={ctx} topk={topk}", flush=True)
    qc, qs, hw, kc, ks, pt = exact_inputs(Q, Hi, ctx, page, ctx + Hi)
    sl = np.array([ctx - 37 * q for q in range(Q)], np.int32)
    sl[-1] = min(sl[-1], topk - 3)                                 # one sequence shorter than topk
    ref_sc = orc.dsa_indexer_scores(qc, qs, hw, kc, ks, pt, sl, page, ctx)
    ref_ix = orc.dsa_indexer_topk(ref_sc, sl, topk)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(d(qc), d(qs), d(hw), d(kc), d(ks), d(pt), d(sl), page, ctx, topk,
                             scores, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(scores.cpu().numpy(), ref_sc)
    np.testing.assert_array_equal(out.cpu().numpy(), ref_ix)


@pytest.mark.gpu
@pytest.mark.parametrize("Q,Hi,ctx,page,topk", [(2, 16, 100000, 64, 2048), (1, 16, 131072, 128, 4096),
                                                (64, 16, 4096, 64, 512)])
def test_gpu_indexer_long_rows_and_many_queries(amd, orc, Q, Hi, ctx, page, topk):
    """Rows beyond one selection workgroup's 32768 keys (100000 and 131072
    positions: 9 and 8 parts, each part's top-k then the top-k of the
    candidates) and 64 queries (4 parts each), bit-exact against the oracle
    on tie-rich exact scores."""
    import torch
    print(f"indexer parts Q={Q} Hi={Hi} ctx={ctx} topk={topk}", flush=True)
    qc, qs, hw, kc, ks, pt = exact_inputs(Q, Hi, ctx, page, ctx + Q)
    sl = np.array([ctx - 1001 * q for q in range(Q)], np.int32)
    ref_sc = orc.dsa_indexer_scores(qc, qs, hw, kc, ks, pt, sl, page, ctx)
    ref_ix = orc.dsa_indexer_topk(ref_sc, sl, topk)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(d(qc), d(qs), d(hw), d(kc), d(ks), d(pt), d(sl), page, ctx, topk,
                             scores, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(scores.cpu().numpy(), ref_sc)
    np.testing.assert_array_equal(out.cpu().numpy(), ref_ix)


@pytest.mark.gpu
def test_gpu_indexer_rejects_unsplittable_long_row(amd):
    """A row above 32768 positions whose parts' candidates would not fit one
    workgroup (2 parts x topk 20000 > 32768) is refused, nothing launched."""
    import torch
    Q, Hi, ctx, page, topk = 1, 16, 40000, 64, 20000
    qc, qs, hw, kc, ks, pt = exact_inputs(Q, Hi, ctx, page, 5)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="max_seq"):
        amd.dsa_indexer_topk_fp8(d(qc), d(qs), d(hw), d(kc), d(ks), d(pt), d(np.array([ctx], np.int32)),
                                 page, ctx, topk, scores, out)


@pytest.mark.gpu
def test_gpu_indexer_empty_and_overlong_sequences(amd, orc):
    """seq_len 0 (every score -inf, every index -1), seq_len past max_seq
    (clamped to max_seq) and seq_len 1, bit-exact against the oracle."""
    import torch
    Q, Hi, ctx, page, topk = 3, 16, 512, 64, 100
    print(f"indexer edge lengths Q={Q} ctx={ctx} topk={topk}", flush=True)
    qc, qs, hw, kc, ks, pt = exact_inputs(Q, Hi, ctx, page, 7)
    sl = np.array([0, ctx + 188, 1], np.int32)
    ref_sc = orc.dsa_indexer_scores(qc, qs, hw, kc, ks, pt, sl, page, ctx)
    ref_ix = orc.dsa_indexer_topk(ref_sc, sl, topk)
    assert (ref_ix[0] == -1).all() and ref_ix[2, 0] == 0 and (ref_ix[2, 1:] == -1).all()
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(d(qc), d(qs), d(hw), d(kc), d(ks), d(pt), d(sl), page, ctx, topk,
                             scores, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(scores.cpu().numpy(), ref_sc)
    np.testing.assert_array_equal(out.cpu().numpy(), ref_ix)


@pytest.mark.gpu
def test_gpu_indexer_random_baseline_shape(amd, orc):
    """BASELINE decode shape on 4 queries: 64 index heads, 32768 positions,
    top-2048, random fp8 data."""
    import torch
    import synth
    Q, Hi, ctx, page, topk = 4, 64, 32768, 64, 2048
    print("indexer random baseline shape", flush=True)
    qc, qs, hw, kc, ks, pt = synth.dsa_indexer(Q, Hi, ctx, page, seed=21)
    sl = torch.tensor([ctx, ctx - 1, 20000, 3001], dtype=torch.int32, device="cuda")
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, pt, sl, page, ctx, topk, scores, out)
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy()
    ref_sc = orc.dsa_indexer_scores(h(qc), h(qs), h(hw), h(kc), h(ks), h(pt), h(sl), page, ctx)
    got_sc = h(scores)
    fin = np.isfinite(ref_sc)
    assert (np.isfinite(got_sc) == fin).all()
    tol = 1e-4 * np.abs(ref_sc[fin]).max()
    assert np.abs(got_sc[fin] - ref_sc[fin]).max() < tol
    ref_ix = orc.dsa_indexer_topk(ref_sc, h(sl), topk)
    got_ix = h(out)
    for q in range(Q):
        assert (np.diff(got_ix[q]) > 0).all()                      # ascending, distinct
        a, b = set(got_ix[q].tolist()), set(ref_ix[q].tolist())
        thr = np.sort(ref_sc[q][:h(sl)[q]])[::-1][topk - 1]
        near = {int(s) for s in np.flatnonzero(np.abs(ref_sc[q] - thr) <= 2 * tol)}
        assert (a ^ b) <= near, (q, len(a ^ b), len(near))
    # the selection is consistent with the GPU's own scores exactly
    gpu_ix = orc.dsa_indexer_topk(got_sc, h(sl), topk)
    np.testing.assert_array_equal(got_ix, gpu_ix)


@pytest.mark.gpu
def test_gpu_indexer_feeds_paged_decode(amd, orc):
    """Indexer -> paged MLA decode on a shared page table, against the
    oracle's decode on the oracle's selection."""
    import torch
    import synth
    Q, Hi, H, ctx, page, topk = 2, 64, 128, 4096, 64, 512
    print("indexer -> decode", flush=True)
    qn, qp, cache, pt, _, pps = synth.dsa_paged(Q, H, 512, 64, topk, page, ctx, seed=31)
    qc, qs, hw, kc, ks, _ = synth.dsa_indexer(Q, Hi, ctx, page, seed=32, page_table=pt)
    sl = torch.full((Q,), ctx, dtype=torch.int32, device="cuda")
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    idx = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, pt, sl, page, ctx, topk, scores, idx)
    out = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    cfg = amd.dsa_config(Q, H, 512, 64, topk, page, cache.shape[0])
    amd.dsa_decode_bf16_paged(qn, qp, cache, pt, idx, out, cfg, pps)
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy()
    gi = h(idx)
    ref_ix = orc.dsa_indexer_topk(h(scores), h(sl), topk)
    np.testing.assert_array_equal(gi, ref_ix)
    ref = orc.dsa_decode_bf16_paged(h(qn).view(np.uint16), h(qp).view(np.uint16),
                                    h(cache).view(np.uint16), h(pt), gi, 512, page)
    got = orc.bf16_to_f32(h(out).view(np.uint16))
    assert np.abs(got - ref).max() < 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("H", [128, 64])
def test_gpu_indexer_short_sequences_feed_paged_decode(amd, orc, H):
    """Sequences shorter than the selection (seq_len < top-k): the indexer
    lists all their positions, then -1; the decode takes the -1 padding as
    selecting nothing, so its output equals attention over the valid
    positions only.  H=128 runs the token-split decode, H=64 the one-block-
    per-32-heads decode."""
    import torch
    import synth
    Q, Hi, ctx, page, topk = 4, 64, 2048, 64, 512
    print(f"indexer (short sequences) -> decode H={H}", flush=True)
    qn, qp, cache, pt, _, pps = synth.dsa_paged(Q, H, 512, 64, topk, page, ctx, seed=33 + H)
    qc, qs, hw, kc, ks, _ = synth.dsa_indexer(Q, Hi, ctx, page, seed=34, page_table=pt)
    seq = [100, 511, 1, ctx]
    sl = torch.tensor(seq, dtype=torch.int32, device="cuda")
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    idx = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, pt, sl, page, ctx, topk, scores, idx)
    out = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    cfg = amd.dsa_config(Q, H, 512, 64, topk, page, cache.shape[0])
    amd.dsa_decode_bf16_paged(qn, qp, cache, pt, idx, out, cfg, pps)
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy()
    gi = h(idx)
    for q, n in enumerate(seq):
        m = min(n, topk)
        assert (gi[q, :m] >= 0).all() and (gi[q, m:] == -1).all()
        if n <= topk:
            np.testing.assert_array_equal(gi[q, :m], np.arange(m))
    np.testing.assert_array_equal(gi, orc.dsa_indexer_topk(h(scores), h(sl), topk))
    ref = orc.dsa_decode_bf16_paged(h(qn).view(np.uint16), h(qp).view(np.uint16),
                                    h(cache).view(np.uint16), h(pt), gi, 512, page)
    got = orc.bf16_to_f32(h(out).view(np.uint16))
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max()
    print(f"short sequences H={H}: max_err={err:.3e}")
    assert err < 1e-2


@pytest.mark.gpu
def test_gpu_indexer_seq_len_past_page_table_capacity(amd, orc):
    """seq_len larger than the page-table row's capacity (pages_per_seq *
    page < max_seq): positions past the capacity are neither scored nor
    selected, so a row with fewer scored positions than top-k is padded with
    -1 instead of listing -inf positions."""
    import torch
    import synth
    Q, Hi, ctx, page, topk = 2, 32, 1024, 64, 512
    print("indexer seq_len past capacity", flush=True)
    qc, qs, hw, kc, ks, pt = synth.dsa_indexer(Q, Hi, ctx, page, seed=35)
    pt_small = pt[:, :4].contiguous()            # capacity 256 positions
    max_seq = ctx
    sl = torch.tensor([ctx, 300], dtype=torch.int32, device="cuda")
    scores = torch.empty((Q, max_seq), dtype=torch.float32, device="cuda")
    idx = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    amd.dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, pt_small, sl, page, max_seq, topk, scores, idx)
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy()
    gi = h(idx)
    for q in range(Q):
        np.testing.assert_array_equal(gi[q, :256], np.arange(256))
        assert (gi[q, 256:] == -1).all()
    assert np.isneginf(h(scores)[:, 256:]).all()
    ref_sc = orc.dsa_indexer_scores(h(qc), h(qs), h(hw), h(kc), h(ks), h(pt_small), h(sl), page, max_seq)
    assert np.isneginf(ref_sc[:, 256:]).all()
    np.testing.assert_array_equal(gi, orc.dsa_indexer_topk(ref_sc, h(sl), topk, cap=256))
