"""Pins for the CPU oracle (oracle/oracle.c), run on the CPU.

Each check uses an independent route to the answer -- a closed form, a
library routine (glibc rand via ctypes, torch's bf16 cast, numpy float64
algebra, a stable argsort), brute force on tiny inputs, or a known-answer
case -- so that a dropped term, a wrong index or a swapped operand in the
oracle fails here.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from cases import DSA_CASES, MOE_CASES


# ------------------------------------------------------------------ generators
def test_random_fill_matches_glibc_rand(orc):
    """utils/cuda_utils.cuh:58 evaluated by hand on glibc's rand()."""
    libc = ctypes.CDLL("libc.so.6")
    libc.srand(42)
    raw = [libc.rand() for _ in range(64)]
    RAND_MAX = 2147483647
    expect = np.array([np.float32(-0.5) + np.float32(np.float32(r) / np.float32(RAND_MAX)) * np.float32(1.0)
                       for r in raw], np.float32)
    orc.srand(42)
    got = orc.random_fill(64, -0.5, 0.5)
    np.testing.assert_array_equal(got, expect)


def test_sparse_indices_are_unique_sorted_and_in_range(orc):
    orc.srand(7)
    idx = orc.gen_sparse_indices(8, 100, 1000, True)
    for row in idx:
        assert len(set(row.tolist())) == 100
        assert (np.diff(row) > 0).all()
        assert row.min() >= 0 and row.max() < 1000
    orc.srand(7)
    raw = orc.gen_sparse_indices(8, 100, 1000, False)
    np.testing.assert_array_equal(np.sort(raw, axis=1), idx)


# ------------------------------------------------------------------ formats
def _e4m3_closed_form(c):
    s = -1.0 if c & 0x80 else 1.0
    e = (c >> 3) & 15
    m = c & 7
    if e == 15 and m == 7:
        return math.nan
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_e4m3_decode_exhaustive(orc):
    codes = np.arange(256, dtype=np.uint8)
    got = orc.e4m3_to_f32(codes)
    for c in range(256):
        ref = _e4m3_closed_form(c)
        if math.isnan(ref):
            assert math.isnan(got[c])
        else:
            assert got[c] == np.float32(ref), c
    assert np.nanmax(got) == 448.0 and np.nanmin(got) == -448.0


def test_e4m3_encode_roundtrip_midpoints_and_saturation(orc):
    vals = [_e4m3_closed_form(c) for c in range(128) if not math.isnan(_e4m3_closed_form(c))]
    vals = sorted(set(vals))
    for c in range(256):
        v = _e4m3_closed_form(c)
        if math.isnan(v):
            continue
        assert orc.f32_to_e4m3_scalar(v) == c, (c, v)
    # midpoints round to the even mantissa; just above/below go to nearest
    for lo, hi in zip(vals[:-1], vals[1:]):
        mid = (lo + hi) / 2.0
        clo, chi = orc.f32_to_e4m3_scalar(lo), orc.f32_to_e4m3_scalar(hi)
        even = clo if (clo & 1) == 0 else chi
        assert orc.f32_to_e4m3_scalar(mid) == even, (lo, hi)
        assert orc.f32_to_e4m3_scalar(np.nextafter(np.float32(mid), np.float32(0))) == clo
        assert orc.f32_to_e4m3_scalar(np.nextafter(np.float32(mid), np.float32(1e9))) == chi
    for big in (448.0, 449.0, 464.0, 1e6, float("inf")):
        assert orc.f32_to_e4m3_scalar(big) == 0x7E
        assert orc.f32_to_e4m3_scalar(-big) == 0xFE
    assert orc.f32_to_e4m3_scalar(float("nan")) == 0x7F


def test_bf16_matches_torch_rne(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, 3.4e38, -3.4e38], np.float32)])
    # exact halfway cases: low 16 bits 0x8000 with even and odd bf16 lsb
    half = (np.arange(64, dtype=np.uint32) << 16 | 0x3F808000).view(np.float32)
    x = np.concatenate([x, half])
    got = orc.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(orc.bf16_to_f32(got), torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_block_quant_rows_and_weights(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    x[1, :128] = 0.0
    q, s = orc.quant_rows_1x128(x)
    assert s[1, 0] == 1.0 and (q[1, :128] == 0).all()
    for r in range(3):
        for b in range(2):
            blk = x[r, 128 * b:128 * (b + 1)]
            amax = np.abs(blk).max()
            if amax > 0:
                assert s[r, b] == np.float32(amax) / np.float32(448.0)
            deq = orc.e4m3_to_f32(q[r, 128 * b:128 * (b + 1)]) * s[r, b]
            # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals
            assert np.all(np.abs(deq - blk) <= np.abs(blk) * 2.0 ** -4 + s[r, b] * 2.0 ** -9 + 1e-30)
            assert np.abs(deq).max() == pytest.approx(amax, rel=1e-6) or amax == 0
    w = rng.standard_normal((256, 384)).astype(np.float32)
    u = rng.uniform(0.5, 2.0, (2, 3)).astype(np.float32)
    wq, ws = orc.quant_weight_128x128(w, u)
    for i in range(2):
        for j in range(3):
            blk = w[128 * i:128 * (i + 1), 128 * j:128 * (j + 1)]
            assert ws[i, j] == np.float32(u[i, j] * np.float32(np.abs(blk).max())) / np.float32(448.0)
            deq = orc.e4m3_to_f32(wq[128 * i:128 * (i + 1), 128 * j:128 * (j + 1)]) * ws[i, j]
            clip = np.clip(blk, -448 * ws[i, j], 448 * ws[i, j])
            assert np.all(np.abs(deq - clip) <= np.abs(clip) * 2.0 ** -4 + ws[i, j] * 2.0 ** -9 + 1e-30)
    np.testing.assert_array_equal(orc.dequant_weight_128x128(wq, ws),
                                  orc.e4m3_to_f32(wq) * np.kron(ws, np.ones((128, 128), np.float32)))


# ------------------------------------------------------------------ routing
def test_topk_known_answers(orc):
    # documented replace-min example: slot order is the insertion history
    idx, wt = orc.topk_row(np.array([0.1, 0.4, 0.3, 0.2], np.float32), 2)
    assert idx.tolist() == [2, 1]
    np.testing.assert_allclose(wt, np.array([0.3, 0.4]) / 0.7, rtol=1e-6)
    # all equal: first K experts, in order, weight 1/K
    idx, wt = orc.topk_row(np.full(8, 0.125, np.float32), 3)
    assert idx.tolist() == [0, 1, 2]
    np.testing.assert_allclose(wt, 1 / 3, rtol=1e-6)
    # equal minimum slots: the FIRST such slot is the victim
    idx, wt = orc.topk_row(np.array([0.3, 0.3, 0.5], np.float32), 2)
    assert idx.tolist() == [2, 1]
    # K = E: every expert, weights = the probabilities (sum 1)
    p = orc.softmax(np.array([1.0, -2.0, 0.5], np.float32))
    idx, wt = orc.topk_row(p, 3)
    assert sorted(idx.tolist()) == [0, 1, 2]
    np.testing.assert_allclose(wt[np.argsort(idx)], p / p.sum(), rtol=1e-6)
    # K > E leaves -1 slots and skips renormalisation (sum <= 0)
    idx, wt = orc.topk_row(np.array([0.6, 0.4], np.float32), 3)
    assert idx.tolist() == [0, 1, -1]


def test_topk_selects_the_k_largest_bruteforce(orc):
    rng = np.random.default_rng(2)
    for _ in range(200):
        E = int(rng.integers(1, 40))
        K = int(rng.integers(1, E + 1))
        p = rng.random(E).astype(np.float32)
        idx, wt = orc.topk_row(p, K)
        assert sorted(idx.tolist()) == sorted(np.argsort(-p, kind="stable")[:K].tolist())
        assert abs(float(wt.sum()) - 1.0) < 1e-5


def test_softmax_matches_float64(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(257).astype(np.float32) * 5
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    np.testing.assert_allclose(orc.softmax(x), ref, rtol=1e-5, atol=1e-9)


def test_route_zero_input_and_duplicate_rows(orc):
    T, E, K, D = 5, 8, 3, 64
    x = np.zeros((T, D), np.float32)
    wg = np.random.default_rng(4).standard_normal((E, D)).astype(np.float32)
    idx, wts = orc.moe_route(x, wg, K)
    assert (idx == np.arange(K)).all()
    np.testing.assert_allclose(wts, 1 / K, rtol=1e-6)
    # expert 5 duplicates expert 2: both have equal logits; at most one more
    # expert may be selected between them only by the slot rule
    wg[5] = wg[2]
    x = np.random.default_rng(5).standard_normal((T, D)).astype(np.float32)
    idx, wts, logits, probs = orc.moe_route(x, wg, K, want_probs=True)
    np.testing.assert_array_equal(logits[:, 5], logits[:, 2])
    ref = x.astype(np.float64) @ wg.astype(np.float64).T
    np.testing.assert_allclose(logits, ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(wts.sum(1), 1.0, rtol=1e-5)


def test_route_non_finite_logits_select_nothing(orc):
    """tests/test_moe.cu:38-68 with a NaN or inf in a token's logits: softmax
    turns every probability of that token into NaN (max is inf, or the sum is
    NaN), `v > slot` is false for NaN, so no expert is inserted: indices stay
    -1 and weights -FLT_MAX (their sum is -inf, not > 0, so they are not
    renormalised).  The other tokens route normally."""
    T, E, K, D = 4, 8, 3, 64
    rng = np.random.default_rng(8)
    x = rng.standard_normal((T, D)).astype(np.float32)
    wg = rng.standard_normal((E, D)).astype(np.float32)
    idx0, wts0 = orc.moe_route(x, wg, K)
    x[1, 5] = np.nan
    x[2, 7] = np.inf
    idx, wts = orc.moe_route(x, wg, K)
    for t in (1, 2):
        assert (idx[t] == -1).all()
        assert (wts[t] == -np.finfo(np.float32).max).all()
    for t in (0, 3):
        np.testing.assert_array_equal(idx[t], idx0[t])
        np.testing.assert_array_equal(wts[t], wts0[t])


def test_route_bias_shifts_logits(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    wg = rng.standard_normal((8, 64)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    _, _, l0, _ = orc.moe_route(x, wg, 2, want_probs=True)
    _, _, l1, _ = orc.moe_route(x, wg, 2, bias=b, want_probs=True)
    np.testing.assert_allclose(l1, l0 + b, rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------ permutation
def test_permute_matches_stable_argsort(orc):
    rng = np.random.default_rng(7)
    for T, E, K in [(1, 4, 2), (37, 8, 2), (200, 16, 4), (64, 64, 8)]:
        idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
        counts, offsets, st, ss = orc.moe_permute(idx, E)
        flat = idx.reshape(-1)
        order = np.argsort(flat, kind="stable")
        np.testing.assert_array_equal(ss, order)
        np.testing.assert_array_equal(st, order // K)
        np.testing.assert_array_equal(counts, np.bincount(flat, minlength=E))
        np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))


def test_permute_skips_invalid_and_duplicate_slots(orc):
    idx = np.array([[1, 1], [0, -1], [2, 0]], np.int32)
    counts, offsets, st, ss = orc.moe_permute(idx, 3)
    assert counts.tolist() == [2, 1, 1]
    assert st.tolist() == [1, 2, 0, 2] and ss.tolist() == [2, 5, 0, 4]


# ------------------------------------------------------------------ expert FFN
def _ffn64(x, w1, w2):
    I = w1.shape[0] // 2
    h = x.astype(np.float64) @ w1.astype(np.float64).T
    g, u = h[:, :I], h[:, I:]
    a = g / (1.0 + np.exp(-g)) * u
    return a @ w2.astype(np.float64).T


def test_single_expert_is_dense_swiglu_ffn(orc):
    x, wg, w1, w2 = orc.reference_moe_inputs(8, 1, 1, 64, 128)
    idx, wts, y = orc.moe_forward_f32(x, wg, w1, w2, 1)
    assert (idx == 0).all() and (wts == 1.0).all()
    np.testing.assert_allclose(y, _ffn64(x, w1[0], w2[0]), rtol=1e-4, atol=1e-6)


def test_identical_experts_give_ffn_regardless_of_routing(orc):
    rng = np.random.default_rng(8)
    T, E, K, D, I = 16, 8, 3, 64, 96
    x = rng.standard_normal((T, D)).astype(np.float32)
    wg = rng.standard_normal((E, D)).astype(np.float32)
    w1 = np.repeat(rng.standard_normal((1, 2 * I, D)).astype(np.float32) / 8, E, 0)
    w2 = np.repeat(rng.standard_normal((1, D, I)).astype(np.float32) / 8, E, 0)
    _, _, y = orc.moe_forward_f32(x, wg, w1, w2, K)
    np.testing.assert_allclose(y, _ffn64(x, w1[0], w2[0]), rtol=1e-4, atol=1e-5)


def test_moe_forward_is_weighted_sum_of_expert_ffns(orc):
    x, wg, w1, w2 = orc.reference_moe_inputs(16, 8, 4, 128, 256)
    idx, wts, y = orc.moe_forward_f32(x, wg, w1, w2, 4)
    ref = np.zeros(y.shape, np.float64)
    for t in range(16):
        for k in range(4):
            ref[t] += wts[t, k] * _ffn64(x[t:t + 1], w1[idx[t, k]], w2[idx[t, k]])[0]
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-6)


def test_bf16_and_fp8_variants_against_float64(orc):
    rng = np.random.default_rng(9)
    T, E, K, D, I = 6, 4, 2, 256, 128
    x = orc.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    wgf = (rng.standard_normal((E, D)) / 16).astype(np.float32)
    w1 = orc.f32_to_bf16((rng.standard_normal((E, 2 * I, D)) / 16).astype(np.float32))
    w2 = orc.f32_to_bf16((rng.standard_normal((E, D, I)) / 11).astype(np.float32))
    idx, wts, y = orc.moe_forward_bf16(x, wgf, w1, w2, K)
    xf, w1f, w2f = orc.bf16_to_f32(x), orc.bf16_to_f32(w1), orc.bf16_to_f32(w2)
    ref = np.zeros((T, D))
    for t in range(T):
        for k in range(K):
            e = idx[t, k]
            I_ = I
            h = xf[t].astype(np.float64) @ w1f[e].astype(np.float64).T
            a = (h[:I_] / (1 + np.exp(-h[:I_])) * h[I_:]).astype(np.float32)
            a = orc.bf16_to_f32(orc.f32_to_bf16(a))  # the bf16 activation storage
            ref[t] += wts[t, k] * (a.astype(np.float64) @ w2f[e].astype(np.float64).T)
    np.testing.assert_allclose(y, ref, rtol=2e-3, atol=2e-4)

    # fp8: quantise the same weights 128x128 and check against float64 on
    # the dequantised values with the same 1x128 activation requantisation
    wgb = orc.f32_to_bf16(wgf)
    u1 = rng.uniform(0.5, 2, (E, 2 * I // 128, D // 128)).astype(np.float32)
    u2 = rng.uniform(0.5, 2, (E, D // 128, I // 128)).astype(np.float32)
    q1, s1, q2, s2 = [], [], [], []
    for e in range(E):
        a, b = orc.quant_weight_128x128(w1f[e], u1[e]); q1.append(a); s1.append(b)
        a, b = orc.quant_weight_128x128(w2f[e], u2[e]); q2.append(a); s2.append(b)
    q1, s1, q2, s2 = map(np.stack, (q1, s1, q2, s2))
    idx8, wts8, y8 = orc.moe_forward_fp8(x, wgb, q1, s1, q2, s2, K)
    xq, xs = orc.quant_rows_1x128(xf)
    xd = orc.e4m3_to_f32(xq) * np.repeat(xs, 128, axis=1)
    ref8 = np.zeros((T, D))
    for t in range(T):
        for k in range(K):
            e = idx8[t, k]
            W1 = orc.dequant_weight_128x128(q1[e], s1[e]).astype(np.float64)
            W2 = orc.dequant_weight_128x128(q2[e], s2[e]).astype(np.float64)
            h = xd[t].astype(np.float64) @ W1.T
            a = (h[:I] / (1 + np.exp(-h[:I])) * h[I:]).astype(np.float32)
            aq, as_ = orc.quant_rows_1x128(a[None, :])
            ad = orc.e4m3_to_f32(aq[0]) * np.repeat(as_[0], 128)
            ref8[t] += wts8[t, k] * (ad.astype(np.float64) @ W2.T)
    err = np.abs(y8 - ref8).max() / np.abs(ref8).max()
    assert err < 2e-2, err
    # routing of the fp8 layer uses the bf16 gate on the bf16 input
    idx_b, _ = orc.moe_route(xf, orc.bf16_to_f32(wgb), K)
    np.testing.assert_array_equal(idx8, idx_b)


def test_zero_input_gives_zero_output(orc):
    x, wg, w1, w2 = orc.reference_moe_inputs(4, 4, 2, 64, 128)
    idx, wts, y = orc.moe_forward_f32(np.zeros_like(x), wg, w1, w2, 2)
    assert (idx == [0, 1]).all() and (y == 0).all()


@pytest.mark.parametrize("name,shape,tol", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_reference_moe_cases_run(orc, name, shape, tol):
    T, E, K, D, I = shape
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    idx, wts, y = orc.moe_forward_f32(x, wg, w1, w2, K)
    assert np.isfinite(y).all()
    np.testing.assert_allclose(wts.sum(1), 1.0, rtol=1e-5)


# ------------------------------------------------------------------ DSA
def _dsa64(qn, qp, kc, kp, v, idx):
    Q, H, Dc = qn.shape
    Dp = qp.shape[2]
    out = np.zeros((Q, H, Dc))
    for q in range(Q):
        K = np.concatenate([kc[idx[q]], kp[idx[q]]], 1).astype(np.float64)
        qq = np.concatenate([qn[q], qp[q]], 1).astype(np.float64)
        s = qq @ K.T / math.sqrt(Dc + Dp)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[q] = p @ v[idx[q]].astype(np.float64)
    return out


def test_dsa_matches_float64_and_special_cases(orc):
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(3, 4, 64, 16, 32, 8, 128)
    out = orc.dsa_forward_f32(qn, qp, kc, kp, v, idx)
    np.testing.assert_allclose(out, _dsa64(qn, qp, kc, kp, v, idx), rtol=1e-4, atol=1e-6)
    # S=1: out = V[idx]
    out1 = orc.dsa_forward_f32(qn, qp, kc, kp, v, idx[:, :1].copy())
    np.testing.assert_array_equal(out1, np.repeat(v[idx[:, 0]][:, None, :], 4, 1))
    # q=0: uniform attention = mean of the selected V rows
    out0 = orc.dsa_forward_f32(np.zeros_like(qn), np.zeros_like(qp), kc, kp, v, idx)
    np.testing.assert_allclose(out0, np.repeat(v[idx].mean(1)[:, None, :], 4, 1), rtol=1e-5, atol=1e-7)
    # permutation invariance of the selected set
    perm = idx[:, ::-1].copy()
    np.testing.assert_allclose(orc.dsa_forward_f32(qn, qp, kc, kp, v, perm), out, rtol=1e-5, atol=1e-7)
    # S = N: dense attention
    full = np.tile(np.arange(128, dtype=np.int32), (3, 1))
    np.testing.assert_allclose(orc.dsa_forward_f32(qn, qp, kc, kp, v, full),
                               _dsa64(qn, qp, kc, kp, v, full), rtol=1e-4, atol=1e-6)


def test_dsa_paged_equals_flat(orc):
    rng = np.random.default_rng(10)
    Q, H, Dc, Dp, S, page, pps = 2, 4, 64, 16, 24, 8, 6
    n_pages = Q * pps
    cache = orc.f32_to_bf16(rng.standard_normal((n_pages * page, Dc + Dp)).astype(np.float32))
    pt = rng.permutation(n_pages).astype(np.int32).reshape(Q, pps)
    logical = np.stack([rng.permutation(pps * page)[:S] for _ in range(Q)]).astype(np.int32)
    qn = orc.f32_to_bf16(rng.standard_normal((Q, H, Dc)).astype(np.float32))
    qp = orc.f32_to_bf16(rng.standard_normal((Q, H, Dp)).astype(np.float32))
    phys = orc.dsa_translate(logical, pt, page)
    assert (phys == pt[np.arange(Q)[:, None], logical // page] * page + logical % page).all()
    out = orc.dsa_decode_bf16_paged(qn, qp, cache, pt, logical, Dc, page)
    cf = orc.bf16_to_f32(cache)
    ref = orc.dsa_forward_f32(orc.bf16_to_f32(qn), orc.bf16_to_f32(qp), cf[:, :Dc].copy(),
                              cf[:, Dc:].copy(), cf[:, :Dc].copy(), phys)
    np.testing.assert_array_equal(out, ref)


def test_dsa_paged_invalid_positions_select_nothing(orc):
    """Selected positions that select nothing (-1 padding, an index past the
    page-table row, a page id of -1 or past the cache) are left out: the
    decode equals the reference restatement (dsa_forward_f32) run on the
    flat rows of the valid positions only, and a query with none gives 0."""
    rng = np.random.default_rng(11)
    Q, H, Dc, Dp, S, page, pps = 3, 4, 64, 16, 24, 8, 6
    n_pages = Q * pps
    cache = orc.f32_to_bf16(rng.standard_normal((n_pages * page, Dc + Dp)).astype(np.float32))
    pt = rng.permutation(n_pages).astype(np.int32).reshape(Q, pps)
    pt[0, 2] = -1                 # an unmapped page
    pt[0, 4] = n_pages + 5        # a page past the cache
    logical = np.stack([rng.permutation(pps * page)[:S] for _ in range(Q)]).astype(np.int32)
    logical[0, -5:] = -1          # padding
    logical[0, 3] = pps * page    # past the row's capacity
    logical[0, 4] = pps * page + 100
    logical[2, :] = -1            # nothing valid
    qn = orc.f32_to_bf16(rng.standard_normal((Q, H, Dc)).astype(np.float32))
    qp = orc.f32_to_bf16(rng.standard_normal((Q, H, Dp)).astype(np.float32))
    phys = orc.dsa_translate(logical, pt, page, cache_rows=n_pages * page)
    # closed form: -1 exactly where the index, the page id or the row is out of range
    ok = (logical >= 0) & (logical < pps * page)
    pg = np.where(ok, pt[np.arange(Q)[:, None], np.clip(logical, 0, pps * page - 1) // page], -1)
    row = pg * page + np.where(ok, logical % page, 0)
    ok &= (pg >= 0) & (row < n_pages * page)
    np.testing.assert_array_equal(phys, np.where(ok, row, -1))
    assert (phys[0] == -1).sum() >= 7 and (phys[1] >= 0).all()
    out = orc.dsa_decode_bf16_paged(qn, qp, cache, pt, logical, Dc, page)
    cf = orc.bf16_to_f32(cache)
    qnf, qpf = orc.bf16_to_f32(qn), orc.bf16_to_f32(qp)
    for q in range(2):
        rows = phys[q][phys[q] >= 0][None, :].astype(np.int32)
        ref = orc.dsa_forward_f32(qnf[q:q + 1], qpf[q:q + 1], cf[:, :Dc].copy(), cf[:, Dc:].copy(),
                                  cf[:, :Dc].copy(), rows)
        np.testing.assert_array_equal(out[q], ref[0])
    assert (out[2] == 0).all()


def test_indexer_topk_capacity(orc):
    """A row scores only min(seq_len, cap) positions: with fewer than top-k of
    them the rest is -1 padding, never a position past the capacity."""
    rng = np.random.default_rng(3)
    sc = rng.standard_normal((2, 64)).astype(np.float32)
    sc[:, 20:] = -np.inf
    sl = np.array([64, 10], np.int32)
    out = orc.dsa_indexer_topk(sc, sl, 32, cap=20)
    np.testing.assert_array_equal(out[0], np.concatenate([np.arange(20), -np.ones(12, int)]))
    np.testing.assert_array_equal(out[1], np.concatenate([np.arange(10), -np.ones(22, int)]))
    out = orc.dsa_indexer_topk(sc, np.array([-4, 0], np.int32), 8)
    assert (out == -1).all()


@pytest.mark.parametrize("name,shape,tol", DSA_CASES, ids=[c[0] for c in DSA_CASES])
def test_reference_dsa_cases_match_float64(orc, name, shape, tol):
    Q, H, Dc, Dp, S, P, N = shape
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(Q, H, Dc, Dp, S, P, N)
    out = orc.dsa_forward_f32(qn, qp, kc, kp, v, idx)
    np.testing.assert_allclose(out, _dsa64(qn, qp, kc, kp, v, idx), rtol=1e-4, atol=1e-6)


# ---------------------------------------------------------------- DSA stages
def _stage_inputs(orc, seed=3, Q=3, H=5, Dc=40, Dp=12, S=17, N=64):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    idx = rng.integers(0, N, (Q, S)).astype(np.int32)
    return f(Q, H, Dc), f(Q, H, Dp), f(N, Dc), f(N, Dp), f(N, Dc), idx


def test_dsa_gather_is_fancy_indexing(orc):
    qn, qp, kc, kp, v, idx = _stage_inputs(orc)
    gkc, gkp, gv = orc.dsa_kv_gather(kc, kp, v, idx)
    np.testing.assert_array_equal(gkc, kc[idx])
    np.testing.assert_array_equal(gkp, kp[idx])
    np.testing.assert_array_equal(gv, v[idx])
    # Dp = 0: no positional part
    g0 = orc.dsa_kv_gather(kc, np.zeros((64, 0), np.float32), v, idx)
    assert g0[1].shape == (3, 17, 0)


def test_dsa_dots_match_float64_and_accumulate(orc):
    qn, qp, kc, kp, v, idx = _stage_inputs(orc)
    gkc, gkp, _ = orc.dsa_kv_gather(kc, kp, v, idx)
    init = np.random.default_rng(4).standard_normal((3, 5, 17)).astype(np.float32)
    dc = np.einsum("qhd,qsd->qhs", qn.astype(np.float64), gkc)
    dp = np.einsum("qhd,qsd->qhs", qp.astype(np.float64), gkp)
    for parts, ref in ((1, dc), (2, dp), (3, dc + dp)):
        out = orc.dsa_dot(qn if parts & 1 else None, qp if parts & 2 else None,
                          gkc if parts & 1 else None, gkp if parts & 2 else None, init, parts)
        np.testing.assert_allclose(out, init + ref, rtol=1e-5, atol=1e-5)
    # one-hot queries pick one column of the gathered rows, exactly
    oh = np.zeros_like(qn)
    oh[:, :, 7] = 1.0
    out = orc.dsa_dot(oh, None, gkc, None, np.zeros((3, 5, 17), np.float32), 1)
    np.testing.assert_array_equal(out, np.repeat(gkc[:, None, :, 7], 5, 1))
    ohp = np.zeros_like(qp)
    ohp[:, :, 3] = 1.0
    out = orc.dsa_dot(np.zeros_like(qn), ohp, gkc, gkp, np.zeros((3, 5, 17), np.float32), 3)
    np.testing.assert_array_equal(out, np.repeat(gkp[:, None, :, 3], 5, 1))


def test_dsa_dot_sums_in_d_order(orc):
    # (1 + 1e8) - 1e8 = 0 in binary32 summed front to back; any other order
    # of these three terms gives 1
    qn = np.ones((1, 1, 3), np.float32)
    kc = np.array([[[1.0, 1e8, -1e8]]], np.float32)
    out = orc.dsa_dot(qn, None, kc, None, np.zeros((1, 1, 1), np.float32), 1)
    assert out[0, 0, 0] == 0.0
    # fused: the positional terms continue the same accumulator
    qp = np.ones((1, 1, 1), np.float32)
    out = orc.dsa_dot(np.ones((1, 1, 2), np.float32), qp, np.array([[[1.0, 1e8]]], np.float32),
                      np.array([[[-1e8]]], np.float32), np.zeros((1, 1, 1), np.float32), 3)
    assert out[0, 0, 0] == 0.0


def test_dsa_softmax_matches_float64(orc):
    rng = np.random.default_rng(6)
    x = (3 * rng.standard_normal((4, 3, 50))).astype(np.float32)
    p = orc.dsa_softmax(x)
    x64 = x.astype(np.float64)
    ref = np.exp(x64 - x64.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    np.testing.assert_allclose(p, ref, rtol=1e-6, atol=1e-8)
    # uniform rows, S a power of two: exactly 1/S
    np.testing.assert_array_equal(orc.dsa_softmax(np.full((2, 2, 64), 0.25, np.float32)),
                                  np.full((2, 2, 64), 1 / 64, np.float32))


def test_dsa_output_proj_matches_float64(orc):
    rng = np.random.default_rng(7)
    attn = rng.random((2, 3, 20)).astype(np.float32)
    v = rng.standard_normal((2, 20, 9)).astype(np.float32)
    out = orc.dsa_output_proj(attn, v)
    np.testing.assert_allclose(out, np.einsum("qhs,qsd->qhd", attn.astype(np.float64), v),
                               rtol=1e-5, atol=1e-6)
    one = np.zeros_like(attn)
    one[:, :, 11] = 1.0
    np.testing.assert_array_equal(orc.dsa_output_proj(one, v), np.repeat(v[:, None, 11], 3, 1))


def test_dsa_stages_compose_to_forward(orc):
    # naive_dsa.cu:435-474: gather, fused dot into zeroed scores, scale,
    # softmax, output projection == cpu_dsa_forward (tests/test_dsa.cu:23-68)
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(4, 4, 64, 16, 64, 16, 256)
    gkc, gkp, gv = orc.dsa_kv_gather(kc, kp, v, idx)
    s = orc.dsa_dot(qn, qp, gkc, gkp, np.zeros((4, 4, 64), np.float32), 3)
    s = s * np.float32(1.0 / math.sqrt(64 + 16))
    out = orc.dsa_output_proj(orc.dsa_softmax(s), gv)
    np.testing.assert_allclose(out, orc.dsa_forward_f32(qn, qp, kc, kp, v, idx), rtol=1e-5, atol=1e-6)
