"""GPU parity of the MoE path, through the C ABI, against the CPU oracle.

Bars: integer outputs (expert indices, permutation, fp8 codes) bit-exact;
fp32 outputs within the reference's max-abs tolerances
(tests/test_moe.cu:204-267, strict <); bf16 outputs within the reference's
1e-2 max-abs of the oracle's fp32 result, widened only where the output's own
rounding (half a bf16 step) plus a 1e-3 allowance exceeds it, i.e. |y| >= 4
(bf16_bar_ok); fp8 outputs within 2e-2 relative (max-abs error over max
|ref|) of the oracle run on the same dequantised fp8 values.
"""
import numpy as np
import pytest
import torch

from cases import MOE_CASES

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    if a.dtype == np.uint8:
        return torch.from_numpy(a).cuda()
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def bf16_np(t):
    return t.cpu().numpy().view(np.uint16)


def announce(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------ formats
@pytest.mark.parametrize("cols", [512, 128, 640, 7168])
def test_quant_rows_bit_exact(amd, orc, cols):
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((37, cols)).astype(np.float32) * np.float32(3.0)
    x[3, :128] = 0.0
    x[5, -128:] *= np.float32(1e-5)                       # subnormal e4m3 codes
    x[7, cols // 256 * 128:][:128] = np.float32(1.0)      # constant block
    x[9, :128] *= np.float32(1e-20)                       # scale below 2^-64: IEEE division path
    x[11] *= np.exp2(np.arange(cols) % 61 - 30).astype(np.float32)  # wide exponent range per block
    xb = orc.f32_to_bf16(x)
    xf = orc.bf16_to_f32(xb)
    q_ref, s_ref = orc.quant_rows_1x128(xf)
    q = torch.empty((37, cols), dtype=torch.uint8, device="cuda")
    s = torch.empty((37, cols // 128), dtype=torch.float32, device="cuda")
    amd.quant_rows_fp8(dev(xb), q, s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), s_ref)
    np.testing.assert_array_equal(host(q), q_ref)


def test_quant_weight_bit_exact(amd, orc):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((256, 384)) * 0.05).astype(np.float32)
    u = rng.uniform(0.5, 2.0, (2, 3)).astype(np.float32)
    q_ref, s_ref = orc.quant_weight_128x128(w, u)
    q = torch.empty((256, 384), dtype=torch.uint8, device="cuda")
    s = torch.empty((2, 3), dtype=torch.float32, device="cuda")
    amd.quant_weight_fp8(dev(w), dev(u), q, s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), s_ref)
    np.testing.assert_array_equal(host(q), q_ref)


# ------------------------------------------------------------------ routing
@pytest.mark.parametrize("name,shape,tol", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_gate_f32_bit_exact_on_reference_cases(amd, orc, name, shape, tol):
    T, E, K, D, I = shape
    announce(f"gate_f32 {name} {shape}")
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    idx_ref, wts_ref = orc.moe_route(x, wg, K)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_f32(dev(x), dev(wg), idx, wts, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6, atol=0)


def _exact_gate_inputs(T, E, D, seed):
    """x and Wg whose products and every partial sum are exact in fp32
    (multiples of 2^-7 far below 2^17), so logits do not depend on the
    summation order and ties occur often."""
    rng = np.random.default_rng(seed)
    x = (rng.integers(-1, 2, (T, D)) * 0.125).astype(np.float32)
    wg = (rng.integers(-2, 3, (E, D)) * 0.0625).astype(np.float32)
    return x, wg


# T = 4133 leaves a ragged last 64-token tile; E = 64 and 16 leave gate
# columns of the 256-expert tile unused
@pytest.mark.parametrize("T,E,K,D", [(64, 256, 8, 7168), (33, 64, 6, 512), (16, 16, 2, 128),
                                     (2048, 256, 8, 7168), (4133, 64, 6, 512), (2050, 16, 2, 128)])
def test_gate_bf16_mfma_bit_exact_on_exact_logits(amd, orc, T, E, K, D):
    announce(f"gate_bf16 exact-logit T={T} E={E} K={K} D={D}")
    x, wg = _exact_gate_inputs(T, E, D, 11)
    xb, wgb = orc.f32_to_bf16(x), orc.f32_to_bf16(wg)
    idx_ref, wts_ref = orc.moe_route(x, wg, K)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16(dev(xb), dev(wgb), idx, wts, amd.moe_config(T, E, K, D, 128))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6, atol=0)


@pytest.mark.parametrize("T,E,K,D", [(1, 256, 8, 7168), (70, 256, 8, 7168), (4096, 256, 8, 7168),
                                     (33, 64, 6, 512), (4133, 64, 6, 512), (2048, 256, 8, 7168)])
def test_gate_fp8_fused_quant_bit_exact(amd, orc, T, E, K, D):
    """Routing of the fp8 layer with the x quantisation fused into the gate
    GEMM (the forward's path): codes and scales bit-identical to the oracle's
    1x128 quantiser, expert indices bit-exact on exactly representable logits."""
    announce(f"gate_fp8 fused quant T={T} E={E} K={K} D={D}")
    cfg = amd.moe_config(T, E, K, D, 128)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    q = torch.empty((T, D), dtype=torch.uint8, device="cuda")
    s = torch.empty((T, D // 128), dtype=torch.float32, device="cuda")
    # 1) exactly representable logits: indices and weights as the oracle's
    x, wg = _exact_gate_inputs(T, E, D, 13)
    xb, wgb = orc.f32_to_bf16(x), orc.f32_to_bf16(wg)
    idx_ref, wts_ref = orc.moe_route(x, wg, K)
    amd.moe_gate_fp8(dev(xb), dev(wgb), idx, wts, q, s, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6, atol=0)
    np.testing.assert_array_equal(host(q), orc.quant_rows_1x128(x)[0])
    # 2) random x over a wide range, an all-zero block and subnormal codes:
    #    e4m3 codes and scales bit-identical to the oracle's quantiser
    rng = np.random.default_rng(T + D)
    x = rng.standard_normal((T, D)).astype(np.float32) * np.float32(4.0)
    x *= np.exp2(rng.integers(-6, 7, (T, 1))).astype(np.float32)
    x[0, :128] = 0.0
    x[-1, -128:] *= np.float32(2.0 ** -12)
    x[-1, -128] = np.float32(1.0)
    xb = orc.f32_to_bf16(x)
    q_ref, s_ref = orc.quant_rows_1x128(orc.bf16_to_f32(xb))
    amd.moe_gate_fp8(dev(xb), dev(wgb), idx, wts, q, s, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), s_ref)
    np.testing.assert_array_equal(host(q), q_ref)


@pytest.mark.parametrize("T", [1024, 4096])
def test_gate_bf16_mfma_random_margin_aware(amd, orc, T):
    """Random N(0,1) inputs at the DSV3 gate shape (16 gate chunks at T=1024,
    4 at T=4096).  GPU (MFMA) and CPU (sequential) logits differ by rounding,
    so the selected set must match wherever the oracle's K-th/(K+1)-th logit
    gap exceeds a bound on that rounding; inside the bound either choice is
    accepted and counted."""
    E, K, D = 256, 8, 7168
    announce(f"gate_bf16 random T={T}")
    rng = np.random.default_rng(12)
    x = orc.bf16_to_f32(orc.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32)))
    wg = orc.bf16_to_f32(orc.f32_to_bf16((rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)))
    idx_ref, wts_ref, logits, _ = orc.moe_route(x, wg, K, want_probs=True)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16(dev(orc.f32_to_bf16(x)), dev(orc.f32_to_bf16(wg)), idx, wts,
                      amd.moe_config(T, E, K, D, 128))
    torch.cuda.synchronize()
    gi, gw = host(idx), host(wts)
    absdot = np.abs(x).astype(np.float64) @ np.abs(wg).astype(np.float64).T   # [T,E]
    bound = 2 * D * 2.0 ** -24 * absdot.max(1)                                  # both sums' error
    srt = np.sort(logits, 1)[:, ::-1]
    margin = srt[:, K - 1] - srt[:, K]
    same_set = np.array([set(gi[t]) == set(idx_ref[t]) for t in range(T)])
    assert same_set[margin > 2 * bound].all()
    same_order = (gi == idx_ref).all(1)
    n_diff = int((~same_order).sum())
    print(f"tokens with different slots: {n_diff} / {T}; near-ties: {(margin <= 2 * bound).sum()}")
    assert n_diff <= max(2, T // 500)
    ok = same_order
    np.testing.assert_allclose(gw[ok], wts_ref[ok], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("xt", ["f32", "bf16"])
@pytest.mark.parametrize("E,K,T,D", [(2, 1, 77, 768), (4, 2, 130, 512), (8, 2, 1000, 4096), (16, 4, 33, 1280),
                                     (8, 2, 4096, 256)])
def test_gate_fp32_weights_lds_path(amd, orc, xt, E, K, T, D):
    """The fp32-gate routing with E in {2, 4, 8, 16} and D a multiple of 256
    (x rows and the gate staged through LDS; fp32 x with E = 2 takes the
    per-lane kernel): the reference's sequential fp32 logits, so indices
    equal the oracle's exactly.  T leaves a ragged last block; D = 256 is a
    single stage, D = 768 / 1280 an odd count of stages."""
    announce(f"gate exact {xt} E={E} K={K} T={T} D={D}")
    rng = np.random.default_rng(E * 1000 + T)
    x = rng.standard_normal((T, D)).astype(np.float32)
    wg = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    cfg = amd.moe_config(T, E, K, D, 64)
    if xt == "f32":
        idx_ref, wts_ref = orc.moe_route(x, wg, K)
        amd.moe_gate_f32(dev(x), dev(wg), idx, wts, cfg)
    else:
        xb = orc.f32_to_bf16(x)
        idx_ref, wts_ref = orc.moe_route(orc.bf16_to_f32(xb), wg, K, bias=b)
        amd.moe_gate_bf16x(dev(xb), dev(wg), dev(b), idx, wts, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6)


def test_gate_bias_and_bf16x(amd, orc):
    T, E, K, D = 128, 8, 2, 1024
    rng = np.random.default_rng(13)
    x = orc.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    wg = (rng.standard_normal((E, D)) / 32).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32)
    idx_ref, wts_ref = orc.moe_route(orc.bf16_to_f32(x), wg, K, bias=b)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16x(dev(x), dev(wg), dev(b), idx, wts, amd.moe_config(T, E, K, D, 64))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6)


@pytest.mark.parametrize("entry,T,E,K,D", [("f32", 64, 256, 8, 512), ("bf16", 1, 256, 8, 7168),
                                           ("bf16", 64, 256, 8, 7168), ("bf16", 4096, 256, 8, 7168)])
def test_gate_non_finite_token_selects_nothing(amd, orc, entry, T, E, K, D):
    """A token with a NaN or inf in x has no finite logit: as in
    tests/test_moe.cu:52-68 no expert is inserted (indices -1, weights
    -FLT_MAX); every other token routes bit-exactly as the oracle's.  Covers
    the fp32 gate and the bf16 MFMA gate's decode (T=1) and chunked top-k
    kernels."""
    announce(f"gate_{entry} non-finite token T={T}")
    x, wg = _exact_gate_inputs(T, E, D, 21)
    bad = [0] if T == 1 else [0, T // 2, T - 1]
    x[bad[0], 3] = np.nan
    if T > 1:
        x[bad[1], D - 1] = np.inf
        x[bad[2], 100] = -np.inf
    idx_ref, wts_ref = orc.moe_route(x, wg, K)
    assert (idx_ref[bad] == -1).all()
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    cfg = amd.moe_config(T, E, K, D, 128)
    if entry == "f32":
        amd.moe_gate_f32(dev(x), dev(wg), idx, wts, cfg)
    else:
        amd.moe_gate_bf16(dev(orc.f32_to_bf16(x)), dev(orc.f32_to_bf16(wg)), idx, wts, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_ref)
    np.testing.assert_array_equal(host(wts)[bad], wts_ref[bad])
    np.testing.assert_allclose(host(wts), wts_ref, rtol=2e-6, atol=0)


# ------------------------------------------------------------------ permutation
# (70, 2048, 4): E > 1024 takes the single-launch kernel; the others the
# three-launch one (incl. a partial last block of 64 tokens and K > E)
# (8256, 256, 8): 129 token blocks, past 8192 tokens: the scan runs as its
# own launch between the count and the scatter
@pytest.mark.parametrize("T,E,K", [(1, 4, 2), (4, 16, 2), (512, 8, 2), (4096, 256, 8), (300, 3, 5),
                                   (8192, 256, 8), (70, 2048, 4), (8256, 256, 8), (20000, 64, 6)])
def test_permute_bit_exact(amd, orc, T, E, K):
    announce(f"permute T={T} E={E} K={K}")
    rng = np.random.default_rng(T + E)
    if K <= E:
        idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    else:  # K > E: the reference leaves -1 slots
        idx = np.full((T, K), -1, np.int32)
        idx[:, :E] = np.stack([rng.permutation(E) for _ in range(T)])
    counts_r, offsets_r, st_r, ss_r = orc.moe_permute(idx, E)
    P = int(offsets_r[-1])
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    st = torch.full((T * K,), -7, dtype=torch.int32, device="cuda")
    ss = torch.full((T * K,), -7, dtype=torch.int32, device="cuda")
    amd.moe_permute(dev(idx), amd.moe_config(T, E, K, 128, 128), counts, offsets, st, ss)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(counts), counts_r)
    np.testing.assert_array_equal(host(offsets), offsets_r)
    np.testing.assert_array_equal(host(st)[:P], st_r)
    np.testing.assert_array_equal(host(ss)[:P], ss_r)


# ------------------------------------------------------------------ stages
def test_gather_scatter_gemm_swiglu_stages(amd, orc):
    T, E, K, D, I = 32, 8, 2, 128, 256
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    idx_r, wts_r = orc.moe_route(x, wg, K)
    cfg = amd.moe_config(T, E, K, D, I)
    dx, didx, dwts = dev(x), dev(idx_r), dev(wts_r)
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    ref = np.zeros((T, D), np.float64)
    for e in range(E):
        gathered = torch.zeros((T, D), dtype=torch.float32, device="cuda")
        tmap = torch.full((T,), -1, dtype=torch.int32, device="cuda")
        cnt = torch.zeros(1, dtype=torch.int32, device="cuda")
        amd.moe_gather_f32(dx, didx, dwts, e, gathered, tmap, cnt, cfg)
        torch.cuda.synchronize()
        c = int(cnt.item())
        toks = [t for t in range(T) if e in idx_r[t]]
        assert c == len(toks) and host(tmap)[:c].tolist() == toks
        np.testing.assert_array_equal(host(gathered)[:c], x[toks])
        if c == 0:
            amd.moe_scatter_f32(gathered, tmap, dwts, didx, e, out, 0, cfg)
            continue
        # naive_gemm takes B [K,N] untransposed
        h = torch.empty((c, 2 * I), dtype=torch.float32, device="cuda")
        amd.naive_gemm_f32(gathered[:c].contiguous(), dev(np.ascontiguousarray(w1[e].T)), h, c, 2 * I, D)
        a = torch.empty((c, I), dtype=torch.float32, device="cuda")
        amd.swiglu_f32(h[:, :I].contiguous(), h[:, I:].contiguous(), a, c * I)
        o = torch.empty((c, D), dtype=torch.float32, device="cuda")
        amd.naive_gemm_f32(a, dev(np.ascontiguousarray(w2[e].T)), o, c, D, I)
        amd.moe_scatter_f32(o, tmap, dwts, didx, e, out, c, cfg)
        hh = x[toks].astype(np.float64) @ w1[e].astype(np.float64).T
        aa = hh[:, :I] / (1 + np.exp(-hh[:, :I])) * hh[:, I:]
        oo = aa @ w2[e].astype(np.float64).T
        for m, t in enumerate(toks):
            ref[t] += wts_r[t, list(idx_r[t]).index(e)] * oo[m]
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(out), ref, rtol=1e-4, atol=1e-6)


# ------------------------------------------------------------------ forward f32
@pytest.mark.parametrize("name,shape,tol", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_forward_f32_reference_cases(amd, orc, name, shape, tol):
    T, E, K, D, I = shape
    announce(f"forward_f32 {name} {shape}")
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    _, _, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K)
    y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    err = np.abs(host(y) - y_ref).max()
    print(f"{name}: max_err={err:.3e}")
    assert err < tol
    assert err < 1e-5 * max(1.0, np.abs(y_ref).max())


@pytest.mark.parametrize("T,E,K,D,I", [(1024, 4, 2, 128, 256), (512, 4, 2, 64, 128),
                                       (600, 3, 2, 64, 128)])
def test_forward_f32_multi_mtile_experts(amd, orc, T, E, K, D, I):
    """Experts of several M-tiles, on the reference's inputs, at the fp32 bar.
    These small layers get 64-row M-tiles (too few UP work items for 256-row
    ones), so an expert of ~256-512 rows splits into 4-8 balanced tiles;
    256-row tiles with a small remainder tile are covered by
    test_forward_every_tile_group_f32_bf16 at I = 2048."""
    announce(f"forward_f32 multi-M-tile experts {(T, E, K, D, I)}")
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    _, _, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K)
    y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    err = np.abs(host(y) - y_ref).max()
    print(f"multi-M-tile f32: max_err={err:.3e}")
    assert err < 1e-5 * max(1.0, np.abs(y_ref).max())


def test_forward_f32_explicit_workspace_and_reuse(amd, orc):
    T, E, K, D, I = 64, 16, 2, 512, 1024
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    _, _, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K)
    cfg = amd.moe_config(T, E, K, D, I)
    ws = amd.alloc_workspace(cfg, amd.AMDMOE_DTYPE_F32)
    ys = []
    for _ in range(3):
        y = torch.empty((T, D), dtype=torch.float32, device="cuda")
        amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), y, cfg, ws=ws)
        ys.append(y)
    torch.cuda.synchronize()
    for y in ys:
        np.testing.assert_array_equal(host(y), host(ys[0]))   # deterministic
    assert np.abs(host(ys[0]) - y_ref).max() < 5e-2
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(amd.AmdMoeError):
        amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), ys[0], cfg, ws=small)


# ------------------------------------------------------------------ forward bf16
def _bf16_case(amd, orc, T, E, K, D, I, bias, sample=None, seed=7):
    import synth
    x, wg, b, w1, w2 = synth.bf16_layer(T, E, D, I, seed=seed, bias=bias)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    amd.moe_forward_bf16(x, wg, b, w1, w2, y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    rows = np.arange(T) if sample is None else sample
    xs = bf16_np(x)[rows]
    idx_r, wts_r, y_ref = orc.moe_forward_bf16(xs, host(wg), bf16_np(w1), bf16_np(w2), K,
                                               bias=None if b is None else host(b))
    yg = orc.bf16_to_f32(bf16_np(y)[rows])
    err = np.abs(yg - y_ref).max()
    print(f"bf16 T={T} E={E} D={D} I={I}: max_err={err:.3e} max|y|={np.abs(y_ref).max():.3f} "
          f"(worst in bf16 steps: {bf16_steps(yg, y_ref):.2f})")
    return err, y_ref, yg


def bf16_steps(got, ref):
    """Largest |got - ref| in units of one bf16 step (2^-7 of the binade) at
    ref: the output is bf16, so its own rounding is half a step."""
    # (values below 2^-7 count with the step at 2^-7: a 1e-2 absolute bar
    # governs them)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -7))) - 7)
    return float((np.abs(got - ref) / step).max())


def bf16_bar_ok(got, ref):
    """The reference's large-case bar (max-abs 1e-2, tests/test_moe.cu:204-267),
    or, where larger, half a bf16 step at |ref| (the output's own rounding:
    the bf16 layer sums its per-expert rows in fp32 and rounds y once) plus
    1e-3 for the rest: the intermediate activation is bf16 in both the GPU
    path and the oracle, and the GPU's SwiGLU (hardware exp2 and reciprocal)
    and fp32 summation order can flip an activation's last bit, each flip
    moving y by ~1e-5 at these shapes.  The widening acts only where
    |y| >= 4 (half a step there is 0.0156)."""
    half = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -100))) - 8)
    bar = np.maximum(1e-2, half + 1e-3)
    return bool((np.abs(got - ref) < bar).all())


def test_forward_bf16_medium_skewed(amd, orc):
    """BASELINE medium config in bf16, with the per-expert logit bias."""
    announce("forward_bf16 medium")
    err, y_ref, yg = _bf16_case(amd, orc, 512, 8, 2, 1024, 2048, bias=True)
    assert bf16_bar_ok(yg, y_ref)


def test_forward_bf16_mixtral_t16(amd, orc):
    announce("forward_bf16 mixtral T=16")
    err, y_ref, yg = _bf16_case(amd, orc, 16, 8, 2, 4096, 14336, bias=False)
    assert bf16_bar_ok(yg, y_ref)


def test_forward_bf16_multi_mtile_experts(amd, orc):
    """~512 rows per expert: each expert spans 2-3 M-tiles of 256 rows.  The
    outputs reach |y| ~ 3, where one bf16 step is 1.6e-2, so the bar is
    relative: 2^-7 of max |y|."""
    announce("forward_bf16 multi-M-tile experts")
    err, y_ref, _ = _bf16_case(amd, orc, 1024, 4, 2, 128, 256, bias=True)
    assert err < 2.0 ** -7 * np.abs(y_ref).max()


# ------------------------------------------------------------------ forward fp8
@pytest.fixture(scope="module")
def dsv3(amd):
    import synth
    announce("generating DSV3 fp8 weights (E=256, D=7168, I=2048)")
    w = synth.dsv3_weights(256, 7168, 2048, seed=1234)
    yield w
    del w
    torch.cuda.empty_cache()


def _fp8_case(amd, orc, weights, T, E, K, D, I, sample=None, seed=1235):
    import synth
    w1q, w1s, w2q, w2s = weights
    x, wg = synth.dsv3_inputs(T, E, D, seed=seed)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    amd.moe_forward_fp8(x, wg, w1q, w1s, w2q, w2s, y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    rows = np.arange(T) if sample is None else np.asarray(sample)
    xs = bf16_np(x)[rows]
    wgn = bf16_np(wg)
    # only the experts the checked tokens use travel to the host
    idx_s, _ = orc.moe_route(orc.bf16_to_f32(xs), orc.bf16_to_f32(wgn), K)
    used = np.unique(idx_s[idx_s >= 0])
    wmap = np.zeros(E, np.int32)
    wmap[used] = np.arange(len(used), dtype=np.int32)
    sel = torch.from_numpy(used).cuda()
    q1 = w1q.index_select(0, sel).cpu().numpy(); s1 = w1s.index_select(0, sel).cpu().numpy()
    q2 = w2q.index_select(0, sel).cpu().numpy(); s2 = w2s.index_select(0, sel).cpu().numpy()
    idx_r, wts_r, y_ref = orc.moe_forward_fp8(xs, wgn, q1, s1, q2, s2, K, wmap=wmap)
    yg = orc.bf16_to_f32(bf16_np(y)[rows])
    rel = np.abs(yg - y_ref).max() / np.abs(y_ref).max()
    print(f"fp8 T={T} E={E}: rel_err={rel:.3e} max|y|={np.abs(y_ref).max():.3f}")
    return rel


def test_forward_fp8_small_full(amd, orc):
    import synth
    announce("forward_fp8 small full")
    w = synth.dsv3_weights(16, 512, 256, seed=77)
    assert _fp8_case(amd, orc, w, 64, 16, 4, 512, 256) < 2e-2


@pytest.mark.parametrize("T", [2, 16, 17])
def test_forward_fp8_decode_sizes(amd, orc, T):
    """Decode-sized batches: a few tokens over many experts (most M-tiles
    one 16-row token tile), parity with the oracle's fp8 forward."""
    import synth
    announce(f"forward_fp8 decode size T={T}")
    w = synth.dsv3_weights(16, 512, 256, seed=78)
    assert _fp8_case(amd, orc, w, T, 16, 4, 512, 256) < 2e-2


def test_forward_fp8_multi_mtile_experts(amd, orc):
    """~256 rows per expert (as DeepSeek-V3 at T=8192): experts take one or
    two M-tiles."""
    import synth
    announce("forward_fp8 multi-M-tile experts")
    w = synth.dsv3_weights(4, 256, 128, seed=81)
    assert _fp8_case(amd, orc, w, 512, 4, 2, 256, 128) < 2e-2


def test_forward_fp8_dsv3_t1(amd, orc, dsv3):
    announce("forward_fp8 dsv3 T=1")
    assert _fp8_case(amd, orc, dsv3, 1, 256, 8, 7168, 2048) < 2e-2


def test_forward_fp8_dsv3_t64_full(amd, orc, dsv3):
    announce("forward_fp8 dsv3 T=64")
    rows = np.arange(0, 64, 4)
    assert _fp8_case(amd, orc, dsv3, 64, 256, 8, 7168, 2048, sample=rows) < 2e-2


def test_forward_fp8_dsv3_t512_sampled(amd, orc, dsv3):
    announce("forward_fp8 dsv3 T=512 sampled")
    rows = np.random.default_rng(5).choice(512, 6, replace=False)
    assert _fp8_case(amd, orc, dsv3, 512, 256, 8, 7168, 2048, sample=rows) < 2e-2


def test_forward_fp8_dsv3_t8192_sampled(amd, orc, dsv3):
    """BASELINE's largest token count: about half the experts span two
    (evenly split) M-tiles."""
    announce("forward_fp8 dsv3 T=8192 sampled")
    rows = np.random.default_rng(6).choice(8192, 6, replace=False)
    assert _fp8_case(amd, orc, dsv3, 8192, 256, 8, 7168, 2048, sample=rows) < 2e-2


def test_forward_fp8_dsv3_t4096_sampled(amd, orc, dsv3):
    announce("forward_fp8 dsv3 T=4096 sampled")
    rows = np.random.default_rng(4).choice(4096, 6, replace=False)
    assert _fp8_case(amd, orc, dsv3, 4096, 256, 8, 7168, 2048, sample=rows) < 2e-2


# ------------------------------------------------------------------ packed weights
def _pack_np(w):
    """The fragment-block order of amdmoe_pack_weights_fp8 restated on the host:
    block (e, n16, kb) holds, at [h][l][16 B], row 16*n16 + (l & 15), bytes
    128*kb + 64*h + 16*(l >> 4) .. +15 of expert e."""
    E, N, K = w.shape
    b = w.reshape(E, N // 16, 16, K // 128, 2, 4, 16)  # e, n16, r, kb, h, q, byte
    return np.ascontiguousarray(b.transpose(0, 1, 3, 4, 5, 2, 6)).reshape(E, N, K)


def test_pack_weights_format(amd):
    announce("pack_weights_fp8 format")
    w = np.random.default_rng(11).integers(0, 256, size=(3, 48, 384), dtype=np.uint8)
    out = torch.empty((3, 48, 384), dtype=torch.uint8, device="cuda")
    amd.pack_weights_fp8(dev(w), out)
    torch.cuda.synchronize()
    assert np.array_equal(host(out), _pack_np(w))
    # lane 17 of block (0, 0, 1), hi half = row 1, bytes 128 + 64 + 16 .. +15
    assert np.array_equal(host(out)[0].reshape(-1)[1 * 2048 + 1024 + 17 * 16:][:16], w[0, 1, 208:224])


def _packed_pair(w1q, w2q):
    p1, p2 = torch.empty_like(w1q), torch.empty_like(w2q)
    import amdmoe
    amdmoe.pack_weights_fp8(w1q, p1)
    amdmoe.pack_weights_fp8(w2q, p2)
    return p1, p2


def test_forward_fp8_packed_bit_identical_small(amd):
    import synth
    announce("forward_fp8_packed small")
    T, E, K, D, I = 64, 16, 4, 512, 256
    w1q, w1s, w2q, w2s = synth.dsv3_weights(E, D, I, seed=78)
    x, wg = synth.dsv3_inputs(T, E, D, seed=79)
    p1, p2 = _packed_pair(w1q, w2q)
    cfg = amd.moe_config(T, E, K, D, I)
    y0 = torch.empty((T, D), dtype=torch.int16, device="cuda")
    y1 = torch.empty_like(y0)
    amd.moe_forward_fp8(x, wg, w1q, w1s, w2q, w2s, y0, cfg)
    amd.moe_forward_fp8_packed(x, wg, p1, w1s, p2, w2s, y1, cfg)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_forward_fp8_packed_bit_identical_dsv3_t4096(amd, dsv3):
    import synth
    announce("forward_fp8_packed dsv3 T=4096")
    w1q, w1s, w2q, w2s = dsv3
    T, E, K, D, I = 4096, 256, 8, 7168, 2048
    x, wg = synth.dsv3_inputs(T, E, D, seed=1236)
    p1, p2 = _packed_pair(w1q, w2q)
    cfg = amd.moe_config(T, E, K, D, I)
    y0 = torch.empty((T, D), dtype=torch.int16, device="cuda")
    y1 = torch.empty_like(y0)
    amd.moe_forward_fp8(x, wg, w1q, w1s, w2q, w2s, y0, cfg)
    amd.moe_forward_fp8_packed(x, wg, p1, w1s, p2, w2s, y1, cfg)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    del p1, p2


# ------------------------------------------------------------------ controlled routing
# Rows per expert chosen so that the grouped GEMM meets every live
# token-tile count of its fp8 main loop (R = 1..16 tiles of 16 rows, both
# register-ring depths: R <= 12 and R > 12), row counts on and just past
# 16-row boundaries, and experts split into two and three M-tiles (more than
# 256 and 512 rows; the permutation splits them evenly into whole 16-row
# tiles).
ROUTED_COUNTS = ([16 * r - 7 for r in range(1, 17)] + [16 * r for r in range(1, 17)]
                 + [1, 2, 15, 17, 255, 257, 270, 300, 400, 511, 512, 513, 600])


def _mtile_rows(cnt, bm=256):
    """Rows of the M-tiles of an expert with cnt rows (the permutation's
    split: ceil(cnt/256) tiles of whole 16-row tiles, as even as possible)."""
    nt = -(-cnt // bm)
    q = -(-cnt // 16)
    base, extra = divmod(q, nt)
    out, first = [], 0
    for j in range(nt):
        r = min(16 * (base + (1 if j < extra else 0)), cnt - first)
        out.append(r)
        first += r
    return out


def _routed_layout(counts, E, K):
    """Token -> experts assignment giving expert i exactly counts[i] rows
    (experts 0..len(counts)-1; the slots left over to make T*K go one each to
    the following experts).  Slots sorted by expert are dealt to tokens
    round-robin (slot j -> token j % T), so an expert never sees one token
    twice as long as its count is at most T."""
    slots = [e for e, c in enumerate(counts) for _ in range(c)]
    T = max(max(counts), -(-len(slots) // K))
    fill = T * K - len(slots)
    assert len(counts) + fill <= E
    slots += list(range(len(counts), len(counts) + fill))
    chosen = [[] for _ in range(T)]
    for j, e in enumerate(slots):
        chosen[j % T].append(e)
    assert all(len(c) == K and len(set(c)) == K for c in chosen)
    return T, chosen


def _routing_columns(chosen, E, D, rng):
    """x [T,D] whose first E columns fix the routing through a one-hot gate
    Wg[e] = e_e (logit e = x[t,e], exact): the token's K experts get 2 + k/8,
    the rest -1; the other columns are N(0,1)."""
    T = len(chosen)
    x = rng.standard_normal((T, D)).astype(np.float32)
    x[:, :E] = -1.0
    for t, es in enumerate(chosen):
        for k, e in enumerate(es):
            x[t, e] = 2.0 + 0.125 * k
    wg = np.zeros((E, D), np.float32)
    wg[np.arange(E), np.arange(E)] = 1.0
    return x, wg


def test_routed_layout_reaches_every_tile_count():
    rs = {r for c in ROUTED_COUNTS for rows in _mtile_rows(c) for r in [-(-rows // 16)]}
    assert rs == set(range(1, 17))
    assert max(len(_mtile_rows(c)) for c in ROUTED_COUNTS) == 3


def test_forward_fp8_every_token_tile_count(amd, orc, dsv3):
    """DSV3 shape (E=256, K=8, D=7168, I=2048) with routing fixed through the
    gate so that experts hold the row counts of ROUTED_COUNTS: every live
    token-tile count R = 1..16 of the fp8 main loop, both register-ring
    depths, two- and three-tile experts.  The full output of the row-major
    and the packed entry is compared with the oracle (relative max error <=
    2e-2 on the same dequantised fp8 values), and the two entries must agree
    bit for bit."""
    import synth
    E, K, D, I = 256, 8, 7168, 2048
    T, chosen = _routed_layout(ROUTED_COUNTS, E, K)
    announce(f"forward_fp8 every token-tile count: T={T}, {len(ROUTED_COUNTS)} sized experts")
    x, wg = _routing_columns(chosen, E, D, np.random.default_rng(1240))
    xb, wgb = orc.f32_to_bf16(x), orc.f32_to_bf16(wg)
    w1q, w1s, w2q, w2s = dsv3
    cfg = amd.moe_config(T, E, K, D, I)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    amd.moe_forward_fp8(dev(xb), dev(wgb), w1q, w1s, w2q, w2s, y, cfg)
    p1, p2 = _packed_pair(w1q, w2q)
    yp = torch.empty_like(y)
    amd.moe_forward_fp8_packed(dev(xb), dev(wgb), p1, w1s, p2, w2s, yp, cfg)
    # the GPU's own routing and permutation: the counts asked for
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16(dev(xb), dev(wgb), idx, wts, cfg)
    torch.cuda.synchronize()
    del p1, p2
    gi = host(idx)
    assert [set(r) for r in gi.tolist()] == [set(c) for c in chosen]
    counts = np.bincount(gi.reshape(-1), minlength=E)
    assert counts[:len(ROUTED_COUNTS)].tolist() == ROUTED_COUNTS
    assert torch.equal(y, yp)
    used = np.unique(gi)
    wmap = np.zeros(E, np.int32)
    wmap[used] = np.arange(len(used), dtype=np.int32)
    sel = torch.from_numpy(used).cuda()
    q1 = w1q.index_select(0, sel).cpu().numpy(); s1 = w1s.index_select(0, sel).cpu().numpy()
    q2 = w2q.index_select(0, sel).cpu().numpy(); s2 = w2s.index_select(0, sel).cpu().numpy()
    idx_r, _, y_ref = orc.moe_forward_fp8(xb, wgb, q1, s1, q2, s2, K, wmap=wmap)
    np.testing.assert_array_equal(np.sort(idx_r, 1), np.sort(gi, 1))
    yg = orc.bf16_to_f32(bf16_np(y))
    rel = np.abs(yg - y_ref).max() / np.abs(y_ref).max()
    # per expert row count: the worst token among those the expert serves
    tok_err = np.abs(yg - y_ref).max(1) / np.abs(y_ref).max()
    worst = {c: float(tok_err[np.flatnonzero((gi == e).any(1))].max())
             for e, c in enumerate(ROUTED_COUNTS)}
    print(f"every tile count: rel_err={rel:.3e}; worst per count: "
          + ", ".join(f"{c}:{v:.1e}" for c, v in worst.items()))
    assert rel < 2e-2


@pytest.mark.parametrize("dtype,I", [("f32", 256), ("bf16", 256), ("f32", 2048), ("bf16", 2048)])
def test_forward_every_tile_group_f32_bf16(amd, orc, dtype, I):
    """fp32 and bf16 main loops are instantiated per group of four 16-row
    tiles (4, 8, 12, 16): routing fixed through the gate gives experts every
    row count of ROUTED_COUNTS (all four groups, split experts); full output
    against the oracle at the fp32 / bf16 bars.  I = 2048 (32 / 64 K-steps)
    runs the down projection with its K split in two (partial rows added
    in the combine)."""
    T, chosen = _routed_layout(ROUTED_COUNTS, 64, 2)
    E, K, D = 64, 2, 128
    announce(f"forward_{dtype} every tile group: T={T} I={I}")
    rng = np.random.default_rng(1250)
    x, wg = _routing_columns(chosen, E, D, rng)
    w1 = (rng.standard_normal((E, 2 * I, D)) / np.sqrt(D)).astype(np.float32)
    w2 = (rng.standard_normal((E, D, I)) / np.sqrt(I)).astype(np.float32)
    cfg = amd.moe_config(T, E, K, D, I)
    if dtype == "f32":
        y = torch.empty((T, D), dtype=torch.float32, device="cuda")
        amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), y, cfg)
        torch.cuda.synchronize()
        idx_r, _, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K)
        err = np.abs(host(y) - y_ref).max()
        bar = 1e-5 * max(1.0, np.abs(y_ref).max())
    else:
        xb, w1b, w2b = orc.f32_to_bf16(x), orc.f32_to_bf16(w1), orc.f32_to_bf16(w2)
        y = torch.empty((T, D), dtype=torch.int16, device="cuda")
        amd.moe_forward_bf16(dev(xb), dev(wg), None, dev(w1b), dev(w2b), y, cfg)
        # the packed-weight entry on every tile group: bit-identical
        p1, p2 = torch.empty_like(dev(w1b)), torch.empty_like(dev(w2b))
        amd.pack_weights_bf16(dev(w1b), p1)
        amd.pack_weights_bf16(dev(w2b), p2)
        yp = torch.empty_like(y)
        amd.moe_forward_bf16_packed(dev(xb), dev(wg), None, p1, p2, yp, cfg)
        torch.cuda.synchronize()
        assert torch.equal(yp, y)
        idx_r, _, y_ref = orc.moe_forward_bf16(xb, wg, w1b, w2b, K)
        err = np.abs(orc.bf16_to_f32(bf16_np(y)) - y_ref).max()
        bar = 2.0 ** -7 * np.abs(y_ref).max()
    counts = np.bincount(idx_r.reshape(-1), minlength=E)
    assert counts[:len(ROUTED_COUNTS)].tolist() == ROUTED_COUNTS
    print(f"{dtype} every tile group: max_err={err:.3e} bar={bar:.3e}")
    assert err < bar


def _tile_edge_sample(amd, idx, cfg, T, E, K, n_rows, seed):
    """Tokens that are the first or the last sorted row of an M-tile, from the
    GPU's own routing and permutation (tokens sort ascending within an
    expert, so these are low and high token ids), where a tile's row bounds
    and masks act; topped up with random tokens to n_rows.  Returns the rows
    and the number of edge tokens among them (all of them when there are at
    most n_rows)."""
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    st = torch.empty(T * K, dtype=torch.int32, device="cuda")
    ss = torch.empty(T * K, dtype=torch.int32, device="cuda")
    amd.moe_permute(idx, cfg, counts, offsets, st, ss)
    torch.cuda.synchronize()
    cn, of, stn = host(counts), host(offsets), host(st)
    edges = []
    for e in range(E):
        first = int(of[e])
        for rows in _mtile_rows(int(cn[e])):
            edges += [int(stn[first]), int(stn[first + rows - 1])]
            first += rows
    rng = np.random.default_rng(seed)
    edge_rows = np.unique(np.array(edges))
    if len(edge_rows) > n_rows:
        edge_rows = np.sort(rng.choice(edge_rows, n_rows, replace=False))
    rest = np.setdiff1d(np.arange(T), edge_rows)
    rows = np.sort(np.concatenate([edge_rows, rng.choice(rest, n_rows - len(edge_rows), replace=False)]))
    assert len(rows) == n_rows
    return rows, len(edge_rows)


@pytest.mark.parametrize("T,n_rows", [(4096, 256), (8192, 640)])
def test_forward_fp8_dsv3_tile_edges(amd, orc, dsv3, T, n_rows):
    """DSV3 T=4096 and T=8192 on the GPU; the oracle checks every token that
    is the first or last row of an M-tile (~180 at T=4096, where each expert
    is one M-tile; several hundred at T=8192, where about half the experts
    split into two) plus random others."""
    import synth
    E, K, D, I = 256, 8, 7168, 2048
    announce(f"forward_fp8 dsv3 T={T}, {n_rows} tile-edge tokens")
    x, wg = synth.dsv3_inputs(T, E, D, seed=1235)
    cfg = amd.moe_config(T, E, K, D, I)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16(x, wg, idx, wts, cfg)
    rows, n_edge = _tile_edge_sample(amd, idx, cfg, T, E, K, n_rows, seed=4)
    print(f"edge tokens checked: {n_edge}")
    assert n_edge >= 100
    assert _fp8_case(amd, orc, dsv3, T, E, K, D, I, sample=rows) < 2e-2


def test_forward_bf16_mixtral_t4096_tile_edges(amd, orc):
    """Mixtral bf16 T=4096 (every expert ~1024 rows, four M-tiles): the
    oracle checks the first and last token of every M-tile plus random
    others, 128 tokens."""
    import synth
    T, E, K, D, I = 4096, 8, 2, 4096, 14336
    announce("forward_bf16 mixtral T=4096 tile edges")
    x, wg, _, _, _ = synth.bf16_layer(T, E, D, I, seed=7, bias=False)
    cfg = amd.moe_config(T, E, K, D, I)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_bf16x(x, wg, None, idx, wts, cfg)
    rows, n_edge = _tile_edge_sample(amd, idx, cfg, T, E, K, 128, seed=5)
    del x, wg
    print(f"edge tokens checked: {n_edge}")
    assert n_edge >= 40
    err, y_ref, yg = _bf16_case(amd, orc, T, E, K, D, I, bias=False, sample=rows, seed=7)
    assert bf16_bar_ok(yg, y_ref)


def test_pack_weights_bf16_is_the_byte_packing(amd):
    """pack_weights_bf16 lays out a bf16 row's 2*cols bytes exactly as
    pack_weights_fp8 lays out a row of that many bytes (whose format
    test_pack_weights_format checks)."""
    w = torch.randint(-32768, 32767, (3, 48, 320), dtype=torch.int16, device="cuda")
    a = torch.empty_like(w)
    b = torch.empty((3, 48, 640), dtype=torch.uint8, device="cuda")
    amd.pack_weights_bf16(w, a)
    amd.pack_weights_fp8(w.view(torch.uint8), b)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.uint8), b)


def test_forward_bf16_packed_bit_identical_mixtral_t256(amd):
    """Mixtral shape (112 N-tiles of UP, 16 of DOWN, experts of ~64 rows):
    the packed-weight bf16 forward equals the row-major one bit for bit."""
    import synth
    T, E, K, D, I = 256, 8, 2, 4096, 14336
    announce("forward_bf16_packed mixtral T=256")
    x, wg, _, w1, w2 = synth.bf16_layer(T, E, D, I, seed=7, bias=False)
    cfg = amd.moe_config(T, E, K, D, I)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    yp = torch.empty_like(y)
    amd.moe_forward_bf16(x, wg, None, w1, w2, y, cfg)
    p1, p2 = torch.empty_like(w1), torch.empty_like(w2)
    amd.pack_weights_bf16(w1, p1)
    amd.pack_weights_bf16(w2, p2)
    del w1, w2
    amd.moe_forward_bf16_packed(x, wg, None, p1, p2, yp, cfg)
    torch.cuda.synchronize()
    assert torch.equal(yp, y)


def test_forward_bf16_packed_bit_identical_mixtral_t4096(amd):
    """Mixtral T=4096 (four full 256-row M-tiles per expert, the down
    projection split in two along I): the packed-weight bf16 forward (4
    waves x 64 weight rows) equals the row-major one (8 waves x 32 rows)
    bit for bit."""
    import synth
    T, E, K, D, I = 4096, 8, 2, 4096, 14336
    announce("forward_bf16_packed mixtral T=4096")
    x, wg, _, w1, w2 = synth.bf16_layer(T, E, D, I, seed=7, bias=False)
    cfg = amd.moe_config(T, E, K, D, I)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    yp = torch.empty_like(y)
    amd.moe_forward_bf16(x, wg, None, w1, w2, y, cfg)
    p1, p2 = torch.empty_like(w1), torch.empty_like(w2)
    amd.pack_weights_bf16(w1, p1)
    amd.pack_weights_bf16(w2, p2)
    del w1, w2
    amd.moe_forward_bf16_packed(x, wg, None, p1, p2, yp, cfg)
    torch.cuda.synchronize()
    assert torch.equal(yp, y)


@pytest.mark.parametrize("T,D,I", [(300, 320, 192), (40, 192, 320)])
def test_forward_bf16_packed_bit_identical_partial_tiles(amd, T, D, I):
    """N-tiles cut short on both projections (I and D multiples of 64 but
    not of 128 / 256: the last UP N-tile has 64 of its 128 columns, the
    last DOWN N-tile 64 of 256), and M-tiles of every tile group: packed
    equals row-major bit for bit."""
    E, K = 16, 4
    announce(f"forward_bf16_packed partial tiles T={T} D={D} I={I}")
    g = torch.Generator(device="cuda")
    g.manual_seed(1251)
    x = (torch.randn((T, D), generator=g, device="cuda")).to(torch.bfloat16).view(torch.int16)
    wg = torch.randn((E, D), generator=g, device="cuda") / D ** 0.5
    w1 = (torch.randn((E, 2 * I, D), generator=g, device="cuda") / D ** 0.5).to(torch.bfloat16).view(torch.int16)
    w2 = (torch.randn((E, D, I), generator=g, device="cuda") / I ** 0.5).to(torch.bfloat16).view(torch.int16)
    cfg = amd.moe_config(T, E, K, D, I)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    yp = torch.empty_like(y)
    amd.moe_forward_bf16(x, wg, None, w1, w2, y, cfg)
    p1, p2 = torch.empty_like(w1), torch.empty_like(w2)
    amd.pack_weights_bf16(w1, p1)
    amd.pack_weights_bf16(w2, p2)
    amd.moe_forward_bf16_packed(x, wg, None, p1, p2, yp, cfg)
    torch.cuda.synchronize()
    assert torch.equal(yp, y)
    assert bool(torch.isfinite(y.view(torch.bfloat16).float()).all())


def test_forward_bf16_mixtral_t256(amd, orc):
    """BASELINE Mixtral config at T=256, every token checked (outputs reach
    |y| ~ 2.6, where bf16_bar_ok is the reference's 1e-2)."""
    announce("forward_bf16 mixtral T=256")
    err, y_ref, yg = _bf16_case(amd, orc, 256, 8, 2, 4096, 14336, bias=False)
    assert bf16_bar_ok(yg, y_ref)


def test_forward_f32_medium_with_bias(amd, orc):
    """BASELINE medium config in fp32 (T=512, E=8, K=2, D=1024, I=2048,
    N(0, 1/fan_in) weights) with the per-expert logit bias ~ N(0, 0.5^2) that
    skews the expert loads, through amdmoe_moe_forward_f32_bias: indices as
    the oracle's and the output within 1e-5 of max |y| (and the reference's
    1e-3)."""
    T, E, K, D, I = 512, 8, 2, 1024, 2048
    announce("forward_f32 medium with bias")
    rng = np.random.default_rng(512)
    x = rng.standard_normal((T, D)).astype(np.float32)
    wg = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32)
    w1 = (rng.standard_normal((E, 2 * I, D)) / np.sqrt(D)).astype(np.float32)
    w2 = (rng.standard_normal((E, D, I)) / np.sqrt(I)).astype(np.float32)
    idx_r, _, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K, bias=b)
    counts = np.bincount(idx_r.reshape(-1), minlength=E)
    print(f"medium f32 expert loads: {counts.tolist()}")
    y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    amd.moe_forward_f32_bias(dev(x), dev(wg), dev(b), dev(w1), dev(w2), y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    err = np.abs(host(y) - y_ref).max()
    print(f"medium f32 with bias: max_err={err:.3e} max|y|={np.abs(y_ref).max():.3f}")
    assert err < 1e-3
    assert err < 1e-5 * max(1.0, np.abs(y_ref).max())


@pytest.mark.parametrize("T,E,K,D,I", [(37, 5, 3, 100, 50), (16, 4, 2, 33, 17), (300, 3, 2, 48, 40),
                                       (9, 2, 2, 1, 1)])
def test_forward_f32_any_shape(amd, orc, T, E, K, D, I):
    """D and I that are not multiples of 32 (the reference takes any shape):
    routing, gather and the whole forward against the oracle at the fp32
    bar, on the reference's input distribution."""
    announce(f"forward_f32 any shape {(T, E, K, D, I)}")
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    idx_r, wts_r, y_ref = orc.moe_forward_f32(x, wg, w1, w2, K)
    cfg = amd.moe_config(T, E, K, D, I)
    y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    amd.moe_forward_f32(dev(x), dev(wg), dev(w1), dev(w2), y, cfg)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_f32(dev(x), dev(wg), idx, wts, cfg)
    g = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    tmap = torch.full((T,), -1, dtype=torch.int32, device="cuda")
    cnt = torch.zeros(1, dtype=torch.int32, device="cuda")
    amd.moe_gather_f32(dev(x), idx, wts, E - 1, g, tmap, cnt, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), idx_r)
    toks = [t for t in range(T) if E - 1 in idx_r[t]]
    assert int(cnt.item()) == len(toks)
    np.testing.assert_array_equal(host(g)[:len(toks)], x[toks])
    err = np.abs(host(y) - y_ref).max()
    print(f"any shape {(T, E, K, D, I)}: max_err={err:.3e}")
    assert err < 1e-3
    assert err < 1e-5 * max(1.0, np.abs(y_ref).max())
