"""GPU parity of the DSA decode path, through the C ABI, against the oracle.

fp32 entry: the reference's 14 cases (tests/test_dsa.cu:162-230) with its
max-abs tolerances (strict <), plus a tighter bound against the oracle.
bf16 paged entry: the BASELINE decode shape, checked per query against the
oracle run on the same bf16 values (max-abs error within 1e-2 of outputs
whose magnitude is O(0.1), i.e. bf16 output rounding plus bf16 P).
"""
import numpy as np
import pytest
import torch

from cases import DSA_CASES

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


@pytest.mark.parametrize("name,shape,tol", DSA_CASES, ids=[c[0] for c in DSA_CASES])
def test_dsa_f32_reference_cases(amd, orc, name, shape, tol):
    Q, H, Dc, Dp, S, P, N = shape
    print(f"dsa_f32 {name} {shape}", flush=True)
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(Q, H, Dc, Dp, S, P, N)
    ref = orc.dsa_forward_f32(qn, qp, kc, kp, v, idx)
    out = torch.full((Q, H, Dc), float("nan"), dtype=torch.float32, device="cuda")
    amd.dsa_forward_f32(dev(qn), dev(qp), dev(kc), dev(kp), dev(v), dev(idx), out,
                        amd.dsa_config(Q, H, Dc, Dp, S, P, N))
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy() - ref).max()
    print(f"{name}: max_err={err:.3e}")
    assert err < tol
    assert err < 1e-6


def _paged_case(amd, orc, Q, H, S, ctx, page=64, check_q=None, seed=5, inputs=None):
    import synth
    if inputs is None:
        inputs = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=seed)
    qn, qp, cache, pt, logical, pps = inputs
    out = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    amd.dsa_decode_bf16_paged(qn, qp, cache, pt, logical, out,
                              amd.dsa_config(Q, H, 512, 64, S, page, Q * ctx), pps)
    torch.cuda.synchronize()
    qs = np.arange(Q) if check_q is None else np.asarray(check_q)
    ptn, lgn = pt.cpu().numpy(), logical.cpu().numpy()
    # only the cache rows the checked queries touch travel to the host
    phys = orc.dsa_translate(lgn[qs], ptn[qs], page)
    rows = torch.from_numpy(phys.reshape(-1).astype(np.int64)).cuda()
    sub = cache.index_select(0, rows).cpu().numpy().view(np.uint16)
    flat = np.arange(len(qs) * S, dtype=np.int32).reshape(len(qs), S)
    cf = orc.bf16_to_f32(sub)
    qnf = orc.bf16_to_f32(qn.cpu().numpy().view(np.uint16)[qs])
    qpf = orc.bf16_to_f32(qp.cpu().numpy().view(np.uint16)[qs])
    ref = orc.dsa_forward_f32(qnf, qpf, cf[:, :512].copy(), cf[:, 512:].copy(), cf[:, :512].copy(), flat)
    got = orc.bf16_to_f32(out.cpu().numpy().view(np.uint16)[qs])
    err = np.abs(got - ref).max()
    print(f"dsa_bf16 Q={Q} H={H} S={S}: max_err={err:.3e} max|ref|={np.abs(ref).max():.3f}")
    return err


def test_dsa_bf16_paged_small(amd, orc):
    print("dsa_bf16 small", flush=True)
    assert _paged_case(amd, orc, 2, 32, 128, 1024) < 1e-2


def test_dsa_bf16_paged_ragged_s(amd, orc):
    """S not a multiple of the 64-token step: the tail is masked."""
    print("dsa_bf16 ragged", flush=True)
    assert _paged_case(amd, orc, 3, 64, 100, 512, seed=6) < 1e-2
    assert _paged_case(amd, orc, 1, 32, 1, 128, seed=7) < 1e-2


def test_dsa_bf16_paged_baseline_shape(amd, orc):
    """B=64, H=128, S=2048 of 32768-token contexts; 16 of the 64 queries
    checked (every fourth, so both ends and every XCD's share of the grid)."""
    print("dsa_bf16 baseline", flush=True)
    assert _paged_case(amd, orc, 64, 128, 2048, 32768, check_q=list(range(0, 64, 4)) + [63]) < 1e-2


# H a multiple of 128: the token-split kernel (workgroup = query x 128 heads
# x split) plus the merge of the splits; H = 32, 64: one workgroup per
# (query, 32 heads)
@pytest.mark.parametrize("Q,H,S,ctx", [
    (8, 128, 100, 512),     # 4 splits of 32, the last one 4 tokens
    (3, 128, 1, 128),       # one token
    (2, 256, 3000, 4096),   # 2 head groups; 64 splits of 64 tokens, the last 17 empty
    (300, 128, 64, 128),    # one split per query (no token split)
    (64, 128, 512, 1024),   # 4 splits of 4 tiles
    (256, 32, 1, 128),      # 32 heads, one position
    (128, 64, 2047, 4096),  # 64 heads, 64-token tiles, the last one ragged
])
def test_dsa_bf16_paged_split_shapes(amd, orc, Q, H, S, ctx):
    print(f"dsa_bf16 split Q={Q} H={H} S={S}", flush=True)
    check = None if Q <= 8 else [0, Q // 2, Q - 1]
    assert _paged_case(amd, orc, Q, H, S, ctx, check_q=check, seed=Q + S) < 1e-2


def test_dsa_bf16_paged_repeat_calls_bit_identical(amd):
    """Calls of different split counts and head groups in a row (sharing
    the decode's cached scratch of partials), each shape's output
    bit-identical across its calls."""
    import synth
    shapes = [(64, 128, 512, 1024), (8, 128, 100, 512), (2, 256, 3000, 4096), (300, 128, 64, 128)]
    cases = []
    for i, (Q, H, S, ctx) in enumerate(shapes):
        inp = synth.dsa_paged(Q, H, 512, 64, S, 64, ctx, seed=30 + i)
        cfg = amd.dsa_config(Q, H, 512, 64, S, 64, Q * ctx)
        cases.append((inp, cfg, torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")))
    first = []
    for rnd in range(3):
        for i, (inp, cfg, out) in enumerate(cases):
            print(f"dsa_bf16 repeat round {rnd} shape {shapes[i]}", flush=True)
            qn, qp, cache, pt, logical, pps = inp
            out.fill_(-1)
            amd.dsa_decode_bf16_paged(qn, qp, cache, pt, logical, out, cfg, pps)
            torch.cuda.synchronize()
            if rnd == 0:
                first.append(out.clone())
            else:
                assert torch.equal(out, first[i]), shapes[i]


def test_dsa_bf16_paged_split_max_jumps(amd, orc):
    """Scores that jump by more than 8 (log2 units) between tiles of a split:
    the path that rescales O to a raised running max.
    Scores come from q_pe . K_p only (q_nope = 0), values from K_c: in every
    128-token split, tile 1 and tile 3 open with a token whose score is
    9.6 resp. 19.2 above the rest and whose V row is -1 (all other V rows
    +1), so the output depends on every tile's share."""
    import synth
    print("dsa_bf16 split max jumps", flush=True)
    Q, H, S, ctx, page = 64, 128, 512, 1024, 64
    qn, qp, cache, pt, logical, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=9)
    bf = lambda v: torch.tensor(v, dtype=torch.float32).to(torch.bfloat16).view(torch.int16)
    qn = torch.zeros_like(qn)
    qp = bf(1.0).expand(Q, H, 64).contiguous().cuda()
    w = torch.zeros(S)     # K_p value of each selected position
    vv = torch.ones(S)     # K_c (= V) value
    for s0 in range(0, S, 128):  # 4 splits of 4 tiles
        w[s0 + 32], vv[s0 + 32] = 2.5, -1.0   # tile 1: +9.6
        w[s0 + 96], vv[s0 + 96] = 5.0, -1.0   # tile 3: +19.2
    phys = torch.from_numpy(orc.dsa_translate(logical.cpu().numpy(), pt.cpu().numpy(), page)
                            .astype(np.int64)).cuda()          # [Q, S]
    rows = torch.empty((Q, S, 576), dtype=torch.float32)
    rows[:, :, :512] = vv[None, :, None]
    rows[:, :, 512:] = w[None, :, None]
    cache.index_copy_(0, phys.reshape(-1), rows.reshape(-1, 576).to(torch.bfloat16).view(torch.int16).cuda())
    err = _paged_case(amd, orc, Q, H, S, ctx, page=page, check_q=[0, 31, 63],
                      inputs=(qn, qp, cache, pt, logical, pps))
    assert err < 1e-2


def test_dsa_bf16_paged_split_large_jump(amd, orc):
    """A tile max ~96 (log2 units) above the split's first tile max (a
    rescale of O by 2^-96): even heads (q_pe = 1) meet tokens with K_p = 25
    and 24.8 in split 2 (V = -1 and +1, so the output depends on both), odd
    heads (q_pe = 0.1) a jump of ~9.6; every other position has score 0 and
    V = 0.5."""
    import synth
    print("dsa_bf16 split large jump", flush=True)
    Q, H, S, ctx, page = 64, 128, 512, 1024, 64
    qn, qp, cache, pt, logical, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=19)
    qn = torch.zeros_like(qn)
    qpe = torch.where(torch.arange(H) % 2 == 0, 1.0, 0.1)[None, :, None].expand(Q, H, 64)
    qp = qpe.to(torch.bfloat16).view(torch.int16).contiguous().cuda()
    w = torch.zeros(S)
    vv = torch.full((S,), 0.5)
    w[256 + 32], vv[256 + 32] = 25.0, -1.0
    w[256 + 40], vv[256 + 40] = 24.8, 1.0
    phys = torch.from_numpy(orc.dsa_translate(logical.cpu().numpy(), pt.cpu().numpy(), page)
                            .astype(np.int64)).cuda()
    rows = torch.empty((Q, S, 576), dtype=torch.float32)
    rows[:, :, :512] = vv[None, :, None]
    rows[:, :, 512:] = w[None, :, None]
    cache.index_copy_(0, phys.reshape(-1), rows.reshape(-1, 576).to(torch.bfloat16).view(torch.int16).cuda())
    err = _paged_case(amd, orc, Q, H, S, ctx, page=page, check_q=[0, 31, 63],
                      inputs=(qn, qp, cache, pt, logical, pps))
    assert err < 1e-2


# ------------------------------------------------------------------ invalid indices
def _invalid_mix(logical, pt, ctx, page, rng, all_invalid_q=None):
    """Plants the index forms that select nothing: -1 padding at the end of a
    row (as the indexer emits for a sequence shorter than the selection),
    indices at or past the page-table row's capacity, and a page-table entry
    of -1 (an unmapped page) or past the cache's last page under some
    selected positions."""
    lg = logical.copy()
    pt = pt.copy()
    Q, S = lg.shape
    n_pages = pt.size
    for q in range(Q):
        npad = rng.integers(0, max(1, S // 3) + 1)
        if npad:
            lg[q, S - npad:] = -1
        if S > 4:
            lg[q, rng.integers(0, S - npad if S - npad > 0 else 1)] = ctx + rng.integers(0, 5 * page)
        if pt.shape[1] > 1:
            pt[q, rng.integers(0, pt.shape[1])] = -1
            pt[q, rng.integers(0, pt.shape[1])] = n_pages + rng.integers(0, 100)
    if all_invalid_q is not None:
        lg[all_invalid_q, :] = -1
    return lg, pt


@pytest.mark.parametrize("Q,H,S,ctx", [
    (6, 128, 300, 1024),   # the token-split kernel (H % 128 == 0)
    (5, 64, 200, 1024),    # one workgroup per 32 heads, 64-token tiles (S <= 2048)
    (3, 32, 2500, 4096),   # one workgroup per 32 heads, 32-token tiles (S > 2048)
    (64, 128, 300, 1024),  # the token-split kernel at the BASELINE query count (4 splits)
])
def test_dsa_bf16_paged_invalid_indices(amd, orc, Q, H, S, ctx):
    """Selected positions that select nothing take no part in the softmax:
    the output equals attention over the valid positions only (the oracle's
    decode, which leaves them out), and a query with no valid position
    gets 0.  Covers all three decode kernels."""
    import synth
    print(f"dsa_bf16 invalid indices Q={Q} H={H} S={S}", flush=True)
    page = 64
    qn, qp, cache, pt, logical, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=Q * 7 + S)
    rng = np.random.default_rng(S)
    lg, ptn = _invalid_mix(logical.cpu().numpy(), pt.cpu().numpy(), ctx, page, rng, all_invalid_q=1)
    out = torch.full((Q, H, 512), 0x7fc0, dtype=torch.int16, device="cuda")
    amd.dsa_decode_bf16_paged(qn, qp, cache, dev(ptn), dev(lg), out,
                              amd.dsa_config(Q, H, 512, 64, S, page, cache.shape[0]), pps)
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy().view(np.uint16)
    ref = orc.dsa_decode_bf16_paged(h(qn), h(qp), h(cache), ptn, lg, 512, page)
    got = orc.bf16_to_f32(h(out))
    assert np.isfinite(got).all()
    assert (got[1] == 0).all()
    err = np.abs(got - ref).max()
    print(f"invalid indices H={H}: max_err={err:.3e}")
    assert err < 1e-2


def test_dsa_bf16_paged_invalid_matches_compacted(amd):
    """GPU against GPU: a row with invalid positions interleaved gives the
    same output as the row holding only its valid positions (padded with -1
    at the end), on the split kernel."""
    import synth
    print("dsa_bf16 invalid == compacted", flush=True)
    Q, H, S, ctx, page = 4, 128, 256, 2048, 64
    qn, qp, cache, pt, logical, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=77)
    lg = logical.cpu().numpy()
    holes = lg.copy()
    holes[:, ::3] = -1
    comp = np.full_like(lg, -1)
    for q in range(Q):
        v = holes[q][holes[q] >= 0]
        comp[q, :len(v)] = v
    cfg = amd.dsa_config(Q, H, 512, 64, S, page, cache.shape[0])
    o1 = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    o2 = torch.empty_like(o1)
    amd.dsa_decode_bf16_paged(qn, qp, cache, pt, dev(holes), o1, cfg, pps)
    amd.dsa_decode_bf16_paged(qn, qp, cache, pt, dev(comp), o2, cfg, pps)
    torch.cuda.synchronize()
    a = o1.cpu().numpy().view(np.uint16)
    b = o2.cpu().numpy().view(np.uint16)
    # different tile/split boundaries: equal to bf16 rounding of fp32 sums
    import oracle
    d = np.abs(oracle.bf16_to_f32(a) - oracle.bf16_to_f32(b)).max()
    assert d < 1e-2


def test_dsa_f32_invalid_indices(amd, orc):
    """dsa_forward_f32: an index outside [0, N) selects nothing; the result
    equals the reference computation on the valid indices only (in order)
    within the reference-case bar (1e-6; device expf vs glibc expf), is
    bit-identical to the same entry called with only the valid indices, and
    a query with none gets 0."""
    Q, H, Dc, Dp, S, N = 4, 8, 64, 16, 96, 512
    print("dsa_f32 invalid indices", flush=True)
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(Q, H, Dc, Dp, S, 64, N)
    idx = idx.copy()
    idx[0, ::5] = -1
    idx[2, 7] = N
    idx[2, 40] = N + 1000
    idx[3, :] = -3
    out = torch.full((Q, H, Dc), float("nan"), dtype=torch.float32, device="cuda")
    amd.dsa_forward_f32(dev(qn), dev(qp), dev(kc), dev(kp), dev(v), dev(idx), out,
                        amd.dsa_config(Q, H, Dc, Dp, S, 64, N))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for q in range(Q):
        valid = idx[q][(idx[q] >= 0) & (idx[q] < N)]
        if len(valid) == 0:
            assert (got[q] == 0).all()
            continue
        vi = valid[None, :].astype(np.int32)
        ref = orc.dsa_forward_f32(qn[q:q + 1], qp[q:q + 1], kc, kp, v, vi)
        assert np.abs(got[q] - ref[0]).max() < 1e-6
        one = torch.empty((1, H, Dc), dtype=torch.float32, device="cuda")
        amd.dsa_forward_f32(dev(qn[q:q + 1]), dev(qp[q:q + 1]), dev(kc), dev(kp), dev(v), dev(vi), one,
                            amd.dsa_config(1, H, Dc, Dp, vi.shape[1], 64, N))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[q], one.cpu().numpy()[0])


def test_dsa_f32_beyond_lds_s20000(amd, orc):
    """S = 20000 selected rows (past what one workgroup's LDS holds; the
    scores go through scratch) with Dc = 48, Dp = 8: equal to the oracle
    within the reference-case bar (1e-6)."""
    Q, H, Dc, Dp, S, N = 2, 3, 48, 8, 20000, 30000
    print("dsa_f32 S=20000", flush=True)
    rng = np.random.default_rng(20000)
    qn = rng.uniform(-0.3, 0.3, (Q, H, Dc)).astype(np.float32)
    qp = rng.uniform(-0.3, 0.3, (Q, H, Dp)).astype(np.float32)
    kc = rng.uniform(-0.3, 0.3, (N, Dc)).astype(np.float32)
    kp = rng.uniform(-0.3, 0.3, (N, Dp)).astype(np.float32)
    v = rng.uniform(-0.3, 0.3, (N, Dc)).astype(np.float32)
    idx = np.stack([np.sort(rng.choice(N, S, replace=False)) for _ in range(Q)]).astype(np.int32)
    ref = orc.dsa_forward_f32(qn, qp, kc, kp, v, idx)
    out = torch.full((Q, H, Dc), float("nan"), dtype=torch.float32, device="cuda")
    amd.dsa_forward_f32(dev(qn), dev(qp), dev(kc), dev(kp), dev(v), dev(idx), out,
                        amd.dsa_config(Q, H, Dc, Dp, S, 64, N))
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy() - ref).max()
    print(f"S=20000: max_err={err:.3e}")
    assert err < 1e-6


def test_dsa_bf16_paged_cache_beyond_4gib(amd, orc):
    """A latent cache of 4.6 GB (beyond the 32-bit offsets of a buffer
    descriptor): half of each query's pages lie above 4 GiB.  The split
    kernel's 64-bit-address variant matches the oracle, and is bit-identical
    to the 32-bit-offset kernel on a compacted copy of the same pages."""
    Q, H, S, page, pps = 2, 128, 512, 64, 64
    N = 4_000_000                                    # cache tokens (4.6 GB)
    print(f"dsa_bf16 cache of {N} tokens ({N * 1152 / 2**30:.2f} GiB)", flush=True)
    rng = np.random.default_rng(4)
    n_pages = N // page
    hi0 = (1 << 32) // (page * 1152) + 1             # first page wholly above 4 GiB
    pages = np.concatenate([rng.choice(hi0, Q * pps // 2, replace=False),
                            rng.choice(np.arange(hi0, n_pages), Q * pps // 2, replace=False)])
    rng.shuffle(pages)
    pt = pages.reshape(Q, pps).astype(np.int32)
    cache = torch.empty((N, 576), dtype=torch.int16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(11)
    rows = torch.from_numpy((pages[:, None] * page + np.arange(page)[None, :]).reshape(-1)).cuda()
    vals = torch.randn((rows.numel(), 576), generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    cache.index_copy_(0, rows, vals)
    logical = np.stack([rng.permutation(pps * page)[:S] for _ in range(Q)]).astype(np.int32)
    qn = torch.randn((Q, H, 512), generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    qp = torch.randn((Q, H, 64), generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    inputs = (qn, qp, cache, dev(pt), dev(logical), pps)
    err = _paged_case(amd, orc, Q, H, S, N // Q, page=page, inputs=inputs)
    assert err < 2e-2
    # the same pages compacted into a cache below 4 GiB: the 32-bit kernel
    out_w = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    amd.dsa_decode_bf16_paged(qn, qp, cache, dev(pt), dev(logical), out_w,
                              amd.dsa_config(Q, H, 512, 64, S, page, N), pps)
    small = cache.index_select(0, rows).contiguous()
    del cache
    pt_small = np.arange(Q * pps, dtype=np.int32).reshape(Q, pps)
    out_s = torch.empty_like(out_w)
    amd.dsa_decode_bf16_paged(qn, qp, small, dev(pt_small), dev(logical), out_s,
                              amd.dsa_config(Q, H, 512, 64, S, page, small.shape[0]), pps)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out_w.cpu().numpy(), out_s.cpu().numpy())


def test_dsa_bf16_paged_long_selection(amd, orc):
    """H = 128 with 10000 selected positions per query (beyond the 4096 that
    the one-workgroup-per-query kernels hold): more splits, same result."""
    print("dsa_bf16 S=10000", flush=True)
    assert _paged_case(amd, orc, 2, 128, 10000, 16384) < 2e-2
