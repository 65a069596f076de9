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
    """B=64, H=128, S=2048 of 32768-token contexts; 4 queries checked."""
    print("dsa_bf16 baseline", flush=True)
    assert _paged_case(amd, orc, 64, 128, 2048, 32768, check_q=[0, 17, 42, 63]) < 1e-2


# H a multiple of 128: the token-split kernel (workgroup = query x 128 heads
# x split) plus the merge of the splits
@pytest.mark.parametrize("Q,H,S,ctx", [
    (8, 128, 100, 512),    # 4 splits of 32, the last one 4 tokens
    (3, 128, 1, 128),      # one token
    (2, 256, 3000, 4096),  # 2 head groups; 64 splits of 64 tokens, the last 17 empty
    (300, 128, 64, 128),   # one split per query (no token split)
    (64, 128, 512, 1024),  # 4 splits of 4 tiles
])
def test_dsa_bf16_paged_split_shapes(amd, orc, Q, H, S, ctx):
    print(f"dsa_bf16 split Q={Q} H={H} S={S}", flush=True)
    check = None if Q <= 8 else [0, Q // 2, Q - 1]
    assert _paged_case(amd, orc, Q, H, S, ctx, check_q=check, seed=Q + S) < 1e-2


def test_dsa_bf16_paged_split_max_jumps(amd, orc):
    """Scores that jump by more than 8 (log2 units) between tiles of a split:
    the path that moves O out of the accumulators and rescales it in memory.
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
