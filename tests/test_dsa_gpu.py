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


def _paged_case(amd, orc, Q, H, S, ctx, page=64, check_q=None, seed=5):
    import synth
    qn, qp, cache, pt, logical, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=seed)
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
