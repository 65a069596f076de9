"""GPU parity of the reference's DSA stage functions (naive_dsa.cuh:31-68)
through the C ABI, against the oracle's restatement of their kernels.

The gather, the three dot products and the output projection form every
value in the reference kernel's order with plain binary32 products and sums,
as the oracle does, so they must match it bit for bit.  The softmax uses the
device expf, so it is held to a few ulp of the oracle (glibc expf).
"""
import math

import numpy as np
import pytest
import torch

from cases import DSA_CASES

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _inputs(shape, seed):
    Q, H, Dc, Dp, S, P, N = shape
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    idx = np.stack([rng.permutation(N)[:S] for _ in range(Q)]).astype(np.int32)
    return f(Q, H, Dc), f(Q, H, Dp), f(N, Dc), f(N, Dp), f(N, Dc), idx


# the reference's DSA matrix, plus shapes off the fast paths (Dc and Dp not
# multiples of 4, Dp = 0, S and H not multiples of the tiles) and a
# BASELINE-sized head/latent geometry
STAGE_CASES = [(n, s) for n, s, _ in DSA_CASES] + [
    ("ragged", (3, 37, 70, 5, 77, 8, 300)),
    ("no-Dp", (2, 8, 64, 0, 40, 8, 128)),
    ("mla", (2, 128, 512, 64, 512, 64, 4096)),
]


@pytest.mark.parametrize("name,shape", STAGE_CASES, ids=[c[0] for c in STAGE_CASES])
def test_dsa_stages_bit_identical(amd, orc, name, shape):
    Q, H, Dc, Dp, S, P, N = shape
    print(f"dsa_stages {name} {shape}", flush=True)
    qn, qp, kc, kp, v, idx = _inputs(shape, seed=11)
    cfg = amd.dsa_config(Q, H, Dc, Dp, S, P, N)
    # gather
    ref_kc, ref_kp, ref_v = orc.dsa_kv_gather(kc, kp, v, idx)
    g = [torch.full(a.shape, float("nan"), device="cuda") for a in (ref_kc, ref_kp, ref_v)]
    amd.dsa_kv_gather_f32(dev(kc), dev(kp), dev(v), dev(idx), *g, cfg)
    torch.cuda.synchronize()
    for got, ref in zip(g, (ref_kc, ref_kp, ref_v)):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)
    # dots, accumulated into nonzero scores
    init = np.random.default_rng(12).standard_normal((Q, H, S)).astype(np.float32)
    for parts, fn, args in (
        (1, amd.dsa_dot_compressed_f32, (dev(qn), g[0])),
        (2, amd.dsa_dot_positional_f32, (dev(qp), g[1])),
        (3, amd.dsa_dot_fused_f32, (dev(qn), dev(qp), g[0], g[1])),
    ):
        ref = orc.dsa_dot(qn if parts & 1 else None, qp if parts & 2 else None,
                          ref_kc if parts & 1 else None, ref_kp if parts & 2 else None, init, parts)
        sc = dev(init)
        fn(*args, sc, cfg)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(sc.cpu().numpy(), ref, err_msg=f"parts={parts}")
    # softmax of the scaled fused scores, then the output projection
    s = orc.dsa_dot(qn, qp, ref_kc, ref_kp, np.zeros((Q, H, S), np.float32), 3)
    s = (s * np.float32(1.0 / math.sqrt(Dc + Dp))).astype(np.float32)
    ref_p = orc.dsa_softmax(s)
    p = dev(s)
    amd.dsa_softmax_f32(p, cfg)
    torch.cuda.synchronize()
    got_p = p.cpu().numpy()
    ulp = np.abs(got_p.view(np.int32).astype(np.int64) - ref_p.view(np.int32).astype(np.int64))
    print(f"{name}: softmax max ulp {ulp.max()}")
    assert ulp.max() <= 4
    out = torch.full((Q, H, Dc), float("nan"), device="cuda")
    amd.dsa_output_proj_f32(dev(ref_p), g[2], out, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), orc.dsa_output_proj(ref_p, ref_v))


def test_dsa_stages_compose_to_forward(amd, orc):
    # the reference's dsa_forward (naive_dsa.cu:435-474) built from the
    # stages on the GPU == this library's fused dsa_forward
    shape = (4, 4, 128, 32, 256, 64, 1024)
    Q, H, Dc, Dp, S, P, N = shape
    qn, qp, kc, kp, v, idx = orc.reference_dsa_inputs(*shape)
    cfg = amd.dsa_config(*shape)
    gkc = torch.empty((Q, S, Dc), device="cuda")
    gkp = torch.empty((Q, S, Dp), device="cuda")
    gv = torch.empty((Q, S, Dc), device="cuda")
    amd.dsa_kv_gather_f32(dev(kc), dev(kp), dev(v), dev(idx), gkc, gkp, gv, cfg)
    sc = torch.zeros((Q, H, S), device="cuda")
    amd.dsa_dot_fused_f32(dev(qn), dev(qp), gkc, gkp, sc, cfg)
    sc *= 1.0 / math.sqrt(Dc + Dp)
    amd.dsa_softmax_f32(sc, cfg)
    out = torch.empty((Q, H, Dc), device="cuda")
    amd.dsa_output_proj_f32(sc, gv, out, cfg)
    fused = torch.empty((Q, H, Dc), device="cuda")
    amd.dsa_forward_f32(dev(qn), dev(qp), dev(kc), dev(kp), dev(v), dev(idx), fused, cfg)
    torch.cuda.synchronize()
    err = (out - fused).abs().max().item()
    print(f"composed vs fused: max_err={err:.3e}")
    assert err < 1e-5


def test_dsa_gather_out_of_range_rows_are_zero(amd, orc):
    Q, H, Dc, Dp, S, P, N = 2, 1, 64, 8, 6, 8, 32
    qn, qp, kc, kp, v, idx = _inputs((Q, H, Dc, Dp, S, P, N), seed=3)
    idx[0, 2] = -1
    idx[1, 4] = N
    g = [torch.full((Q, S, d), float("nan"), device="cuda") for d in (Dc, Dp, Dc)]
    amd.dsa_kv_gather_f32(dev(kc), dev(kp), dev(v), dev(idx), *g, amd.dsa_config(Q, H, Dc, Dp, S, P, N))
    torch.cuda.synchronize()
    ok = (idx >= 0) & (idx < N)
    safe = np.where(ok, idx, 0)
    for got, src in zip(g, (kc, kp, v)):
        exp = np.where(ok[:, :, None], src[safe], 0.0).astype(np.float32)
        np.testing.assert_array_equal(got.cpu().numpy(), exp)
