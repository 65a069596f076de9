"""The frozen fixtures of tests/golden/reference_cases.npz (written by
tests/golden/make_golden.py from the reference's own 13 MoE and 14 DSA cases).

CPU: the oracle reproduces every fixture bit for bit (inputs, routing,
outputs), so a change to the oracle or to the glibc-rand input generation
cannot go unnoticed.  GPU: the HIP path meets the fixtures -- expert indices
of the fp32 gate bit-identical, routing weights within a few ulp (device
expf against glibc's, both within their documented error), outputs within
the reference's tolerances (strict <)."""
import os

import numpy as np
import pytest

from cases import DSA_CASES, MOE_CASES

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_cases.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.fixture(scope="module")
def make(orc):
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(GOLDEN), "make_golden.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


@pytest.mark.parametrize("name,shape,tol", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_oracle_reproduces_moe_fixture(gold, make, name, shape, tol):
    got = make.moe_case(shape)
    for k in ("in_sha", "route_sha", "out_sha"):
        assert str(gold[f"moe/{name}/{k}"]) == got[k], k
    np.testing.assert_array_equal(gold[f"moe/{name}/idx"], got["idx"])
    np.testing.assert_array_equal(gold[f"moe/{name}/head"], got["head"])


@pytest.mark.parametrize("name,shape,tol", DSA_CASES, ids=[c[0] for c in DSA_CASES])
def test_oracle_reproduces_dsa_fixture(gold, make, name, shape, tol):
    got = make.dsa_case(shape)
    for k in ("in_sha", "out_sha"):
        assert str(gold[f"dsa/{name}/{k}"]) == got[k], k
    np.testing.assert_array_equal(gold[f"dsa/{name}/head"], got["head"])


def test_fixture_known_answers(gold):
    """Properties the fixtures must have whatever produced them: weights of
    each token sum to 1; the single-expert case routes everything to expert
    0 with weight 1; full routing (K = E) lists every expert once."""
    for name, (T, E, K, D, I), _ in MOE_CASES:
        wts = gold[f"moe/{name}/wts"]
        np.testing.assert_allclose(wts.sum(1), 1.0, rtol=1e-6)
    assert (gold["moe/single-expert/idx"] == 0).all()
    np.testing.assert_array_equal(gold["moe/single-expert/wts"], 1.0)
    idx = gold["moe/full-routing/idx"]
    assert all(sorted(r) == [0, 1, 2, 3] for r in idx)


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,tol", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_gpu_meets_moe_fixture(amd, orc, gold, name, shape, tol):
    import torch
    T, E, K, D, I = shape
    print(f"golden moe {name} {shape}", flush=True)
    x, wg, w1, w2 = orc.reference_moe_inputs(T, E, K, D, I)
    cfg = amd.moe_config(T, E, K, D, I)
    dx, dwg = torch.from_numpy(x).cuda(), torch.from_numpy(wg).cuda()
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amd.moe_gate_f32(dx, dwg, idx, wts, cfg)
    y = torch.full((T, D), float("nan"), dtype=torch.float32, device="cuda")
    amd.moe_forward_f32(dx, dwg, torch.from_numpy(w1).cuda(), torch.from_numpy(w2).cuda(), y, cfg)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy(), gold[f"moe/{name}/idx"])
    np.testing.assert_allclose(wts.cpu().numpy(), gold[f"moe/{name}/wts"], rtol=2e-6, atol=0)
    head = gold[f"moe/{name}/head"]
    assert np.abs(y.cpu().numpy()[:head.shape[0]] - head).max() < tol


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,tol", DSA_CASES, ids=[c[0] for c in DSA_CASES])
def test_gpu_meets_dsa_fixture(amd, orc, gold, name, shape, tol):
    import torch
    Q, H, Dc, Dp, S, P, N = shape
    print(f"golden dsa {name} {shape}", flush=True)
    arrs = orc.reference_dsa_inputs(Q, H, Dc, Dp, S, P, N)
    out = torch.full((Q, H, Dc), float("nan"), dtype=torch.float32, device="cuda")
    amd.dsa_forward_f32(*(torch.from_numpy(a).cuda() for a in arrs), out,
                        amd.dsa_config(Q, H, Dc, Dp, S, P, N))
    torch.cuda.synchronize()
    head = gold[f"dsa/{name}/head"]
    assert np.abs(out.cpu().numpy()[0, :head.shape[0]] - head).max() < tol
