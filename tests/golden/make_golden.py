"""Writes tests/golden/reference_cases.npz: the CPU oracle's results on the
reference's own 13 MoE and 14 DSA test cases (tests/test_moe.cu:204-267,
tests/test_dsa.cu:162-230), whose inputs are regenerated bit-identically by
glibc rand() (srand(42), utils/cuda_utils.cuh:56-60).

The reference ships no golden vectors and its CPU oracle cannot be built in
this image (it lives in CUDA translation units), so these fixtures are the
oracle restatement's outputs, frozen: they pin it against drift (checked by
tests/test_golden.py) and give the GPU path a fixture to meet.  Stored per
case: sha256 of the generated inputs, of the output, of the routing, the
routing itself (MoE: expert indices and weights, T x K) and the first rows of
the output.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle  # noqa: E402
from cases import DSA_CASES, MOE_CASES  # noqa: E402

HEAD_ROWS = 2


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def moe_case(shape):
    T, E, K, D, I = shape
    x, wg, w1, w2 = oracle.reference_moe_inputs(T, E, K, D, I)
    idx, wts, y = oracle.moe_forward_f32(x, wg, w1, w2, K)
    return {"in_sha": sha(x, wg, w1, w2), "out_sha": sha(y), "route_sha": sha(idx, wts),
            "idx": idx, "wts": wts, "head": y[:HEAD_ROWS].copy()}


def dsa_case(shape):
    Q, H, Dc, Dp, S, P, N = shape
    qn, qp, kc, kp, v, idx = oracle.reference_dsa_inputs(Q, H, Dc, Dp, S, P, N)
    out = oracle.dsa_forward_f32(qn, qp, kc, kp, v, idx)
    return {"in_sha": sha(qn, qp, kc, kp, v, idx), "out_sha": sha(out), "idx": idx,
            "head": out[0, :HEAD_ROWS].copy()}


def build():
    data = {}
    for name, shape, _ in MOE_CASES:
        for k, v in moe_case(shape).items():
            data[f"moe/{name}/{k}"] = np.asarray(v)
    for name, shape, _ in DSA_CASES:
        for k, v in dsa_case(shape).items():
            data[f"dsa/{name}/{k}"] = np.asarray(v)
    return data


if __name__ == "__main__":
    oracle.lib()
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_cases.npz")
    np.savez_compressed(out, **build())
    print(f"wrote {out} ({os.path.getsize(out)} bytes)")
