"""The activation quantisers divide a block's values by its scale with one
correctly rounded reciprocal per block and one FMA correction per value
(div_rn in csrc/common.hpp): q0 = RN(v r), q = RN(q0 + RN(v - s q0) r),
r = RN(1/s).  Markstein's theorem makes q the correctly rounded quotient;
this checks the identity against IEEE fp32 division on bf16 values and
block scales s = RN(amax/448) >= 2^-64 (the range where the kernels take
it), with the FMA's single rounding computed exactly."""
import numpy as np


def _bf16(x):
    u = x.astype(np.float32).view(np.uint32)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.view(np.float32)


def test_reciprocal_with_fma_correction_is_the_rounded_quotient():
    rng = np.random.default_rng(20261202)
    f32 = np.float32
    checked = 0
    for lo, hi, span in ((-30, 30, 12), (-60, -40, 40), (-8, 8, 1)):
        n = 400_000
        v = _bf16((rng.standard_normal(n) * np.exp2(rng.uniform(lo, hi, n))).astype(np.float32))
        fac = np.where(rng.random(n) < 0.1, 1.0, np.exp2(rng.uniform(0, span, n)))
        amax = np.maximum(_bf16(np.abs(v).astype(np.float64) * fac), np.abs(v))
        keep = (amax > 0) & (amax / 448 >= 2.0 ** -64)
        v, amax = v[keep], amax[keep]
        s = (amax / f32(448.0)).astype(np.float32)
        r = (f32(1.0) / s).astype(np.float32)
        q0 = (v * r).astype(np.float32)
        # RN(v - s q0): s q0 is exact in fp64 and the difference is exact
        # (Sterbenz: v and s q0 are within a factor of two)
        res = (v.astype(np.float64) - s.astype(np.float64) * q0.astype(np.float64)).astype(np.float32)
        t = res.astype(np.float64) * r.astype(np.float64)  # exact
        tot = q0.astype(np.float64) + t
        q = tot.astype(np.float32)
        # the fp64 sum is exact unless its two-sum error is nonzero; a second
        # rounding can then only differ on an exact fp32 midpoint
        err = t - (tot - q0.astype(np.float64))
        half = np.abs(np.spacing(q)).astype(np.float64) / 2
        assert not np.any((err != 0) & (np.abs(tot - q.astype(np.float64)) == half))
        np.testing.assert_array_equal(q, (v / s).astype(np.float32))
        checked += v.size
    assert checked > 1_000_000
