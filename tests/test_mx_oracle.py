"""The oracle's OCP Microscaling (MX) codec and MXFP4 layer, pinned on the CPU.

The MX formats have no counterpart in the reference (fp32 only); the
oracle restates the OCP MX specification v1.0 and these checks pin it: the
E2M1 element table against the specification's value list, every E8M0 code
against 2^(E-127), E2M1 round-to-nearest-even against a brute-force nearest
search with ties to the even mantissa, the block conversion's shared
exponent (floor(log2 max|v|) - emax_elem) on known answers, the nibble
packing, and the MXFP4 layer against a float64 numpy restatement."""
import numpy as np
import pytest

E2M1_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]   # OCP MX v1.0, FP4 E2M1


def test_e2m1_table_is_the_specification_list(orc):
    got = [orc.e2m1_to_f32(c) for c in range(16)]
    assert got[:8] == E2M1_VALUES
    assert got[8:] == [-v for v in E2M1_VALUES]
    assert np.signbit(got[8])


def test_e8m0_every_code(orc):
    for c in range(255):
        assert orc.e8m0_to_f32(c) == np.ldexp(np.float32(1.0), c - 127)
    assert np.isnan(orc.e8m0_to_f32(255))


def test_e2m1_encode_round_trip_and_rne(orc):
    for c in range(16):
        assert orc.f32_to_e2m1_scalar(orc.e2m1_to_f32(c)) == c
    vals = np.array(E2M1_VALUES)
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-7, 7, 4000), np.arange(-6.5, 6.75, 0.25)]).astype(np.float32)
    for x in xs:
        a = abs(float(x))
        d = np.abs(vals - a)
        best = np.flatnonzero(d == d.min())
        if a >= 6.0:
            want = 7
        elif len(best) == 1:
            want = int(best[0])
        else:                     # a tie: the code with the even mantissa bit
            want = int([b for b in best if b % 2 == 0][0])
        want |= 8 if np.signbit(x) else 0
        assert orc.f32_to_e2m1_scalar(x) == want, x


@pytest.mark.parametrize("bits,emax,top", [(4, 2, 6.0), (8, 8, 448.0)])
def test_block_shared_exponent_known_answers(orc, bits, emax, top):
    # all 1.0: shared exponent 0 - emax, elements 2^emax
    q, s = orc.mx_quant_rows(np.ones((1, 32), np.float32), bits)
    assert s[0, 0] == 127 - emax
    deq = orc.mx_dequant_rows(q, s, bits)
    np.testing.assert_array_equal(deq, 1.0)
    # max exactly the element format's largest normal: scale 1, values kept
    x = np.zeros((1, 32), np.float32)
    x[0, 5] = top
    x[0, 9] = -top / 2
    q, s = orc.mx_quant_rows(x, bits)
    assert s[0, 0] == 127
    np.testing.assert_array_equal(orc.mx_dequant_rows(q, s, bits), x)
    # all zero: E = 0, elements 0
    q, s = orc.mx_quant_rows(np.zeros((2, 64), np.float32), bits)
    assert (s == 0).all() and (q == 0).all()
    # scaling by 2^k moves only the scale
    rng = np.random.default_rng(bits)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    q0, s0 = orc.mx_quant_rows(x, bits)
    q1, s1 = orc.mx_quant_rows(x * np.float32(2.0 ** 11), bits)
    np.testing.assert_array_equal(q0, q1)
    np.testing.assert_array_equal(s1.astype(int), s0.astype(int) + 11)


@pytest.mark.parametrize("bits", [4, 8])
def test_block_conversion_matches_spec_restatement(orc, bits):
    """Every element is the format's RNE of v / X with X = 2^(floor(log2
    max|v|) - emax), saturated; numpy restatement with the oracle's own
    scalar encoders only for the final rounding (pinned above)."""
    rng = np.random.default_rng(7 + bits)
    x = (rng.standard_normal((8, 128)) * np.exp2(rng.integers(-20, 20, (8, 1)))).astype(np.float32)
    x[2, :32] = 0.0
    q, s = orc.mx_quant_rows(x, bits)
    emax = 2 if bits == 4 else 8
    for r in range(8):
        for b in range(4):
            blk = x[r, 32 * b:32 * b + 32]
            amax = np.abs(blk).max()
            e8 = 0 if amax == 0 else int(np.clip(np.floor(np.log2(amax)) - emax + 127, 0, 254))
            assert s[r, b] == e8
            v = blk * np.float32(2.0 ** (127 - e8))
            for j in range(32):
                c = orc.f32_to_e2m1_scalar(v[j]) if bits == 4 else orc.f32_to_e4m3_scalar(v[j])
                i = 32 * b + j
                got = (q[r, i // 2] >> (4 * (i & 1))) & 15 if bits == 4 else q[r, i]
                assert got == c


def test_fp4_nibble_packing(orc):
    x = np.zeros((1, 32), np.float32)
    x[0, 0], x[0, 1], x[0, 30], x[0, 31] = 0.5, 1.0, -3.0, 6.0
    q, s = orc.mx_quant_rows(x, 4)
    assert s[0, 0] == 127                   # max 6 -> floor(log2 6) - 2 = 0
    assert q[0, 0] == (2 << 4) | 1          # element 0 low nibble, element 1 high
    assert q[0, 15] == (7 << 4) | (8 | 5)


def _mx_deq(orc, q, s, bits):
    rows = q.shape[0] * (q.shape[1] if q.ndim == 3 else 1)
    return orc.mx_dequant_rows(q.reshape(rows, -1), s.reshape(rows, -1), bits)


def test_mxfp4_layer_matches_float64_restatement(orc):
    """Routing as the fp8 layer; x and the SwiGLU output as MXFP8 (the oracle's
    own quantiser, pinned above), weights dequantised from MXFP4; the FFNs
    and the ascending-expert weighted sum in float64."""
    rng = np.random.default_rng(3)
    T, E, K, D, I = 24, 6, 2, 64, 96
    xb = orc.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    wgb = orc.f32_to_bf16((rng.standard_normal((E, D)) / 8).astype(np.float32))
    w1 = (rng.standard_normal((E, 2 * I, D)) / 8).astype(np.float32)
    w2 = (rng.standard_normal((E, D, I)) / 10).astype(np.float32)
    w1q, w1s = orc.mx_quant_rows(w1.reshape(-1, D), 4)
    w2q, w2s = orc.mx_quant_rows(w2.reshape(-1, I), 4)
    w1q, w1s = w1q.reshape(E, 2 * I, D // 2), w1s.reshape(E, 2 * I, D // 32)
    w2q, w2s = w2q.reshape(E, D, I // 2), w2s.reshape(E, D, I // 32)
    idx, wts, y = orc.moe_forward_mxfp4(xb, wgb, w1q, w1s, w2q, w2s, K)
    idx_r, wts_r = orc.moe_route(orc.bf16_to_f32(xb), orc.bf16_to_f32(wgb), K)
    np.testing.assert_array_equal(idx, idx_r)
    xq, xs = orc.mx_quant_rows(orc.bf16_to_f32(xb), 8)
    xd = orc.mx_dequant_rows(xq, xs, 8).astype(np.float64)
    W1 = orc.mx_dequant_rows(w1q.reshape(-1, D // 2), w1s.reshape(-1, D // 32), 4).reshape(E, 2 * I, D)
    W2 = orc.mx_dequant_rows(w2q.reshape(-1, I // 2), w2s.reshape(-1, I // 32), 4).reshape(E, D, I)
    ref = np.zeros((T, D))
    for t in range(T):
        for e in sorted(set(idx[t].tolist())):
            h = W1[e].astype(np.float64) @ xd[t]
            a = h[:I] / (1 + np.exp(-h[:I])) * h[I:]
            aq, as_ = orc.mx_quant_rows(a.astype(np.float32)[None, :], 8)
            a = orc.mx_dequant_rows(aq, as_, 8)[0].astype(np.float64)
            ref[t] += wts[t, list(idx[t]).index(e)] * (W2[e].astype(np.float64) @ a)
    # the oracle rounds each sum in fp32 (measured 6e-8 of max |y| here; an
    # MXFP8 code moved by that rounding would show as ~1e-3)
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()
