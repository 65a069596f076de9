"""GPU parity of the MXFP4 expert layer (OCP MX: E2M1 weights and E4M3
activations with E8M0 scales per 32 along K), through the C ABI, against
the oracle's restatement of the OCP MX specification (tests/test_mx_oracle.py
pins it).  No counterpart in the reference (fp32 only; its roadmap names
NVFP4 experts, whose AMD analogue this is).

Bars: quantiser codes and scales bit-exact; the fragment packing equal to a
numpy restatement; the layer within 2e-2 relative (max-abs error over
max |y|) of the oracle on the same dequantised values."""
import numpy as np
import pytest
import torch

from test_moe_gpu import ROUTED_COUNTS, _routed_layout, _routing_columns, announce, bf16_np, dev, host

pytestmark = pytest.mark.gpu


def _wide(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    x *= np.exp2(rng.integers(-12, 13, (shape[0], 1))).astype(np.float32)
    return x


@pytest.mark.parametrize("rows,cols", [(64, 512), (7, 96), (3, 7168)])
def test_quant_weight_mxfp4_bit_exact(amd, orc, rows, cols):
    rng = np.random.default_rng(rows * cols)
    w = _wide(rng, (rows, cols))
    w[0, :32] = 0.0                                   # zero block
    w[1, 32:64] = np.float32(6.0)                     # block max exactly 6
    w[-1, -32:] *= np.float32(2.0 ** -130)            # E8M0 clamp at 0 (subnormal fp32)
    q_ref, s_ref = orc.mx_quant_rows(w, 4)
    q = torch.empty((rows, cols // 2), dtype=torch.uint8, device="cuda")
    s = torch.empty((rows, cols // 32), dtype=torch.uint8, device="cuda")
    amd.quant_weight_mxfp4(dev(w), q, s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), s_ref)
    np.testing.assert_array_equal(host(q), q_ref)


@pytest.mark.parametrize("rows,cols", [(37, 512), (1, 7168), (64, 2048)])
def test_quant_rows_mxfp8_bit_exact(amd, orc, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = orc.f32_to_bf16(_wide(rng, (rows, cols)))
    xf = orc.bf16_to_f32(x)
    q_ref, s_ref = orc.mx_quant_rows(xf, 8)
    q = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    s = torch.empty((rows, cols // 32), dtype=torch.uint8, device="cuda")
    amd.quant_rows_mxfp8(dev(x), q, s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), s_ref)
    np.testing.assert_array_equal(host(q), q_ref)


def _pack_np(q, s):
    """Fragment order restated: block (e, n16, kb) holds at [lane 16g + r]
    the 16 code bytes 64kb + 16g.. of row 16n16 + r, and its scale byte
    4kb + g."""
    E, N, K2 = q.shape
    K = 2 * K2
    qb = q.reshape(E, N // 16, 16, K // 128, 4, 16)          # e, n16, r, kb, g, byte
    qp = qb.transpose(0, 1, 3, 4, 2, 5).reshape(E, N, K2)
    sb = s.reshape(E, N // 16, 16, K // 128, 4)              # e, n16, r, kb, g
    sp = sb.transpose(0, 1, 3, 4, 2).reshape(E, N, K // 32)
    return np.ascontiguousarray(qp), np.ascontiguousarray(sp)


def test_pack_weights_mxfp4_format(amd):
    rng = np.random.default_rng(5)
    E, N, K = 3, 48, 384
    q = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    s = rng.integers(0, 256, (E, N, K // 32), dtype=np.uint8)
    qp = torch.empty_like(dev(q))
    sp = torch.empty_like(dev(s))
    amd.pack_weights_mxfp4(dev(q), dev(s), qp, sp)
    torch.cuda.synchronize()
    rq, rs = _pack_np(q, s)
    np.testing.assert_array_equal(host(qp), rq)
    np.testing.assert_array_equal(host(sp), rs)
    # lane 17 of block (0, 0, 1): row 1, code bytes 64 + 16 .. +15, scale 4 + 1
    assert np.array_equal(host(qp)[0].reshape(-1)[1024 + 17 * 16:][:16], q[0, 1, 80:96])
    assert host(sp)[0].reshape(-1)[64 + 17] == s[0, 1, 5]


def _mx_case(amd, orc, weights, x, wg, K, sample=None):
    """weights: row-major (w1q, w1s, w2q, w2s) device tensors; x, wg bf16 bit
    views on the device.  Packs, runs the forward, checks `sample` rows."""
    w1q, w1s, w2q, w2s = weights
    T, D = x.shape
    E = wg.shape[0]
    I = w2q.shape[2] * 2
    packed = []
    for q, s in ((w1q, w1s), (w2q, w2s)):
        qp, sp = torch.empty_like(q), torch.empty_like(s)
        amd.pack_weights_mxfp4(q, s, qp, sp)
        packed += [qp, sp]
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")
    amd.moe_forward_mxfp4(x, wg, *packed, y, amd.moe_config(T, E, K, D, I))
    torch.cuda.synchronize()
    del packed
    rows = np.arange(T) if sample is None else np.asarray(sample)
    xs = bf16_np(x)[rows]
    wgn = bf16_np(wg)
    idx_s, _ = orc.moe_route(orc.bf16_to_f32(xs), orc.bf16_to_f32(wgn), K)
    used = np.unique(idx_s[idx_s >= 0])
    wmap = np.zeros(E, np.int32)
    wmap[used] = np.arange(len(used), dtype=np.int32)
    sel = torch.from_numpy(used).cuda()
    q1, s1 = w1q.index_select(0, sel).cpu().numpy(), w1s.index_select(0, sel).cpu().numpy()
    q2, s2 = w2q.index_select(0, sel).cpu().numpy(), w2s.index_select(0, sel).cpu().numpy()
    _, _, y_ref = orc.moe_forward_mxfp4(xs, wgn, q1, s1, q2, s2, K, wmap=wmap)
    yg = orc.bf16_to_f32(bf16_np(y)[rows])
    rel = np.abs(yg - y_ref).max() / np.abs(y_ref).max()
    print(f"mxfp4 T={T} E={E} D={D} I={I}: rel_err={rel:.3e} max|y|={np.abs(y_ref).max():.3f}")
    return rel


def test_forward_mxfp4_small_full(amd, orc):
    import synth
    announce("forward_mxfp4 small full")
    T, E, K, D, I = 64, 16, 4, 512, 256
    w = synth.mxfp4_weights(E, D, I, seed=71, packed=False)
    x, wg = synth.dsv3_inputs(T, E, D, seed=72)
    assert _mx_case(amd, orc, w, x, wg, K) < 2e-2


def test_forward_mxfp4_every_token_tile_count(amd, orc):
    """Routing fixed through the gate so that experts hold every row count
    of ROUTED_COUNTS: each live token-tile count R = 1..16 of the MX main
    loop, both register-ring depths, experts of two and three M-tiles; the
    full output against the oracle."""
    import synth
    E, K, D, I = 64, 8, 2048, 1024
    T, chosen = _routed_layout(ROUTED_COUNTS, E, K)
    announce(f"forward_mxfp4 every token-tile count: T={T}")
    x, wg = _routing_columns(chosen, E, D, np.random.default_rng(1260))
    w = synth.mxfp4_weights(E, D, I, seed=73, packed=False)
    assert _mx_case(amd, orc, w, dev(orc.f32_to_bf16(x)), dev(orc.f32_to_bf16(wg)), K) < 2e-2


@pytest.fixture(scope="module")
def dsv3_mx(amd):
    import synth
    announce("generating DSV3 MXFP4 weights (E=256, D=7168, I=2048)")
    w = synth.mxfp4_weights(256, 7168, 2048, seed=1234, packed=False)
    yield w
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,n_check", [(1, 1), (64, 16), (4096, 48)])
def test_forward_mxfp4_dsv3(amd, orc, dsv3_mx, T, n_check):
    import synth
    announce(f"forward_mxfp4 dsv3 T={T}")
    x, wg = synth.dsv3_inputs(T, 256, 7168, seed=1237)
    rows = np.sort(np.random.default_rng(T).choice(T, n_check, replace=False))
    assert _mx_case(amd, orc, dsv3_mx, x, wg, 8, sample=rows) < 2e-2
