"""numpy front-end for the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, as the checker.  The product library never
imports it and has no CPU fallback.

Every function mirrors one C function of oracle.c, which cites the reference
file:line it restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_L, _I, _F = ctypes.c_long, ctypes.c_int, ctypes.c_float


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_srand": (None, [ctypes.c_uint]),
            "orc_set_threads": (None, [_I]),
            "orc_get_threads": (_I, []),
            "orc_random_fill": (None, [_f32p, _L, _F, _F]),
            "orc_gen_sparse_indices": (None, [_i32p, _I, _I, _I, _I]),
            "orc_max_abs_error": (_F, [_f32p, _f32p, _L]),
            "orc_mean_abs_error": (_F, [_f32p, _f32p, _L]),
            "orc_f32_to_bf16_array": (None, [_f32p, _u16p, _L]),
            "orc_bf16_to_f32_array": (None, [_u16p, _f32p, _L]),
            "orc_e4m3_to_f32_array": (None, [_u8p, _f32p, _L]),
            "orc_f32_to_e4m3": (ctypes.c_uint8, [_F]),
            "orc_quant_rows_1x128": (None, [_f32p, _L, _I, _u8p, _f32p]),
            "orc_quant_weight_128x128": (None, [_f32p, _I, _I, _f32p, _u8p, _f32p]),
            "orc_softmax": (None, [_f32p, _I]),
            "orc_topk_row": (None, [_f32p, _I, _I, _i32p, _f32p]),
            "orc_moe_route": (None, [_f32p, _f32p, ctypes.c_void_p, _I, _I, _I, _I,
                                     _i32p, _f32p, ctypes.c_void_p, ctypes.c_void_p]),
            "orc_moe_permute": (None, [_i32p, _I, _I, _I, _i32p, _i32p, _i32p, _i32p]),
            "orc_moe_forward_f32": (None, [_f32p, _f32p, _f32p, _f32p, ctypes.c_void_p,
                                           _I, _I, _I, _I, _I, _i32p, _f32p, _f32p]),
            "orc_moe_forward_bf16": (None, [_u16p, _f32p, _u16p, _u16p, ctypes.c_void_p,
                                            _I, _I, _I, _I, _I, _i32p, _f32p, _f32p]),
            "orc_dequant_weight_128x128": (None, [_u8p, _f32p, _I, _I, _f32p]),
            "orc_moe_forward_fp8": (None, [_u16p, _I, _u16p, _u8p, _f32p, _u8p, _f32p,
                                           ctypes.c_void_p, _I, _I, _I, _I, _i32p, _f32p, _f32p]),
            "orc_e8m0_to_f32": (_F, [ctypes.c_uint8]),
            "orc_e2m1_to_f32": (_F, [ctypes.c_uint8]),
            "orc_f32_to_e2m1": (ctypes.c_uint8, [_F]),
            "orc_mx_quant_rows": (None, [_f32p, _L, _I, _I, _u8p, _u8p]),
            "orc_mx_dequant_rows": (None, [_u8p, _u8p, _L, _I, _I, _f32p]),
            "orc_moe_forward_mxfp4": (None, [_u16p, _I, _u16p, _u8p, _u8p, _u8p, _u8p,
                                             ctypes.c_void_p, _I, _I, _I, _I, _i32p, _f32p, _f32p]),
            "orc_dsa_kv_gather": (None, [_f32p, ctypes.c_void_p, _f32p, _i32p, _f32p,
                                         ctypes.c_void_p, _f32p, _I, _I, _I, _I]),
            "orc_dsa_dot": (None, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_void_p, _f32p, _I, _I, _I, _I, _I, _I]),
            "orc_dsa_softmax": (None, [_f32p, _L, _I]),
            "orc_dsa_output_proj": (None, [_f32p, _f32p, _f32p, _I, _I, _I, _I]),
            "orc_dsa_forward_f32": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _i32p, _f32p,
                                           _I, _I, _I, _I, _I]),
            "orc_dsa_translate": (None, [_i32p, _i32p, _I, _I, _I, _I, _L, _i32p]),
            "orc_dsa_decode_bf16_paged": (None, [_u16p, _u16p, _u16p, _i32p, _i32p, _f32p,
                                                 _I, _I, _I, _I, _I, _I, _I, _L]),
            "orc_dsa_indexer_scores": (None, [_u8p, _f32p, _f32p, _u8p, _f32p, _i32p, _i32p,
                                              _I, _I, _I, _I, _I, _f32p]),
            "orc_dsa_indexer_topk": (None, [_f32p, _i32p, _I, _I, _I, _I, _i32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _opt(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n):
    """Threads of the oracle's parallel loops (1 = the reference's single thread)."""
    lib().orc_set_threads(int(n))


def get_threads():
    return int(lib().orc_get_threads())


# ---------------------------------------------------------------- generators
def srand(seed):
    lib().orc_srand(seed)


def random_fill(n, lo, hi):
    """utils/cuda_utils.cuh:56-60 on the current glibc rand() stream."""
    out = np.empty(n, np.float32)
    lib().orc_random_fill(out, n, lo, hi)
    return out


def gen_sparse_indices(Q, S, N, sort_rows=True):
    """tests/test_dsa.cu:73-85 (sort_rows=False keeps the draw order)."""
    out = np.empty(Q * S, np.int32)
    lib().orc_gen_sparse_indices(out, Q, S, N, int(sort_rows))
    return out.reshape(Q, S)


def reference_moe_inputs(T, E, K, D, I, seed=42):
    """Inputs of tests/test_moe.cu:151-164 (srand(seed); x, Wg, W1, W2)."""
    srand(seed)
    x = random_fill(T * D, -0.5, 0.5).reshape(T, D)
    wg = random_fill(E * D, -0.5, 0.5).reshape(E, D)
    w1 = random_fill(E * 2 * I * D, -0.1, 0.1).reshape(E, 2 * I, D)
    w2 = random_fill(E * D * I, -0.1, 0.1).reshape(E, D, I)
    return x, wg, w1, w2


def reference_dsa_inputs(Q, H, Dc, Dp, S, P, N, seed=42):
    """Inputs of tests/test_dsa.cu:101-115."""
    srand(seed)
    qn = random_fill(Q * H * Dc, -0.3, 0.3).reshape(Q, H, Dc)
    qp = random_fill(Q * H * Dp, -0.3, 0.3).reshape(Q, H, Dp)
    kc = random_fill(N * Dc, -0.3, 0.3).reshape(N, Dc)
    kp = random_fill(N * Dp, -0.3, 0.3).reshape(N, Dp)
    v = random_fill(N * Dc, -0.3, 0.3).reshape(N, Dc)
    idx = gen_sparse_indices(Q, S, N, True)
    return qn, qp, kc, kp, v, idx


# ---------------------------------------------------------------- formats
def f32_to_bf16(a):
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_bf16_array(a.reshape(-1), out.reshape(-1), a.size)
    return out


def bf16_to_f32(a):
    a = _c(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_bf16_to_f32_array(a.reshape(-1), out.reshape(-1), a.size)
    return out


def e4m3_to_f32(a):
    a = _c(a, np.uint8)
    out = np.empty(a.shape, np.float32)
    lib().orc_e4m3_to_f32_array(a.reshape(-1), out.reshape(-1), a.size)
    return out


def f32_to_e4m3_scalar(v):
    return int(lib().orc_f32_to_e4m3(float(v)))


def quant_rows_1x128(x):
    x = _c(x, np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // 128), np.float32)
    lib().orc_quant_rows_1x128(x, rows, cols, q, s)
    return q, s


def quant_weight_128x128(w, u):
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows // 128, cols // 128), np.float32)
    lib().orc_quant_weight_128x128(w, rows, cols, _c(u, np.float32), q, s)
    return q, s


def dequant_weight_128x128(q, s):
    q = _c(q, np.uint8)
    rows, cols = q.shape
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequant_weight_128x128(q, _c(s, np.float32), rows, cols, out)
    return out


# ---------------------------------------------------------------- MoE
def softmax(row):
    r = _c(row, np.float32).copy()
    lib().orc_softmax(r, r.size)
    return r


def topk_row(p, K):
    p = _c(p, np.float32)
    idx = np.empty(K, np.int32)
    wt = np.empty(K, np.float32)
    lib().orc_topk_row(p, p.size, K, idx, wt)
    return idx, wt


def moe_route(x, wg, K, bias=None, want_probs=False):
    x = _c(x, np.float32)
    wg = _c(wg, np.float32)
    T, D = x.shape
    E = wg.shape[0]
    idx = np.empty((T, K), np.int32)
    wts = np.empty((T, K), np.float32)
    logits = np.empty((T, E), np.float32)
    probs = np.empty((T, E), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_moe_route(x, wg, _opt(b), T, E, K, D, idx, wts, _opt(logits), _opt(probs))
    if want_probs:
        return idx, wts, logits, probs
    return idx, wts


def moe_permute(idx, E):
    idx = _c(idx, np.int32)
    T, K = idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    st = np.full(T * K, -1, np.int32)
    ss = np.full(T * K, -1, np.int32)
    lib().orc_moe_permute(idx, T, K, E, counts, offsets, st, ss)
    n = int(offsets[E])
    return counts, offsets, st[:n], ss[:n]


def moe_forward_f32(x, wg, w1, w2, K, bias=None):
    x, wg, w1, w2 = (_c(a, np.float32) for a in (x, wg, w1, w2))
    T, D = x.shape
    E = wg.shape[0]
    I = w1.shape[1] // 2
    idx = np.empty((T, K), np.int32)
    wts = np.empty((T, K), np.float32)
    y = np.empty((T, D), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_moe_forward_f32(x, wg, w1, w2, _opt(b), T, E, K, D, I, idx, wts, y)
    return idx, wts, y


def moe_forward_bf16(x_bf16, wg_f32, w1_bf16, w2_bf16, K, bias=None):
    x, w1, w2 = (_c(a, np.uint16) for a in (x_bf16, w1_bf16, w2_bf16))
    wg = _c(wg_f32, np.float32)
    T, D = x.shape
    E = wg.shape[0]
    I = w1.shape[1] // 2
    idx = np.empty((T, K), np.int32)
    wts = np.empty((T, K), np.float32)
    y = np.empty((T, D), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_moe_forward_bf16(x, wg, w1, w2, _opt(b), T, E, K, D, I, idx, wts, y)
    return idx, wts, y


def moe_forward_fp8(x_bf16_rows, wg_bf16, w1q, w1s, w2q, w2s, K, wmap=None):
    """wmap[e] = slot of expert e in the weight arrays (None: identity)."""
    x = _c(x_bf16_rows, np.uint16)
    wg = _c(wg_bf16, np.uint16)
    w1q, w2q = _c(w1q, np.uint8), _c(w2q, np.uint8)
    w1s, w2s = _c(w1s, np.float32), _c(w2s, np.float32)
    n, D = x.shape
    E = wg.shape[0]
    I = w1q.shape[1] // 2
    idx = np.empty((n, K), np.int32)
    wts = np.empty((n, K), np.float32)
    y = np.empty((n, D), np.float32)
    wm = None if wmap is None else _c(wmap, np.int32)
    lib().orc_moe_forward_fp8(x, n, wg, w1q, w1s, w2q, w2s, _opt(wm), E, K, D, I, idx, wts, y)
    return idx, wts, y


# ---------------------------------------------------------------- MX (OCP microscaling)
def e8m0_to_f32(c):
    return float(lib().orc_e8m0_to_f32(int(c)))


def e2m1_to_f32(c):
    return float(lib().orc_e2m1_to_f32(int(c)))


def f32_to_e2m1_scalar(v):
    return int(lib().orc_f32_to_e2m1(float(v)))


def mx_quant_rows(x, elem_bits):
    """Rows -> (codes, E8M0 scales [rows, cols/32]); fp4 codes packed two per
    byte (even element in the low nibble) [rows, cols/2], fp8 [rows, cols]."""
    x = _c(x, np.float32)
    rows, cols = x.shape
    q = np.zeros((rows, cols // 2 if elem_bits == 4 else cols), np.uint8)
    s = np.empty((rows, cols // 32), np.uint8)
    lib().orc_mx_quant_rows(x, rows, cols, elem_bits, q, s)
    return q, s


def mx_dequant_rows(q, s, elem_bits):
    q, s = _c(q, np.uint8), _c(s, np.uint8)
    rows = s.shape[0]
    cols = s.shape[1] * 32
    out = np.empty((rows, cols), np.float32)
    lib().orc_mx_dequant_rows(q, s, rows, cols, elem_bits, out)
    return out


def moe_forward_mxfp4(x_bf16_rows, wg_bf16, w1q, w1s, w2q, w2s, K, wmap=None):
    """MXFP4 expert weights (row-major E2M1 + E8M0 per 32), MXFP8 activations."""
    x = _c(x_bf16_rows, np.uint16)
    wg = _c(wg_bf16, np.uint16)
    w1q, w1s, w2q, w2s = (_c(a, np.uint8) for a in (w1q, w1s, w2q, w2s))
    n, D = x.shape
    E = wg.shape[0]
    I = w2q.shape[2] * 2
    idx = np.empty((n, K), np.int32)
    wts = np.empty((n, K), np.float32)
    y = np.empty((n, D), np.float32)
    wm = None if wmap is None else _c(wmap, np.int32)
    lib().orc_moe_forward_mxfp4(x, n, wg, w1q, w1s, w2q, w2s, _opt(wm), E, K, D, I, idx, wts, y)
    return idx, wts, y


# ---------------------------------------------------------------- DSA
def dsa_forward_f32(qn, qp, kc, kp, v, idx):
    qn, qp, kc, kp, v = (_c(a, np.float32) for a in (qn, qp, kc, kp, v))
    idx = _c(idx, np.int32)
    Q, H, Dc = qn.shape
    Dp = qp.shape[2]
    S = idx.shape[1]
    out = np.empty((Q, H, Dc), np.float32)
    lib().orc_dsa_forward_f32(qn, qp, kc, kp, v, idx, out, Q, H, Dc, Dp, S)
    return out


def dsa_kv_gather(kc, kp, v, idx):
    """naive_dsa.cu:13-60 -> (gathered_kc, gathered_kp, gathered_v)."""
    kc, kp, v = (_c(a, np.float32) for a in (kc, kp, v))
    idx = _c(idx, np.int32)
    Q, S = idx.shape
    Dc, Dp = kc.shape[1], kp.shape[1]
    gkc = np.empty((Q, S, Dc), np.float32)
    gkp = np.empty((Q, S, Dp), np.float32)
    gv = np.empty((Q, S, Dc), np.float32)
    lib().orc_dsa_kv_gather(kc, kp.ctypes.data if Dp else None, v, idx, gkc,
                            gkp.ctypes.data if Dp else None, gv, Q, S, Dc, Dp)
    return gkc, gkp, gv


def dsa_dot(qn, qp, kc, kp, scores, parts):
    """naive_dsa.cu:89-276; parts 1 = compressed, 2 = positional, 3 = fused.
    Returns scores + the dots (the input is not modified)."""
    out = _c(scores, np.float32).copy()
    Q, H, S = out.shape
    arrs = [None if a is None else _c(a, np.float32) for a in (qn, qp, kc, kp)]
    Dc = arrs[0].shape[2] if arrs[0] is not None else 0
    Dp = arrs[1].shape[2] if arrs[1] is not None else 0
    ptr = [None if a is None else a.ctypes.data for a in arrs]
    lib().orc_dsa_dot(*ptr, out, Q, H, S, Dc, Dp, parts)
    return out


def dsa_softmax(scores):
    """naive_dsa.cu:278-296 on a copy of scores [..., S]."""
    out = _c(scores, np.float32).copy()
    S = out.shape[-1]
    lib().orc_dsa_softmax(out, out.size // S if S else 0, S)
    return out


def dsa_output_proj(attn, v):
    """naive_dsa.cu:300-316: attn [Q,H,S], v [Q,S,Dc] -> [Q,H,Dc]."""
    attn, v = _c(attn, np.float32), _c(v, np.float32)
    Q, H, S = attn.shape
    Dc = v.shape[2]
    out = np.empty((Q, H, Dc), np.float32)
    lib().orc_dsa_output_proj(attn, v, out, Q, H, S, Dc)
    return out


def dsa_translate(logical, page_table, page, cache_rows=0):
    """Physical cache row of each selected logical index, -1 where it selects
    nothing (index outside the page-table row, negative page id, row at or
    past cache_rows when cache_rows > 0)."""
    logical = _c(logical, np.int32)
    pt = _c(page_table, np.int32)
    Q, S = logical.shape
    out = np.empty((Q, S), np.int32)
    lib().orc_dsa_translate(logical, pt, Q, S, pt.shape[1], page, cache_rows, out)
    return out


def dsa_decode_bf16_paged(qn, qp, cache, page_table, logical, Dc, page):
    """Paged decode over the valid selected tokens only (see dsa_translate);
    0 for a query with none."""
    qn, qp, cache = (_c(a, np.uint16) for a in (qn, qp, cache))
    pt = _c(page_table, np.int32)
    logical = _c(logical, np.int32)
    Q, H, _ = qn.shape
    Dp = qp.shape[2]
    S = logical.shape[1]
    out = np.empty((Q, H, Dc), np.float32)
    lib().orc_dsa_decode_bf16_paged(qn, qp, cache, pt, logical, out, Q, H, Dc, Dp, S,
                                    pt.shape[1], page, cache.shape[0])
    return out


# ---------------------------------------------------------------- indexer
def dsa_indexer_scores(qc, qs, hw, kc, ks, page_table, seq_len, page, max_seq):
    """Lightning-indexer scores (double precision, rounded once to fp32):
    score[q,s] = ks[row] * sum_j hw[q,j] qs[q,j] relu(q[q,j,:] . k[row,:]),
    -inf past seq_len[q]."""
    qc, kc = _c(qc, np.uint8), _c(kc, np.uint8)
    qs, hw, ks = (_c(a, np.float32) for a in (qs, hw, ks))
    pt, sl = _c(page_table, np.int32), _c(seq_len, np.int32)
    Q, Hi, _ = qc.shape
    out = np.empty((Q, max_seq), np.float32)
    lib().orc_dsa_indexer_scores(qc, qs, hw, kc, ks, pt, sl, Q, Hi, page, pt.shape[1], max_seq, out)
    return out


def dsa_indexer_topk(scores, seq_len, topk, cap=0):
    """The topk positions per row by score (ties: lower position), in
    ascending position order, padded with -1; a row holds min(seq_len, cap)
    candidate positions (cap <= 0: the row length)."""
    scores = _c(scores, np.float32)
    sl = _c(seq_len, np.int32)
    Q, max_seq = scores.shape
    out = np.empty((Q, topk), np.int32)
    lib().orc_dsa_indexer_topk(scores, sl, Q, max_seq, cap, topk, out)
    return out
