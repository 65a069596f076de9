"""ctypes binding of libamdmoe.so (the C ABI in include/amdmoe.h).

Thin plumbing for Python callers (tests, bench): tensors are torch CUDA
tensors, passed to the library as raw device pointers.  There is no CPU or
PyTorch fallback: if the HIP library is missing or a call fails, this raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libamdmoe.so")

AMDMOE_DTYPE_F32 = 0
AMDMOE_DTYPE_BF16 = 1
AMDMOE_DTYPE_FP8 = 2
AMDMOE_DTYPE_MXFP4 = 3

# Exported symbols, in the order include/amdmoe.h declares them.
SYMBOLS = [
    "amdmoe_last_error", "amdmoe_version", "amdmoe_moe_workspace_bytes",
    "amdmoe_moe_forward_f32", "amdmoe_moe_forward_f32_bias", "amdmoe_moe_forward_bf16",
    "amdmoe_moe_forward_bf16_packed", "amdmoe_moe_forward_fp8",
    "amdmoe_moe_forward_fp8_packed", "amdmoe_moe_forward_mxfp4", "amdmoe_quant_weight_mxfp4",
    "amdmoe_quant_rows_mxfp8", "amdmoe_pack_weights_mxfp4", "amdmoe_moe_forward_fp8_packed_noalloc",
    "amdmoe_pack_weights_fp8", "amdmoe_pack_weights_bf16",
    "amdmoe_moe_gate_f32", "amdmoe_moe_gate_bf16x", "amdmoe_moe_gate_bf16", "amdmoe_moe_gate_fp8",
    "amdmoe_moe_gather_f32", "amdmoe_moe_permute", "amdmoe_naive_gemm_f32",
    "amdmoe_swiglu_f32", "amdmoe_moe_scatter_f32", "amdmoe_quant_rows_fp8",
    "amdmoe_quant_weight_fp8", "amdmoe_set_stage_events", "amdmoe_dsa_forward_f32",
    "amdmoe_dsa_decode_bf16_paged", "amdmoe_dsa_indexer_topk_fp8", "amdmoe_dsa_kv_gather_f32",
    "amdmoe_dsa_dot_compressed_f32",
    "amdmoe_dsa_dot_positional_f32", "amdmoe_dsa_dot_fused_f32", "amdmoe_dsa_softmax_f32",
    "amdmoe_dsa_output_proj_f32",
]


class MoeConfig(ctypes.Structure):
    """Layout-identical to the reference's MoeConfig (naive_moe.cuh:9-15)."""
    _fields_ = [("num_tokens", ctypes.c_int), ("num_experts", ctypes.c_int),
                ("top_k", ctypes.c_int), ("hidden_dim", ctypes.c_int),
                ("intermediate_dim", ctypes.c_int)]


class DsaConfig(ctypes.Structure):
    """Layout-identical to the reference's DsaConfig (naive_dsa.cuh:9-17)."""
    _fields_ = [("num_queries", ctypes.c_int), ("num_heads", ctypes.c_int),
                ("head_dim_compressed", ctypes.c_int), ("head_dim_positional", ctypes.c_int),
                ("num_selected_kv", ctypes.c_int), ("page_size", ctypes.c_int),
                ("total_kv_tokens", ctypes.c_int)]


class AmdMoeError(RuntimeError):
    pass


_lib = None
_P = ctypes.c_void_p


def load():
    """Load libamdmoe.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AmdMoeError(f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(LIB_PATH)
    cfgp = ctypes.POINTER(MoeConfig)
    dcfgp = ctypes.POINTER(DsaConfig)
    I, L_, SZ = ctypes.c_int, ctypes.c_long, ctypes.c_size_t
    sigs = {
        "amdmoe_last_error": (ctypes.c_char_p, []),
        "amdmoe_version": (ctypes.c_char_p, []),
        "amdmoe_moe_workspace_bytes": (I, [cfgp, I, ctypes.POINTER(SZ)]),
        "amdmoe_moe_forward_f32": (I, [_P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_f32_bias": (I, [_P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_bf16": (I, [_P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_bf16_packed": (I, [_P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_fp8": (I, [_P, _P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_fp8_packed": (I, [_P, _P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_moe_forward_mxfp4": (I, [_P, _P, _P, _P, _P, _P, _P, cfgp, _P, SZ, _P]),
        "amdmoe_quant_weight_mxfp4": (I, [_P, L_, I, _P, _P, _P]),
        "amdmoe_quant_rows_mxfp8": (I, [_P, L_, I, _P, _P, _P]),
        "amdmoe_pack_weights_mxfp4": (I, [_P, _P, I, I, I, _P, _P, _P]),
        "amdmoe_moe_forward_fp8_packed_noalloc": (I, [_P, _P, _P, _P, _P, _P, _P, cfgp, _P]),
        "amdmoe_pack_weights_fp8": (I, [_P, I, I, I, _P, _P]),
        "amdmoe_pack_weights_bf16": (I, [_P, I, I, I, _P, _P]),
        "amdmoe_moe_gate_f32": (I, [_P, _P, _P, _P, cfgp, _P]),
        "amdmoe_moe_gate_bf16x": (I, [_P, _P, _P, _P, _P, cfgp, _P]),
        "amdmoe_moe_gate_bf16": (I, [_P, _P, _P, _P, cfgp, _P]),
        "amdmoe_moe_gate_fp8": (I, [_P, _P, _P, _P, _P, _P, cfgp, _P]),
        "amdmoe_moe_gather_f32": (I, [_P, _P, _P, I, _P, _P, _P, cfgp, _P]),
        "amdmoe_moe_permute": (I, [_P, cfgp, _P, _P, _P, _P, _P]),
        "amdmoe_naive_gemm_f32": (I, [_P, _P, _P, I, I, I, _P]),
        "amdmoe_swiglu_f32": (I, [_P, _P, _P, I, _P]),
        "amdmoe_moe_scatter_f32": (I, [_P, _P, _P, _P, I, _P, I, cfgp, _P]),
        "amdmoe_quant_rows_fp8": (I, [_P, L_, I, _P, _P, _P]),
        "amdmoe_quant_weight_fp8": (I, [_P, L_, I, _P, _P, _P, _P]),
        "amdmoe_set_stage_events": (I, [ctypes.POINTER(_P)]),
        "amdmoe_dsa_forward_f32": (I, [_P, _P, _P, _P, _P, _P, _P, dcfgp, _P]),
        "amdmoe_dsa_decode_bf16_paged": (I, [_P, _P, _P, _P, _P, _P, dcfgp, I, _P]),
        "amdmoe_dsa_indexer_topk_fp8": (I, [_P, _P, _P, _P, _P, L_, _P, _P, I, I, I, I, I, I,
                                            _P, _P, _P]),
        "amdmoe_dsa_kv_gather_f32": (I, [_P, _P, _P, _P, _P, _P, _P, dcfgp, _P]),
        "amdmoe_dsa_dot_compressed_f32": (I, [_P, _P, _P, dcfgp, _P]),
        "amdmoe_dsa_dot_positional_f32": (I, [_P, _P, _P, dcfgp, _P]),
        "amdmoe_dsa_dot_fused_f32": (I, [_P, _P, _P, _P, _P, dcfgp, _P]),
        "amdmoe_dsa_softmax_f32": (I, [_P, dcfgp, _P]),
        "amdmoe_dsa_output_proj_f32": (I, [_P, _P, _P, dcfgp, _P]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc):
    if rc != 0:
        raise AmdMoeError(f"amdmoe error {rc}: {load().amdmoe_last_error().decode()}")


def _ptr(t):
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous(), "expected a contiguous device tensor"
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def moe_config(T, E, K, D, I):
    return MoeConfig(T, E, K, D, I)


def dsa_config(Q, H, Dc, Dp, S, P, N):
    return DsaConfig(Q, H, Dc, Dp, S, P, N)


def workspace_bytes(cfg, dtype):
    n = ctypes.c_size_t(0)
    _check(load().amdmoe_moe_workspace_bytes(ctypes.byref(cfg), dtype, ctypes.byref(n)))
    return n.value


def alloc_workspace(cfg, dtype, device="cuda"):
    import torch
    return torch.empty(workspace_bytes(cfg, dtype), dtype=torch.uint8, device=device)


def _ws(ws):
    return (None, 0) if ws is None else (_ptr(ws), ws.numel())


def moe_forward_f32(x, wg, w1, w2, y, cfg, ws=None, stream=None):
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_f32(_ptr(x), _ptr(wg), _ptr(w1), _ptr(w2), _ptr(y),
                                         ctypes.byref(cfg), p, n, _stream(stream)))


def moe_forward_f32_bias(x, wg, bias, w1, w2, y, cfg, ws=None, stream=None):
    """amdmoe_moe_forward_f32 with a per-expert logit bias [E] (None: no bias)."""
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_f32_bias(_ptr(x), _ptr(wg), _ptr(bias), _ptr(w1), _ptr(w2),
                                              _ptr(y), ctypes.byref(cfg), p, n, _stream(stream)))


def moe_forward_bf16(x, wg, bias, w1, w2, y, cfg, ws=None, stream=None):
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_bf16(_ptr(x), _ptr(wg), _ptr(bias), _ptr(w1), _ptr(w2),
                                          _ptr(y), ctypes.byref(cfg), p, n, _stream(stream)))


def moe_forward_bf16_packed(x, wg, bias, w1p, w2p, y, cfg, ws=None, stream=None):
    """amdmoe_moe_forward_bf16 with W1/W2 in pack_weights_bf16 order."""
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_bf16_packed(_ptr(x), _ptr(wg), _ptr(bias), _ptr(w1p), _ptr(w2p),
                                                 _ptr(y), ctypes.byref(cfg), p, n, _stream(stream)))


def pack_weights_bf16(w, out, stream=None):
    """Repack bf16 expert weights w [E, rows, cols] (int16 bit-view device tensor) into out
    (same shape) in fragment-block order."""
    E, rows, cols = w.shape
    _check(load().amdmoe_pack_weights_bf16(_ptr(w), E, rows, cols, _ptr(out), _stream(stream)))


def moe_forward_fp8(x, wg, w1, w1s, w2, w2s, y, cfg, ws=None, stream=None):
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_fp8(_ptr(x), _ptr(wg), _ptr(w1), _ptr(w1s), _ptr(w2),
                                         _ptr(w2s), _ptr(y), ctypes.byref(cfg), p, n,
                                         _stream(stream)))


def moe_forward_fp8_packed(x, wg, w1p, w1s, w2p, w2s, y, cfg, ws=None, stream=None):
    """amdmoe_moe_forward_fp8 with W1/W2 in pack_weights_fp8 order."""
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_fp8_packed(_ptr(x), _ptr(wg), _ptr(w1p), _ptr(w1s), _ptr(w2p),
                                                _ptr(w2s), _ptr(y), ctypes.byref(cfg), p, n,
                                                _stream(stream)))


def moe_forward_mxfp4(x, wg, w1p, w1sp, w2p, w2sp, y, cfg, ws=None, stream=None):
    """MXFP4 experts (fragment order, pack_weights_mxfp4), MXFP8 activations."""
    p, n = _ws(ws)
    _check(load().amdmoe_moe_forward_mxfp4(_ptr(x), _ptr(wg), _ptr(w1p), _ptr(w1sp), _ptr(w2p),
                                           _ptr(w2sp), _ptr(y), ctypes.byref(cfg), p, n,
                                           _stream(stream)))


def quant_weight_mxfp4(w, q, s, stream=None):
    rows, cols = w.shape
    _check(load().amdmoe_quant_weight_mxfp4(_ptr(w), rows, cols, _ptr(q), _ptr(s), _stream(stream)))


def quant_rows_mxfp8(x, q, s, stream=None):
    rows, cols = x.shape
    _check(load().amdmoe_quant_rows_mxfp8(_ptr(x), rows, cols, _ptr(q), _ptr(s), _stream(stream)))


def pack_weights_mxfp4(q, s, qp, sp, stream=None):
    """q [E, rows, cols/2], s [E, rows, cols/32] (uint8) -> fragment order."""
    E, rows, half = q.shape
    _check(load().amdmoe_pack_weights_mxfp4(_ptr(q), _ptr(s), E, rows, 2 * half, _ptr(qp), _ptr(sp),
                                            _stream(stream)))


NOALLOC_SCRATCH_BYTES = 64 << 20


def moe_forward_fp8_packed_noalloc(x, wg, w1p, w1s, w2p, w2s, y, cfg, stream=None):
    """amdmoe_moe_forward_fp8_packed with the library's fixed per-GPU scratch
    (no allocation; workspace at most NOALLOC_SCRATCH_BYTES)."""
    _check(load().amdmoe_moe_forward_fp8_packed_noalloc(_ptr(x), _ptr(wg), _ptr(w1p), _ptr(w1s),
                                                        _ptr(w2p), _ptr(w2s), _ptr(y),
                                                        ctypes.byref(cfg), _stream(stream)))


def pack_weights_fp8(w, out, stream=None):
    """Repack e4m3 expert weights w [E, rows, cols] (uint8 device tensor) into out (same shape
    and size) in fragment-block order."""
    E, rows, cols = w.shape
    _check(load().amdmoe_pack_weights_fp8(_ptr(w), E, rows, cols, _ptr(out), _stream(stream)))


def moe_gate_f32(x, wg, idx, wts, cfg, stream=None):
    _check(load().amdmoe_moe_gate_f32(_ptr(x), _ptr(wg), _ptr(idx), _ptr(wts), ctypes.byref(cfg),
                                      _stream(stream)))


def moe_gate_bf16x(x, wg, bias, idx, wts, cfg, stream=None):
    _check(load().amdmoe_moe_gate_bf16x(_ptr(x), _ptr(wg), _ptr(bias), _ptr(idx), _ptr(wts),
                                        ctypes.byref(cfg), _stream(stream)))


def moe_gate_bf16(x, wg, idx, wts, cfg, stream=None):
    _check(load().amdmoe_moe_gate_bf16(_ptr(x), _ptr(wg), _ptr(idx), _ptr(wts),
                                       ctypes.byref(cfg), _stream(stream)))


def moe_gate_fp8(x, wg, idx, wts, xq, xs, cfg, stream=None):
    _check(load().amdmoe_moe_gate_fp8(_ptr(x), _ptr(wg), _ptr(idx), _ptr(wts), _ptr(xq), _ptr(xs),
                                      ctypes.byref(cfg), _stream(stream)))


def moe_gather_f32(x, idx, wts, expert, gathered, token_map, count, cfg, stream=None):
    _check(load().amdmoe_moe_gather_f32(_ptr(x), _ptr(idx), _ptr(wts), expert, _ptr(gathered),
                                        _ptr(token_map), _ptr(count), ctypes.byref(cfg),
                                        _stream(stream)))


def moe_permute(idx, cfg, counts, offsets, sorted_token, sorted_slot, stream=None):
    _check(load().amdmoe_moe_permute(_ptr(idx), ctypes.byref(cfg), _ptr(counts), _ptr(offsets),
                                     _ptr(sorted_token), _ptr(sorted_slot), _stream(stream)))


def naive_gemm_f32(A, B, C, M, N, K, stream=None):
    _check(load().amdmoe_naive_gemm_f32(_ptr(A), _ptr(B), _ptr(C), M, N, K, _stream(stream)))


def swiglu_f32(gate, up, out, n, stream=None):
    _check(load().amdmoe_swiglu_f32(_ptr(gate), _ptr(up), _ptr(out), n, _stream(stream)))


def moe_scatter_f32(eo, token_map, wts, idx, expert, out, count, cfg, stream=None):
    _check(load().amdmoe_moe_scatter_f32(_ptr(eo), _ptr(token_map), _ptr(wts), _ptr(idx), expert,
                                         _ptr(out), count, ctypes.byref(cfg), _stream(stream)))


def quant_rows_fp8(x, q, s, stream=None):
    rows, cols = x.shape
    _check(load().amdmoe_quant_rows_fp8(_ptr(x), rows, cols, _ptr(q), _ptr(s), _stream(stream)))


def quant_weight_fp8(w, u, q, s, stream=None):
    rows, cols = w.shape
    _check(load().amdmoe_quant_weight_fp8(_ptr(w), rows, cols, _ptr(u), _ptr(q), _ptr(s),
                                          _stream(stream)))


class StageEvents:
    """Seven torch.cuda.Events recorded by the next forward at its stage
    boundaries (see amdmoe_set_stage_events)."""
    NAMES = ["route", "quant_x", "permute", "gemm_up", "gemm_down", "combine"]

    def __init__(self):
        import torch
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(7)]
        for e in self.events:   # torch creates the HIP event on first record
            e.record()
        self._arr = (_P * 7)(*[ctypes.c_void_p(e.cuda_event) for e in self.events])

    def arm(self):
        _check(load().amdmoe_set_stage_events(self._arr))

    @staticmethod
    def disarm():
        _check(load().amdmoe_set_stage_events(None))

    def stage_ms(self):
        return {n: self.events[i].elapsed_time(self.events[i + 1]) for i, n in enumerate(self.NAMES)}


def dsa_forward_f32(qn, qp, kc, kp, v, idx, out, cfg, stream=None):
    _check(load().amdmoe_dsa_forward_f32(_ptr(qn), _ptr(qp), _ptr(kc), _ptr(kp), _ptr(v),
                                         _ptr(idx), _ptr(out), ctypes.byref(cfg),
                                         _stream(stream)))


def dsa_decode_bf16_paged(qn, qp, cache, page_table, logical, out, cfg, pages_per_seq,
                          stream=None):
    _check(load().amdmoe_dsa_decode_bf16_paged(_ptr(qn), _ptr(qp), _ptr(cache), _ptr(page_table),
                                               _ptr(logical), _ptr(out), ctypes.byref(cfg),
                                               pages_per_seq, _stream(stream)))


# the reference's DSA stage functions (naive_dsa.cuh:31-68)
def dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, page_table, seq_len, page, max_seq, topk, scores,
                         out, stream=None):
    Q, Hi, _ = qc.shape
    _check(load().amdmoe_dsa_indexer_topk_fp8(_ptr(qc), _ptr(qs), _ptr(hw), _ptr(kc), _ptr(ks),
                                              kc.shape[0], _ptr(page_table), _ptr(seq_len), Q, Hi,
                                              page, page_table.shape[1], max_seq, topk,
                                              _ptr(scores), _ptr(out), _stream(stream)))


def dsa_kv_gather_f32(kc, kp, v, idx, gkc, gkp, gv, cfg, stream=None):
    _check(load().amdmoe_dsa_kv_gather_f32(_ptr(kc), _ptr(kp), _ptr(v), _ptr(idx), _ptr(gkc),
                                           _ptr(gkp), _ptr(gv), ctypes.byref(cfg), _stream(stream)))


def dsa_dot_compressed_f32(qn, kc, scores, cfg, stream=None):
    _check(load().amdmoe_dsa_dot_compressed_f32(_ptr(qn), _ptr(kc), _ptr(scores),
                                                ctypes.byref(cfg), _stream(stream)))


def dsa_dot_positional_f32(qp, kp, scores, cfg, stream=None):
    _check(load().amdmoe_dsa_dot_positional_f32(_ptr(qp), _ptr(kp), _ptr(scores),
                                                ctypes.byref(cfg), _stream(stream)))


def dsa_dot_fused_f32(qn, qp, kc, kp, scores, cfg, stream=None):
    _check(load().amdmoe_dsa_dot_fused_f32(_ptr(qn), _ptr(qp), _ptr(kc), _ptr(kp), _ptr(scores),
                                           ctypes.byref(cfg), _stream(stream)))


def dsa_softmax_f32(scores, cfg, stream=None):
    _check(load().amdmoe_dsa_softmax_f32(_ptr(scores), ctypes.byref(cfg), _stream(stream)))


def dsa_output_proj_f32(attn, v, out, cfg, stream=None):
    _check(load().amdmoe_dsa_output_proj_f32(_ptr(attn), _ptr(v), _ptr(out), ctypes.byref(cfg),
                                             _stream(stream)))
