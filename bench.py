#!/usr/bin/env python3
"""Benchmark of the MoE forward hot path on one MI355X.

Workload (BASELINE.json metric and configs[3]): DeepSeek-V3-shape FP8
block-scale MoE layer, T=4096 tokens, E=256 experts, top-8, D=7168,
I=2048, SwiGLU; e4m3 expert weights with fp32 128x128 scales, x bf16
quantised 1x128 in the forward, bf16 gate and output.  Synthetic data
(seeded on the GPU); all inputs resident in HBM before timing.

A step = one full layer forward (routing, x quantisation, permutation,
both grouped GEMMs, combine).  Prints ONE JSON line on stdout; progress
goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "llm-sys-project_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer tokens/s + % fp8 MFMA peak (1 MI355X, DSV3 shape T=4096)"
FP8_PEAK = 5.0e15       # dense fp8 MFMA, FLOP/s
HBM_PEAK = 8.0e12       # bytes/s
ROOF_KERNEL = "grouped_gemm_kernel<fp8, UP, packed>"  # the dominant kernel


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def moe_bytes(T, E_active, K, D, I):
    """Algorithmic HBM bytes: (layer, up-projection kernel) per launch."""
    w1 = E_active * (2 * I * D + (2 * I // 128) * (D // 128) * 4)
    w2 = E_active * (D * I + (D // 128) * (I // 128) * 4)
    layer = w1 + w2 + T * D * 2 + 256 * D * 2 + T * D * 2
    P = T * K
    up = w1 + T * D + T * (D // 128) * 4 + P * I + P * (I // 128) * 4
    return layer, up


def cpu_baseline(x, wg, w1q, w1s, w2q, w2s, K, n_tokens):
    """The CPU oracle (restatement of tests/test_moe.cu:32-140 with the fp8
    formats) on a sample of tokens of the same workload."""
    import numpy as np
    import torch

    import oracle
    rows = np.arange(n_tokens)
    xs = x[:n_tokens].cpu().numpy().view(np.uint16)
    wgn = wg.cpu().numpy().view(np.uint16)
    idx, _ = oracle.moe_route(oracle.bf16_to_f32(xs), oracle.bf16_to_f32(wgn), K)
    used = np.unique(idx)
    wmap = np.zeros(wg.shape[0], np.int32)
    wmap[used] = np.arange(len(used), dtype=np.int32)
    sel = torch.from_numpy(used).cuda()
    q1, s1 = w1q.index_select(0, sel).cpu().numpy(), w1s.index_select(0, sel).cpu().numpy()
    q2, s2 = w2q.index_select(0, sel).cpu().numpy(), w2s.index_select(0, sel).cpu().numpy()
    oracle.lib()
    threads = oracle.get_threads()
    t0 = time.perf_counter()
    oracle.moe_forward_fp8(xs, wgn, q1, s1, q2, s2, K, wmap=wmap)
    dt = time.perf_counter() - t0
    del q1, s1, q2, s2
    return {"value": len(rows) / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{len(rows)} tokens of the T=4096 DSV3 fp8 workload (routing, x/act "
                      f"quantisation, {len(used)} experts dequantised, combine); {dt:.1f} s",
            "cpu_model": cpu_model(),
            "single_core": cpu_single_core(K, x.shape[1], w2q.shape[2])}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_single_core(K, D, I, n_tokens=16):
    """The faithful restatement of the reference's CPU oracle
    (tests/test_moe.cu:32-140: fp32 weights, sequential sums) on ONE core,
    at the DSV3 per-token shape: each token runs K expert FFNs of D x I
    (a K-expert layer, E = K, so every token uses every expert: the
    per-token work 6*K*D*I of the DSV3 layer; only the gate, E*D per token,
    is smaller).  Timed on n_tokens tokens; the T=4096 time is that
    extrapolated linearly in T (the oracle's cost is linear in T*K)."""
    import numpy as np
    import torch

    import oracle
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    E = K
    x = torch.randn((n_tokens, D), generator=g, device="cuda").cpu().numpy()
    wg = (torch.randn((E, D), generator=g, device="cuda") / D ** 0.5).cpu().numpy()
    w1 = (torch.randn((E, 2 * I, D), generator=g, device="cuda") / D ** 0.5).cpu().numpy()
    w2 = (torch.randn((E, D, I), generator=g, device="cuda") / I ** 0.5).cpu().numpy()
    prev = oracle.get_threads()
    oracle.set_threads(1)
    try:
        t0 = time.perf_counter()
        oracle.moe_forward_f32(x, wg, w1, w2, K)
        dt = time.perf_counter() - t0
    finally:
        oracle.set_threads(prev)
    del w1, w2
    tps = n_tokens / dt
    return {"value": round(tps, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "t4096_s_extrapolated": round(4096 / tps, 1),
            "sample": f"{n_tokens} tokens, fp32 restatement of cpu_moe_forward on one core, "
                      f"K={K} experts of D={D}, I={I} per token (DSV3 per-token work); "
                      f"{dt:.1f} s; T=4096 extrapolated linearly"}


def dsa_bench(amdmoe, synth, iters=20, cpu=False):
    """BASELINE DSA decode: B=64, H=128, Dc=512, Dp=64, S=2048 of 32768.

    Calls rotate over four decode batches (queries and selected positions)
    over one 2.42 GB cache: each batch reads 151 MB of KV rows, the four
    together ~580 MB of distinct rows, more than twice the 256 MB MALL, so a
    timed call cannot find its rows cached by the call before."""
    import torch
    Q, H, S, page, ctx = 64, 128, 2048, 64, 32768
    qn, qp, cache, pt, lg, pps = synth.dsa_paged(Q, H, 512, 64, S, page, ctx, seed=5)
    sets = [(qn, qp, lg)] + [synth.dsa_queries(Q, H, 512, 64, S, ctx, seed=s) for s in (6, 7, 8)]
    cfg = amdmoe.dsa_config(Q, H, 512, 64, S, page, Q * ctx)
    out = torch.empty((Q, H, 512), dtype=torch.int16, device="cuda")
    for a_, b_, c_ in sets:
        amdmoe.dsa_decode_bf16_paged(a_, b_, cache, pt, c_, out, cfg, pps)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(iters):
        a_, b_, c_ = sets[i % len(sets)]
        amdmoe.dsa_decode_bf16_paged(a_, b_, cache, pt, c_, out, cfg, pps)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / iters
    nbytes = Q * (S * 1152 + H * 576 * 2 + H * 512 * 2 + S * 4 + (ctx // page) * 4)
    flops = Q * H * S * (2 * 576 + 2 * 512)
    res = {"us_per_call": round(us, 2), "queries_per_s": round(Q / (us * 1e-6), 1),
           "hbm_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
           "hbm_frac": round(nbytes / (us * 1e-6) / HBM_PEAK, 4),
           "bf16_mfma_frac": round(flops / (us * 1e-6) / 2.5e15, 4),
           "rotation": f"{len(sets)} batches over one cache"}
    if cpu:
        res["cpu_baseline"] = dsa_cpu_baseline(qn, qp, cache, pt, lg, page)
    del sets, cache
    torch.cuda.empty_cache()
    return res


def dsa_cpu_baseline(qn, qp, cache, pt, lg, page, n_single=8):
    """The oracle's restatement of the reference's cpu_dsa_forward
    (tests/test_dsa.cu:23-68: per query gather of the selected rows, then per
    head sequential fp32 dots, softmax and output sums) on the same decode
    batch, its bf16 values decoded to fp32 and the selected rows gathered
    through the page table beforehand (not timed): all 64 queries on every
    host thread, and n_single queries on one core."""
    import numpy as np
    import torch

    import oracle
    Q, H, _ = qn.shape
    S = lg.shape[1]
    phys = oracle.dsa_translate(lg.cpu().numpy(), pt.cpu().numpy(), page)
    rows = cache.index_select(0, torch.from_numpy(phys.reshape(-1).astype(np.int64)).cuda())
    rows = oracle.bf16_to_f32(rows.cpu().numpy().view(np.uint16))          # [Q*S, 576]
    kc, kp = rows[:, :512].copy(), rows[:, 512:].copy()
    qnf = oracle.bf16_to_f32(qn.cpu().numpy().view(np.uint16))
    qpf = oracle.bf16_to_f32(qp.cpu().numpy().view(np.uint16))
    flat = np.arange(Q * S, dtype=np.int32).reshape(Q, S)
    oracle.lib()
    threads = oracle.get_threads()
    t0 = time.perf_counter()
    oracle.dsa_forward_f32(qnf, qpf, kc, kp, kc, flat)
    dt = time.perf_counter() - t0
    prev = oracle.get_threads()
    oracle.set_threads(1)
    try:
        n = min(n_single, Q)
        t0 = time.perf_counter()
        oracle.dsa_forward_f32(qnf[:n], qpf[:n], kc, kp, kc, flat[:n])
        dt1 = time.perf_counter() - t0
    finally:
        oracle.set_threads(prev)
    return {"value": round(Q / dt, 2), "unit": "queries/s", "cores": threads, "kind": "port",
            "sample": f"all {Q} queries of one BASELINE decode batch (H={H}, S={S}, Dc=512, Dp=64), "
                      f"restatement of cpu_dsa_forward over OpenMP threads; {dt:.1f} s",
            "cpu_model": cpu_model(),
            "single_core": {"value": round(n / dt1, 3), "unit": "queries/s", "cores": 1, "kind": "port",
                            "sample": f"{n} queries on one core (the reference's single-threaded "
                                      f"loop); {dt1:.1f} s"}}


def indexer_bench(amdmoe, synth, iters=20):
    """Lightning indexer at the decode shape: 64 queries, 64 fp8 index heads,
    32768 positions each, top-2048 (the indices dsa_decode consumes)."""
    import torch
    Q, Hi, ctx, page, topk = 64, 64, 32768, 64, 2048
    qc, qs, hw, kc, ks, pt = synth.dsa_indexer(Q, Hi, ctx, page, seed=41)
    sl = torch.full((Q,), ctx, dtype=torch.int32, device="cuda")
    scores = torch.empty((Q, ctx), dtype=torch.float32, device="cuda")
    out = torch.empty((Q, topk), dtype=torch.int32, device="cuda")
    ms = _time_calls(lambda: amdmoe.dsa_indexer_topk_fp8(qc, qs, hw, kc, ks, pt, sl, page, ctx, topk,
                                                        scores, out), iters)
    # keys + their scales once, q and head data, scores written and read back, indices
    nbytes = Q * ctx * (128 + 4) + Q * Hi * (128 + 8) + Q * (ctx // page) * 4 + 2 * Q * ctx * 4 + Q * topk * 4
    flops = 2 * Q * ctx * Hi * 128
    del qc, qs, hw, kc, ks, pt, scores, out
    return {"us_per_call": round(ms * 1e3, 2), "queries_per_s": round(Q / (ms * 1e-3), 1),
            "hbm_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4),
            "fp8_mfma_frac": round(flops / (ms * 1e-3) / FP8_PEAK, 4),
            "shape": f"Q={Q} Hi={Hi} ctx={ctx} top-{topk}"}


def mxfp4_bench(amdmoe, synth, iters=20, tokens=(1, 64, 4096)):
    """The MXFP4 expert layer (OCP MX: E2M1 weights, E4M3 activations, E8M0
    scales per 32; no counterpart in the reference) at the DSV3 shape, per
    token count: ms per layer, tokens/s, and the HBM floor of the bytes that
    must cross (active experts' fp4 weights + scales, x, gate, y)."""
    import torch
    E, K, D, I = 256, 8, 7168, 2048
    w1p, w1s, w2p, w2s = synth.mxfp4_weights(E, D, I, seed=1234)
    xa, wg = synth.dsv3_inputs(max(tokens), E, D, seed=99)
    rows = {}
    for T in tokens:
        x = xa[:T].contiguous()
        cfg = amdmoe.moe_config(T, E, K, D, I)
        ws = amdmoe.alloc_workspace(cfg, amdmoe.AMDMOE_DTYPE_MXFP4)
        y = torch.empty((T, D), dtype=torch.int16, device="cuda")
        idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
        wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
        amdmoe.moe_gate_bf16(x, wg, idx, wts, cfg)
        torch.cuda.synchronize()
        act = int(torch.unique(idx).numel())
        ms = _time_calls(lambda: amdmoe.moe_forward_mxfp4(x, wg, w1p, w1s, w2p, w2s, y, cfg, ws=ws), iters)
        nbytes = act * 3 * I * D * (0.5 + 1 / 32) + E * D * 2 + 2 * T * D * 2
        flops = 6 * T * K * D * I
        rows[f"T{T}"] = {"ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                         "experts_active": act, "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                         "hbm_floor_ms": round(nbytes / HBM_PEAK * 1e3, 4),
                         "floor_frac": round(nbytes / HBM_PEAK / (ms * 1e-3), 4)}
        log(f"[bench] mxfp4 T={T}: {rows[f'T{T}']}")
        del x, y, ws
    del w1p, w1s, w2p, w2s, xa, wg
    torch.cuda.empty_cache()
    return rows


def _time_calls(fn, iters, warmup=3):
    """Mean ms of fn() over iters calls, hip events on torch's current stream
    (the stream every amdmoe wrapper launches on by default)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def sweep(amdmoe, synth, iters, only=None):
    """Every MoE / DSA configuration of BASELINE.json, one row each (only
    those whose row name matches the regular expression `only`, if given:
    a profiler run can then cover one configuration alone).

    floor_ms = max(algorithmic HBM bytes / 8 TB/s, FLOPs / dense peak) --
    the roofline of the whole layer; attainable = floor_ms / ms."""
    import re

    import torch
    rows = []

    def want(name):
        return only is None or re.search(only, name) is not None

    def row(name, dtype, T, E, K, D, I, ms, w_bytes, act_bytes, peak, active):
        flops = 6 * T * K * D * I
        nbytes = w_bytes + act_bytes
        floor = max(nbytes / HBM_PEAK, flops / peak) * 1e3
        r = {"config": name, "dtype": dtype, "T": T, "E": E, "K": K, "D": D, "I": I,
             "experts_active": active, "ms": round(ms, 4),
             "tokens_per_s": round(T / (ms * 1e-3), 1),
             "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
             "mfma_peak_frac": round(flops / (ms * 1e-3) / peak, 4),
             "hbm_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
             "floor_ms": round(floor, 4), "attainable_frac": round(floor / ms, 4)}
        log(f"[sweep] {name:34s} {ms:9.4f} ms  {r['tokens_per_s']:12.1f} tok/s  "
            f"{r['tflops']:8.2f} TFLOP/s  {100 * r['mfma_peak_frac']:5.1f}% peak  "
            f"{100 * r['attainable_frac']:5.1f}% of floor {floor:.4f} ms")
        rows.append(r)

    def active_experts(idx_fn, T, E, K):
        idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
        wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
        idx_fn(idx, wts)
        torch.cuda.synchronize()
        return int(torch.unique(idx).numel())

    # tiny and medium fp32 (reference signature: no gate bias), medium bf16 with bias
    for name, (T, E, K, D, I) in (("tiny_fp32", (4, 4, 2, 64, 128)),
                                  ("medium_fp32", (512, 8, 2, 1024, 2048))):
        if not want(name):
            continue
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        x = torch.randn((T, D), generator=g, device="cuda")
        wg = torch.randn((E, D), generator=g, device="cuda") / D ** 0.5
        w1 = torch.randn((E, 2 * I, D), generator=g, device="cuda") / D ** 0.5
        w2 = torch.randn((E, D, I), generator=g, device="cuda") / I ** 0.5
        y = torch.empty((T, D), device="cuda")
        cfg = amdmoe.moe_config(T, E, K, D, I)
        ws = amdmoe.alloc_workspace(cfg, amdmoe.AMDMOE_DTYPE_F32)
        act = active_experts(lambda i, w: amdmoe.moe_gate_f32(x, wg, i, w, cfg), T, E, K)
        ms = _time_calls(lambda: amdmoe.moe_forward_f32(x, wg, w1, w2, y, cfg, ws=ws), iters)
        row(name, "f32", T, E, K, D, I, ms, act * 3 * I * D * 4 + E * D * 4,
            2 * T * D * 4, 157.3e12, act)
        del x, wg, w1, w2, y, ws
    bf16_cfgs = [("medium_bf16_bias", (512, 8, 2, 1024, 2048), True)]
    bf16_cfgs += [(f"mixtral_bf16_T{T}", (T, 8, 2, 4096, 14336), False) for T in (16, 256, 4096)]
    layer, packed = None, None
    for name, (T, E, K, D, I), bias in bf16_cfgs:
        # the Mixtral rows come in both weight layouts: row-major (the
        # reference's) and fragment-block packed (amdmoe_pack_weights_bf16)
        lays = [(name, False)] + ([(name + "_packed", True)] if D == 4096 else [])
        lays = [(n, pk) for n, pk in lays if want(n)]
        if not lays:
            continue
        if layer is None or layer[0] != (E, D, I, bias) or layer[1].shape[0] < T:
            layer, packed = None, None
            torch.cuda.empty_cache()
            Tg = 4096 if D == 4096 else T
            layer = ((E, D, I, bias),) + synth.bf16_layer(Tg, E, D, I, seed=7, bias=bias)
        xa, wg, b, w1, w2 = layer[1:]
        if packed is None and any(pk for _, pk in lays):
            packed = (torch.empty_like(w1), torch.empty_like(w2))
            amdmoe.pack_weights_bf16(w1, packed[0])
            amdmoe.pack_weights_bf16(w2, packed[1])
        x = xa[:T].contiguous()
        y = torch.empty((T, D), dtype=torch.int16, device="cuda")
        cfg = amdmoe.moe_config(T, E, K, D, I)
        ws = amdmoe.alloc_workspace(cfg, amdmoe.AMDMOE_DTYPE_BF16)
        act = active_experts(lambda i, w: amdmoe.moe_gate_bf16x(x, wg, b, i, w, cfg), T, E, K)
        for n, pk in lays:
            if pk:
                fwd = lambda: amdmoe.moe_forward_bf16_packed(x, wg, b, packed[0], packed[1], y, cfg,
                                                             ws=ws)
            else:
                fwd = lambda: amdmoe.moe_forward_bf16(x, wg, b, w1, w2, y, cfg, ws=ws)
            ms = _time_calls(fwd, iters)
            row(n, "bf16", T, E, K, D, I, ms, act * 3 * I * D * 2 + E * D * 4,
                2 * T * D * 2, 2.5e15, act)
        del x, y, ws
    layer, packed = None, None
    torch.cuda.empty_cache()
    # DeepSeek-V3 fp8 block-scale, packed (headline layout) and row-major
    E, K, D, I = 256, 8, 7168, 2048
    fp8_tokens = [T for T in (1, 64, 512, 4096, 8192)
                  if want(f"dsv3_fp8_T{T}_packed") or want(f"dsv3_fp8_T{T}_row-major")]
    mx_tokens = tuple(T for T in (1, 64, 512, 4096, 8192) if want(f"dsv3_mxfp4_T{T}"))
    if not fp8_tokens:
        return _sweep_mx(amdmoe, synth, iters, mx_tokens, row, rows)
    w1q, w1s, w2q, w2s = synth.dsv3_weights(E, D, I, seed=1234)
    w1p, w2p = torch.empty_like(w1q), torch.empty_like(w2q)
    amdmoe.pack_weights_fp8(w1q, w1p)
    amdmoe.pack_weights_fp8(w2q, w2p)
    xa, wg = synth.dsv3_inputs(8192, E, D, seed=99)
    for T in fp8_tokens:
        x = xa[:T].contiguous()
        y = torch.empty((T, D), dtype=torch.int16, device="cuda")
        cfg = amdmoe.moe_config(T, E, K, D, I)
        ws = amdmoe.alloc_workspace(cfg, amdmoe.AMDMOE_DTYPE_FP8)
        act = active_experts(lambda i, w: amdmoe.moe_gate_bf16(x, wg, i, w, cfg), T, E, K)
        wb = act * (3 * I * D + ((2 * I // 128) * (D // 128) + (D // 128) * (I // 128)) * 4) + E * D * 2
        for lay, (a1, a2, fwd) in (("packed", (w1p, w2p, amdmoe.moe_forward_fp8_packed)),
                                   ("row-major", (w1q, w2q, amdmoe.moe_forward_fp8))):
            if not want(f"dsv3_fp8_T{T}_{lay}"):
                continue
            ms = _time_calls(lambda: fwd(x, wg, a1, w1s, a2, w2s, y, cfg, ws=ws), iters)
            row(f"dsv3_fp8_T{T}_{lay}", "fp8_e4m3", T, E, K, D, I, ms, wb, 2 * T * D * 2,
                FP8_PEAK, act)
        del x, y, ws
    del w1q, w1s, w2q, w2s, w1p, w2p, xa, wg
    torch.cuda.empty_cache()
    return _sweep_mx(amdmoe, synth, iters, mx_tokens, row, rows)


def _sweep_mx(amdmoe, synth, iters, tokens, row, rows):
    """The MXFP4 rows of the sweep."""
    if not tokens:
        return rows
    for name, r in mxfp4_bench(amdmoe, synth, iters, tokens=tokens).items():
        T = int(name[1:])
        row(f"dsv3_mxfp4_{name}", "mxfp4", T, 256, 8, 7168, 2048, r["ms"],
            r["experts_active"] * 3 * 2048 * 7168 * (0.5 + 1 / 32) + 256 * 7168 * 2, 2 * T * 7168 * 2,
            FP8_PEAK, r["experts_active"])
    return rows


def kernel_label(name):
    """Short label of a demangled kernel name from a rocprofv3 CSV."""
    import re
    base = name.split("(")[0].replace("void ", "").replace("amdmoe::", "").strip()
    m = re.match(r"grouped_gemm_kernel<(\d), (\d), (true|false)>", base)
    if m:
        dt = ("f32", "bf16", "fp8", "MX")[int(m.group(1))]
        mode = ("UP", "DOWN")[int(m.group(2))]
        lay = "packed" if m.group(3) == "true" else "row-major"
        return f"grouped_gemm_kernel<{dt}, {mode}, {lay}>"
    m = re.match(r"grouped_gemm_bf16_w4_kernel<(\d)>", base)
    if m:
        return f"grouped_gemm_bf16_w4_kernel<{('UP', 'DOWN')[int(m.group(1))]}>"
    m = re.match(r"indexer_topk_kernel<(\d+), (\d)>", base)
    if m:
        return f"indexer_topk_kernel<{m.group(1)}, {('full', 'part', 'merge')[int(m.group(2))]}>"
    return base


def pmc_averages(csv_dir):
    """{kernel label: {counter: mean per dispatch}} of a rocprofv3 --pmc run
    (each counter summed over its hardware-instance rows per dispatch, then
    averaged over the kernel's dispatches), with "dispatches" and, when the
    CSV has timestamps, "duration_us"."""
    import csv
    import glob
    from collections import defaultdict
    files = glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {csv_dir}")
    per = defaultdict(lambda: defaultdict(float))
    dur = {}
    for fn in files:
        with open(fn) as f:
            for r in csv.DictReader(f):
                key = (kernel_label(r["Kernel_Name"]), r["Dispatch_Id"])
                per[key][r["Counter_Name"]] += float(r["Counter_Value"])
                if r.get("End_Timestamp"):
                    dur[key] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
    agg = defaultdict(lambda: defaultdict(list))
    for key, cv in per.items():
        for c, v in cv.items():
            agg[key[0]][c].append(v)
        if key in dur:
            agg[key[0]]["duration_us"].append(dur[key])
    return {k: dict({c: sum(v) / len(v) for c, v in cs.items()},
                    dispatches=max(len(v) for v in cs.values())) for k, cs in agg.items()}


def traffic_summary(fetch_dir, write_dir, out_md, out_json, command,
                    title="HBM traffic per launch: DSV3 fp8 MoE layer, T=4096 (+ DSA decode)"):
    """HBM bytes per launch from a FETCH_SIZE run and a WRITE_SIZE run of the
    same command with --calibrate-copy: the 1 GiB device-to-device copy
    (rocclr copyBuffer dispatches, 1 GiB read + 1 GiB written in all) gives
    the factor from each counter's KiB to true bytes."""
    fa, wa = pmc_averages(fetch_dir), pmc_averages(write_dir)
    cal = [k for k in fa if "copyBuffer" in k]
    if not cal:
        raise SystemExit("no copy-kernel dispatches: run with --calibrate-copy")
    c = cal[0]
    per_dispatch_kib = (1 << 30) / 1024 / fa[c]["dispatches"]
    f_fetch = per_dispatch_kib / fa[c]["FETCH_SIZE"]
    f_write = per_dispatch_kib / wa[c]["WRITE_SIZE"]
    rows, kernels = [], {}
    for k in sorted(fa, key=lambda k: -fa[k]["FETCH_SIZE"]):
        if not k or k.startswith("at::") or k.startswith("rocprim") or k not in wa or k == c:
            continue
        fb = fa[k]["FETCH_SIZE"] * 1024 * f_fetch
        wb = wa[k]["WRITE_SIZE"] * 1024 * f_write
        kernels[k] = {"fetch_kib": fa[k]["FETCH_SIZE"], "write_kib": wa[k]["WRITE_SIZE"],
                      "bytes": fb + wb}
        rows.append(f"| `{k}` | {fa[k]['FETCH_SIZE']:.4g} | {wa[k]['WRITE_SIZE']:.4g} | "
                    f"{(fb + wb) / 1e9:.3f} GB |")
    lines = [f"# {title}", "",
             "Two counter runs and the summary (from the repository root on the GPU box):", "",
             "```", command, "```", "",
             f"Calibration: `--calibrate-copy` runs one 1 GiB device-to-device copy first "
             f"(`{c}`, {fa[c]['dispatches']} dispatches).  Per dispatch FETCH_SIZE reads "
             f"{fa[c]['FETCH_SIZE']:.0f} KiB and WRITE_SIZE {wa[c]['WRITE_SIZE']:.0f} KiB of "
             f"{per_dispatch_kib:.0f} KiB moved each way, so bytes = FETCH_SIZE x 1024 x "
             f"{f_fetch:.2f} + WRITE_SIZE x 1024 x {f_write:.2f}.", "",
             "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes / launch (calibrated) |",
             "|---|---:|---:|---:|"] + rows
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(out_json, "w") as f:
        json.dump({"factor_fetch": f_fetch, "factor_write": f_write, "kernels": kernels}, f, indent=1)
    print("\n".join(lines))


def stats_summary(csv_dir, out_md, title, command):
    """This library's kernels from a rocprofv3 --kernel-trace --stats run
    (kernel_stats.csv) as a markdown table."""
    import csv
    import glob
    files = glob.glob(os.path.join(csv_dir, "**", "*kernel_stats.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_stats.csv under {csv_dir}")
    lines = [f"# {title}", "", "Command (from the repository root on the GPU box):", "", "```",
             command, "```", "",
             "Rows: this library's kernels (torch and rocprim kernels of the synthetic-data "
             "setup omitted).", "",
             "| kernel | calls | average us | min us | max us | total share |",
             "|---|---:|---:|---:|---:|---:|"]
    for r in csv.DictReader(open(files[0])):
        k = kernel_label(r["Name"])
        if not k or k.startswith("at::") or k.startswith("rocprim") or "elementwise" in k:
            continue
        lines.append(f"| `{k}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                     f"{float(r['Percentage']):.1f}% |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def pmc_summary(csv_dir, out_md, title, command):
    """Per-kernel averages of a rocprofv3 --pmc run (counter_collection CSV):
    each counter summed over its dimension rows per dispatch, then averaged
    over the kernel's dispatches.  Writes a markdown table to out_md."""
    import csv
    import glob
    from collections import defaultdict
    files = glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {csv_dir}")
    per = defaultdict(lambda: defaultdict(float))   # (kernel, dispatch) -> counter -> value
    dur = {}
    for fn in files:
        with open(fn) as f:
            for r in csv.DictReader(f):
                key = (kernel_label(r["Kernel_Name"]), r["Dispatch_Id"])
                per[key][r["Counter_Name"]] += float(r["Counter_Value"])
                if r.get("End_Timestamp"):
                    dur[key] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
    agg = defaultdict(lambda: defaultdict(list))
    counters = []
    for (k, _d), cv in per.items():
        for c, v in cv.items():
            agg[k][c].append(v)
            if c not in counters:
                counters.append(c)
        if (k, _d) in dur:
            agg[k]["duration_us"].append(dur[(k, _d)])
    if dur:
        counters.append("duration_us")
    # derived columns, where their counters were collected:
    #   clock GHz   = GRBM_GUI_ACTIVE / 8 (one count per XCD) / duration
    #   MFMA busy   = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs)
    #   MFMA TF/s   = (SQ_INSTS_VALU_MFMA_MOPS_F8 + _BF16) x 512 / duration
    #   LDS conflict = SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS
    #   L2 hit      = TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)
    derived = []
    have = set(counters)
    if {"GRBM_GUI_ACTIVE", "duration_us"} <= have:
        derived.append(("clock GHz", lambda a: a["GRBM_GUI_ACTIVE"] / 8 / a["duration_us"] / 1e3))
    if {"GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES"} <= have:
        derived.append(("MFMA busy", lambda a: a["SQ_VALU_MFMA_BUSY_CYCLES"] / (a["GRBM_GUI_ACTIVE"] / 8 * 1024)))
    mops = [c for c in ("SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_BF16") if c in have]
    if mops and "duration_us" in have:
        derived.append(("MFMA TF/s", lambda a: sum(a[c] for c in mops) * 512 / (a["duration_us"] * 1e-6) / 1e12))
    if {"SQ_LDS_BANK_CONFLICT", "SQ_ACTIVE_INST_LDS"} <= have:
        derived.append(("LDS conflict", lambda a: a["SQ_LDS_BANK_CONFLICT"] / max(a["SQ_ACTIVE_INST_LDS"], 1.0)))
    if {"TCC_HIT_sum", "TCC_MISS_sum"} <= have:
        derived.append(("L2 hit", lambda a: a["TCC_HIT_sum"] / max(a["TCC_HIT_sum"] + a["TCC_MISS_sum"], 1.0)))
    lines = [f"# {title}", "", "Command (from the repository root on the GPU box):", "", "```",
             command, "```", "",
             "Per kernel: each counter summed over its hardware instances per dispatch, averaged "
             "over the kernel's dispatches."]
    if derived:
        lines += ["", "Derived: clock GHz = GRBM_GUI_ACTIVE / 8 (one count per XCD) / duration; "
                  "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs); "
                  "MFMA TF/s = MFMA_MOPS x 512 / duration (padded rows included); LDS conflict = "
                  "SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS; L2 hit = TCC_HIT / (TCC_HIT + TCC_MISS).  "
                  "For kernels of a few microseconds GRBM_GUI_ACTIVE also counts the dispatch, so their "
                  "clock column reads high.  Rows: this library's kernels (torch and rocprim kernels of "
                  "the synthetic-data setup omitted)."]
    lines += ["", "| kernel | dispatches | " + " | ".join(counters + [d[0] for d in derived]) + " |",
              "|---|---:|" + "---:|" * (len(counters) + len(derived))]
    for k in sorted(agg, key=lambda k: -max(sum(v) for v in agg[k].values())):
        if not k or k.startswith("at::") or k.startswith("rocprim"):
            continue  # torch / rocprim kernels of the synthetic-data setup
        n = max(len(v) for v in agg[k].values())
        avg = {c: sum(agg[k][c]) / len(agg[k][c]) if agg[k][c] else float("nan") for c in counters}
        vals = [avg[c] for c in counters]
        dv = []
        for name, f in derived:
            try:
                x = f(avg)
                dv.append(f"{100 * x:.1f}%" if name in ("MFMA busy", "LDS conflict", "L2 hit") else f"{x:.3g}")
            except (ZeroDivisionError, KeyError):
                dv.append("-")
        lines.append(f"| `{k}` | {n} | " + " | ".join([f"{v:.4g}" for v in vals] + dv) + " |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-summary":
        # bench.py --pmc-summary CSV_DIR OUT_MD TITLE COMMAND
        pmc_summary(*sys.argv[2:6])
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--stats-summary":
        # bench.py --stats-summary CSV_DIR OUT_MD TITLE COMMAND
        stats_summary(*sys.argv[2:6])
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--traffic-summary":
        # bench.py --traffic-summary FETCH_DIR WRITE_DIR OUT_MD OUT_JSON COMMAND [TITLE]
        traffic_summary(*sys.argv[2:8])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--sweep", metavar="JSON",
                    help="instead of the headline line, time every BASELINE MoE config and "
                         "write the rows to JSON")
    ap.add_argument("--only", metavar="REGEX",
                    help="with --sweep: only the rows whose config name matches (e.g. one "
                         "configuration per profiler run)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--cpu-sample", type=int, default=1024, help="tokens for the CPU baseline (0: skip)")
    ap.add_argument("--skip-dsa", action="store_true")
    ap.add_argument("--skip-mx", action="store_true", help="skip the MXFP4 layer rows")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "moe_dsv3_fp8_T4096_traffic.json"),
                    help="measured HBM bytes per launch (FETCH_SIZE/WRITE_SIZE counter runs, "
                         "calibrated on a copy kernel; see the .md beside it)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one 1 GiB device-to-device copy kernel (a known-size "
                         "reference for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    import torch

    import amdmoe
    import synth
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.sweep:
        import re
        rows = sweep(amdmoe, synth, args.steps, args.only)
        md = ["| config | ms | tokens/s | TFLOP/s | % dense peak | floor ms | % of floor |",
              "|---|---:|---:|---:|---:|---:|---:|"]
        for r in rows:
            md.append(f"| {r['config']} | {r['ms']:.4f} | {r['tokens_per_s']:.0f} | {r['tflops']:.1f} | "
                      f"{100 * r['mfma_peak_frac']:.1f}% | {r['floor_ms']:.4f} | "
                      f"{100 * r['attainable_frac']:.1f}% |")
        if args.only is None or re.search(args.only, "dsa_decode_B64_H128_S2048"):
            d = {"config": "dsa_decode_B64_H128_S2048", **dsa_bench(amdmoe, synth)}
            log(f"[sweep] dsa: {d}")
            rows.append(d)
            md.append(f"| {d['config']} (bf16, paged) | {d['us_per_call'] / 1e3:.4f} | "
                      f"{d['queries_per_s']:.0f} queries/s | {100 * d['bf16_mfma_frac']:.1f}% of bf16 | | "
                      f"{0.0212:.4f} | {100 * d['hbm_frac']:.1f}% of HBM peak |")
        if args.only is None or re.search(args.only, "dsa_indexer"):
            ix = indexer_bench(amdmoe, synth)
            log(f"[sweep] dsa indexer: {ix}")
            rows.append({"config": "dsa_indexer", **ix})
            md.append(f"| dsa_indexer ({ix['shape']}, fp8) | {ix['us_per_call'] / 1e3:.4f} | "
                      f"{ix['queries_per_s']:.0f} queries/s | {100 * ix['fp8_mfma_frac']:.1f}% of fp8 | | | "
                      f"{100 * ix['hbm_frac']:.1f}% of HBM peak |")
        with open(args.sweep, "w") as f:
            json.dump(rows, f, indent=1)
        with open(os.path.splitext(args.sweep)[0] + ".md", "w") as f:
            f.write("\n".join(md) + "\n")
        return
    T, E, K, D, I = args.tokens, 256, 8, 7168, 2048
    log(f"[bench] generating DSV3 fp8 weights E={E} D={D} I={I}")
    w1q, w1s, w2q, w2s = synth.dsv3_weights(E, D, I, seed=1234)
    x, wg = synth.dsv3_inputs(T, E, D, seed=99)
    cfg = amdmoe.moe_config(T, E, K, D, I)
    ws = amdmoe.alloc_workspace(cfg, amdmoe.AMDMOE_DTYPE_FP8)
    y = torch.empty((T, D), dtype=torch.int16, device="cuda")

    # active experts (for the algorithmic byte count)
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
    amdmoe.moe_gate_bf16(x, wg, idx, wts, cfg)
    torch.cuda.synchronize()
    e_active = int(torch.unique(idx).numel())

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        amdmoe.moe_forward_fp8(x, wg, w1q, w1s, w2q, w2s, y, cfg, ws=ws)
    torch.cuda.synchronize()

    def timed(forward):
        # the step time comes from a pass without stage events (their seven
        # event records per step are instrumentation, not the layer); the
        # stage times from a second pass of the same length with them
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for i in range(args.steps):
            forward()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        stage = [amdmoe.StageEvents() for _ in range(args.steps)]
        torch.cuda.synchronize()
        for i in range(args.steps):
            stage[i].arm()
            forward()
        amdmoe.StageEvents.disarm()
        torch.cuda.synchronize()
        per_stage = {n: sum(s.stage_ms()[n] for s in stage) / args.steps for n in amdmoe.StageEvents.NAMES}
        log(f"[bench] {ms:.4f} ms/step; stage ms: " + ", ".join(f"{k}={v:.4f}" for k, v in per_stage.items()))
        return ms, per_stage

    # headline: the expert weights in fragment-block order, packed once at
    # load (amdmoe_pack_weights_fp8; the DSV3 path's in-memory format)
    w1p, w2p = torch.empty_like(w1q), torch.empty_like(w2q)
    amdmoe.pack_weights_fp8(w1q, w1p)
    amdmoe.pack_weights_fp8(w2q, w2p)
    for _ in range(args.warmup):
        amdmoe.moe_forward_fp8_packed(x, wg, w1p, w1s, w2p, w2s, y, cfg, ws=ws)
    log(f"[bench] timing {args.steps} steps (packed weights)")
    ms, per_stage = timed(lambda: amdmoe.moe_forward_fp8_packed(x, wg, w1p, w1s, w2p, w2s, y, cfg, ws=ws))
    del w1p, w2p

    # the same layer on row-major weights (the drop-in layout of the C ABI)
    log(f"[bench] timing {args.steps} steps (row-major weights)")
    ms_r, per_stage_r = timed(lambda: amdmoe.moe_forward_fp8(x, wg, w1q, w1s, w2q, w2s, y, cfg, ws=ws))

    flops = 6 * T * K * D * I
    layer_bytes, up_bytes = moe_bytes(T, e_active, K, D, I)
    up_ms = per_stage["gemm_up"]
    achieved = up_bytes / (up_ms * 1e-3) / 1e9
    traffic = None
    if args.traffic and os.path.exists(args.traffic) and T == 4096:
        traffic = json.load(open(args.traffic))["kernels"].get(ROOF_KERNEL, {}).get("bytes")
    result = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {"workload": f"dsv3_fp8_blockscale_moe_T{T}", "T": T, "E": E, "K": K, "D": D,
                   "I": I, "experts_active": e_active,
                   "weights": "e4m3 + fp32 128x128 scales; W1/W2 in MFMA fragment-block order, "
                              "packed once at load (amdmoe_pack_weights_fp8)"},
        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "fp8_peak_frac": round(flops / (ms * 1e-3) / FP8_PEAK, 4),
        "layer_hbm_frac": round(layer_bytes / (ms * 1e-3) / HBM_PEAK, 4),
        "stage_ms": {k: round(v, 4) for k, v in per_stage.items()},
        "row_major_weights": {"note": "same layer, W1/W2 row-major as given to the drop-in "
                                      "amdmoe_moe_forward_fp8",
                              "value": round(T / (ms_r * 1e-3), 1), "ms_per_step": round(ms_r, 4),
                              "fp8_peak_frac": round(flops / (ms_r * 1e-3) / FP8_PEAK, 4),
                              "stage_ms": {k: round(v, 4) for k, v in per_stage_r.items()}},
        "roofline": {"kernel": ROOF_KERNEL + " (GEMM1 + SwiGLU + requant)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved / (HBM_PEAK / 1e9), 4),
                     "traffic": round(traffic) if traffic else None, "algorithmic_bytes": up_bytes},
    }
    if not args.skip_mx:
        log("[bench] MXFP4 layer")
        result["mxfp4_layer"] = mxfp4_bench(amdmoe, synth)
    if not args.skip_dsa:
        log("[bench] DSA decode")
        result["dsa_decode"] = dsa_bench(amdmoe, synth, cpu=args.cpu_sample > 0)
        log("[bench] DSA indexer")
        result["dsa_indexer"] = indexer_bench(amdmoe, synth)
    if args.cpu_sample > 0:
        log(f"[bench] CPU baseline on {args.cpu_sample} tokens")
        result["cpu_baseline"] = cpu_baseline(x, wg, w1q, w1s, w2q, w2s, K, args.cpu_sample)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
