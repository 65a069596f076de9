"""Synthetic inputs of the BASELINE workloads, generated on the GPU.

torch supplies device memory and seeded normals (plumbing); the fp8 block
quantisation of the expert weights runs through the library's own HIP
kernel (amdmoe_quant_weight_fp8).  Shapes and distributions:
  - DeepSeek-V3 fp8 layer: W1 [E,2I,D], W2 [E,D,I] ~ N(0, 1/fan_in), e4m3
    with fp32 128x128 scales u*amax/448, u ~ U(0.5, 2); x ~ N(0,1) bf16;
    Wg ~ N(0, 1/D) bf16.
  - Mixtral / medium bf16 layer: bf16 x ~ N(0,1), bf16 W ~ N(0, 1/fan_in),
    fp32 gate ~ N(0, 1/D); optional per-expert logit bias ~ N(0, 0.5^2).
  - DSA decode: bf16 latent cache ~ N(0,1) in pages, page table a random
    permutation of physical pages, indices uniform without replacement.
"""
import torch

import amdmoe


def _gen(seed, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def dsv3_weights(E, D, I, seed=1234, device="cuda"):
    """fp8 block-scale expert weights, built one expert at a time."""
    g = _gen(seed, device)
    w1q = torch.empty((E, 2 * I, D), dtype=torch.uint8, device=device)
    w2q = torch.empty((E, D, I), dtype=torch.uint8, device=device)
    w1s = torch.empty((E, 2 * I // 128, D // 128), dtype=torch.float32, device=device)
    w2s = torch.empty((E, D // 128, I // 128), dtype=torch.float32, device=device)
    for e in range(E):
        w = torch.randn((2 * I, D), generator=g, device=device) * (1.0 / D ** 0.5)
        u = torch.rand((2 * I // 128, D // 128), generator=g, device=device) * 1.5 + 0.5
        amdmoe.quant_weight_fp8(w, u, w1q[e], w1s[e])
        w = torch.randn((D, I), generator=g, device=device) * (1.0 / I ** 0.5)
        u = torch.rand((D // 128, I // 128), generator=g, device=device) * 1.5 + 0.5
        amdmoe.quant_weight_fp8(w, u, w2q[e], w2s[e])
        del w, u
    torch.cuda.synchronize()
    return w1q, w1s, w2q, w2s


def mxfp4_weights(E, D, I, seed=1234, device="cuda", packed=True):
    """MXFP4 expert weights of the DSV3 layer shape: W1 [E,2I,D], W2 [E,D,I]
    ~ N(0, 1/fan_in) quantised by amdmoe_quant_weight_mxfp4 (E2M1, E8M0 per
    32 along K), built one expert at a time; packed (fragment order,
    amdmoe_pack_weights_mxfp4) unless packed=False, which returns the
    row-major codes and scales."""
    g = _gen(seed, device)
    w1q = torch.empty((E, 2 * I, D // 2), dtype=torch.uint8, device=device)
    w1s = torch.empty((E, 2 * I, D // 32), dtype=torch.uint8, device=device)
    w2q = torch.empty((E, D, I // 2), dtype=torch.uint8, device=device)
    w2s = torch.empty((E, D, I // 32), dtype=torch.uint8, device=device)
    for e in range(E):
        w = torch.randn((2 * I, D), generator=g, device=device) * (1.0 / D ** 0.5)
        amdmoe.quant_weight_mxfp4(w, w1q[e], w1s[e])
        w = torch.randn((D, I), generator=g, device=device) * (1.0 / I ** 0.5)
        amdmoe.quant_weight_mxfp4(w, w2q[e], w2s[e])
        del w
    if not packed:
        torch.cuda.synchronize()
        return w1q, w1s, w2q, w2s
    out = []
    for q, s in ((w1q, w1s), (w2q, w2s)):
        qp, sp = torch.empty_like(q), torch.empty_like(s)
        amdmoe.pack_weights_mxfp4(q, s, qp, sp)
        out += [qp, sp]
    torch.cuda.synchronize()
    return tuple(out)


def dsv3_inputs(T, E, D, seed=99, device="cuda"):
    """x bf16 [T,D] ~ N(0,1) and gate bf16 [E,D] ~ N(0, 1/D), as int16 bit views."""
    g = _gen(seed, device)
    x = torch.randn((T, D), generator=g, device=device).to(torch.bfloat16)
    wg = (torch.randn((E, D), generator=g, device=device) * (1.0 / D ** 0.5)).to(torch.bfloat16)
    return x.view(torch.int16), wg.view(torch.int16)


def bf16_layer(T, E, D, I, seed=7, bias=False, device="cuda"):
    """bf16 x, W1, W2 (int16 bit views), fp32 gate and optional fp32 bias."""
    g = _gen(seed, device)
    x = torch.randn((T, D), generator=g, device=device).to(torch.bfloat16)
    wg = torch.randn((E, D), generator=g, device=device) * (1.0 / D ** 0.5)
    w1 = (torch.randn((E, 2 * I, D), generator=g, device=device) * (1.0 / D ** 0.5)).to(torch.bfloat16)
    w2 = (torch.randn((E, D, I), generator=g, device=device) * (1.0 / I ** 0.5)).to(torch.bfloat16)
    b = torch.randn((E,), generator=g, device=device) * 0.5 if bias else None
    return x.view(torch.int16), wg, b, w1.view(torch.int16), w2.view(torch.int16)


def dsa_paged(Q, H, Dc, Dp, S, page, ctx, seed=5, device="cuda"):
    """Paged bf16 latent cache and per-query logical indices.

    Each query owns ctx tokens = ctx/page pages; the page table maps them to
    a random permutation of all physical pages; each query selects S
    distinct logical positions (unsorted)."""
    g = _gen(seed, device)
    pps = ctx // page
    n_pages = Q * pps
    cache = torch.randn((n_pages * page, Dc + Dp), generator=g, device=device).to(torch.bfloat16)
    pt = torch.randperm(n_pages, generator=g, device=device).to(torch.int32).reshape(Q, pps)
    logical = torch.stack([torch.randperm(ctx, generator=g, device=device)[:S] for _ in range(Q)])
    logical = logical.to(torch.int32).contiguous()
    qn = torch.randn((Q, H, Dc), generator=g, device=device).to(torch.bfloat16)
    qp = torch.randn((Q, H, Dp), generator=g, device=device).to(torch.bfloat16)
    return (qn.view(torch.int16), qp.view(torch.int16), cache.view(torch.int16), pt, logical, pps)


def dsa_queries(Q, H, Dc, Dp, S, ctx, seed, device="cuda"):
    """Another decode batch over an existing cache (dsa_paged's layout):
    bf16 q_nope / q_pe ~ N(0,1) and S distinct logical positions per query."""
    g = _gen(seed, device)
    logical = torch.stack([torch.randperm(ctx, generator=g, device=device)[:S] for _ in range(Q)])
    qn = torch.randn((Q, H, Dc), generator=g, device=device).to(torch.bfloat16)
    qp = torch.randn((Q, H, Dp), generator=g, device=device).to(torch.bfloat16)
    return qn.view(torch.int16), qp.view(torch.int16), logical.to(torch.int32).contiguous()


def dsa_indexer(Q, Hi, ctx, page, seed=9, page_table=None, device="cuda"):
    """Lightning-indexer inputs: fp8 e4m3 query heads [Q,Hi,128] and keys
    [Q*ctx,128] (paged like the latent cache), each row quantised with one
    fp32 scale (amdmoe_quant_rows_fp8: amax/448), per-head weights
    ~ N(0, 1/Hi), and a page table (a random permutation of all pages unless
    one is given)."""
    g = _gen(seed, device)
    pps = ctx // page
    q = torch.randn((Q * Hi, 128), generator=g, device=device).to(torch.bfloat16)
    k = torch.randn((Q * ctx, 128), generator=g, device=device).to(torch.bfloat16)
    qc = torch.empty((Q * Hi, 128), dtype=torch.uint8, device=device)
    qs = torch.empty((Q * Hi, 1), dtype=torch.float32, device=device)
    kc = torch.empty((Q * ctx, 128), dtype=torch.uint8, device=device)
    ks = torch.empty((Q * ctx, 1), dtype=torch.float32, device=device)
    amdmoe.quant_rows_fp8(q.view(torch.int16), qc, qs)
    amdmoe.quant_rows_fp8(k.view(torch.int16), kc, ks)
    hw = torch.randn((Q, Hi), generator=g, device=device) * (1.0 / Hi ** 0.5)
    if page_table is None:
        page_table = torch.randperm(Q * pps, generator=g, device=device).to(torch.int32).reshape(Q, pps)
    return (qc.reshape(Q, Hi, 128), qs.reshape(Q, Hi), hw.contiguous(), kc, ks.reshape(Q * ctx),
            page_table)
