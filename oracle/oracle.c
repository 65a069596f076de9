/*
 * CPU oracle for the MoE forward and DSA sparse-decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/, the
 * smoke() entry of __graft_entry__.py and the cpu_baseline leg of bench.py may
 * load it.  The product library (llm-sys-project_amd/) never links, loads or
 * falls back to it.
 *
 * It restates, op for op, the reference's own CPU implementation:
 *   - cpu_softmax           tests/test_moe.cu:14-20  (identical in tests/test_dsa.cu:15-21)
 *   - cpu_silu              tests/test_moe.cu:22-24
 *   - cpu_moe_forward       tests/test_moe.cu:32-140
 *   - cpu_dsa_forward       tests/test_dsa.cu:23-68
 *   - random_fill           utils/cuda_utils.cuh:56-60   (glibc rand(), same expression)
 *   - gen_sparse_indices    tests/test_dsa.cu:73-85
 *   - max/mean_abs_error    utils/cuda_utils.cuh:70-85
 * and the reference's DSA GPU stage kernels (their loops are scalar too):
 *   - dsa_kv_gather         kernels/dsa/naive_dsa.cu:13-60
 *   - dsa_dot_*             kernels/dsa/naive_dsa.cu:89-134, 157-206, 208-276
 *   - dsa_softmax           kernels/dsa/naive_dsa.cu:278-296
 *   - dsa_output_proj       kernels/dsa/naive_dsa.cu:300-316
 * and adds the BASELINE-defined formats the reference does not have:
 *   - OCP fp8 e4m3 ("E4M3FN") encode/decode, bf16 round-to-nearest-even,
 *   - 1x128 activation / 128x128 weight block quantisation,
 *   - the bf16 and fp8-block-scale variants of the MoE forward,
 *   - paged address translation for the DSA decode.
 *
 * Build with -O2 -ffp-contract=off (no -ffast-math, no -march=native) so the
 * arithmetic is plain IEEE binary32 in source order, like the reference's
 * scalar loops.  OpenMP parallel loops only split independent output rows;
 * every output element keeps the reference's accumulation order, so results
 * are bit-identical for any thread count.
 *
 * Parity pins (see tests/test_oracle.py): exhaustive fp8 code table vs the
 * closed-form decode; bf16 RNE closed form; routing known-answer tests
 * (x=0, duplicated gate rows, K=E, E=1); brute-force counting sort for the
 * permutation; float64 textbook GEMM/SwiGLU for the expert FFN; identical
 * experts => y = FFN(x); DSA S=1, q=0, S=N-dense and index-permutation
 * invariance; paged == flat translation; DSA stages: gather == fancy
 * indexing, dots and output projection == float64 products (one-hot inputs
 * exact), softmax == float64 softmax (uniform rows exact), and the stages
 * composed as naive_dsa.cu:435-474 == cpu_dsa_forward.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* generators (glibc rand(): same expression as the reference)         */
/* ------------------------------------------------------------------ */

/* Threads of the oracle's parallel loops (the reference's CPU oracle is
 * single-threaded; 1 reproduces it, more only split independent rows or
 * output columns, so results are identical for any count). */
EXPORT void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
EXPORT int orc_get_threads(void) { return omp_get_max_threads(); }

/* utils/cuda_utils.cuh:56-60 */
EXPORT void orc_srand(unsigned seed) { srand(seed); }

EXPORT void orc_random_fill(float* data, long n, float lo, float hi) {
    for (long i = 0; i < n; i++)
        data[i] = lo + (float)rand() / RAND_MAX * (hi - lo);
}

/* tests/test_dsa.cu:73-85: partial Fisher-Yates per query, then sort. */
static int cmp_int(const void* a, const void* b) {
    int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

EXPORT void orc_gen_sparse_indices(int* indices, int Q, int S, int total_kv, int sort_rows) {
    int* pool = (int*)malloc(sizeof(int) * (size_t)total_kv);
    for (int q = 0; q < Q; q++) {
        for (int i = 0; i < total_kv; i++) pool[i] = i;
        for (int i = 0; i < S; i++) {
            int j = i + rand() % (total_kv - i);
            int t = pool[i]; pool[i] = pool[j]; pool[j] = t;
        }
        if (sort_rows) qsort(pool, (size_t)S, sizeof(int), cmp_int);
        for (int s = 0; s < S; s++) indices[(size_t)q * S + s] = pool[s];
    }
    free(pool);
}

/* utils/cuda_utils.cuh:70-85 */
EXPORT float orc_max_abs_error(const float* a, const float* b, long n) {
    float mx = 0.0f;
    for (long i = 0; i < n; i++) {
        float d = fabsf(a[i] - b[i]);
        if (d > mx) mx = d;
    }
    return mx;
}

EXPORT float orc_mean_abs_error(const float* a, const float* b, long n) {
    double sum = 0.0;
    for (long i = 0; i < n; i++) sum += fabsf(a[i] - b[i]);
    return (float)(sum / (double)n);
}

/* ------------------------------------------------------------------ */
/* number formats                                                      */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16: upper 16 bits of binary32, round to nearest even; NaN stays NaN. */
EXPORT uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

EXPORT float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

EXPORT void orc_f32_to_bf16_array(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

EXPORT void orc_bf16_to_f32_array(const uint16_t* in, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* OCP 8-bit FP, E4M3 ("E4M3FN"): bias 7, no infinities, S.1111.111 = NaN,
 * max normal 448 = S.1111.110, subnormals m/8 * 2^-6. */
EXPORT float orc_e4m3_to_f32(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m / 8.0f, -6);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

/* Round to nearest even with saturation to +-448 (the "satfinite" mode). */
EXPORT uint8_t orc_f32_to_e4m3(float f) {
    if (isnan(f)) return 0x7f;
    uint8_t sign = signbit(f) ? 0x80 : 0x00;
    float a = fabsf(f);
    if (a >= 448.0f) return sign | 0x7e;
    /* smallest normal is 2^-6; subnormal spacing is 2^-9 */
    int e;
    frexpf(a, &e);              /* a = f * 2^e, f in [0.5,1) => exponent e-1 */
    int ex = e - 1;
    if (ex < -6) ex = -6;       /* subnormal range shares the 2^-9 spacing */
    float step = ldexpf(1.0f, ex - 3);
    float q = a / step;         /* exact: power-of-two scaling */
    float r = rintf(q);         /* round half to even (default rounding mode) */
    float v = r * step;
    /* re-encode v (v <= 448 since 448 is representable and a < 448) */
    if (v == 0.0f) return sign;
    int e2;
    frexpf(v, &e2);
    int ex2 = e2 - 1;
    uint8_t code;
    if (ex2 < -6) {
        code = (uint8_t)(int)(v / ldexpf(1.0f, -9));          /* subnormal mantissa */
    } else {
        int mant = (int)(v / ldexpf(1.0f, ex2 - 3)) - 8;      /* 0..7 */
        code = (uint8_t)(((ex2 + 7) << 3) | mant);
    }
    return sign | code;
}

EXPORT void orc_e4m3_to_f32_array(const uint8_t* in, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = orc_e4m3_to_f32(in[i]);
}

/* 1x128 block quantisation of rows: scale = amax/448, q = e4m3(v/scale).
 * An all-zero block gets scale 1 so that dequantisation stays exact. */
EXPORT void orc_quant_rows_1x128(const float* x, long rows, int cols,
                                 uint8_t* q, float* scales) {
    int nb = cols / 128;
    for (long r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const float* src = x + r * cols + b * 128;
            float amax = 0.0f;
            for (int j = 0; j < 128; j++) amax = fmaxf(amax, fabsf(src[j]));
            float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            scales[r * nb + b] = s;
            for (int j = 0; j < 128; j++) q[r * cols + b * 128 + j] = orc_f32_to_e4m3(src[j] / s);
        }
    }
}

/* 128x128 block quantisation of a [rows, cols] weight with a per-block scale
 * multiplier u (BASELINE: u ~ U(0.5, 2)); scale = u * amax / 448. */
EXPORT void orc_quant_weight_128x128(const float* w, int rows, int cols, const float* u,
                                     uint8_t* q, float* scales) {
    int rb = rows / 128, cb = cols / 128;
    for (int i = 0; i < rb; i++) {
        for (int j = 0; j < cb; j++) {
            float amax = 0.0f;
            for (int r = 0; r < 128; r++)
                for (int c = 0; c < 128; c++)
                    amax = fmaxf(amax, fabsf(w[(size_t)(i * 128 + r) * cols + j * 128 + c]));
            float s = amax > 0.0f ? u[i * cb + j] * amax / 448.0f : 1.0f;
            scales[i * cb + j] = s;
            for (int r = 0; r < 128; r++)
                for (int c = 0; c < 128; c++) {
                    size_t o = (size_t)(i * 128 + r) * cols + j * 128 + c;
                    q[o] = orc_f32_to_e4m3(w[o] / s);
                }
        }
    }
}

/* ------------------------------------------------------------------ */
/* MoE: routing                                                        */
/* ------------------------------------------------------------------ */

/* tests/test_moe.cu:14-20 */
EXPORT void orc_softmax(float* data, int n) {
    float mx = -FLT_MAX;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, data[i]);
    float s = 0.0f;
    for (int i = 0; i < n; i++) { data[i] = expf(data[i] - mx); s += data[i]; }
    for (int i = 0; i < n; i++) data[i] /= s;
}

/* tests/test_moe.cu:22-24 */
static inline float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* Replace-min top-K over probabilities in ascending expert order, then
 * renormalise by the slot-order sum (tests/test_moe.cu:52-68). */
EXPORT void orc_topk_row(const float* p, int E, int K, int* idx, float* wt) {
    for (int k = 0; k < K; k++) { idx[k] = -1; wt[k] = -FLT_MAX; }
    for (int e = 0; e < E; e++) {
        float v = p[e];
        int min_k = 0;
        for (int k = 1; k < K; k++)
            if (wt[k] < wt[min_k]) min_k = k;
        if (v > wt[min_k]) { wt[min_k] = v; idx[min_k] = e; }
    }
    float s = 0.0f;
    for (int k = 0; k < K; k++) s += wt[k];
    if (s > 0.0f) for (int k = 0; k < K; k++) wt[k] /= s;
}

/* Gate logits (sequential fp32 sum over d, tests/test_moe.cu:42-45), an
 * optional per-expert bias (the BASELINE medium config's skew; the
 * reference has none), softmax, top-K.  x and Wg are fp32 here; the bf16
 * variants decode to fp32 first, which is exact.  probs_out (optional)
 * receives the softmax probabilities, logits_out the raw logits. */
EXPORT void orc_moe_route(const float* x, const float* Wg, const float* bias,
                          int T, int E, int K, int D,
                          int* idx, float* wts, float* logits_out, float* probs_out) {
    #pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)E);
        #pragma omp for schedule(static)
        for (int t = 0; t < T; t++) {
            for (int e = 0; e < E; e++) {
                float sum = 0.0f;
                for (int d = 0; d < D; d++)
                    sum += x[(size_t)t * D + d] * Wg[(size_t)e * D + d];
                if (bias) sum += bias[e];
                row[e] = sum;
                if (logits_out) logits_out[(size_t)t * E + e] = sum;
            }
            orc_softmax(row, E);
            if (probs_out) memcpy(probs_out + (size_t)t * E, row, sizeof(float) * (size_t)E);
            orc_topk_row(row, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
        }
        free(row);
    }
}

/* ------------------------------------------------------------------ */
/* MoE: permutation (the reference gather order, tests/test_moe.cu:76-83) */
/* ------------------------------------------------------------------ */

/* For each expert e ascending: tokens t ascending whose slot list holds e
 * (first matching slot k; a token is listed once per expert).
 * sorted_token[p], sorted_slot[p] = t*K + k, counts[e], offsets[E+1]. */
EXPORT void orc_moe_permute(const int* idx, int T, int K, int E,
                            int* counts, int* offsets, int* sorted_token, int* sorted_slot) {
    int p = 0;
    for (int e = 0; e < E; e++) {
        offsets[e] = p;
        int c = 0;
        for (int t = 0; t < T; t++) {
            for (int k = 0; k < K; k++) {
                if (idx[t * K + k] == e) {
                    sorted_token[p] = t;
                    sorted_slot[p] = t * K + k;
                    p++; c++;
                    break;
                }
            }
        }
        counts[e] = c;
    }
    offsets[E] = p;
}

/* ------------------------------------------------------------------ */
/* MoE: full forward                                                   */
/* ------------------------------------------------------------------ */

/* Expert FFN + combine given routing, with optional rounding hooks that
 * mirror a storage precision of the intermediate activation:
 *   act_mode 0: fp32 (reference), 1: bf16 RNE, 2: e4m3 1x128 blocks.
 * w1/w2 are fp32 (already dequantised where applicable). */
/* ------------------------------------------------------------------ */
/* OCP Microscaling (MX) formats, OCP MX specification v1.0: a block of  */
/* 32 elements shares one E8M0 scale X = 2^(E-127) (E = 255 is NaN);     */
/* elements are FP4 E2M1 (0, 0.5, 1, 1.5, 2, 3, 4, 6 and negatives) or  */
/* FP8 E4M3.  Conversion from fp32 (spec section 6.3): shared exponent =  */
/* floor(log2(max |v|)) - emax_elem (E2M1: 2, E4M3: 8), clamped to the    */
/* E8M0 range; each element = RNE(v / X), saturated to the element's     */
/* largest normal.  No counterpart in the reference (fp32 only); the      */
/* format of this build's MXFP4 expert weights and MXFP8 activations.     */
/* An all-zero block gets E = 0.                                          */
/* ------------------------------------------------------------------ */
EXPORT float orc_e8m0_to_f32(uint8_t c) { return c == 255 ? NAN : ldexpf(1.0f, (int)c - 127); }

/* E2M1: sign, 2 exponent bits (bias 1), 1 mantissa bit; exponent 0 is
 * subnormal (m * 0.5). */
EXPORT float orc_e2m1_to_f32(uint8_t c) {
    int e = (c >> 1) & 3, m = c & 1;
    float v = e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1);
    return (c & 8) ? -v : v;
}

/* Round to nearest even E2M1, saturating at 6 (NaN also gives the largest
 * magnitude: E2M1 has no NaN).  Within a binade the representable values
 * are the multiples of a step (0.5 below 2, 1 in [2,4), 2 in [4,6]) whose
 * parity is the mantissa bit, so RNE is rint on a / step. */
EXPORT uint8_t orc_f32_to_e2m1(float f) {
    uint8_t sign = signbit(f) ? 8 : 0;
    float a = fabsf(f);
    if (isnan(f) || a >= 6.0f) return sign | 7;
    float step = a < 2.0f ? 0.5f : (a < 4.0f ? 1.0f : 2.0f);
    float r = rintf(a / step) * step;
    uint8_t code = r < 2.0f ? (uint8_t)(r * 2.0f) : (r < 4.0f ? (uint8_t)(4 + (int)(r - 2.0f))
                                                             : (r < 6.0f ? 6 : 7));
    return sign | code;
}

/* One 32-element block: returns the E8M0 code, writes the element codes
 * (elem_bits 4: E2M1, one code per byte here; 8: E4M3). */
static uint8_t mx_block(const float* v, int elem_bits, uint8_t* codes) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    int e8 = 0;
    if (amax > 0.0f) {
        int e;
        frexpf(amax, &e);                      /* floor(log2 amax) = e - 1 */
        e8 = e - 1 - (elem_bits == 4 ? 2 : 8) + 127;
        if (e8 < 0) e8 = 0;
        if (e8 > 254) e8 = 254;
    }
    float inv = ldexpf(1.0f, 127 - e8);        /* 1 / X, a power of two: exact */
    for (int i = 0; i < 32; i++)
        codes[i] = elem_bits == 4 ? orc_f32_to_e2m1(v[i] * inv) : orc_f32_to_e4m3(v[i] * inv);
    return (uint8_t)e8;
}

/* Rows of cols values (cols % 32 == 0) -> MX: fp4 codes packed two per byte
 * (element 2j in the low nibble) [rows, cols/2], or fp8 codes [rows, cols];
 * scales E8M0 [rows, cols/32]. */
EXPORT void orc_mx_quant_rows(const float* x, long rows, int cols, int elem_bits, uint8_t* q,
                              uint8_t* s) {
    uint8_t c[32];
    for (long r = 0; r < rows; r++)
        for (int b = 0; b < cols / 32; b++) {
            s[r * (cols / 32) + b] = mx_block(x + r * cols + 32 * b, elem_bits, c);
            for (int j = 0; j < 32; j++) {
                long i = r * cols + 32 * b + j;
                if (elem_bits == 4) {
                    if (j & 1) q[i / 2] |= (uint8_t)(c[j] << 4);
                    else q[i / 2] = c[j];
                } else {
                    q[i] = c[j];
                }
            }
        }
}

EXPORT void orc_mx_dequant_rows(const uint8_t* q, const uint8_t* s, long rows, int cols,
                                int elem_bits, float* out) {
    for (long r = 0; r < rows; r++)
        for (int j = 0; j < cols; j++) {
            long i = r * cols + j;
            float e = elem_bits == 4 ? orc_e2m1_to_f32((q[i / 2] >> (4 * (i & 1))) & 15)
                                     : orc_e4m3_to_f32(q[i]);
            out[i] = e * orc_e8m0_to_f32(s[r * (cols / 32) + j / 32]);
        }
}

static void expert_ffn_rows(const float* xrows, int cnt, const float* w1_e, const float* w2_e,
                            int D, int I, int act_mode, float* g2 /* [cnt, D] */) {
    float* g1 = (float*)malloc(sizeof(float) * 2 * (size_t)I);
    float* act = (float*)malloc(sizeof(float) * (size_t)I);
    uint8_t* q = (uint8_t*)malloc((size_t)I);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(I / 128 + 1));
    for (int m = 0; m < cnt; m++) {
        const float* xr = xrows + (size_t)m * D;
        /* GEMM1 tests/test_moe.cu:88-98 (threads split output columns) */
        #pragma omp parallel for schedule(static)
        for (int n = 0; n < 2 * I; n++) {
            float sum = 0.0f;
            for (int d = 0; d < D; d++) sum += xr[d] * w1_e[(size_t)n * D + d];
            g1[n] = sum;
        }
        /* SwiGLU tests/test_moe.cu:100-110 */
        for (int j = 0; j < I; j++) act[j] = orc_silu(g1[j]) * g1[I + j];
        if (act_mode == 1) {
            for (int j = 0; j < I; j++) act[j] = orc_bf16_to_f32(orc_f32_to_bf16(act[j]));
        } else if (act_mode == 2) {
            orc_quant_rows_1x128(act, 1, I, q, sc);
            for (int j = 0; j < I; j++) act[j] = orc_e4m3_to_f32(q[j]) * sc[j / 128];
        } else if (act_mode == 3) {
            /* MXFP8: E4M3 elements, one E8M0 scale per 32 (the MXFP4 layer) */
            for (int b = 0; b < I / 32; b++) {
                const uint8_t e8 = mx_block(act + 32 * b, 8, q + 32 * b);
                for (int j = 0; j < 32; j++)
                    act[32 * b + j] = orc_e4m3_to_f32(q[32 * b + j]) * orc_e8m0_to_f32(e8);
            }
        }
        /* GEMM2 tests/test_moe.cu:112-121 */
        #pragma omp parallel for schedule(static)
        for (int n = 0; n < D; n++) {
            float sum = 0.0f;
            for (int j = 0; j < I; j++) sum += act[j] * w2_e[(size_t)n * I + j];
            g2[(size_t)m * D + n] = sum;
        }
    }
    free(g1); free(act); free(q); free(sc);
}

/* Reference forward (tests/test_moe.cu:32-140), fp32.  gate_bias may be
 * NULL (the reference has no bias).  idx/wts/y are outputs. */
EXPORT void orc_moe_forward_f32(const float* x, const float* Wg, const float* W1, const float* W2,
                                const float* gate_bias, int T, int E, int K, int D, int I,
                                int* idx, float* wts, float* y) {
    orc_moe_route(x, Wg, gate_bias, T, E, K, D, idx, wts, NULL, NULL);
    memset(y, 0, sizeof(float) * (size_t)T * D);
    int* tmap = (int*)malloc(sizeof(int) * (size_t)T);
    float* xr = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* g2 = (float*)malloc(sizeof(float) * (size_t)T * D);
    for (int e = 0; e < E; e++) {
        int cnt = 0;
        for (int t = 0; t < T; t++)
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { tmap[cnt++] = t; break; }
        if (cnt == 0) continue;
        for (int m = 0; m < cnt; m++)
            memcpy(xr + (size_t)m * D, x + (size_t)tmap[m] * D, sizeof(float) * (size_t)D);
        expert_ffn_rows(xr, cnt, W1 + (size_t)e * 2 * I * D, W2 + (size_t)e * D * I, D, I, 0, g2);
        /* scatter tests/test_moe.cu:123-132 */
        for (int m = 0; m < cnt; m++) {
            int t = tmap[m];
            float w = 0.0f;
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { w = wts[t * K + k]; break; }
            for (int d = 0; d < D; d++) y[(size_t)t * D + d] += w * g2[(size_t)m * D + d];
        }
    }
    free(tmap); free(xr); free(g2);
}

/* bf16 variant (BASELINE medium-bf16 / Mixtral): x, W1, W2 bf16; gate fp32;
 * the intermediate activation is held in bf16 (act_mode 1), as the GPU path
 * stores it.  Output y stays fp32 (the caller rounds for comparison). */
EXPORT void orc_moe_forward_bf16(const uint16_t* x, const float* Wg, const uint16_t* W1,
                                 const uint16_t* W2, const float* gate_bias,
                                 int T, int E, int K, int D, int I,
                                 int* idx, float* wts, float* y) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)T * D);
    orc_bf16_to_f32_array(x, xf, (long)T * D);
    orc_moe_route(xf, Wg, gate_bias, T, E, K, D, idx, wts, NULL, NULL);
    memset(y, 0, sizeof(float) * (size_t)T * D);
    int* tmap = (int*)malloc(sizeof(int) * (size_t)T);
    float* xr = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* g2 = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* w1f = (float*)malloc(sizeof(float) * (size_t)2 * I * D);
    float* w2f = (float*)malloc(sizeof(float) * (size_t)D * I);
    for (int e = 0; e < E; e++) {
        int cnt = 0;
        for (int t = 0; t < T; t++)
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { tmap[cnt++] = t; break; }
        if (cnt == 0) continue;
        orc_bf16_to_f32_array(W1 + (size_t)e * 2 * I * D, w1f, (long)2 * I * D);
        orc_bf16_to_f32_array(W2 + (size_t)e * D * I, w2f, (long)D * I);
        for (int m = 0; m < cnt; m++)
            memcpy(xr + (size_t)m * D, xf + (size_t)tmap[m] * D, sizeof(float) * (size_t)D);
        expert_ffn_rows(xr, cnt, w1f, w2f, D, I, 1, g2);
        for (int m = 0; m < cnt; m++) {
            int t = tmap[m];
            float w = 0.0f;
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { w = wts[t * K + k]; break; }
            for (int d = 0; d < D; d++) y[(size_t)t * D + d] += w * g2[(size_t)m * D + d];
        }
    }
    free(xf); free(tmap); free(xr); free(g2); free(w1f); free(w2f);
}

/* Dequantise one expert's [rows, cols] e4m3 weight with [rows/128, cols/128]
 * fp32 block scales into fp32. */
EXPORT void orc_dequant_weight_128x128(const uint8_t* q, const float* s, int rows, int cols,
                                       float* out) {
    int cb = cols / 128;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++)
            out[(size_t)r * cols + c] =
                orc_e4m3_to_f32(q[(size_t)r * cols + c]) * s[(r / 128) * cb + c / 128];
}

/* FP8 block-scale variant (BASELINE DSV3 config), evaluated for an
 * arbitrary subset of tokens (each token's output depends only on its own
 * row, so a subset equals the full forward restricted to it):
 *   x bf16 [n, D] (the selected rows), Wg bf16 [E, D];
 *   routing as the reference on fp32 logits of the bf16 values;
 *   x quantised 1x128 to e4m3 and dequantised; weights dequantised from
 *   e4m3 + 128x128 fp32 scales (W1 [E,2I,D], W2 [E,D,I]);
 *   the intermediate activation requantised 1x128 (act_mode 2);
 *   combine in ascending expert order in fp32.
 * Expert e's weights sit at slot wmap[e] of the w1q/w1s/w2q/w2s arrays
 * (wmap NULL: slot e), so a caller may pass only the experts the selected
 * tokens use; only those are dequantised. */
EXPORT void orc_moe_forward_fp8(const uint16_t* x, int n, const uint16_t* Wg,
                                const uint8_t* w1q, const float* w1s,
                                const uint8_t* w2q, const float* w2s, const int* wmap,
                                int E, int K, int D, int I,
                                int* idx, float* wts, float* y) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* wgf = (float*)malloc(sizeof(float) * (size_t)E * D);
    orc_bf16_to_f32_array(x, xf, (long)n * D);
    orc_bf16_to_f32_array(Wg, wgf, (long)E * D);
    orc_moe_route(xf, wgf, NULL, n, E, K, D, idx, wts, NULL, NULL);
    /* activation quantisation 1x128 -> dequantised values */
    uint8_t* xq = (uint8_t*)malloc((size_t)n * D);
    float* xs = (float*)malloc(sizeof(float) * (size_t)n * (D / 128));
    orc_quant_rows_1x128(xf, n, D, xq, xs);
    for (long i = 0; i < (long)n * D; i++) xf[i] = orc_e4m3_to_f32(xq[i]) * xs[i / 128];
    memset(y, 0, sizeof(float) * (size_t)n * D);
    int* tmap = (int*)malloc(sizeof(int) * (size_t)n);
    float* xr = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* g2 = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* w1f = (float*)malloc(sizeof(float) * (size_t)2 * I * D);
    float* w2f = (float*)malloc(sizeof(float) * (size_t)D * I);
    int nb_d = D / 128, nb_i = I / 128;
    for (int e = 0; e < E; e++) {
        int cnt = 0;
        for (int t = 0; t < n; t++)
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { tmap[cnt++] = t; break; }
        if (cnt == 0) continue;
        size_t ws = wmap ? (size_t)wmap[e] : (size_t)e;
        orc_dequant_weight_128x128(w1q + ws * 2 * I * D, w1s + ws * (2 * I / 128) * nb_d,
                                   2 * I, D, w1f);
        orc_dequant_weight_128x128(w2q + ws * D * I, w2s + ws * nb_d * nb_i, D, I, w2f);
        for (int m = 0; m < cnt; m++)
            memcpy(xr + (size_t)m * D, xf + (size_t)tmap[m] * D, sizeof(float) * (size_t)D);
        expert_ffn_rows(xr, cnt, w1f, w2f, D, I, 2, g2);
        for (int m = 0; m < cnt; m++) {
            int t = tmap[m];
            float w = 0.0f;
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { w = wts[t * K + k]; break; }
            for (int d = 0; d < D; d++) y[(size_t)t * D + d] += w * g2[(size_t)m * D + d];
        }
    }
    free(xf); free(wgf); free(xq); free(xs); free(tmap); free(xr); free(g2); free(w1f); free(w2f);
}

/* MXFP4 layer (this build's extension of the fp8 layer): expert weights
 * E2M1 with E8M0 scales per 32 along K (W1 q [E',2I,D/2], s [E',2I,D/32];
 * W2 q [E',D,I/2], s [E',D,I/32], row-major, element 2j in the low nibble),
 * activations MXFP8 (x and the SwiGLU output quantised per 32 columns).
 * Routing as orc_moe_forward_fp8 (bf16 x and gate); wmap as there. */
EXPORT void orc_moe_forward_mxfp4(const uint16_t* x, int n, const uint16_t* Wg,
                                  const uint8_t* w1q, const uint8_t* w1s,
                                  const uint8_t* w2q, const uint8_t* w2s, const int* wmap,
                                  int E, int K, int D, int I,
                                  int* idx, float* wts, float* y) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* wgf = (float*)malloc(sizeof(float) * (size_t)E * D);
    orc_bf16_to_f32_array(x, xf, (long)n * D);
    orc_bf16_to_f32_array(Wg, wgf, (long)E * D);
    orc_moe_route(xf, wgf, NULL, n, E, K, D, idx, wts, NULL, NULL);
    uint8_t* xq = (uint8_t*)malloc((size_t)n * D);
    uint8_t* xs = (uint8_t*)malloc((size_t)n * (D / 32));
    orc_mx_quant_rows(xf, n, D, 8, xq, xs);
    orc_mx_dequant_rows(xq, xs, n, D, 8, xf);
    memset(y, 0, sizeof(float) * (size_t)n * D);
    int* tmap = (int*)malloc(sizeof(int) * (size_t)n);
    float* xr = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* g2 = (float*)malloc(sizeof(float) * (size_t)n * D);
    float* w1f = (float*)malloc(sizeof(float) * (size_t)2 * I * D);
    float* w2f = (float*)malloc(sizeof(float) * (size_t)D * I);
    for (int e = 0; e < E; e++) {
        int cnt = 0;
        for (int t = 0; t < n; t++)
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { tmap[cnt++] = t; break; }
        if (cnt == 0) continue;
        size_t ws = wmap ? (size_t)wmap[e] : (size_t)e;
        orc_mx_dequant_rows(w1q + ws * 2 * I * (D / 2), w1s + ws * 2 * I * (D / 32), 2 * I, D, 4, w1f);
        orc_mx_dequant_rows(w2q + ws * D * (I / 2), w2s + ws * D * (I / 32), D, I, 4, w2f);
        for (int m = 0; m < cnt; m++)
            memcpy(xr + (size_t)m * D, xf + (size_t)tmap[m] * D, sizeof(float) * (size_t)D);
        expert_ffn_rows(xr, cnt, w1f, w2f, D, I, 3, g2);
        for (int m = 0; m < cnt; m++) {
            int t = tmap[m];
            float w = 0.0f;
            for (int k = 0; k < K; k++)
                if (idx[t * K + k] == e) { w = wts[t * K + k]; break; }
            for (int d = 0; d < D; d++) y[(size_t)t * D + d] += w * g2[(size_t)m * D + d];
        }
    }
    free(xf); free(wgf); free(xq); free(xs); free(tmap); free(xr); free(g2); free(w1f); free(w2f);
}

/* ------------------------------------------------------------------ */
/* DSA sparse decode                                                   */
/* ------------------------------------------------------------------ */

/* tests/test_dsa.cu:23-68, flat indices into [N, *] caches. */
EXPORT void orc_dsa_forward_f32(const float* q_nope, const float* q_pe,
                                const float* kv_c, const float* kv_p, const float* v_cache,
                                const int* sparse_indices, float* output,
                                int Q, int H, int Dc, int Dp, int S) {
    float scale = 1.0f / sqrtf((float)(Dc + Dp));
    #pragma omp parallel for schedule(dynamic)
    for (int q = 0; q < Q; q++) {
        float* kc = (float*)malloc(sizeof(float) * (size_t)S * Dc);
        float* kp = (float*)malloc(sizeof(float) * (size_t)S * (Dp > 0 ? Dp : 1));
        float* v = (float*)malloc(sizeof(float) * (size_t)S * Dc);
        float* scores = (float*)malloc(sizeof(float) * (size_t)S);
        for (int s = 0; s < S; s++) {
            long idx = sparse_indices[(size_t)q * S + s];
            for (int d = 0; d < Dc; d++) kc[(size_t)s * Dc + d] = kv_c[idx * Dc + d];
            for (int d = 0; d < Dp; d++) kp[(size_t)s * Dp + d] = kv_p[idx * Dp + d];
            for (int d = 0; d < Dc; d++) v[(size_t)s * Dc + d] = v_cache[idx * Dc + d];
        }
        for (int h = 0; h < H; h++) {
            const float* qn = q_nope + ((size_t)q * H + h) * Dc;
            const float* qp = q_pe + ((size_t)q * H + h) * Dp;
            for (int s = 0; s < S; s++) {
                float sum_c = 0.0f, sum_p = 0.0f;
                for (int d = 0; d < Dc; d++) sum_c += qn[d] * kc[(size_t)s * Dc + d];
                for (int d = 0; d < Dp; d++) sum_p += qp[d] * kp[(size_t)s * Dp + d];
                scores[s] = (sum_c + sum_p) * scale;
            }
            orc_softmax(scores, S);
            for (int d = 0; d < Dc; d++) {
                float sum = 0.0f;
                for (int s = 0; s < S; s++) sum += scores[s] * v[(size_t)s * Dc + d];
                output[((size_t)q * H + h) * Dc + d] = sum;
            }
        }
        free(kc); free(kp); free(v); free(scores);
    }
}

/* The stage functions of naive_dsa.cuh:31-68, in the order of operations of
 * their kernels (one thread's sequential loop per output value). */

/* naive_dsa.cu:13-60: gathered_*[q,s,:] = cache[idx[q,s], :]. */
EXPORT void orc_dsa_kv_gather(const float* kv_c, const float* kv_p, const float* v_cache,
                              const int* idx, float* gkc, float* gkp, float* gv,
                              int Q, int S, int Dc, int Dp) {
    for (long r = 0; r < (long)Q * S; r++) {
        long row = idx[r];
        memcpy(gkc + r * Dc, kv_c + row * Dc, sizeof(float) * (size_t)Dc);
        if (Dp > 0) memcpy(gkp + r * Dp, kv_p + row * Dp, sizeof(float) * (size_t)Dp);
        memcpy(gv + r * Dc, v_cache + row * Dc, sizeof(float) * (size_t)Dc);
    }
}

/* naive_dsa.cu:89-134 (parts = 1: q_nope . kc), 157-206 (parts = 2:
 * q_pe . kp), 208-276 (parts = 3: the concatenation, one accumulator):
 * sum over d in order, then scores[q,h,s] += sum. */
EXPORT void orc_dsa_dot(const float* qn, const float* qp, const float* kc, const float* kp,
                        float* scores, int Q, int H, int S, int Dc, int Dp, int parts) {
    #pragma omp parallel for schedule(static)
    for (int q = 0; q < Q; q++)
        for (int h = 0; h < H; h++)
            for (int s = 0; s < S; s++) {
                float sum = 0.0f;
                if (parts & 1) {
                    const float* a = qn + ((size_t)q * H + h) * Dc;
                    const float* b = kc + ((size_t)q * S + s) * Dc;
                    for (int d = 0; d < Dc; d++) sum += a[d] * b[d];
                }
                if (parts & 2) {
                    const float* a = qp + ((size_t)q * H + h) * Dp;
                    const float* b = kp + ((size_t)q * S + s) * Dp;
                    for (int d = 0; d < Dp; d++) sum += a[d] * b[d];
                }
                scores[((size_t)q * H + h) * S + s] += sum;
            }
}

/* naive_dsa.cu:278-296: per row, e = expf(x - max) (summed in order), then
 * x = e * (1 / sum).  (The CPU oracle of tests/test_dsa.cu divides instead.) */
EXPORT void orc_dsa_softmax(float* scores, long rows, int S) {
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; r++) {
        float* row = scores + r * S;
        float mx = -FLT_MAX;
        for (int s = 0; s < S; s++) mx = fmaxf(mx, row[s]);
        float sum = 0.0f;
        for (int s = 0; s < S; s++) {
            row[s] = expf(row[s] - mx);
            sum += row[s];
        }
        float inv = 1.0f / sum;
        for (int s = 0; s < S; s++) row[s] *= inv;
    }
}

/* naive_dsa.cu:300-316: out[q,h,d] = sum over s in order of
 * attn[q,h,s] * v[q,s,d]. */
EXPORT void orc_dsa_output_proj(const float* attn, const float* v, float* out,
                                int Q, int H, int S, int Dc) {
    #pragma omp parallel for schedule(static)
    for (int q = 0; q < Q; q++)
        for (int h = 0; h < H; h++)
            for (int d = 0; d < Dc; d++) {
                float sum = 0.0f;
                for (int s = 0; s < S; s++)
                    sum += attn[((size_t)q * H + h) * S + s] * v[((size_t)q * S + s) * Dc + d];
                out[((size_t)q * H + h) * Dc + d] = sum;
            }
}

/* Paged address translation (BASELINE DSA config; the reference has no page
 * table): logical index i of query q lives at physical token
 * page_table[q][i / page] * page + i % page. */
/* Physical row of a selected token, or -1 when it selects nothing: logical
 * index outside [0, pages_per_seq * page), a negative page id, or a row at
 * or past cache_rows (cache_rows <= 0: unbounded). */
static long dsa_phys_row(const int* pt_row, int i, int pages_per_seq, int page, long cache_rows) {
    if (i < 0 || (long)i >= (long)pages_per_seq * page) return -1;
    int pg = pt_row[i / page];
    if (pg < 0) return -1;
    long row = (long)pg * page + i % page;
    if (cache_rows > 0 && row >= cache_rows) return -1;
    return row;
}

EXPORT void orc_dsa_translate(const int* logical, const int* page_table, int Q, int S,
                              int pages_per_seq, int page, long cache_rows, int* physical) {
    for (int q = 0; q < Q; q++)
        for (int s = 0; s < S; s++)
            physical[(size_t)q * S + s] = (int)dsa_phys_row(
                page_table + (size_t)q * pages_per_seq, logical[(size_t)q * S + s], pages_per_seq,
                page, cache_rows);
}

/* bf16 paged MLA-absorbed decode: one latent cache [Ntok, Dc+Dp] bf16 whose
 * first Dc columns are K_c and also V, last Dp columns K_p.  Math as
 * orc_dsa_forward_f32 on the decoded values; out fp32 [Q, H, Dc].  Selected
 * tokens that select nothing (dsa_phys_row == -1, e.g. the -1 padding of a
 * sequence shorter than the selection) are left out: the softmax runs over
 * the valid tokens only, in their order, and a query with none gets 0. */
EXPORT void orc_dsa_decode_bf16_paged(const uint16_t* q_nope, const uint16_t* q_pe,
                                      const uint16_t* cache, const int* page_table,
                                      const int* logical, float* output,
                                      int Q, int H, int Dc, int Dp, int S,
                                      int pages_per_seq, int page, long cache_rows) {
    int Dt = Dc + Dp;
    float scale = 1.0f / sqrtf((float)(Dc + Dp));
    #pragma omp parallel for schedule(dynamic)
    for (int q = 0; q < Q; q++) {
        float* kc = (float*)malloc(sizeof(float) * (size_t)S * Dc);
        float* kp = (float*)malloc(sizeof(float) * (size_t)S * (Dp > 0 ? Dp : 1));
        float* scores = (float*)malloc(sizeof(float) * (size_t)S);
        float* qn = (float*)malloc(sizeof(float) * (size_t)Dc);
        float* qp = (float*)malloc(sizeof(float) * (size_t)(Dp > 0 ? Dp : 1));
        int nv = 0;  /* valid tokens, compacted in selection order */
        for (int s = 0; s < S; s++) {
            long phys = dsa_phys_row(page_table + (size_t)q * pages_per_seq,
                                     logical[(size_t)q * S + s], pages_per_seq, page, cache_rows);
            if (phys < 0) continue;
            const uint16_t* row = cache + phys * Dt;
            for (int d = 0; d < Dc; d++) kc[(size_t)nv * Dc + d] = orc_bf16_to_f32(row[d]);
            for (int d = 0; d < Dp; d++) kp[(size_t)nv * Dp + d] = orc_bf16_to_f32(row[Dc + d]);
            nv++;
        }
        if (nv == 0) {
            memset(output + (size_t)q * H * Dc, 0, sizeof(float) * (size_t)H * Dc);
            free(kc); free(kp); free(scores); free(qn); free(qp);
            continue;
        }
        for (int h = 0; h < H; h++) {
            for (int d = 0; d < Dc; d++) qn[d] = orc_bf16_to_f32(q_nope[((size_t)q * H + h) * Dc + d]);
            for (int d = 0; d < Dp; d++) qp[d] = orc_bf16_to_f32(q_pe[((size_t)q * H + h) * Dp + d]);
            for (int s = 0; s < nv; s++) {
                float sum_c = 0.0f, sum_p = 0.0f;
                for (int d = 0; d < Dc; d++) sum_c += qn[d] * kc[(size_t)s * Dc + d];
                for (int d = 0; d < Dp; d++) sum_p += qp[d] * kp[(size_t)s * Dp + d];
                scores[s] = (sum_c + sum_p) * scale;
            }
            orc_softmax(scores, nv);
            for (int d = 0; d < Dc; d++) {
                float sum = 0.0f;
                for (int s = 0; s < nv; s++) sum += scores[s] * kc[(size_t)s * Dc + d];
                output[((size_t)q * H + h) * Dc + d] = sum;
            }
        }
        free(kc); free(kp); free(scores); free(qn); free(qp);
    }
}

/* ------------------------------------------------------------------ indexer
 * DeepSeek-V3.2's lightning indexer, the producer of the sparse indices the
 * decode consumes (absent from the reference; the formula is the published
 * one, I[t,s] = sum_j w[t,j] * ReLU(q[t,j] . k[s])), in the fp8 form the
 * library takes: q codes e4m3 [Q,Hi,128] with scales [Q,Hi], per-head
 * weights [Q,Hi], key codes e4m3 [rows,128] with a scale per row, keys in
 * pages through page_table.  Scores are computed in double and rounded once:
 *   score[q,s] = ks[row] * sum_j (w[q,j] * qs[q,j]) * relu(sum_d q[q,j,d] k[row,d])
 * for s < seq_len[q]; row = page_table[q][s / page] * page + s % page. */
EXPORT void orc_dsa_indexer_scores(const uint8_t* qc, const float* qs, const float* hw,
                                   const uint8_t* kc, const float* ks, const int* page_table,
                                   const int* seq_len, int Q, int Hi, int page, int pages_per_seq,
                                   int max_seq, float* scores) {
    #pragma omp parallel for schedule(dynamic)
    for (int q = 0; q < Q; q++) {
        float qf[128];
        double* wq = (double*)malloc(sizeof(double) * (size_t)Hi);
        float* qv = (float*)malloc(sizeof(float) * (size_t)Hi * 128);
        for (int j = 0; j < Hi; j++) {
            wq[j] = (double)hw[(size_t)q * Hi + j] * (double)qs[(size_t)q * Hi + j];
            for (int d = 0; d < 128; d++) qv[(size_t)j * 128 + d] = orc_e4m3_to_f32(qc[((size_t)q * Hi + j) * 128 + d]);
        }
        /* positions past seq_len or past the page-table row's capacity score -inf */
        long len = seq_len[q] < (long)pages_per_seq * page ? seq_len[q] : (long)pages_per_seq * page;
        for (int s = 0; s < max_seq; s++) {
            if (s >= len) { scores[(size_t)q * max_seq + s] = -INFINITY; continue; }
            long row = (long)page_table[(size_t)q * pages_per_seq + s / page] * page + s % page;
            for (int d = 0; d < 128; d++) qf[d] = orc_e4m3_to_f32(kc[row * 128 + d]);
            double tot = 0.0;
            for (int j = 0; j < Hi; j++) {
                double dot = 0.0;
                for (int d = 0; d < 128; d++) dot += (double)qv[(size_t)j * 128 + d] * (double)qf[d];
                tot += wq[j] * (dot > 0.0 ? dot : 0.0);
            }
            scores[(size_t)q * max_seq + s] = (float)(tot * (double)ks[row]);
        }
        free(wq);
        free(qv);
    }
}

/* The topk positions of each row with the largest scores (ties: the lower
 * position wins; -0 equals +0), listed in ascending position order; rows
 * shorter than topk are padded with -1. */
static int g_topk_len;
static const float* g_topk_row;
static int cmp_score_desc(const void* a, const void* b) {
    int i = *(const int*)a, j = *(const int*)b;
    float x = g_topk_row[i], y = g_topk_row[j];
    if (x > y) return -1;
    if (x < y) return 1;
    return i - j;
}
EXPORT void orc_dsa_indexer_topk(const float* scores, const int* seq_len, int Q, int max_seq,
                                 int cap, int topk, int* out) {
    /* cap: positions scored per row (the page-table row's capacity), <= 0: max_seq */
    int* pos = (int*)malloc(sizeof(int) * (size_t)(max_seq > 0 ? max_seq : 1));
    int lim = cap > 0 && cap < max_seq ? cap : max_seq;
    for (int q = 0; q < Q; q++) {
        int n = seq_len[q] < lim ? seq_len[q] : lim;
        if (n < 0) n = 0;
        for (int s = 0; s < n; s++) pos[s] = s;
        g_topk_row = scores + (size_t)q * max_seq;
        g_topk_len = n;
        qsort(pos, (size_t)n, sizeof(int), cmp_score_desc);
        int m = n < topk ? n : topk;
        qsort(pos, (size_t)m, sizeof(int), cmp_int);
        for (int k = 0; k < topk; k++) out[(size_t)q * topk + k] = k < m ? pos[k] : -1;
    }
    free(pos);
}
