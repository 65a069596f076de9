// naive_dsa.h -- C++ drop-in for the reference's DSA operator header
// (kernels/dsa/naive_dsa.cuh): dsa_forward, which the reference's tests and
// benchmarks call, and the six stage functions it is composed of.  Same
// struct, names, argument order and meaning, `hipStream_t stream = 0`;
// errors print and exit like CUDA_CHECK (utils/cuda_utils.cuh:13-21).  The
// BASELINE paged bf16 decode is amdmoe_dsa_decode_bf16_paged in amdmoe.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "amdmoe.h"

namespace amdmoe_dropin_dsa {
inline void check(int rc, const char* file, int line) {
    if (rc != AMDMOE_OK) {
        std::fprintf(stderr, "HIP error at %s:%d: %s\n", file, line, amdmoe_last_error());
        std::exit(EXIT_FAILURE);
    }
}
}  // namespace amdmoe_dropin_dsa

// naive_dsa.cuh:81-87
inline void dsa_forward(const float* q_nope, const float* q_pe, const float* kv_cache_compressed,
                        const float* kv_cache_positional, const float* v_cache,
                        const int* sparse_indices, float* output, const DsaConfig& cfg,
                        hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(
        amdmoe_dsa_forward_f32(q_nope, q_pe, kv_cache_compressed, kv_cache_positional, v_cache,
                               sparse_indices, output, &cfg, stream),
        __FILE__, __LINE__);
}

// naive_dsa.cuh:31-36
inline void dsa_kv_gather(const float* kv_cache_compressed, const float* kv_cache_positional,
                          const float* v_cache, const int* sparse_indices, float* gathered_kc,
                          float* gathered_kp, float* gathered_v, const DsaConfig& cfg,
                          hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(
        amdmoe_dsa_kv_gather_f32(kv_cache_compressed, kv_cache_positional, v_cache,
                                 sparse_indices, gathered_kc, gathered_kp, gathered_v, &cfg,
                                 stream),
        __FILE__, __LINE__);
}

// naive_dsa.cuh:42-43
inline void dsa_dot_compressed(const float* q_nope, const float* kc, float* scores,
                               const DsaConfig& cfg, hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(amdmoe_dsa_dot_compressed_f32(q_nope, kc, scores, &cfg, stream),
                               __FILE__, __LINE__);
}

// naive_dsa.cuh:49-50
inline void dsa_dot_positional(const float* q_pe, const float* kp, float* scores,
                               const DsaConfig& cfg, hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(amdmoe_dsa_dot_positional_f32(q_pe, kp, scores, &cfg, stream),
                               __FILE__, __LINE__);
}

// naive_dsa.cuh:54-57
inline void dsa_dot_fused(const float* q_nope, const float* q_pe, const float* kc,
                          const float* kp, float* scores, const DsaConfig& cfg,
                          hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(amdmoe_dsa_dot_fused_f32(q_nope, q_pe, kc, kp, scores, &cfg, stream),
                               __FILE__, __LINE__);
}

// naive_dsa.cuh:61
inline void dsa_softmax(float* scores, const DsaConfig& cfg, hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(amdmoe_dsa_softmax_f32(scores, &cfg, stream), __FILE__, __LINE__);
}

// naive_dsa.cuh:67-68
inline void dsa_output_proj(const float* attn, const float* v, float* output,
                            const DsaConfig& cfg, hipStream_t stream = 0) {
    ::amdmoe_dropin_dsa::check(amdmoe_dsa_output_proj_f32(attn, v, output, &cfg, stream),
                               __FILE__, __LINE__);
}
