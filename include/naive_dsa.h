// naive_dsa.h -- C++ drop-in for the reference's DSA operator header
// (kernels/dsa/naive_dsa.cuh), for the entry point the reference's tests
// and benchmarks call: dsa_forward.  Same struct, name, argument order and
// meaning, `hipStream_t stream = 0`; errors print and exit like CUDA_CHECK
// (utils/cuda_utils.cuh:13-21).  The BASELINE paged bf16 decode is
// amdmoe_dsa_decode_bf16_paged in amdmoe.h.
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
