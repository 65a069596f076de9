// naive_moe.h -- C++ drop-in for the reference's MoE operator header
// (kernels/moe/naive_moe.cuh).  Same struct, same function names, same
// argument order and meaning, `hipStream_t stream = 0` in place of
// `cudaStream_t stream = 0`.  Each function forwards to the C ABI in
// amdmoe.h; on failure it prints "HIP error at <file>:<line>: <message>"
// and exits with EXIT_FAILURE, as the reference's CUDA_CHECK does
// (utils/cuda_utils.cuh:13-21).
//
// Differences a caller can observe:
//   - moe_forward does not block the host (the reference synchronises once
//     per expert, naive_moe.cu:427-429); synchronise before reading `output`.
//   - none in the shapes accepted: moe_forward takes any D and I (multiples
//     of 32 run the MFMA grouped GEMM, others a bounds-checked fp32 GEMM);
//     shapes the reference mishandles (D > 1024 in its scatter launch,
//     element counts past 2^31) work here, and K > 64 is rejected with an
//     error instead.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "amdmoe.h"

namespace amdmoe_dropin {
inline void check(int rc, const char* file, int line) {
    if (rc != AMDMOE_OK) {
        std::fprintf(stderr, "HIP error at %s:%d: %s\n", file, line, amdmoe_last_error());
        std::exit(EXIT_FAILURE);
    }
}
}  // namespace amdmoe_dropin

#define AMDMOE_DROPIN_CHECK(call) ::amdmoe_dropin::check((call), __FILE__, __LINE__)

// naive_moe.cuh:27-29
inline void moe_gate(const float* input, const float* gate_weight, int* expert_indices,
                     float* expert_weights, const MoeConfig& cfg, hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_moe_gate_f32(input, gate_weight, expert_indices, expert_weights,
                                            &cfg, stream));
}

// naive_moe.cuh:38-41
inline void moe_gather(const float* input, const int* expert_indices, const float* expert_weights,
                       int expert_id, float* gathered, int* token_map, int* count,
                       const MoeConfig& cfg, hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_moe_gather_f32(input, expert_indices, expert_weights, expert_id,
                                              gathered, token_map, count, &cfg, stream));
}

// naive_moe.cuh:44-45
inline void naive_gemm(const float* A, const float* B, float* C, int M, int N, int K,
                       hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_naive_gemm_f32(A, B, C, M, N, K, stream));
}

// naive_moe.cuh:50-51
inline void swiglu(const float* gate, const float* up, float* out, int n,
                   hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_swiglu_f32(gate, up, out, n, stream));
}

// naive_moe.cuh:59-62
inline void moe_scatter(const float* expert_out, const int* token_map,
                        const float* expert_weights, const int* expert_indices, int expert_id,
                        float* output, int count, const MoeConfig& cfg, hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_moe_scatter_f32(expert_out, token_map, expert_weights,
                                               expert_indices, expert_id, output, count, &cfg,
                                               stream));
}

// naive_moe.cuh:74-76
inline void moe_forward(const float* input, const float* gate_weight, const float* w1,
                        const float* w2, float* output, const MoeConfig& cfg,
                        hipStream_t stream = 0) {
    AMDMOE_DROPIN_CHECK(amdmoe_moe_forward_f32(input, gate_weight, w1, w2, output, &cfg, nullptr,
                                               0, stream));
}
