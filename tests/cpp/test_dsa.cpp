// test_dsa -- the reference's DSA correctness suite (tests/test_dsa.cu) run
// through the drop-in header naive_dsa.h: the same 14 cases, seeds, fill
// order, sorted sparse indices, tolerances and output format, checked
// against the CPU oracle (oracle/oracle.c, a restatement of
// cpu_dsa_forward).  Exit status 0 iff every case passes.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/naive_dsa.h"

extern "C" {
void orc_srand(unsigned seed);
void orc_random_fill(float* data, long n, float lo, float hi);
void orc_gen_sparse_indices(int* indices, int Q, int S, int total_kv, int sort_rows);
void orc_dsa_forward_f32(const float* q_nope, const float* q_pe, const float* kv_c,
                         const float* kv_p, const float* v_cache, const int* sparse_indices,
                         float* output, int Q, int H, int Dc, int Dp, int S);
float orc_max_abs_error(const float* a, const float* b, long n);
float orc_mean_abs_error(const float* a, const float* b, long n);
}

#define HIP_OK(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,       \
                         hipGetErrorString(e_));                                       \
            std::exit(EXIT_FAILURE);                                                   \
        }                                                                              \
    } while (0)

template <typename T> static T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

static bool run_test(const char* name, const DsaConfig& c, float tol) {
    std::printf("  %-40s  ", name);
    const int Q = c.num_queries, H = c.num_heads, Dc = c.head_dim_compressed,
              Dp = c.head_dim_positional, S = c.num_selected_kv, N = c.total_kv_tokens;
    orc_srand(42);
    std::vector<float> qn((size_t)Q * H * Dc), qp((size_t)Q * H * Dp), kc((size_t)N * Dc),
        kp((size_t)N * Dp), v((size_t)N * Dc), ref((size_t)Q * H * Dc), got((size_t)Q * H * Dc);
    std::vector<int> idx((size_t)Q * S);
    orc_random_fill(qn.data(), (long)qn.size(), -0.3f, 0.3f);
    orc_random_fill(qp.data(), (long)qp.size(), -0.3f, 0.3f);
    orc_random_fill(kc.data(), (long)kc.size(), -0.3f, 0.3f);
    orc_random_fill(kp.data(), (long)kp.size(), -0.3f, 0.3f);
    orc_random_fill(v.data(), (long)v.size(), -0.3f, 0.3f);
    orc_gen_sparse_indices(idx.data(), Q, S, N, 1);
    orc_dsa_forward_f32(qn.data(), qp.data(), kc.data(), kp.data(), v.data(), idx.data(), ref.data(),
                        Q, H, Dc, Dp, S);
    float *dqn = upload(qn), *dqp = upload(qp), *dkc = upload(kc), *dkp = upload(kp), *dv = upload(v);
    int* didx = upload(idx);
    float* dout = nullptr;
    HIP_OK(hipMalloc(&dout, got.size() * sizeof(float)));
    dsa_forward(dqn, dqp, dkc, dkp, dv, didx, dout, c);
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(got.data(), dout, got.size() * sizeof(float), hipMemcpyDeviceToHost));
    const float mx = orc_max_abs_error(ref.data(), got.data(), (long)got.size());
    const float mean = orc_mean_abs_error(ref.data(), got.data(), (long)got.size());
    const bool pass = mx < tol;
    std::printf("max=%.6e  mean=%.6e  %s\n", mx, mean, pass ? "PASS" : "FAIL");
    for (float* p : {dqn, dqp, dkc, dkp, dv, dout}) HIP_OK(hipFree(p));
    HIP_OK(hipFree(didx));
    return pass;
}

int main() {
    std::printf("=== DSA Correctness Tests ===\n\n");
    struct { const char* name; DsaConfig cfg; float tol; } cases[] = {
        {"tiny   (Q=2,H=2,Dc=32,S=16)", {2, 2, 32, 8, 16, 8, 64}, 1e-3f},
        {"small  (Q=4,H=4,Dc=64,S=64)", {4, 4, 64, 16, 64, 16, 256}, 1e-3f},
        {"medium (Q=8,H=8,Dc=128,S=128)", {8, 8, 128, 32, 128, 32, 512}, 1e-2f},
        {"large  (Q=4,H=4,Dc=128,S=256)", {4, 4, 128, 32, 256, 64, 1024}, 1e-2f},
        {"single-query (Q=1,H=4,S=32)", {1, 4, 64, 16, 32, 8, 128}, 1e-3f},
        {"single-head (Q=4,H=1,S=64)", {4, 1, 64, 16, 64, 16, 256}, 1e-3f},
        {"minimal-S (Q=4,H=4,S=4)", {4, 4, 64, 16, 4, 4, 256}, 1e-3f},
        {"pos-heavy (Dc=32,Dp=64,S=64)", {4, 4, 32, 64, 64, 16, 256}, 1e-3f},
        {"tiny-Dp (Dc=128,Dp=4,S=64)", {4, 4, 128, 4, 64, 16, 256}, 1e-2f},
        {"many-heads (Q=4,H=32,S=64)", {4, 32, 64, 16, 64, 16, 256}, 1e-2f},
        {"many-queries (Q=32,H=4,S=64)", {32, 4, 64, 16, 64, 16, 512}, 1e-2f},
        {"full-cache (Q=4,S=N=128)", {4, 4, 64, 16, 128, 16, 128}, 1e-3f},
        {"large-cache (N=4096,S=128)", {4, 4, 128, 32, 128, 64, 4096}, 1e-2f},
        {"stress (Q=16,H=16,Dc=128,S=256)", {16, 16, 128, 32, 256, 64, 2048}, 5e-2f},
    };
    int passed = 0, total = 0;
    for (auto& c : cases) {
        total++;
        if (run_test(c.name, c.cfg, c.tol)) passed++;
    }
    std::printf("\nResults: %d / %d passed\n", passed, total);
    return passed == total ? 0 : 1;
}
