// test_moe -- the reference's MoE correctness suite (tests/test_moe.cu) run
// through the drop-in header naive_moe.h: the same 13 cases, seeds, fill
// order, tolerances (strict <) and output format.  The expected output comes
// from the CPU oracle library (oracle/oracle.c, a restatement of the
// reference's cpu_moe_forward).  Exit status 0 iff every case passes.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/naive_moe.h"

extern "C" {
void orc_srand(unsigned seed);
void orc_random_fill(float* data, long n, float lo, float hi);
void orc_moe_forward_f32(const float* x, const float* Wg, const float* W1, const float* W2,
                         const float* gate_bias, int T, int E, int K, int D, int I, int* idx,
                         float* wts, float* y);
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

static float* upload(const std::vector<float>& h) {
    float* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(float)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    return d;
}

static bool run_test(const char* name, const MoeConfig& cfg, float tol) {
    std::printf("  %-30s  ", name);
    const int T = cfg.num_tokens, E = cfg.num_experts, K = cfg.top_k, D = cfg.hidden_dim,
              I = cfg.intermediate_dim;
    orc_srand(42);
    std::vector<float> x((size_t)T * D), g((size_t)E * D), w1((size_t)E * 2 * I * D), w2((size_t)E * D * I);
    orc_random_fill(x.data(), (long)x.size(), -0.5f, 0.5f);
    orc_random_fill(g.data(), (long)g.size(), -0.5f, 0.5f);
    orc_random_fill(w1.data(), (long)w1.size(), -0.1f, 0.1f);
    orc_random_fill(w2.data(), (long)w2.size(), -0.1f, 0.1f);
    std::vector<int> idx((size_t)T * K);
    std::vector<float> wts((size_t)T * K), ref((size_t)T * D), got((size_t)T * D);
    orc_moe_forward_f32(x.data(), g.data(), w1.data(), w2.data(), nullptr, T, E, K, D, I, idx.data(),
                        wts.data(), ref.data());
    float *dx = upload(x), *dg = upload(g), *dw1 = upload(w1), *dw2 = upload(w2), *dy = nullptr;
    HIP_OK(hipMalloc(&dy, (size_t)T * D * sizeof(float)));
    moe_forward(dx, dg, dw1, dw2, dy, cfg);
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(got.data(), dy, got.size() * sizeof(float), hipMemcpyDeviceToHost));
    const float mx = orc_max_abs_error(ref.data(), got.data(), (long)got.size());
    const float mean = orc_mean_abs_error(ref.data(), got.data(), (long)got.size());
    const bool pass = mx < tol;
    std::printf("max_err=%.6e  mean_err=%.6e  %s\n", mx, mean, pass ? "PASS" : "FAIL");
    for (float* p : {dx, dg, dw1, dw2, dy}) HIP_OK(hipFree(p));
    return pass;
}

int main() {
    std::printf("=== MoE Correctness Tests ===\n\n");
    struct { const char* name; MoeConfig cfg; float tol; } cases[] = {
        {"small  (T=4, E=4, D=64)", {4, 4, 2, 64, 128}, 1e-3f},
        {"medium (T=32, E=8, D=128)", {32, 8, 2, 128, 256}, 1e-3f},
        {"large  (T=64, E=8, D=256)", {64, 8, 2, 256, 512}, 1e-2f},
        {"topk4  (T=16, E=8, K=4)", {16, 8, 4, 128, 256}, 1e-2f},
        {"single-token (T=1, E=4)", {1, 4, 2, 64, 128}, 1e-3f},
        {"single-expert (T=8, E=1, K=1)", {8, 1, 1, 64, 128}, 1e-3f},
        {"topk1  (T=32, E=16, K=1)", {32, 16, 1, 128, 256}, 1e-2f},
        {"wide-ffn (T=16, D=64, I=512)", {16, 4, 2, 64, 512}, 1e-2f},
        {"narrow-ffn (T=16, D=256, I=64)", {16, 4, 2, 256, 64}, 1e-2f},
        {"sparse-routing (T=4, E=16)", {4, 16, 2, 128, 256}, 1e-3f},
        {"many-tokens (T=128, E=8)", {128, 8, 2, 128, 256}, 1e-2f},
        {"full-routing (T=8, E=4, K=4)", {8, 4, 4, 64, 128}, 1e-3f},
        {"stress (T=64, E=16, D=512)", {64, 16, 2, 512, 1024}, 5e-2f},
    };
    int passed = 0, total = 0;
    for (auto& c : cases) {
        total++;
        if (run_test(c.name, c.cfg, c.tol)) passed++;
    }
    std::printf("\nResults: %d / %d passed\n", passed, total);
    return passed == total ? 0 : 1;
}
