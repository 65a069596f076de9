// bench_moe -- the reference's MoE latency benchmark (benchmarks/bench_moe.cu)
// run through the drop-in header: same six configs, same argv
// ([warmup=10] [iters=50]), same table, inputs filled with the same glibc
// rand() expression after srand(123), each call timed with events on the
// null stream.  Unlike the reference, moe_forward does not synchronise
// internally, so the timer covers exactly the launched work.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/naive_moe.h"

#define HIP_OK(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,       \
                         hipGetErrorString(e_));                                       \
            std::exit(EXIT_FAILURE);                                                   \
        }                                                                              \
    } while (0)

// utils/cuda_utils.cuh:56-60
static void random_fill(float* data, size_t n, float lo, float hi) {
    for (size_t i = 0; i < n; i++) data[i] = lo + static_cast<float>(rand()) / static_cast<float>(RAND_MAX) * (hi - lo);
}

static float* upload(const std::vector<float>& h) {
    float* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(float)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    return d;
}

static void bench_one(const char* label, const MoeConfig& cfg, int warmup, int iters) {
    const int T = cfg.num_tokens, E = cfg.num_experts, D = cfg.hidden_dim, I = cfg.intermediate_dim;
    std::vector<float> x((size_t)T * D), g((size_t)E * D), w1((size_t)E * 2 * I * D), w2((size_t)E * D * I);
    random_fill(x.data(), x.size(), -0.5f, 0.5f);
    random_fill(g.data(), g.size(), -0.5f, 0.5f);
    random_fill(w1.data(), w1.size(), -0.1f, 0.1f);
    random_fill(w2.data(), w2.size(), -0.1f, 0.1f);
    float *dx = upload(x), *dg = upload(g), *dw1 = upload(w1), *dw2 = upload(w2), *dy = nullptr;
    HIP_OK(hipMalloc(&dy, (size_t)T * D * sizeof(float)));
    for (int i = 0; i < warmup; i++) moe_forward(dx, dg, dw1, dw2, dy, cfg);
    HIP_OK(hipDeviceSynchronize());
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    std::vector<float> times(iters);
    for (int i = 0; i < iters; i++) {
        HIP_OK(hipEventRecord(a, 0));
        moe_forward(dx, dg, dw1, dw2, dy, cfg);
        HIP_OK(hipEventRecord(b, 0));
        HIP_OK(hipEventSynchronize(b));
        HIP_OK(hipEventElapsedTime(&times[i], a, b));
    }
    std::sort(times.begin(), times.end());
    float mean = 0.0f;
    for (float t : times) mean += t;
    mean /= iters;
    std::printf("  %-28s  %8.3f  %8.3f  %8.3f  %8.3f  %12.0f\n", label, times.front(), mean,
                times[iters / 2], times.back(), T / (mean * 1e-3f));
    HIP_OK(hipEventDestroy(a));
    HIP_OK(hipEventDestroy(b));
    for (float* p : {dx, dg, dw1, dw2, dy}) HIP_OK(hipFree(p));
}

int main(int argc, char** argv) {
    int warmup = 10, iters = 50;
    if (argc > 1) warmup = std::atoi(argv[1]);
    if (argc > 2) iters = std::atoi(argv[2]);
    std::printf("=== MoE Kernel Benchmark (gfx950) ===\n");
    std::printf("    warmup=%d  iters=%d\n\n", warmup, iters);
    std::printf("  %-28s  %8s  %8s  %8s  %8s  %12s\n", "Config", "Min(ms)", "Mean(ms)", "Med(ms)",
                "Max(ms)", "Tok/s");
    std::printf("  %s\n", std::string(96, '-').c_str());
    srand(123);
    struct { const char* label; MoeConfig cfg; } configs[] = {
        {"T=16,E=4,K=2,D=64,I=128", {16, 4, 2, 64, 128}},
        {"T=32,E=8,K=2,D=128,I=256", {32, 8, 2, 128, 256}},
        {"T=64,E=8,K=2,D=256,I=512", {64, 8, 2, 256, 512}},
        {"T=128,E=8,K=2,D=256,I=512", {128, 8, 2, 256, 512}},
        {"T=64,E=8,K=4,D=256,I=512", {64, 8, 4, 256, 512}},
        {"T=128,E=16,K=2,D=512,I=1024", {128, 16, 2, 512, 1024}},
    };
    for (auto& c : configs) bench_one(c.label, c.cfg, warmup, iters);
    std::printf("\n");
    return 0;
}
