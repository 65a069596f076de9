// bench_dsa -- the reference's DSA latency benchmark (benchmarks/bench_dsa.cu)
// through the drop-in header: same six configs, argv [warmup=10] [iters=50],
// same table with Q/s, inputs from glibc rand() after srand(123) and the
// reference's sorted sparse-index generator.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/naive_dsa.h"

#define HIP_OK(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,       \
                         hipGetErrorString(e_));                                       \
            std::exit(EXIT_FAILURE);                                                   \
        }                                                                              \
    } while (0)

static void random_fill(float* data, size_t n, float lo, float hi) {
    for (size_t i = 0; i < n; i++) data[i] = lo + static_cast<float>(rand()) / static_cast<float>(RAND_MAX) * (hi - lo);
}

// tests/test_dsa.cu:73-85 (partial Fisher-Yates, then sorted)
static void gen_sparse_indices(int* indices, int Q, int S, int N) {
    std::vector<int> pool(N);
    for (int q = 0; q < Q; q++) {
        std::iota(pool.begin(), pool.end(), 0);
        for (int i = 0; i < S; i++) std::swap(pool[i], pool[i + rand() % (N - i)]);
        std::sort(pool.begin(), pool.begin() + S);
        for (int s = 0; s < S; s++) indices[q * S + s] = pool[s];
    }
}

template <typename T> static T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

static void bench_one(const char* label, const DsaConfig& c, int warmup, int iters) {
    const int Q = c.num_queries, H = c.num_heads, Dc = c.head_dim_compressed,
              Dp = c.head_dim_positional, S = c.num_selected_kv, N = c.total_kv_tokens;
    std::vector<float> qn((size_t)Q * H * Dc), qp((size_t)Q * H * Dp), kc((size_t)N * Dc),
        kp((size_t)N * Dp), v((size_t)N * Dc);
    std::vector<int> idx((size_t)Q * S);
    random_fill(qn.data(), qn.size(), -0.3f, 0.3f);
    random_fill(qp.data(), qp.size(), -0.3f, 0.3f);
    random_fill(kc.data(), kc.size(), -0.3f, 0.3f);
    random_fill(kp.data(), kp.size(), -0.3f, 0.3f);
    random_fill(v.data(), v.size(), -0.3f, 0.3f);
    gen_sparse_indices(idx.data(), Q, S, N);
    float *dqn = upload(qn), *dqp = upload(qp), *dkc = upload(kc), *dkp = upload(kp), *dv = upload(v);
    int* didx = upload(idx);
    float* dout = nullptr;
    HIP_OK(hipMalloc(&dout, (size_t)Q * H * Dc * sizeof(float)));
    for (int i = 0; i < warmup; i++) dsa_forward(dqn, dqp, dkc, dkp, dv, didx, dout, c);
    HIP_OK(hipDeviceSynchronize());
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    std::vector<float> times(iters);
    for (int i = 0; i < iters; i++) {
        HIP_OK(hipEventRecord(a, 0));
        dsa_forward(dqn, dqp, dkc, dkp, dv, didx, dout, c);
        HIP_OK(hipEventRecord(b, 0));
        HIP_OK(hipEventSynchronize(b));
        HIP_OK(hipEventElapsedTime(&times[i], a, b));
    }
    std::sort(times.begin(), times.end());
    float mean = 0.0f;
    for (float t : times) mean += t;
    mean /= iters;
    std::printf("  %-40s  %8.3f  %8.3f  %8.3f  %8.3f  %10.0f\n", label, times.front(), mean,
                times[iters / 2], times.back(), Q / (mean * 1e-3f));
    HIP_OK(hipEventDestroy(a));
    HIP_OK(hipEventDestroy(b));
    for (float* p : {dqn, dqp, dkc, dkp, dv, dout}) HIP_OK(hipFree(p));
    HIP_OK(hipFree(didx));
}

int main(int argc, char** argv) {
    int warmup = 10, iters = 50;
    if (argc > 1) warmup = std::atoi(argv[1]);
    if (argc > 2) iters = std::atoi(argv[2]);
    std::printf("=== DSA Kernel Benchmark (gfx950) ===\n");
    std::printf("    warmup=%d  iters=%d\n\n", warmup, iters);
    std::printf("  %-40s  %8s  %8s  %8s  %8s  %10s\n", "Config", "Min(ms)", "Mean(ms)", "Med(ms)",
                "Max(ms)", "Q/s");
    std::printf("  %s\n", std::string(100, '-').c_str());
    srand(123);
    struct { const char* label; DsaConfig cfg; } configs[] = {
        {"Q=4,H=4,Dc=64,Dp=16,S=64,N=256", {4, 4, 64, 16, 64, 16, 256}},
        {"Q=8,H=8,Dc=128,Dp=32,S=128,N=512", {8, 8, 128, 32, 128, 32, 512}},
        {"Q=16,H=8,Dc=128,Dp=32,S=256,N=1024", {16, 8, 128, 32, 256, 64, 1024}},
        {"Q=8,H=16,Dc=256,Dp=64,S=256,N=2048", {8, 16, 256, 64, 256, 64, 2048}},
        {"Q=4,H=16,Dc=512,Dp=64,S=512,N=4096", {4, 16, 512, 64, 512, 64, 4096}},
        {"Q=8,H=16,Dc=512,Dp=64,S=1024,N=8192", {8, 16, 512, 64, 1024, 64, 8192}},
    };
    for (auto& c : configs) bench_one(c.label, c.cfg, warmup, iters);
    std::printf("\n");
    return 0;
}
