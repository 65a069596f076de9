"""The reference's own test matrices (configs and tolerances), shared by the
CPU and GPU suites."""

# tests/test_moe.cu:204-267 -- (name, (T, E, K, D, I), tol)
MOE_CASES = [
    ("small", (4, 4, 2, 64, 128), 1e-3),
    ("medium", (32, 8, 2, 128, 256), 1e-3),
    ("large", (64, 8, 2, 256, 512), 1e-2),
    ("topk4", (16, 8, 4, 128, 256), 1e-2),
    ("single-token", (1, 4, 2, 64, 128), 1e-3),
    ("single-expert", (8, 1, 1, 64, 128), 1e-3),
    ("topk1", (32, 16, 1, 128, 256), 1e-2),
    ("wide-ffn", (16, 4, 2, 64, 512), 1e-2),
    ("narrow-ffn", (16, 4, 2, 256, 64), 1e-2),
    ("sparse-routing", (4, 16, 2, 128, 256), 1e-3),
    ("many-tokens", (128, 8, 2, 128, 256), 1e-2),
    ("full-routing", (8, 4, 4, 64, 128), 1e-3),
    ("stress", (64, 16, 2, 512, 1024), 5e-2),
]

# tests/test_dsa.cu:162-230 -- (name, (Q, H, Dc, Dp, S, P, N), tol)
DSA_CASES = [
    ("tiny", (2, 2, 32, 8, 16, 8, 64), 1e-3),
    ("small", (4, 4, 64, 16, 64, 16, 256), 1e-3),
    ("medium", (8, 8, 128, 32, 128, 32, 512), 1e-2),
    ("large", (4, 4, 128, 32, 256, 64, 1024), 1e-2),
    ("single-query", (1, 4, 64, 16, 32, 8, 128), 1e-3),
    ("single-head", (4, 1, 64, 16, 64, 16, 256), 1e-3),
    ("minimal-S", (4, 4, 64, 16, 4, 4, 256), 1e-3),
    ("pos-heavy", (4, 4, 32, 64, 64, 16, 256), 1e-3),
    ("tiny-Dp", (4, 4, 128, 4, 64, 16, 256), 1e-2),
    ("many-heads", (4, 32, 64, 16, 64, 16, 256), 1e-2),
    ("many-queries", (32, 4, 64, 16, 64, 16, 512), 1e-2),
    ("full-cache", (4, 4, 64, 16, 128, 16, 128), 1e-3),
    ("large-cache", (4, 4, 128, 32, 128, 64, 4096), 1e-2),
    ("stress", (16, 16, 128, 32, 256, 64, 2048), 5e-2),
]
