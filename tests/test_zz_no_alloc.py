"""The no-allocation fp8 forward (amdmoe_moe_forward_fp8_packed_noalloc),
through the C ABI: the same result as amdmoe_moe_forward_fp8_packed with an
explicit workspace, bit for bit, on two calls in a row whose second input is
smaller (the library's per-GPU scratch keeps the first call's contents), no
change in free device memory across calls, and a clear error for a
configuration whose workspace exceeds the fixed scratch."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(amd, E, D, I, seed):
    import synth
    w1q, w1s, w2q, w2s = synth.dsv3_weights(E, D, I, seed=seed)
    p1, p2 = torch.empty_like(w1q), torch.empty_like(w2q)
    amd.pack_weights_fp8(w1q, p1)
    amd.pack_weights_fp8(w2q, p2)
    return p1, w1s, p2, w2s


def test_noalloc_forward_equals_packed_forward(amd):
    import synth
    E, K, D, I = 64, 8, 2048, 1024
    print("noalloc fp8 forward: E=64 K=8 D=2048 I=1024, T=300 then T=37", flush=True)
    p1, s1, p2, s2 = _layer(amd, E, D, I, seed=901)
    for T, seed in ((300, 902), (37, 903), (37, 904)):
        cfg = amd.moe_config(T, E, K, D, I)
        assert amd.workspace_bytes(cfg, amd.AMDMOE_DTYPE_FP8) <= amd.NOALLOC_SCRATCH_BYTES
        x, wg = synth.dsv3_inputs(T, E, D, seed=seed)
        ws = amd.alloc_workspace(cfg, amd.AMDMOE_DTYPE_FP8)
        y_ref = torch.empty((T, D), dtype=torch.int16, device="cuda")
        y = torch.full((T, D), -1, dtype=torch.int16, device="cuda")
        amd.moe_forward_fp8_packed(x, wg, p1, s1, p2, s2, y_ref, cfg, ws=ws)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        amd.moe_forward_fp8_packed_noalloc(x, wg, p1, s1, p2, s2, y, cfg)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert torch.equal(y, y_ref), f"T={T}"
        if seed != 902:  # after the first call on this device: nothing allocated
            assert free1 == free0
        print(f"noalloc T={T}: bit-identical to the packed forward", flush=True)


def test_noalloc_rejects_configs_beyond_its_scratch(amd):
    E, K, D, I = 256, 8, 7168, 2048
    cfg = amd.moe_config(4096, E, K, D, I)
    assert amd.workspace_bytes(cfg, amd.AMDMOE_DTYPE_FP8) > amd.NOALLOC_SCRATCH_BYTES
    t = torch.empty(16, dtype=torch.int16, device="cuda")
    w = torch.empty(16, dtype=torch.uint8, device="cuda")
    s = torch.empty(16, dtype=torch.float32, device="cuda")
    with pytest.raises(amd.AmdMoeError, match="no-allocation"):
        amd.moe_forward_fp8_packed_noalloc(t, t, w, s, w, s, t, cfg)
