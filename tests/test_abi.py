"""Host-side checks of the C ABI (no GPU needed): the library loads, exports
every entry point include/amdmoe.h declares, and rejects bad arguments
before touching the device."""
import ctypes
import os
import re

import pytest

import amdmoe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "amdmoe.h")).read()
    return sorted(set(re.findall(r"\b(amdmoe_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(amdmoe.SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(amdmoe.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_config_structs_match_reference_layout():
    # MoeConfig {T,E,K,D,I} and DsaConfig {Q,H,Dc,Dp,S,P,N}: plain ints in order
    assert ctypes.sizeof(amdmoe.MoeConfig) == 5 * 4
    assert [f[0] for f in amdmoe.MoeConfig._fields_] == [
        "num_tokens", "num_experts", "top_k", "hidden_dim", "intermediate_dim"]
    assert ctypes.sizeof(amdmoe.DsaConfig) == 7 * 4
    assert [f[0] for f in amdmoe.DsaConfig._fields_] == [
        "num_queries", "num_heads", "head_dim_compressed", "head_dim_positional",
        "num_selected_kv", "page_size", "total_kv_tokens"]


def test_workspace_size_is_computed_on_the_host():
    small = amdmoe.workspace_bytes(amdmoe.moe_config(4, 4, 2, 64, 128), amdmoe.AMDMOE_DTYPE_F32)
    big = amdmoe.workspace_bytes(amdmoe.moe_config(4096, 256, 8, 7168, 2048), amdmoe.AMDMOE_DTYPE_FP8)
    assert 0 < small < big
    # dominant terms at the DSV3 shape: bf16 pair rows (P*D*2) + fp8 activation (P*I)
    P = 4096 * 8
    assert big >= P * 7168 * 2 + P * 2048


def test_fp32_takes_any_hidden_and_intermediate_dim():
    # the reference's moe_forward takes any D and I (naive_moe.cu:400-471)
    for cfg in [(4, 4, 2, 60, 128), (5, 5, 3, 100, 50), (1, 1, 1, 1, 1)]:
        assert amdmoe.workspace_bytes(amdmoe.moe_config(*cfg), amdmoe.AMDMOE_DTYPE_F32) > 0


@pytest.mark.parametrize("cfg,dtype,msg", [
    ((4, 0, 2, 64, 128), 0, "num_experts"),
    ((4, 4, 0, 64, 128), 0, "top_k"),
    ((4, 4, 2, 96, 128), 1, "multiples of 64"),
    ((4, 4, 2, 192, 128), 2, "multiples of 128"),
    ((-1, 4, 2, 64, 128), 0, "num_tokens"),
])
def test_invalid_configs_are_rejected(cfg, dtype, msg):
    with pytest.raises(amdmoe.AmdMoeError, match=msg):
        amdmoe.workspace_bytes(amdmoe.moe_config(*cfg), dtype)


def test_forward_validates_before_device_work():
    lib = amdmoe.load()
    cfg = amdmoe.moe_config(4, 4, 99, 64, 128)
    rc = lib.amdmoe_moe_forward_f32(None, None, None, None, None, ctypes.byref(cfg), None, 0, None)
    assert rc == 1 and b"top_k" in lib.amdmoe_last_error()
    cfg = amdmoe.moe_config(4, 4, 2, 64, 128)
    rc = lib.amdmoe_moe_forward_f32(None, None, None, None, None, ctypes.byref(cfg), None, 0, None)
    assert rc == 1 and b"null" in lib.amdmoe_last_error()
    # empty batch is a no-op
    cfg = amdmoe.moe_config(0, 4, 2, 64, 128)
    assert lib.amdmoe_moe_forward_f32(None, None, None, None, None, ctypes.byref(cfg), None, 0, None) == 0
    dcfg = amdmoe.dsa_config(1, 48, 512, 64, 16, 64, 1024)
    rc = lib.amdmoe_dsa_decode_bf16_paged(None, None, None, None, None, None, ctypes.byref(dcfg), 1, None)
    assert rc == 1 and b"multiple of 32" in lib.amdmoe_last_error()
    dcfg = amdmoe.dsa_config(1, 32, 256, 64, 16, 64, 1024)
    rc = lib.amdmoe_dsa_decode_bf16_paged(None, None, None, None, None, None, ctypes.byref(dcfg), 1, None)
    assert rc == 1 and b"Dc=512" in lib.amdmoe_last_error()


def test_workspace_too_small_is_reported():
    lib = amdmoe.load()
    cfg = amdmoe.moe_config(4, 4, 2, 64, 128)
    rc = lib.amdmoe_moe_forward_f32(ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256),
                                    ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.byref(cfg),
                                    ctypes.c_void_p(4096), 16, None)
    assert rc == 3 and b"workspace" in lib.amdmoe_last_error()


def test_pack_weights_validates_before_device_work():
    lib = amdmoe.load()
    p = ctypes.c_void_p(4096)
    assert lib.amdmoe_pack_weights_fp8(None, 1, 16, 128, p, None) == 1
    assert b"null" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_fp8(p, 1, 24, 128, ctypes.c_void_p(8192), None) == 1
    assert b"16" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_fp8(p, 1, 16, 192, ctypes.c_void_p(8192), None) == 1
    assert b"128" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_fp8(p, 1, 16, 128, p, None) == 1
    assert b"in-place" in lib.amdmoe_last_error()


def test_pack_weights_bf16_validates_before_device_work():
    lib = amdmoe.load()
    p = ctypes.c_void_p(4096)
    assert lib.amdmoe_pack_weights_bf16(None, 1, 16, 64, p, None) == 1
    assert b"null" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_bf16(p, 1, 16, 96, ctypes.c_void_p(8192), None) == 1
    assert b"multiple of 64" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_bf16(p, 1, 24, 64, ctypes.c_void_p(8192), None) == 1
    assert b"16" in lib.amdmoe_last_error()
    assert lib.amdmoe_pack_weights_bf16(p, 1, 16, 64, p, None) == 1
    assert b"in-place" in lib.amdmoe_last_error()
    # the packed bf16 forward checks its configuration and pointers like the row-major one
    cfg = amdmoe.moe_config(4, 4, 2, 96, 128)
    rc = lib.amdmoe_moe_forward_bf16_packed(None, None, None, None, None, None, ctypes.byref(cfg), None, 0, None)
    assert rc == 1 and b"multiples of 64" in lib.amdmoe_last_error()
    cfg = amdmoe.moe_config(4, 4, 2, 64, 128)
    rc = lib.amdmoe_moe_forward_bf16_packed(None, None, None, None, None, None, ctypes.byref(cfg), None, 0, None)
    assert rc == 1 and b"null" in lib.amdmoe_last_error()
