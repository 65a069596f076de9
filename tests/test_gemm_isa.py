"""The grouped GEMM's in-flight weight registers are never touched before
their wait (see tests/isa_hazards.py), checked on the gfx950 assembly of
every csrc/moe_gemm_*.hip variant file as the library's Makefile compiles
it (the files compile in parallel)."""
import glob
import os
import shutil
import subprocess

import pytest

from isa_hazards import sgpr_hazards, violations

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRCS = sorted(glob.glob(os.path.join(ROOT, "llm-sys-project_amd", "csrc", "moe_gemm_*.hip")))
HIPCC = "/opt/rocm/bin/hipcc"


def test_checker_flags_a_copy_before_the_wait():
    asm = "\n".join([
        "_Zk:", "\tbuffer_load_dwordx4 v[2:5], v1, s[0:3], s4 offen offset:0",
        "\tv_mov_b32_e32 v9, v3", "\ts_waitcnt vmcnt(0)", "\ts_endpgm"])
    assert len(violations(asm)) == 1
    clean = asm.replace("\tv_mov_b32_e32 v9, v3\n\ts_waitcnt vmcnt(0)", "\ts_waitcnt vmcnt(0)\n\tv_mov_b32_e32 v9, v3")
    assert violations(clean) == []


def test_checker_counts_newer_loads_before_a_wait_covers():
    # vmcnt(1) leaves the newest load in flight: it covers the first load
    # only when another vector-memory instruction was issued after it
    asm = "\n".join([
        "_Zk:", "\tbuffer_load_dwordx4 v[2:5], v1, s[0:3], s4 offen offset:0",
        "\ts_waitcnt vmcnt(1)", "\tv_mov_b32_e32 v9, v3", "\ts_waitcnt vmcnt(0)", "\ts_endpgm"])
    assert len(violations(asm)) == 1
    covered = asm.replace("offset:0\n", "offset:0\n\tglobal_store_dword v1, v6, s[6:7]\n")
    assert violations(covered) == []


def test_sgpr_checker_flags_a_valu_written_soffset():
    asm = "\n".join([
        "_Zk:", "\tv_readfirstlane_b32 s4, v3",
        "\tbuffer_load_dwordx4 v[2:5], v1, s[0:3], s4 offen offset:0", "\ts_endpgm"])
    assert len(sgpr_hazards(asm)) == 1
    padded = asm.replace("s4, v3\n", "s4, v3\n\ts_nop 4\n")
    assert sgpr_hazards(padded) == []
    salu = asm.replace("v_readfirstlane_b32 s4, v3", "s_add_i32 s4, s5, 64")
    assert sgpr_hazards(salu) == []


def test_checker_follows_branches_to_a_use():
    asm = "\n".join([
        "_Zk:", "\tbuffer_load_dwordx4 v[2:5], v1, s[0:3], s4 offen offset:0",
        "\ts_cbranch_scc1 .LBB0_2", "\ts_waitcnt vmcnt(0)", ".LBB0_2:",
        "\tv_add_u32_e32 v4, v6, v7", "\ts_waitcnt vmcnt(0)", "\ts_endpgm"])
    assert len(violations(asm)) == 1


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc missing")
def test_grouped_gemm_weight_loads_are_never_touched_in_flight(tmp_path):
    assert len(SRCS) >= 7, SRCS
    procs = []
    for src in SRCS:
        out = tmp_path / (os.path.basename(src)[:-4] + ".s")
        procs.append((src, out, subprocess.Popen(
            [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "--cuda-device-only", "-S", src, "-o", str(out)],
            stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)))
    for src, out, p in procs:
        _, err = p.communicate()
        assert p.returncode == 0, (src, err[-2000:])
        asm = out.read_text()
        assert asm.count("buffer_load_dwordx4 v[") > 0, src
        if "_mx_" in src:
            assert asm.count("buffer_load_ubyte v") > 0, src
        bad = violations(asm)
        assert bad == [], (src, bad[:5])
        bad = sgpr_hazards(asm)
        assert bad == [], (src, bad[:5])
