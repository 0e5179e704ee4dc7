"""The sip and gulp kernels' untracked payload loads (and the raw twin's), checked on their gfx950
assembly: no instruction between a load and its `s_waitcnt` touches the
load's destination registers (no spill, copy or reuse of an in-flight
register). The checker itself is pinned on small hand-written programs, each
with one planted mistake or one pattern it must accept.

Runs on the CPU: hipcc cross-compiles the device code to assembly.
"""

import os
import re
import shutil
import subprocess

import pytest

from tests.asm_inflight import analyse, kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


def _flagged(body):
    return analyse(body)[0]


def test_read_before_wait_is_flagged():
    body = """
    buffer_load_dword v1, v2, s[0:3], s4 offen
    v_add_u32_e32 v3, v1, v1
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert len(_flagged(body)) == 1


def test_read_after_wait_is_clean():
    body = """
    buffer_load_dword v1, v2, s[0:3], s4 offen
    s_waitcnt vmcnt(0)
    v_add_u32_e32 v3, v1, v1
    s_endpgm
    """
    assert _flagged(body) == []


def test_partial_wait_retires_only_the_older_loads():
    # stage A (v1, v[2:3]) then stage B (v4, v[5:6]); vmcnt(2) completes A only
    body = """
    buffer_load_dword v1, v10, s[0:3], s4 offen
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
    buffer_load_dword v4, v10, s[0:3], s5 offen
    buffer_load_dwordx2 v[5:6], v11, s[0:3], s5 offen
    s_waitcnt vmcnt(2)
    v_add_u32_e32 v7, v1, v3
    v_add_u32_e32 v8, v4, v4
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    hz = _flagged(body)
    assert len(hz) == 1 and "v8, v4, v4" in hz[0][2]


def test_a_load_to_lds_holds_no_register_but_counts_in_vmcnt():
    # a buffer load with the lds modifier writes LDS, not its first operand
    # (its address): reusing that register is fine. It still counts in
    # vmcnt: vmcnt(1) after it retires the older load, so v1 is ready (were
    # it not counted, v1's load would be the one left in flight)
    body = """
    buffer_load_dword v1, v10, s[0:3], s4 offen
    buffer_load_dword v2, s[0:3], 0 offen lds
    v_mov_b32_e32 v2, 0
    s_waitcnt vmcnt(1)
    v_add_u32_e32 v3, v1, v1
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert _flagged(body) == []
    # without the vmcnt(1), the read of v1 is flagged (and only it)
    hz = _flagged(body.replace("s_waitcnt vmcnt(1)", ""))
    assert len(hz) == 1 and "v3, v1, v1" in hz[0][2]


def test_spill_and_reuse_of_an_inflight_register_are_flagged():
    body = """
    buffer_load_dword v1, v12, s[28:31], s18 offen
    scratch_store_dword off, v1, off offset:32
    v_lshrrev_b32_e32 v1, 4, v0
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert len(_flagged(body)) == 2


def test_a_path_that_skips_the_newer_loads_is_flagged():
    # on the taken branch stage B is never issued, so vmcnt(2) leaves A in flight
    body = """
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
    s_cmp_eq_u32 s6, 0
    s_cbranch_scc1 .LBB0_2
    buffer_load_dwordx2 v[5:6], v11, s[0:3], s5 offen
.LBB0_2:
    s_waitcnt vmcnt(2)
    v_add_u32_e32 v7, v2, v3
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert len(_flagged(body)) == 1


def test_two_load_variants_of_a_uniform_branch_are_not_mixed():
    # the compiler's form of `t ? load(b) : load(a)`: s[4:5] steers the
    # second branch, so exactly one variant issues on every path
    body = """
    s_mov_b64 s[4:5], -1
    s_and_b64 vcc, exec, s[6:7]
    s_cbranch_vccnz .LBB0_2
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
    s_mov_b64 s[4:5], 0
.LBB0_2:
    s_andn2_b64 vcc, exec, s[4:5]
    s_cbranch_vccnz .LBB0_4
    buffer_load_dwordx2 v[2:3], v11, s[8:11], s4 offen
.LBB0_4:
    buffer_load_dwordx2 v[5:6], v11, s[0:3], s5 offen
    s_waitcnt vmcnt(1)
    v_add_u32_e32 v7, v2, v3
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert _flagged(body) == []


def test_execz_inside_a_divergent_region_keeps_both_edges():
    # exec may be empty inside the saveexec region: the skip edge is real
    body = """
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
    v_cmp_ne_u32_e32 vcc, 0, v0
    s_and_saveexec_b64 s[6:7], vcc
    s_cbranch_execz .LBB0_2
    buffer_load_dwordx2 v[5:6], v11, s[0:3], s5 offen
.LBB0_2:
    s_or_b64 exec, exec, s[6:7]
    s_waitcnt vmcnt(1)
    v_add_u32_e32 v7, v2, v3
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert len(_flagged(body)) == 1


def test_execnz_with_full_exec_skips_the_other_variant():
    # the compiler's form of `t ? load(b) : load(a)` steered by exec: with
    # exec full the first variant branches over the second
    body = """
    s_cmp_eq_u32 s6, 0
    s_cbranch_scc1 .LBB0_2
    buffer_load_dwordx2 v[2:3], v11, s[8:11], s4 offen
    s_cbranch_execnz .LBB0_3
.LBB0_2:
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
.LBB0_3:
    buffer_load_dwordx2 v[5:6], v11, s[0:3], s5 offen
    s_waitcnt vmcnt(1)
    v_add_u32_e32 v7, v2, v3
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert _flagged(body) == []


def test_execnz_inside_a_divergent_region_keeps_both_edges():
    body = """
    v_cmp_ne_u32_e32 vcc, 0, v0
    s_and_saveexec_b64 s[6:7], vcc
    buffer_load_dwordx2 v[2:3], v11, s[8:11], s4 offen
    s_cbranch_execnz .LBB0_3
    buffer_load_dwordx2 v[2:3], v11, s[0:3], s4 offen
.LBB0_3:
    s_or_b64 exec, exec, s[6:7]
    s_waitcnt vmcnt(0)
    s_endpgm
    """
    assert len(_flagged(body)) == 1


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not installed")
    out = tmp_path_factory.mktemp("asm") / "kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-I", os.path.join(ROOT, "include"),
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           os.path.join(ROOT, "drinkme_amd", "csrc", "kernels.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def test_every_sip_and_gulp_kernel_keeps_its_inflight_registers(kernel_asm):
    ks = kernels(kernel_asm, r"k_gemv_(sip|gulp)I")
    # sip: 3 kinds x M = 1, 2, 4, 8; gulp: 2 x 4, and 8-wave workgroups at M = 1, 2, 4; the raw twin:
    # 2 x (M = 1, 2, 4, 8, and M = 4, 8 as gulp); the decode: sip and gulp; the matrix policy's gulp
    # M = 4 in quad units and its twin, unphased and phased
    assert len(ks) == 41
    for name, body in ks.items():
        hazards, reached, total = analyse(body)
        assert reached == total, f"{name}: walked {reached} of {total} blocks"
        assert not hazards, f"{name}: {len(hazards)} in-flight register uses, first {hazards[0][2]!r}"


def test_no_scratch_and_no_vgpr_spill_in_kernels_with_untracked_loads(kernel_asm):
    """A VGPR spill, or any scratch access, between an untracked load and its
    wait would move registers the compiler thinks are ready; SGPR spills go
    to lanes of VGPRs (v_writelane / v_readlane), which the in-flight walk
    above watches like any other register write or read. So: no scratch
    instruction, no private segment, no VGPR spill and no AGPR in any of
    these kernels; SGPR spills are counted and reported."""
    from tests.asm_inflight import metadata

    ks = kernels(kernel_asm, r"k_gemv_(sip|gulp)I")
    md = metadata(kernel_asm)
    sgpr_spills = {}
    for name, body in ks.items():
        assert name in md, f"{name}: no metadata"
        assert md[name].get("vgpr_spill_count", 0) == 0, f"{name}: {md[name]['vgpr_spill_count']} VGPR spills"
        assert "scratch_" not in body, f"{name}: scratch access"
        # nor a private segment at all: a frame the compiler reserves (an SGPR spill slot it then
        # placed in VGPR lanes) leaves no instruction but still has every dispatch set up scratch
        assert md[name].get("private_segment_fixed_size", 0) == 0, \
            f"{name}: {md[name]['private_segment_fixed_size']}-byte private segment"
        # the in-flight walk tracks VGPRs and SGPRs: a kernel that used AGPRs (as spill space, or an
        # MFMA's accumulators) would need the walk extended first
        assert md[name].get("agpr_count", 0) == 0 and not re.search(r"v_accvgpr|\ba\[?\d", body), \
            f"{name}: AGPRs in use"
        sgpr_spills[name] = md[name].get("sgpr_spill_count", 0)
        assert body.count("v_writelane_b32") >= sgpr_spills[name] > 0 or sgpr_spills[name] == 0
    print("SGPR spills (to VGPR lanes):", {k[20:60]: v for k, v in sgpr_spills.items() if v})


def _plan_constants(tmp_path):
    """kSipStaticLds and kGulpStaticLds as the host's plans use them."""
    src = tmp_path / "lds.cpp"
    src.write_text('#include <cstdio>\n#include "plan.h"\n'
                   'int main() { printf("%zu %zu\\n", dmx::kSipStaticLds, dmx::kGulpStaticLds); }\n')
    exe = tmp_path / "lds"
    subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "drinkme_amd", "csrc"), str(src), "-o", str(exe)],
                   check=True, timeout=120)
    sip, gulp = (int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.split())
    return sip, gulp


def test_static_lds_fits_what_the_plans_reserve(kernel_asm, tmp_path):
    """The host plans a launch's dynamic LDS (activation rows, row partials)
    around the kernels' static tables: a kernel whose static LDS outgrew
    the reserved figure would leave the plan's two workgroups per CU (or its
    column phases) unable to fit, and fail to launch. Each sip and gulp
    kernel's group segment, from its code-object metadata, fits in its
    family's figure."""
    from tests.asm_inflight import metadata

    sip_lds, gulp_lds = _plan_constants(tmp_path)
    md = metadata(kernel_asm)
    seen = 0
    for name, fields in md.items():
        fam = "gulp" if "k_gemv_gulp" in name else "sip" if "k_gemv_sip" in name else None
        if fam is None:
            continue
        seen += 1
        # the raw twins mirroring gulp (k_gemv_sip<false, M, PH, 2>, and 4 under the matrix policy) run
        # gulp's plan; at M = 1, 2 the twins of both run k_gemv_sip<false, M, PH, 1> under either plan
        twin = re.search(r"k_gemv_sipILb0ELi(\d)ELb[01]ELi([124])E", name)
        gulp_plan = fam == "gulp" or (twin and (twin.group(2) in "24" or twin.group(1) in "12"))
        limit = gulp_lds if gulp_plan else sip_lds
        assert fields["group_segment_fixed_size"] <= limit, (name, fields["group_segment_fixed_size"], limit)
    assert seen == 41
