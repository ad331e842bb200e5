"""The AMDGCN audit of the trusted kernels (`pck.cuda.isa_audit`): each rule on hand-written
assembly fragments, the build flags, and the audit of the real gfx950 builds (hipcc, no GPU)."""

from __future__ import annotations

import shutil

import pytest

from pck import _build
from pck.cuda import isa_audit as audit


def kernel(body: str, denorm32: int = 3, denorm64: int = 3, ieee: int = 1) -> str:
    return f"""\t.text
k:
{body}
\ts_endpgm
\t.amdhsa_kernel k
\t\t.amdhsa_float_denorm_mode_32 {denorm32}
\t\t.amdhsa_float_denorm_mode_16_64 {denorm64}
\t\t.amdhsa_ieee_mode {ieee}
\t.end_amdhsa_kernel
"""


def test_clean_fragment_passes() -> None:
    assert audit.violations("gemv.hip", kernel("\tv_add_f32_e32 v1, v2, v3\n\tv_mul_f32_e32 v4, v1, v5")) == []


@pytest.mark.parametrize("op", ["v_pk_fma_f32 v[0:1], v[2:3], v[4:5], v[6:7]", "v_pk_add_f32 v[0:1], v[2:3], v[4:5]"])
def test_packed_fp32_is_flagged_everywhere(op: str) -> None:
    assert any("packed FP32" in v for v in audit.violations("checker.hip", kernel(f"\t{op}")))


@pytest.mark.parametrize("op", ["s_store_dword s1, s[2:3], 0x0", "s_atomic_add s1, s[2:3], 0x0", "s_dcache_wb"])
def test_scalar_memory_writes_are_flagged(op: str) -> None:
    assert any("scalar-memory" in v for v in audit.violations("member.hip", kernel(f"\t{op}")))


@pytest.mark.parametrize(("d32", "d64", "ieee"), [(0, 3, 1), (3, 2, 1), (3, 3, 0)])
def test_kernel_modes(d32: int, d64: int, ieee: int) -> None:
    assert audit.violations("bcheck.hip", kernel("\tv_add_f32_e32 v1, v2, v3", d32, d64, ieee))


def test_fused_fp32_in_a_tree_source_only() -> None:
    fma = kernel("\tv_fmac_f32_e32 v1, v2, v3")
    assert any("multiply-add" in v for v in audit.violations("bgemm.hip", fma))
    assert audit.violations("sampling.hip", fma) == []  # the split expf term is a stated FMA
    idiom = kernel("\tv_fmamk_f32 v1, v2, 0xcf800000, v1\n\tv_fmamk_f32 v1, v2, 0x4f800000, v1")
    assert audit.violations("gemv.hip", idiom) == []  # 64-bit integer division
    assert audit.violations("gemv.hip", kernel("\tv_fmamk_f32 v1, v2, 0x3f800000, v1"))


def test_transcendentals_only_in_the_expf_sources() -> None:
    exp = kernel("\tv_exp_f32_e32 v1, v2")
    assert audit.violations("checker.hip", exp)
    assert audit.violations("member.hip", exp) == []


def test_reciprocals_only_in_their_idioms() -> None:
    int_div = kernel(
        "\tv_rcp_f32_e32 v1, v1\n\tv_mov_b32_e32 v7, v6\n\tv_xor_b32_e32 v7, v8, v6\n"
        "\tv_mul_f32_e32 v1, 0x5f7ffffc, v1"
    )
    assert audit.violations("bgemm.hip", int_div) == []
    assert audit.violations("bgemm.hip", kernel("\tv_rcp_f32_e32 v1, v2\n\tv_mul_f32_e32 v3, v1, v4"))
    ieee_div = kernel("\tv_rcp_f64_e32 v[2:3], v[0:1]\n\tv_fma_f64 v[4:5], v[0:1], v[2:3], 1.0\n\tv_div_fixup_f64 v[6:7], v[4:5], v[0:1], v[8:9]")
    assert audit.violations("sampling.hip", ieee_div) == []
    assert audit.violations("sampling.hip", kernel("\tv_rcp_f64_e32 v[2:3], v[0:1]\n\tv_mul_f64 v[4:5], v[2:3], v[6:7]"))
    ieee_div32 = kernel("\tv_div_scale_f32 v2, s[0:1], v1, v1, v0\n\tv_rcp_f32_e32 v3, v2\n"
                        "\tv_fma_f32 v4, -v2, v3, 1.0\n\tv_div_fixup_f32 v5, v4, v1, v0")
    assert audit.violations("quantize.hip", ieee_div32) == []
    # the fused refinement of that sequence is still a multiply-add in a tree source
    assert any("multiply-add" in v for v in audit.violations("template.hip", ieee_div32))


def test_rounding_mode_writes_only_in_the_upward_add_window() -> None:
    on, off = audit.UPWARD_ON, audit.UPWARD_OFF
    window = f"\t{on}\n\ts_nop 1\n\tv_add_f64 v[2:3], v[2:3], v[4:5]\n\t{off}\n\ts_nop 1"
    assert audit.violations("checker.hip", kernel(window)) == []
    inside = f"\t{on}\n\tv_fma_f64 v[2:3], v[2:3], v[4:5], v[6:7]\n\t{off}"
    assert any("under the upward" in v for v in audit.violations("checker.hip", kernel(inside)))
    assert any("left set" in v for v in audit.violations("gemv.hip", kernel(f"\t{on}\n\tv_add_f64 v[2:3], v[2:3], v[4:5]")))
    for other in ("s_setreg_b32 hwreg(HW_REG_MODE, 0, 4), s2", "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 4, 4), 0",
                  "s_round_mode 0x1", "s_denorm_mode 0x0", off):  # fmt: skip
        assert any("hardware-register" in v for v in audit.violations("bcheck.hip", kernel(f"\t{other}")))


def test_build_flags() -> None:
    assert audit.check_flags(_build.HIPCC_FLAGS) == []
    assert audit.check_flags([*_build.HIPCC_FLAGS, "-ffast-math"]) == ["forbidden flag -ffast-math"]
    loose = [f for f in _build.HIPCC_FLAGS if f != "-ffp-contract=off"]
    assert audit.check_flags(loose) == ["missing flag -ffp-contract=off"]


@pytest.mark.skipif(shutil.which("hipcc") is None and not _build.Path("/opt/rocm/bin/hipcc").exists(), reason="needs hipcc")
def test_the_trusted_builds_pass() -> None:
    assert audit.audit() == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not _build.Path("/opt/rocm/bin/hipcc").exists(), reason="needs hipcc")
def test_the_other_library_sources_pass_the_same_rules() -> None:
    """The agent's templates (bit-exact trees, so no multiply-add), their INT8 copy and the
    read stream: every source built into the library is audited."""
    assert set(audit.LIBRARY_HIP) == set(_build.SOURCES)
    assert audit.audit(audit.OTHER_HIP) == []
