"""The library's hipcc flags do what the numerics rely on, shown on the gfx950 assembly of a
probe kernel built here (no GPU needed):

- `-Xclang -target-feature -Xclang -packed-fp32-ops` takes effect in the device pass: the same
  float2 multiply-add code compiles to a packed FP32 FMA without it and to none with it (the
  "not a recognized feature" warning comes from the x86 host pass only);
- `-ffp-contract=off` keeps a separate multiply and add (no FMA) where the source writes them;
- the build treats warnings as errors.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from pck import _build

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                                reason="needs hipcc")  # fmt: skip

PROBE = """
#include <hip/hip_runtime.h>
__global__ void probe(float2* a, const float2* b, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    float2 u = a[i], v = b[i];
    u.x = u.x * v.x + v.y;
    u.y = u.y * v.y + v.x;
    a[i] = u;
  }
}
"""
PACKED_FEATURE = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def device_asm(tmp_path: Path, flags: list[str]) -> tuple[str, str]:
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / "probe.s"
    cmd = [_build.hipcc(), f"--offload-arch={_build.ARCH}", "-O3", *flags, "--cuda-device-only",
           "-Wno-unused-command-line-argument", "-S", str(src), "-o", str(out)]  # fmt: skip
    res = subprocess.run(cmd, capture_output=True, text=True, check=True)
    return out.read_text(), res.stderr


def opcodes(asm: str) -> list[str]:
    return [ln.split()[0] for ln in asm.splitlines() if ln.startswith("\tv_")]


def test_packed_fp32_feature_applies_to_device_code(tmp_path: Path) -> None:
    without, _ = device_asm(tmp_path, [])
    with_flag, stderr = device_asm(tmp_path, PACKED_FEATURE)
    assert any(op.startswith("v_pk_fma_f32") for op in opcodes(without))
    assert not any(op.startswith("v_pk_") and op.endswith("_f32") for op in opcodes(with_flag))
    assert "not a recognized feature" not in stderr  # device-only compile: no host pass


def test_contraction_off_keeps_mul_and_add(tmp_path: Path) -> None:
    asm, _ = device_asm(tmp_path, ["-ffp-contract=off", *PACKED_FEATURE])
    ops = opcodes(asm)
    assert not any(op.startswith(("v_fma_f32", "v_fmac_f32")) for op in ops)
    assert any(op.startswith("v_mul_f32") for op in ops) and any(op.startswith("v_add_f32") for op in ops)


def test_library_flags() -> None:
    flags = _build.HIPCC_FLAGS
    for required in ("-ffp-contract=off", "-fno-fast-math", "-Werror", "-Wall", "-Wextra"):
        assert required in flags
    at = flags.index("-target-feature")
    assert flags[at - 1 : at + 3] == PACKED_FEATURE
