"""Audit the AMDGCN assembly of the trusted kernels (this build's counterpart of the
reference's PTX audit, `src/pck/cuda/ptx_audit.py`).

The checkers' bounds assume IEEE arithmetic as written: no contraction of separate multiplies
and adds, no fast-math, subnormals preserved, and `expf` only where its error is part of a
stated bound.  The bit-exact product trees (tree GEMV, batched product) must be FP32 adds of
the products, never fused.  This script compiles each trusted HIP source for gfx950 with the
library's own flags (`pck._build`) to assembly and reports:

- build flags that allow contraction, fast math or flushed subnormals, or that leave packed
  FP32 instructions enabled;
- packed FP32 instructions (`v_pk_fma_f32`, `v_pk_mul_f32`, `v_pk_add_f32`) anywhere;
- scalar-memory writes or atomics (`s_store*`, `s_buffer_store*`, `s_atomic*`,
  `s_buffer_atomic*`, `s_dcache_wb*`, `s_scratch_store*`) anywhere;
- a kernel whose FP32 or FP16/FP64 denormal mode is not "preserve" (3), or IEEE mode off;
- in the tree sources, any FP32 multiply-add (`v_fma_f32`, `v_fmac_f32`, `v_mad_f32`,
  `v_mac_f32`, mixed or dot forms) other than the integer-division idiom, `v_fmamk_f32` with
  the constants 2^32 or -2^32;
- approximate FP32 transcendentals (`v_exp_f32`, `v_log_f32`, `v_rsq_*`, `v_sqrt_*`) outside
  the sources whose bounds take `expf`'s error as a hypothesis (membership, set sampling);
- `v_rcp_f32` other than in the integer-division idiom (the first instruction that reads its
  result multiplies it by 0x5f7ffffc) or inside an IEEE division sequence (a
  `v_div_fixup_f32` within the next 40 vector instructions), and `v_rcp_f64` other than inside
  an IEEE division sequence (a `v_div_fixup_f64` within the next 40 vector instructions);
- any write of a hardware register (`s_setreg*`, `s_round_mode`, `s_denorm_mode`) other than
  the checkers' upward-add window: the FP64 rounding field set to round toward +inf, then
  only `v_add_f64` and `s_nop`, then the field set back to round to nearest even (an
  unclosed window, or any other instruction inside one, is reported).

The library's other sources (the agent's templates, their INT8 copy, the read stream) are held
to the same rules: the templates are bit-exact FP32 trees like the trusted GEMV.

Run:  python -m pck.cuda.isa_audit        (needs hipcc; reads only assembly built here)
"""

from __future__ import annotations

import re
import subprocess
import sys
import tempfile
from collections.abc import Sequence
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from pck import _build

TRUSTED_HIP = ("gemv.hip", "bgemm.hip", "checker.hip", "bcheck.hip", "member.hip", "sampling.hip")
OTHER_HIP = ("template.hip", "quantize.hip", "measure.hip")  # built into the library, untrusted
LIBRARY_HIP = TRUSTED_HIP + OTHER_HIP
TREE_SOURCES = {"gemv.hip", "bgemm.hip", "template.hip"}  # bit-exact FP32 trees: adds only
EXP_SOURCES = {"member.hip", "sampling.hip"}  # bounds that take expf's error as a hypothesis

REQUIRED_FLAGS = ("-ffp-contract=off", "-fno-fast-math", "-packed-fp32-ops")
FORBIDDEN_FLAGS = re.compile(
    r"^(-ffast-math|-funsafe-math-optimizations|-ffp-contract=(fast|on)|"
    r"-fgpu-flush-denormals-to-zero|-fno-honor-(nans|infinities)|-freciprocal-math|"
    r"-fassociative-math|-cl-fast-relaxed-math|-ffinite-math-only)$"
)

PACKED_FP32 = re.compile(r"^v_pk_(fma|mul|add)_f32")
SCALAR_WRITE = re.compile(r"^s_(store|buffer_store|atomic|buffer_atomic|dcache_wb|scratch_store)")
FP32_MULADD = re.compile(r"^v_(fma|fmac|mad|mac|fmamk|fmaak|madmk|madak)_f32|^v_(fma|mad)_mix|^v_dot\d")
INT_DIV_FMAMK = re.compile(r"^v_fmamk_f32\b.*,\s*0x(4f800000|cf800000)\s*,")
TRANSCENDENTAL = re.compile(r"^v_(exp|log)_f32|^v_(rsq|sqrt)_f(16|32|64)")
INT_DIV_MUL = re.compile(r"^v_mul_f32\w*\s.*0x5f7ffffc")
MODE_WRITE = re.compile(r"^s_(setreg\w*|round_mode|denorm_mode)$")
UPWARD_ON = "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 1"
UPWARD_OFF = "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 0"
UPWARD_BODY = re.compile(r"^(s_nop|v_add_f64)$")

_INSN = re.compile(r"^\s+([a-z][a-z0-9_]*)(?:\s+(.*))?$")
_KERNEL = re.compile(r"^\s*\.amdhsa_kernel\s+(\S+)")
_MODE = re.compile(r"^\s*\.amdhsa_(float_denorm_mode_32|float_denorm_mode_16_64|ieee_mode)\s+(\d+)")


def instructions(asm: str) -> list[str]:
    """Instruction lines (opcode and operands, comments removed), directives and labels
    excluded."""
    out = []
    for line in asm.splitlines():
        line = line.split(";", 1)[0].rstrip()
        m = _INSN.match(line)
        if m and not line.lstrip().startswith("."):
            out.append(f"{m.group(1)} {m.group(2) or ''}".strip())
    return out


def kernel_modes(asm: str) -> dict[str, dict[str, int]]:
    """Per kernel descriptor: its FP denormal modes and IEEE mode."""
    modes: dict[str, dict[str, int]] = {}
    current = None
    for line in asm.splitlines():
        m = _KERNEL.match(line)
        if m:
            current = m.group(1)
            modes[current] = {}
            continue
        if current is not None:
            mm = _MODE.match(line)
            if mm:
                modes[current][mm.group(1)] = int(mm.group(2))
            elif line.strip() == ".end_amdhsa_kernel":
                current = None
    return modes


def violations(source: str, asm: str) -> list[str]:
    """Everything in this source's assembly that breaks the rules of the module docstring."""
    found: list[str] = []
    insns = instructions(asm)

    def vector_window(i: int, count: int) -> list[str]:
        """The next ``count`` vector instructions after i (the scheduler interleaves scalar
        and memory instructions into these sequences)."""
        out = []
        for j in range(i + 1, len(insns)):
            if insns[j].startswith("v_"):
                out.append(insns[j])
                if len(out) == count:
                    break
        return out

    def first_reader(i: int) -> str:
        """The first later instruction that reads the 32-bit destination register of
        instruction i (within 40 instructions)."""
        operands = insns[i].split(" ", 1)[1] if " " in insns[i] else ""
        dest = operands.split(",", 1)[0].strip()
        reads = re.compile(rf"(?<![\w\[:]){re.escape(dest)}(?![\w\]:])")
        for j in range(i + 1, min(len(insns), i + 41)):
            ops = insns[j].split(" ", 1)[1] if " " in insns[j] else ""
            if "," in ops and reads.search(ops.split(",", 1)[1]):
                return insns[j]
        return ""

    upward = False  # inside an upward-add window
    for i, ins in enumerate(insns):
        op = ins.split(" ", 1)[0]
        if ins == UPWARD_ON and not upward:
            upward = True
        elif ins == UPWARD_OFF and upward:
            upward = False
        elif MODE_WRITE.match(op):
            found.append(f"{source}: hardware-register write outside the upward-add window: {ins}")
        elif upward and not UPWARD_BODY.match(op):
            found.append(f"{source}: instruction under the upward rounding mode: {ins}")
        if PACKED_FP32.match(op):
            found.append(f"{source}: packed FP32 instruction: {ins}")
        if SCALAR_WRITE.match(op):
            found.append(f"{source}: scalar-memory write or atomic: {ins}")
        if source in TREE_SOURCES and FP32_MULADD.match(op) and not INT_DIV_FMAMK.match(ins):
            found.append(f"{source}: FP32 multiply-add in a bit-exact tree source: {ins}")
        if TRANSCENDENTAL.match(op) and source not in EXP_SOURCES:
            found.append(f"{source}: approximate transcendental outside the expf sources: {ins}")
        if op.startswith("v_rcp_f32") and not INT_DIV_MUL.match(first_reader(i)):
            if not any(w.startswith("v_div_fixup_f32") for w in vector_window(i, 40)):
                found.append(
                    f"{source}: v_rcp_f32 outside the integer-division idiom and IEEE division: {ins}"
                )
        if op.startswith("v_rcp_f64"):
            if not any(w.startswith("v_div_fixup_f64") for w in vector_window(i, 40)):
                found.append(f"{source}: v_rcp_f64 outside an IEEE division sequence: {ins}")
    if upward:
        found.append(f"{source}: upward rounding mode left set at the end of the code")
    modes = kernel_modes(asm)
    if not modes:
        found.append(f"{source}: no kernel descriptors found")
    for kernel, m in modes.items():
        if m.get("float_denorm_mode_32") != 3 or m.get("float_denorm_mode_16_64") != 3:
            found.append(f"{source}: {kernel} does not preserve subnormals ({m})")
        if m.get("ieee_mode") != 1:
            found.append(f"{source}: {kernel} runs with IEEE mode off ({m})")
    return found


def check_flags(flags: Sequence[str]) -> list[str]:
    """Problems with the library's compiler flags."""
    problems = [f"forbidden flag {f}" for f in flags if FORBIDDEN_FLAGS.match(f)]
    problems += [f"missing flag {f}" for f in REQUIRED_FLAGS if f not in flags]
    return problems


def compile_to_asm(source: str, out_dir: Path) -> str:
    """gfx950 assembly of one trusted source, with the library's flags."""
    out = out_dir / f"{source}.s"
    cmd = [
        _build.hipcc(), *_build.HIPCC_FLAGS, *_build.SOURCE_FLAGS.get(source, []),
        f"-I{_build.INCLUDE}", f"-I{_build.CSRC}", "--cuda-device-only", "-S",
        # hipcc adds --hip-link, which a compile to assembly does not use
        "-Wno-unused-command-line-argument", str(_build.CSRC / source), "-o", str(out),
    ]  # fmt: skip
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{res.stderr}")
    return out.read_text()


def audit(sources: Sequence[str] = TRUSTED_HIP) -> list[str]:
    """Every violation over the given trusted sources and the build flags."""
    found = check_flags(_build.HIPCC_FLAGS)
    with tempfile.TemporaryDirectory() as tmp, ThreadPoolExecutor(len(sources)) as pool:
        texts = list(pool.map(lambda s: compile_to_asm(s, Path(tmp)), sources))
    for source, asm in zip(sources, texts, strict=True):
        found += violations(source, asm)
    return found


def main() -> int:
    found = audit(LIBRARY_HIP)
    for line in found:
        print(line)
    print(f"{len(LIBRARY_HIP)} sources audited, {len(found)} violation(s)")
    return 1 if found else 0


if __name__ == "__main__":
    sys.exit(main())
