"""Builds libpck_hip.so, the gfx950 HIP library behind `pck.cuda` and `pck.member`, and
libpck_probe.so, the probes of device arithmetic that tests run (`pck.cuda.probe`), with the
same flags.

Run ``python -m pck._build`` (with ``proof-carrying-kernels_amd`` on ``sys.path``) or call
`build`.  hipcc cross-compiles for gfx950 without a GPU.  The library lands next to this file
so it travels with the source tree; it is never installed into site-packages.

Flags that the numerics depend on:
  -ffp-contract=off   no mul + add -> FMA contraction (the GEMV adds rounded products, and the
                      checker's error-free transformations need separate roundings);
  no -ffast-math and no denormal flushing (kernel descriptors keep FP32/FP64 denormals);
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed FP32 instructions (v_pk_add/mul/fma_f32) in any kernel.  The
                      gfx950 device pass applies it (without it hipcc -O3 forms v_pk_fma_f32
                      from ordinary float2 code; tests/test_build_flags.py shows both); the x86
                      host pass prints "'-packed-fp32-ops' is not a recognized feature for this
                      target (ignoring feature)", which concerns host code only;
  -Wall -Wextra -Werror   every warning of the device and host passes fails the build.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIBRARY = PACKAGE / "libpck_hip.so"
SOURCES = (
    "gemv.hip",
    "bgemm.hip",
    "checker.hip",
    "bcheck.hip",
    "member.hip",
    "sampling.hip",
    "measure.hip",
    "template.hip",  # the agent's templates: kernels under test, outside the trusted set
    "quantize.hip",  # their INT8 weight copy
)
PROBE_LIBRARY = PACKAGE / "libpck_probe.so"
PROBE_SOURCES = ("probe.hip",)
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Wall",
    "-Wextra",
    "-Werror",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

# Per-source additions.  bcheck.hip keeps its matrix-core accumulators in ordinary VGPRs: with
# the default accumulator-register form the compiler copies every accumulator between register
# files on each loop pass (measured 6% of the batched checker's time).
SOURCE_FLAGS = {"bcheck.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libpck_hip.so)")
    return found


def _compile(src: Path, obj: Path) -> None:
    extra = SOURCE_FLAGS.get(src.name, [])
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")


def _link(objects: list[Path], library: Path) -> None:
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking {library.name} failed:\n{res.stderr}")
    os.replace(tmp, library)


def build(verbose: bool = False) -> Path:
    """Compile every source in csrc/, link libpck_hip.so and libpck_probe.so; returns the
    path of libpck_hip.so."""
    out_dir = ROOT / "_build"
    out_dir.mkdir(exist_ok=True)
    names = [s for s in SOURCES + PROBE_SOURCES if (CSRC / s).exists()]
    sources = [CSRC / s for s in names]
    objects = {s: out_dir / (Path(s).stem + ".o") for s in names}
    jobs = min(len(sources), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(_compile, sources, [objects[s] for s in names]))
    _link([objects[s] for s in SOURCES if s in objects], LIBRARY)
    _link([objects[s] for s in PROBE_SOURCES if s in objects], PROBE_LIBRARY)
    if verbose:
        print(f"built {LIBRARY} and {PROBE_LIBRARY.name}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
