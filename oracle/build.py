"""TEST INFRASTRUCTURE — builds liboracle_model.so from the oracle's C restatements.

gcc -O2 with -ffp-contract=off and no fast math: every float operation in the model is one
IEEE round-to-nearest SSE operation and subnormals are kept (the default MXCSR).  OpenMP only
splits rows across threads; the per-row arithmetic is sequential.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCES = ("gemv_model.c",)
LIBRARY = HERE / "liboracle_model.so"
FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
         "-Wall", "-Werror"]  # fmt: skip


def build() -> Path:
    cmd = ["gcc", *FLAGS, *(str(HERE / s) for s in SOURCES), "-o", str(LIBRARY)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the oracle's C model failed:\n{res.stderr}")
    return LIBRARY


if __name__ == "__main__":
    print(build())
