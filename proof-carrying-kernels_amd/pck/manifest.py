"""Pinned checker hash and per-variant manifests (reference `src/pck/manifest.py`).

The trusted checker's files are hash-pinned in ``checker_lock.json``: `verify_pinned` raises
if the code on disk does not match, and a test keeps the lock current.  On MI355X the trusted
set is this build's: the host checkers and constants, the HIP kernels of the checkers and of
the products whose trees they bound, the rounding helpers, the C ABI header, the ctypes
signatures and the build script (its compiler flags are part of what the bounds assume:
no contraction, no fast math, no packed FP32).  A `Manifest` records what a certified variant
rests on: its config, the spec's parameters, the checker hash, the Lean hash when the Lean
sources are present (they are not in this build), the theorem names and the commit.

Update the lock after a deliberate change to a trusted file:
  python -m pck.manifest --update
"""

from __future__ import annotations

import argparse
import functools
import hashlib
import json
import subprocess
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any

SRC = Path(__file__).parent  # proof-carrying-kernels_amd/pck
PACKAGE_ROOT = SRC.parent  # proof-carrying-kernels_amd
ROOT = PACKAGE_ROOT.parent  # the repository
LOCK = SRC / "checker_lock.json"
TRUSTED = (
    "pck/fp.py",
    "pck/member.py",
    "pck/vllm_plugin.py",  # builds every input to the in-vLLM membership verdicts
    "pck/cuda/checker.py",
    "pck/cuda/sampling.py",
    "pck/cuda/batched.py",  # the batched product's tree height, which sets tau
    "pck/cuda/gemv.py",
    "pck/cuda/_lib.py",  # the ctypes signatures of the ABI
    "pck/_build.py",  # compiler flags: -ffp-contract=off, -fno-fast-math, no packed FP32
    "csrc/rounding.h",
    "csrc/check_pair.h",
    "csrc/checker.hip",
    "csrc/bcheck.hip",
    "csrc/sampling.hip",
    "csrc/member.hip",
    "csrc/gemv.hip",  # the tree whose height the b = 1 bound uses, and carried checks
    "csrc/bgemm.hip",  # the batched product's order
    "../include/pck_hip.h",
)
THEOREMS = {
    "T1 no false alarms": "PCK.t1_block",
    "T2 guaranteed detection": "PCK.t2_block",
    "T3 safe runtime threshold": "PCK.t3_no_false_alarm",
    "T4 randomized detection": "PCK.t4_computed",
    "T4 spread errors": "PCK.t4_spread_computed",
}
"""What a GEMV certificate rests on (the reference's Lean names, lean/PCK/*.lean)."""


class CheckerMismatch(RuntimeError):
    """The checker on disk is not the pinned one."""


_HASHES: dict[Path, tuple[tuple[int, int], str]] = {}


def _file_hash(path: Path) -> str:
    """SHA-256 of a file, re-read only when its modification time or size changes."""
    st = path.stat()
    stamp = (st.st_mtime_ns, st.st_size)
    cached = _HASHES.get(path)
    if cached is None or cached[0] != stamp:
        cached = (stamp, hashlib.sha256(path.read_bytes()).hexdigest())
        _HASHES[path] = cached
    return cached[1]


def file_hashes() -> dict[str, str]:
    return {name: _file_hash((PACKAGE_ROOT / name).resolve()) for name in TRUSTED}


def combined(hashes: dict[str, str]) -> str:
    """One hash over (name, file hash) pairs in name order."""
    text = "".join(f"{name}\0{digest}\n" for name, digest in sorted(hashes.items()))
    return hashlib.sha256(text.encode()).hexdigest()


def checker_hash() -> str:
    return combined(file_hashes())


def pinned() -> dict[str, Any]:
    data: dict[str, Any] = json.loads(LOCK.read_text())
    return data


def verify_pinned() -> None:
    """Raise `CheckerMismatch` naming the changed files if the checker is not the pinned one."""
    lock = pinned()
    if checker_hash() == lock["checker"]:
        return
    now = file_hashes()
    changed = sorted(name for name in TRUSTED if lock["files"].get(name) != now[name])
    raise CheckerMismatch(
        f"trusted checker differs from the pinned one ({', '.join(changed)}); "
        "review the change, then run: python -m pck.manifest --update"
    )


def lean_hash() -> str | None:
    """Hash of the Lean sources and build configuration (None where they are absent, as in
    this build)."""
    lean = ROOT / "lean"
    if not (lean / "lakefile.toml").exists():
        return None
    files = sorted(lean.glob("PCK/**/*.lean")) + [
        lean / n for n in ("PCK.lean", "lakefile.toml", "lake-manifest.json", "lean-toolchain")
    ]
    h = hashlib.sha256()
    for f in files:
        h.update(str(f.relative_to(lean)).encode() + b"\0" + _file_hash(f).encode() + b"\0")
    return h.hexdigest()


def git_commit() -> str | None:
    return _git_commit(ROOT)


@functools.cache
def _git_commit(root: Path) -> str | None:
    """HEAD of the checkout at ``root``, once per process."""
    try:
        out = subprocess.run(
            ["git", "rev-parse", "HEAD"], cwd=root, capture_output=True, text=True, check=True
        )
    except (OSError, subprocess.CalledProcessError):
        return None
    return out.stdout.strip() or None


@dataclass(frozen=True)
class Manifest:
    """What one certified variant rests on (reference `manifest.py:132-159`)."""

    task: str
    config: dict[str, Any]
    slot_code: str | None
    spec: dict[str, int]
    speedup: float
    checker: str = field(default_factory=checker_hash)
    lean: str | None = field(default_factory=lean_hash)
    theorems: dict[str, str] = field(default_factory=lambda: dict(THEOREMS))
    commit: str | None = field(default_factory=git_commit)

    def to_json(self) -> str:
        return json.dumps(asdict(self), indent=2, sort_keys=True) + "\n"

    @classmethod
    def from_json(cls, text: str) -> Manifest:
        return cls(**json.loads(text))

    def problems(self) -> list[str]:
        """Why this manifest does not match the pinned checker and current proofs."""
        out = []
        if self.checker != pinned()["checker"]:
            out.append("checker hash differs from the pinned checker")
        current = lean_hash()
        if current is not None and self.lean != current:
            out.append("Lean sources differ from the ones the certificate was made with")
        return out


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--update", action="store_true", help="re-pin the current checker")
    args = parser.parse_args()
    hashes = file_hashes()
    if args.update:
        LOCK.write_text(json.dumps({"checker": combined(hashes), "files": hashes}, indent=2) + "\n")
        print(f"pinned {combined(hashes)}")
        return
    try:
        verify_pinned()
        print(f"checker matches the pin {checker_hash()}")
    except CheckerMismatch as e:
        print(e)


if __name__ == "__main__":
    main()
