"""The pinned trusted checker and per-variant certificates (interface of the reference's
`src/pck/manifest.py`: `verify_pinned`, `CheckerMismatch`, `Manifest`, ``--update``).

What is pinned.  The verdicts of this build rest on three things, and the lock
(``checker_lock.json``) records all three:

- the trusted source files: the host-side constants and wrappers, the HIP kernels of the
  checkers and of the products whose trees the thresholds bound, the rounding helpers, the C
  ABI header and the ctypes signatures (`TRUSTED`), each by its SHA-256;
- the compiler flags and target the library is built with (`pck._build`): no contraction, no
  fast math, no packed FP32, gfx950.  They are recorded as data, so a change of flags is
  reported as such, not as an anonymous change of the build script;
- a digest over both, which is what a certificate quotes (`checker_hash`).

`verify_pinned` raises `CheckerMismatch` naming every file or setting that differs from the
lock.  After a reviewed change: ``python -m pck.manifest --update``.

A `Manifest` is the certificate of one variant: its task, config, slot code, the spec's
parameters, the speedup, the checker digest, the digest of Lean sources when a ``lean/``
directory is present (this build has none), the theorems it rests on and the commit.
"""

from __future__ import annotations

import argparse
import hashlib
import json
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any

PACKAGE = Path(__file__).resolve().parent  # proof-carrying-kernels_amd/pck
PACKAGE_ROOT = PACKAGE.parent  # proof-carrying-kernels_amd
ROOT = PACKAGE_ROOT.parent  # the repository
LOCK = PACKAGE / "checker_lock.json"
LOCK_FORMAT = 2

# Paths relative to PACKAGE_ROOT.
TRUSTED = (
    "pck/fp.py",
    "pck/checker.py",  # the CPU blocked checker
    "pck/sampling.py",  # the CPU set-sampling checker
    "pck/member.py",
    "pck/vllm_plugin.py",  # builds every input to the in-vLLM membership verdicts
    "pck/cuda/checker.py",
    "pck/cuda/sampling.py",
    "pck/cuda/batched.py",  # the batched product's tree height, which sets tau
    "pck/cuda/gemv.py",
    "pck/cuda/_lib.py",  # the ctypes signatures of the ABI
    "csrc/rounding.h",
    "csrc/check_pair.h",
    "csrc/rowsum_check.h",
    "csrc/checker.hip",
    "csrc/bcheck.hip",
    "csrc/sampling.hip",
    "csrc/member.hip",
    "csrc/gemv.hip",  # the tree whose height the b = 1 bound uses; in-pass sums; carried checks
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
"""The reference's Lean theorems a GEMV certificate rests on (lean/PCK/*.lean there)."""


class CheckerMismatch(RuntimeError):
    """The trusted checker on disk, or its build settings, differ from the lock."""


_DIGESTS: dict[Path, tuple[int, int, str]] = {}


def digest_file(path: Path) -> str:
    """SHA-256 of a file, streamed; recomputed only when its size or modification time
    changes (a proof-gated evaluation checks the pin before every episode)."""
    st = path.stat()
    cached = _DIGESTS.get(path)
    if cached is not None and cached[:2] == (st.st_size, st.st_mtime_ns):
        return cached[2]
    h = hashlib.sha256()
    with path.open("rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    _DIGESTS[path] = (st.st_size, st.st_mtime_ns, h.hexdigest())
    return h.hexdigest()


def build_settings() -> dict[str, Any]:
    """The compiler settings the thresholds assume, as the library is built."""
    from pck import _build

    return {
        "arch": _build.ARCH,
        "flags": list(_build.HIPCC_FLAGS),
        "source_flags": {k: list(v) for k, v in sorted(_build.SOURCE_FLAGS.items())},
    }


def current_state() -> dict[str, Any]:
    """Digests of the trusted files and the build settings, as the lock stores them."""
    files = {name: digest_file(PACKAGE_ROOT / name) for name in TRUSTED}
    return {"files": files, "build": build_settings()}


def digest_state(state: dict[str, Any]) -> str:
    """One digest over a state: canonical JSON (sorted keys, no whitespace) of files and
    build settings."""
    canonical = json.dumps(
        {"files": state["files"], "build": state["build"]}, sort_keys=True, separators=(",", ":")
    )
    return hashlib.sha256(canonical.encode()).hexdigest()


def checker_hash() -> str:
    """The digest a certificate quotes for the checker on disk."""
    return digest_state(current_state())


def pinned() -> dict[str, Any]:
    """The lock: {"format", "checker", "files", "build"}."""
    data: dict[str, Any] = json.loads(LOCK.read_text())
    return data


def differences(lock: dict[str, Any], state: dict[str, Any]) -> list[str]:
    """Every trusted file and build setting on which ``state`` departs from ``lock``."""
    out = []
    names = sorted(set(lock.get("files", {})) | set(state["files"]))
    out += [n for n in names if lock.get("files", {}).get(n) != state["files"].get(n)]
    build = lock.get("build", {})
    out += [f"build {k}" for k in sorted(state["build"]) if build.get(k) != state["build"][k]]
    return out


def verify_pinned() -> None:
    """Raise `CheckerMismatch` naming what changed if the trusted checker on disk (files or
    build settings) is not the pinned one."""
    lock = pinned()
    state = current_state()
    changed = differences(lock, state)
    if lock.get("format") != LOCK_FORMAT:
        changed.append("lock format")
    if not changed and digest_state(state) == lock.get("checker"):
        return
    changed = changed or ["lock digest"]
    raise CheckerMismatch(
        f"trusted checker differs from the pinned one ({', '.join(changed)}); review the change, "
        "then run: python -m pck.manifest --update"
    )


def write_lock(path: Path | None = None) -> str:
    """Pin the current state; returns its digest."""
    state = current_state()
    digest = digest_state(state)
    lock = {"format": LOCK_FORMAT, "checker": digest, **state}
    (path or LOCK).write_text(json.dumps(lock, indent=2, sort_keys=True) + "\n")
    return digest


def lean_hash() -> str | None:
    """Digest of the Lean sources and their build configuration under ``ROOT/lean`` (None
    when there is no such directory, as in this build: its thresholds carry the reference's
    theorems, which are not rebuilt here)."""
    lean = ROOT / "lean"
    if not lean.is_dir():
        return None
    wanted = [p for p in sorted(lean.rglob("*")) if p.is_file() and (
        p.suffix == ".lean" or p.name in ("lakefile.toml", "lake-manifest.json", "lean-toolchain")
    ) and ".lake" not in p.parts]  # fmt: skip
    listing = {str(p.relative_to(lean)): digest_file(p) for p in wanted}
    return hashlib.sha256(json.dumps(listing, sort_keys=True).encode()).hexdigest()


def git_commit(root: Path | None = None) -> str | None:
    """The commit checked out at ``root`` (default: the repository), read from ``.git``
    directly (HEAD, a loose ref or packed-refs); None outside a checkout."""
    git = (root or ROOT) / ".git"
    try:
        head = (git / "HEAD").read_text().strip()
    except OSError:
        return None
    if not head.startswith("ref: "):
        return head or None
    ref = head[5:]
    try:
        return (git / ref).read_text().strip() or None
    except OSError:
        pass
    try:
        for line in (git / "packed-refs").read_text().splitlines():
            parts = line.split()
            if len(parts) == 2 and parts[1] == ref:
                return parts[0]
    except OSError:
        pass
    return None


@dataclass(frozen=True)
class Manifest:
    """The certificate of one variant (the reference's fields, `src/pck/manifest.py:132-159`)."""

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
        """Why this certificate does not stand against the pinned checker and current proofs."""
        out = []
        if self.checker != pinned()["checker"]:
            out.append("checker hash differs from the pinned checker")
        lean = lean_hash()
        if lean is not None and self.lean != lean:
            out.append("Lean sources differ from the ones the certificate was made with")
        return out


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="Pin or verify the trusted checker.")
    parser.add_argument("--update", action="store_true", help="pin the checker on disk")
    args = parser.parse_args(argv)
    if args.update:
        print(f"pinned {write_lock()}")
        return 0
    try:
        verify_pinned()
    except CheckerMismatch as err:
        print(err)
        return 1
    print(f"checker matches the pin {checker_hash()}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
