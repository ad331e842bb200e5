"""The trusted-checker pin (`pck.manifest`): the lock matches the tree, every kind of change is
caught and named (a file's bytes, a compiler flag, the target, an added or dropped file, an old
lock format), certificates round-trip and go stale when the checker moves, and the commit is
read from a checkout's .git in each of its forms."""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from pck import _build, manifest
from pck.manifest import CheckerMismatch, Manifest


@pytest.fixture
def lock_copy(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> Path:
    """A private lock of the current state, installed as the module's LOCK."""
    path = tmp_path / "lock.json"
    monkeypatch.setattr(manifest, "LOCK", path)
    manifest.write_lock(path)
    return path


def test_the_committed_lock_pins_the_tree() -> None:
    """Fails after any edit to a trusted file or flag: review it, then re-pin
    (python -m pck.manifest --update)."""
    manifest.verify_pinned()
    lock = manifest.pinned()
    assert set(lock["files"]) == set(manifest.TRUSTED)
    assert lock["build"]["arch"] == "gfx950"
    assert "-ffp-contract=off" in lock["build"]["flags"]


def test_every_trusted_path_is_a_file() -> None:
    for name in manifest.TRUSTED:
        assert (manifest.PACKAGE_ROOT / name).is_file(), name


def test_one_changed_byte_is_named(lock_copy: Path, tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(manifest, "PACKAGE_ROOT", tmp_path / "pkg")
    (tmp_path / "pkg").mkdir()
    for name in manifest.TRUSTED:  # mirror the trusted files, then alter one byte of one
        dst = (tmp_path / "pkg" / name).resolve()
        dst.parent.mkdir(parents=True, exist_ok=True)
        dst.write_bytes((Path(_build.ROOT) / name).resolve().read_bytes())
    manifest.write_lock(lock_copy)
    manifest.verify_pinned()
    target = (tmp_path / "pkg" / "csrc/rounding.h")
    data = bytearray(target.read_bytes())
    data[-2] ^= 1
    target.write_bytes(bytes(data))
    with pytest.raises(CheckerMismatch, match=r"\(csrc/rounding\.h\)"):
        manifest.verify_pinned()


def test_a_flag_change_is_named(lock_copy: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    flags = [f for f in _build.HIPCC_FLAGS if f != "-ffp-contract=off"] + ["-ffp-contract=fast"]
    monkeypatch.setattr(_build, "HIPCC_FLAGS", flags)
    with pytest.raises(CheckerMismatch, match="build flags"):
        manifest.verify_pinned()


def test_a_target_change_is_named(lock_copy: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(_build, "ARCH", "gfx942")
    with pytest.raises(CheckerMismatch, match="build arch"):
        manifest.verify_pinned()


def test_added_and_dropped_files_are_named(lock_copy: Path) -> None:
    lock = json.loads(lock_copy.read_text())
    lock["files"]["csrc/extra.hip"] = "0" * 64
    del lock["files"]["csrc/bcheck.hip"]
    lock_copy.write_text(json.dumps(lock))
    with pytest.raises(CheckerMismatch, match=r"csrc/bcheck\.hip, csrc/extra\.hip"):
        manifest.verify_pinned()


def test_an_old_lock_format_is_refused(lock_copy: Path) -> None:
    lock = json.loads(lock_copy.read_text())
    lock["format"] = 1
    lock_copy.write_text(json.dumps(lock))
    with pytest.raises(CheckerMismatch, match="lock format"):
        manifest.verify_pinned()


def test_digest_is_canonical() -> None:
    state = manifest.current_state()
    shuffled = {"build": dict(reversed(list(state["build"].items()))),
                "files": dict(reversed(list(state["files"].items())))}  # fmt: skip
    assert manifest.digest_state(shuffled) == manifest.digest_state(state) == manifest.checker_hash()


def test_certificates_round_trip_and_go_stale(lock_copy: Path) -> None:
    cert = Manifest("4096x4096-gauss", {"layout": "row"}, None, {"h_spec": 23}, 1.25)
    assert Manifest.from_json(cert.to_json()) == cert
    assert cert.problems() == [] and cert.lean is None
    assert cert.theorems["T3 safe runtime threshold"] == "PCK.t3_no_false_alarm"
    other = Manifest("t", {}, "slot", {}, 1.0, checker="f" * 64)
    assert other.problems() == ["checker hash differs from the pinned checker"]


def test_lean_sources_enter_the_certificate(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(manifest, "ROOT", tmp_path)
    assert manifest.lean_hash() is None
    (tmp_path / "lean/PCK").mkdir(parents=True)
    (tmp_path / "lean/PCK/T3.lean").write_text("theorem t3 : True := trivial\n")
    (tmp_path / "lean/lakefile.toml").write_text("name = 'PCK'\n")
    first = manifest.lean_hash()
    (tmp_path / "lean/PCK/T3.lean").write_text("theorem t3 : 1 = 1 := rfl\n")
    assert first is not None and manifest.lean_hash() not in (None, first)


def test_commit_from_each_form_of_git_head(tmp_path: Path) -> None:
    sha = "0123456789abcdef0123456789abcdef01234567"
    git = tmp_path / ".git"
    assert manifest.git_commit(tmp_path) is None
    git.mkdir()
    (git / "HEAD").write_text(sha + "\n")  # detached
    assert manifest.git_commit(tmp_path) == sha
    (git / "HEAD").write_text("ref: refs/heads/main\n")
    (git / "packed-refs").write_text(f"# pack-refs with: peeled\n{sha} refs/heads/main\n")
    assert manifest.git_commit(tmp_path) == sha
    (git / "refs/heads").mkdir(parents=True)
    (git / "refs/heads/main").write_text("f" * 40 + "\n")  # a loose ref wins
    assert manifest.git_commit(tmp_path) == "f" * 40
    assert manifest.git_commit() is not None  # this checkout


def test_cli(lock_copy: Path, capsys: pytest.CaptureFixture[str]) -> None:
    assert manifest.main([]) == 0 and "matches the pin" in capsys.readouterr().out
    lock = json.loads(lock_copy.read_text())
    lock["checker"] = "0" * 64
    lock_copy.write_text(json.dumps(lock))
    assert manifest.main([]) == 1
    assert manifest.main(["--update"]) == 0
    manifest.verify_pinned()
