"""The C ABI of libpck_hip.so, checked without a GPU: the library loads, exports every function
the headers under include/ declare (include/pck_probe.h: libpck_probe.so, the probes of device
arithmetic), and the ctypes mirrors of its structs have the header's layout (gcc compiles the
header and prints sizeof / offsetof)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from pck.cuda import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "pck_hip.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


PROBE_HEADER = ROOT / "include" / "pck_probe.h"


def declared_functions(headers: list[Path] | None = None) -> list[str]:
    """Every pck_* function that the headers (default: those of libpck_hip.so) declare."""
    names: set[str] = set()
    for header in headers if headers is not None else [h for h in HEADERS if h != PROBE_HEADER]:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(pck_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_the_entry_points() -> None:
    names = declared_functions()
    for expected in (
        "pck_gemv_bf16_naive",
        "pck_gemv_bf16_coalesced",
        "pck_gemv_fp8_coalesced",
        "pck_gemv_group",
        "pck_blocked_check",
        "pck_check_members",
        "pck_sampling_check",
        "pck_sampling_scratch_words",
        "pck_error_string",
        "pck_gemv_template",
        "pck_gemv_template_q8",
        "pck_gemv_column",
        "pck_column_tiles",
        "pck_quantize_rows_q8",
    ):
        assert expected in names


def test_library_exports_every_declared_function() -> None:
    handle = _lib.lib()
    for name in declared_functions():
        assert hasattr(handle, name), name
    assert set(declared_functions()) >= set(_lib.SIGNATURES) | set(_lib.SIZE_QUERIES)
    from pck.cuda import template

    assert set(declared_functions()) >= set(template.SIGNATURES) | {"pck_column_tiles"}


def test_probe_library_exports_its_header() -> None:
    from pck.cuda import probe

    names = declared_functions([PROBE_HEADER])
    assert set(names) == set(probe.SIGNATURES)
    handle = probe.lib()
    for name in names:
        assert hasattr(handle, name), name
    subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-Wall", "-Werror", "-x", "c",
                    str(PROBE_HEADER)], check=True)  # fmt: skip


def test_template_header_compiles_as_c_and_argument_counts_match(tmp_path: Path) -> None:
    """The template header is plain C, and each ctypes signature has the prototype's arity."""
    from pck.cuda import template

    src = tmp_path / "t.c"
    src.write_text('#include "pck_template.h"\nint main(void) { return 0; }\n')
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{HEADER.parent}", str(src), "-o",
                    str(tmp_path / "t")], check=True)
    text = re.sub(r"/\*.*?\*/", "", (HEADER.parent / "pck_template.h").read_text(), flags=re.S)
    for name, argtypes in template.SIGNATURES.items():
        params = re.search(name + r"\s*\(([^)]*)\)", text, flags=re.S)
        assert params is not None, name
        assert len(params.group(1).split(",")) == len(argtypes), name


def test_column_tiles_without_a_gpu() -> None:
    from pck.cuda.template import column_tiles

    assert column_tiles(0, 8) == 0 and column_tiles(1, 8) == 1 and column_tiles(256, 8) == 1
    assert column_tiles(257 * 2, 2) == 9 and column_tiles(64, 3) == -1


def test_error_strings() -> None:
    assert _lib.lib().pck_error_string(0) == b"no error"
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(1, "probe")


LAYOUT_PROGRAM = r"""
#include <stddef.h>
#include <stdio.h>
#include "pck_hip.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("PckGemv %zu\nPckCheckDesc %zu\nPckCheckBatch %zu\nPckBatchCheckDesc %zu\n",
         sizeof(PckGemv), sizeof(PckCheckDesc), sizeof(PckCheckBatch), sizeof(PckBatchCheckDesc));
  F(PckGemv, W) F(PckGemv, m) F(PckGemv, n)
  F(PckCheckDesc, tau) F(PckCheckDesc, n) F(PckCheckDesc, seg_len) F(PckCheckDesc, block)
  F(PckCheckDesc, segments) F(PckCheckDesc, coef) F(PckCheckDesc, tau_floor)
  F(PckCheckBatch, start) F(PckCheckBatch, count)
  F(PckBatchCheckDesc, X) F(PckBatchCheckDesc, n) F(PckBatchCheckDesc, batch) F(PckBatchCheckDesc, tau_floor)
  return 0;
}
"""


def test_struct_layouts_match_the_header(tmp_path: Path) -> None:
    src = tmp_path / "layout.c"
    src.write_text(LAYOUT_PROGRAM)
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.rsplit(" ", 1) for line in lines if line)
    structs = {"PckGemv": _lib.PckGemv, "PckCheckDesc": _lib.PckCheckDesc, "PckCheckBatch": _lib.PckCheckBatch,
               "PckBatchCheckDesc": _lib.PckBatchCheckDesc}
    for key, value in got.items():
        if "." in key:
            struct, field = key.split(".")
            assert getattr(structs[struct], field).offset == int(value), key
        else:
            assert ctypes.sizeof(structs[key]) == int(value), key


def _check_descs(shapes: list[tuple[int, int, int, int, int]], x_offset: int = 0) -> ctypes.Array:
    """Descriptors (n, block, num_blocks, checks, batch) with placeholder device addresses: the
    plan only validates and sizes them, it never dereferences a pointer."""
    descs = (_lib.PckBatchCheckDesc * len(shapes))()
    for i, (n, block, nb, checks, batch) in enumerate(shapes):
        d = descs[i]
        base = 0x10000000 * (i + 1)
        d.c, d.a, d.r = base, base + 0x1000000, base + 0x2000000
        d.X, d.Y = base + 0x3000000 + x_offset, base + 0x4000000
        d.passed, d.rho, d.tau = base + 0x5000000, base + 0x6000000, base + 0x7000000
        d.n, d.block, d.num_blocks, d.checks, d.batch = n, block, nb, checks, batch
        d.coef, d.geps, d.tau_floor = 1.0, 1e-7, 0.0
    return descs


def _workspace(descs: ctypes.Array) -> tuple[int, int]:
    need = ctypes.c_int64(-1)
    err = _lib.lib().pck_batch_check_workspace(descs, len(descs), ctypes.byref(need))
    return err, need.value


def test_batch_check_plan_sizes_the_llama_layer() -> None:
    """The Llama-3-8B layer at B = 256, b = 128, K = 1: the shortest segment (a multiple of 256
    columns) that keeps the partial grid within 256 workgroups is 2048 columns, 2 for n = 4096
    and 7 for n = 14336 (10 x 8 x 2 + 1 x 8 x 7 = 216 workgroups; 1792 would give 304), so the
    partials hold 256 x (48 x 2 + 32 x 2 + 224 x 2 + 32 x 7) FP64 pairs: 3,407,872 bytes."""
    layer = [(4096, 128, 48, 1, 256), (4096, 128, 32, 1, 256), (4096, 128, 224, 1, 256),
             (14336, 128, 32, 1, 256)]  # fmt: skip
    assert _workspace(_check_descs(layer)) == (0, 3_407_872)


def test_batch_check_plan_rejects_what_32_bit_offsets_cannot_address() -> None:
    # one finish workgroup reads 64 columns of nb * b rows: below 2^31 bytes passes
    assert _workspace(_check_descs([(8, 128, 65535, 1, 16)]))[0] == 0
    assert _workspace(_check_descs([(8, 128, 65536, 1, 16)]))[0] != 0
    # each partial array (pairs x batch x segments FP64 values) stays below 2^31 bytes
    assert _workspace(_check_descs([(8, 4, 1 << 14, 1, (1 << 14) - 64)]))[0] == 0
    assert _workspace(_check_descs([(8, 4, 1 << 14, 1, 1 << 14)]))[0] != 0
    # X must be 16-byte aligned
    assert _workspace(_check_descs([(4096, 128, 32, 1, 128)], x_offset=8))[0] != 0
