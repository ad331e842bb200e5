"""The agent's GEMV templates on the GPU against their CPU models, bit for bit (the reference's
tests/gpu/test_template_cuda.py cases: every row-major, INT8 and column-major config on random
shapes, the scalar path on misaligned inputs, bad knobs rejected, repeated column calls), plus
the INT8 copy made on the GPU against the CPU model, and launches larger than one workgroup
per row tile, where the column template's ticket merge has many workgroups to order."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle.template import emulate, emulate_column, quantize_rows
from pck.agent.column import ColumnConfig, column_space
from pck.agent.config import KernelConfig, int8_space, row_space
from pck.cuda import column_tiles, gemv_column, gemv_template, row_q8
from pck.fp import bf16

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def to_gpu(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).cuda()


@settings(max_examples=300, deadline=None)
@given(
    st.sampled_from(row_space()),
    st.integers(1, 40),
    st.integers(1, 3000),
    st.integers(0, 2**32 - 1),
)
def test_row_template_matches_its_model(cfg: KernelConfig, m: int, n: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n) * 2.0 ** rng.integers(-8, 9, n))
    got = gemv_template(to_gpu(W), to_gpu(x), cfg).cpu().numpy()
    np.testing.assert_array_equal(got, emulate(cfg, W, x))


@settings(max_examples=200, deadline=None)
@given(
    st.sampled_from(int8_space()),
    st.integers(1, 40),
    st.integers(1, 3000),
    st.integers(0, 2**32 - 1),
)
def test_int8_template_matches_its_model(cfg: KernelConfig, m: int, n: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n) * 2.0 ** rng.integers(-8, 9, n))
    # the BF16 weights passed beside the copy are not read
    got = gemv_template(torch.zeros(1, device="cuda"), to_gpu(x), cfg, row_q8(W))
    np.testing.assert_array_equal(got.cpu().numpy(), emulate(cfg, W, x))


@pytest.mark.parametrize("seed", range(4))
def test_int8_copy_matches_the_cpu_model(seed: int) -> None:
    rng = np.random.default_rng(seed)
    m, n = 37, 128 * 5 + 77
    W = (rng.standard_normal((m, n)) * 10.0 ** rng.integers(-3, 3, (m, 1))).astype(np.float32)
    W[3, :128] = 0  # an all-zero group
    W[4, 128:256] = 0.5  # a flat group: every value 127
    W[5, :4] = [127.0, 2.5, -3.5, 0.5]  # ties to even at scale 1
    W[5, 4:128] = 0
    want_q, want_s = quantize_rows(W)
    for source in (W, torch.from_numpy(W)):  # FP32 input from NumPy and from torch
        Wq, S = row_q8(source)
        np.testing.assert_array_equal(Wq.cpu().numpy(), want_q)
        np.testing.assert_array_equal(S.cpu().numpy(), want_s)
    Wb = bf16(W)  # a BF16 tensor is read as BF16
    Wq, S = row_q8(to_gpu(Wb))
    want_q, want_s = quantize_rows(Wb)
    np.testing.assert_array_equal(Wq.cpu().numpy(), want_q)
    np.testing.assert_array_equal(S.cpu().numpy(), want_s)


@pytest.mark.parametrize(
    "cfg",
    [KernelConfig(threads=t, vec=v, unroll=u) for t in (64, 512) for v in (1, 2, 4, 8) for u in (1, 4)]
    + [KernelConfig(threads=t, vec=v, unroll=u, weights="int8") for t in (64, 512)
       for v in (1, 2, 4, 8, 16) for u in (1, 4)],
)
def test_vector_path_for_every_width(cfg: KernelConfig) -> None:
    """n a multiple of 128 and aligned tensors: every vec takes its wide loads (random shapes
    rarely give n % 16 == 0, so they mostly exercise the element path)."""
    rng = np.random.default_rng(cfg.vec * 10 + cfg.unroll)
    W = bf16(rng.standard_normal((33, 1280)) * 0.02)
    x = bf16(rng.standard_normal(1280))
    q8 = row_q8(W) if cfg.weights == "int8" else None
    got = gemv_template(to_gpu(W), to_gpu(x), cfg, q8).cpu().numpy()
    np.testing.assert_array_equal(got, emulate(cfg, W, x))


def test_int8_template_needs_a_matching_int8_copy() -> None:
    rng = np.random.default_rng(2)
    W = bf16(rng.standard_normal((16, 300)) * 0.02)
    x = to_gpu(bf16(rng.standard_normal(300)))
    cfg = KernelConfig(weights="int8")
    with pytest.raises(ValueError, match="INT8 copy"):
        gemv_template(to_gpu(W), x, cfg)
    Wq, S = row_q8(W)
    with pytest.raises(RuntimeError, match="shape"):
        gemv_template(to_gpu(W), x, cfg, (Wq, S[:, :1].contiguous()))
    with pytest.raises(RuntimeError, match="int8"):
        gemv_template(to_gpu(W), x, cfg, (Wq.float(), S))


@pytest.mark.parametrize(
    "cfg",
    [KernelConfig(vec=v, unroll=u) for v in (1, 2, 4, 8) for u in (1, 2, 4)]
    + [KernelConfig(vec=v, weights="int8") for v in (4, 16)]
    + [KernelConfig(vec=8, acc="bf16", skip_tail=True, threads=64)],
)
def test_misaligned_x_takes_the_element_path(cfg: KernelConfig) -> None:
    rng = np.random.default_rng(0)
    W = bf16(rng.standard_normal((8, 1025)) * 0.02)
    x = bf16(rng.standard_normal(1025))
    xc = to_gpu(np.concatenate([[0.0], x]))[1:]  # 2-byte aligned only
    q8 = row_q8(W) if cfg.weights == "int8" else None
    got = gemv_template(to_gpu(W), xc, cfg, q8).cpu().numpy()
    np.testing.assert_array_equal(got, emulate(cfg, W, x))


def test_llama_shapes_on_the_default_and_exploit_knobs() -> None:
    """4096 x 4096 and 1024 x 14336 (many workgroups, long chains)."""
    rng = np.random.default_rng(7)
    for m, n in ((4096, 4096), (1024, 14336)):
        W = bf16(rng.standard_normal((m, n)) * 0.02)
        x = bf16(rng.standard_normal(n))
        Wg, xg = to_gpu(W), to_gpu(x)
        for cfg in (KernelConfig(), KernelConfig(threads=512, rows_per_block=2, vec=4, unroll=4),
                    KernelConfig(acc="bf16", partials="bf16", out="bf16")):
            np.testing.assert_array_equal(gemv_template(Wg, xg, cfg).cpu().numpy(), emulate(cfg, W, x))
        cfg = KernelConfig(vec=16, unroll=2, weights="int8")
        got = gemv_template(Wg, xg, cfg, row_q8(Wg)).cpu().numpy()
        np.testing.assert_array_equal(got, emulate(cfg, W, x))


def test_bad_rows_per_block_and_threads_are_rejected() -> None:
    from pck.cuda.template import _template

    W = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="launch failed"):
        _template(W, x, 64, 4, 8, 1, 0)  # 16 lanes per row
    with pytest.raises(RuntimeError, match="rows_per_block must divide threads"):
        _template(W, x, 64, 3, 8, 1, 0)
    with pytest.raises(RuntimeError, match="launch failed"):
        _template(W, x, 64, 1, 3, 1, 0)  # vec 3
    with pytest.raises(RuntimeError, match="threads"):
        _template(W, x, 48, 1, 8, 1, 0)


@settings(max_examples=300, deadline=None)
@given(
    st.sampled_from(column_space()),
    st.integers(1, 80),
    st.integers(1, 3000),
    st.integers(0, 2**32 - 1),
)
def test_column_template_matches_its_model(cfg: ColumnConfig, rows: int, n: int, seed: int) -> None:
    m = rows * cfg.vec  # the kernel needs m % vec == 0
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n) * 2.0 ** rng.integers(-8, 3, n))
    got = gemv_column(to_gpu(W.T), to_gpu(x), cfg).cpu().numpy()
    np.testing.assert_array_equal(got, emulate_column(cfg, W, x))


def test_column_template_rejects_rows_not_divisible_by_vec() -> None:
    WT = torch.zeros(16, 12, dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(16, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="launch failed"):
        gemv_column(WT, x, ColumnConfig(vec=8))


def test_column_template_merges_identically_on_repeated_calls() -> None:
    """4096 x 14336 with 64 grid splits (16 row tiles of 64 workgroups each) and with 2: the
    second launch merges the splits in a fixed order, call after call."""
    rng = np.random.default_rng(1)
    W = bf16(rng.standard_normal((4096, 14336)) * 0.02)
    x = bf16(rng.standard_normal(14336))
    WT, xg = to_gpu(W.T), to_gpu(x)
    for cfg in (ColumnConfig(threads=256, vec=4, splits=64), ColumnConfig(threads=32, vec=8, splits=2)):
        first = gemv_column(WT, xg, cfg)
        for _ in range(5):
            assert torch.equal(gemv_column(WT, xg, cfg), first)
        np.testing.assert_array_equal(first.cpu().numpy(), emulate_column(cfg, W, x))
    assert column_tiles(4096, 4) == 32


def test_column_calls_on_two_streams_overlap_safely() -> None:
    """Each call has its own scratch, so launches on two streams at once give the same bits."""
    rng = np.random.default_rng(9)
    W = bf16(rng.standard_normal((2048, 4096)) * 0.02)
    xs = [bf16(rng.standard_normal(4096)) for _ in range(2)]
    WT = to_gpu(W.T)
    cfg = ColumnConfig(threads=128, vec=8, splits=32)
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = []
    torch.cuda.synchronize()
    for stream, x in zip(streams, xs):
        with torch.cuda.stream(stream):
            outs.append([gemv_column(WT, to_gpu(x), cfg) for _ in range(4)])
    torch.cuda.synchronize()
    for got, x in zip(outs, xs):
        want = emulate_column(cfg, W, x)
        for y in got:
            np.testing.assert_array_equal(y.cpu().numpy(), want)


def test_column_skip_reads_fewer_columns_and_matches_the_model() -> None:
    rng = np.random.default_rng(6)
    W = bf16(rng.standard_normal((512, 4096)) * 0.02)
    x = bf16(rng.standard_normal(4096) * 0.05)  # many activations below 0.05
    cfg = ColumnConfig(threads=128, vec=8, splits=8, skip_below=0.05)
    got = gemv_column(to_gpu(W.T), to_gpu(x), cfg).cpu().numpy()
    np.testing.assert_array_equal(got, emulate_column(cfg, W, x))
    assert not np.array_equal(got, emulate_column(ColumnConfig(threads=128, vec=8, splits=8), W, x))


def test_native_entries_take_the_pybind_arguments() -> None:
    """The template launches with the reference's pybind argument lists (bindings.cpp)."""
    from pck.cuda.template import _column, _template, _template_q8

    rng = np.random.default_rng(8)
    W = bf16(rng.standard_normal((64, 700)) * 0.02)
    x = bf16(rng.standard_normal(700))
    Wg, xg = to_gpu(W), to_gpu(x)
    cfg = KernelConfig(threads=128, rows_per_block=2, vec=4, unroll=2, out="bf16")
    np.testing.assert_array_equal(_template(Wg, xg, 128, 2, 4, 2, 4).cpu().numpy(), emulate(cfg, W, x))
    Wq, S = row_q8(W)
    q = KernelConfig(threads=64, vec=2, weights="int8")
    np.testing.assert_array_equal(_template_q8(Wq, S, xg, 64, 1, 2, 1).cpu().numpy(), emulate(q, W, x))
    tickets = torch.zeros(4, dtype=torch.int32, device="cuda")
    c = ColumnConfig(threads=64, vec=2, splits=4)
    got = _column(to_gpu(W.T), xg, tickets, 64, 2, 4, 0.0).cpu().numpy()
    np.testing.assert_array_equal(got, emulate_column(c, W, x))
    assert not tickets.any()
    with pytest.raises(RuntimeError, match="tickets"):
        _column(to_gpu(W.T), xg, torch.zeros(0, dtype=torch.int32, device="cuda"), 64, 2, 4, 0.0)


@pytest.mark.parametrize(
    "cfg",
    [
        KernelConfig(),
        KernelConfig(threads=128, rows_per_block=2, vec=4, unroll=4),
        ColumnConfig(),
        KernelConfig(acc="bf16"),
        KernelConfig(partials="bf16"),
        KernelConfig(out="bf16"),
        KernelConfig(threads=64, skip_tail=True),
        KernelConfig(vec=16, weights="int8"),
        ColumnConfig(skip_below=0.3),
    ],
    ids=str,
)
def test_the_trusted_checker_judges_template_outputs_like_the_cpu_checker(cfg) -> None:  # type: ignore[no-untyped-def]
    """What the templates exist for: their GPU outputs go to the trusted GPU checker at the
    config's own tree height, and its verdicts equal the CPU checker's on the same signs.
    Honest configs pass every block; each exploit is rejected."""
    from oracle.checker import BlockedChecker
    from pck.agent.config import is_exploit
    from pck.cuda import GpuBlockedChecker

    m, n = 512, 2000  # n is not a multiple of a 64-lane x 8-column tile: skip_tail drops 464
    rng = np.random.default_rng(11)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    Wg, xg = to_gpu(W), to_gpu(x)
    if isinstance(cfg, ColumnConfig):
        y = gemv_column(to_gpu(W.T), xg, cfg)
    else:
        y = gemv_template(Wg, xg, cfg, row_q8(W) if cfg.weights == "int8" else None)
    np.testing.assert_array_equal(y.cpu().numpy(), emulate(cfg, W, x))
    height = cfg.tree_height(n)
    checker = GpuBlockedChecker(Wg, 64, height, checks=8, generator=torch.Generator().manual_seed(4))
    gpu = checker.verdict(xg, y).cpu().numpy()
    cpu = BlockedChecker(W, x, 64, height).verdict_with_signs(
        y.cpu().numpy(), checker.r.cpu().numpy().astype(np.float64)
    )[0].all(0)
    np.testing.assert_array_equal(gpu, cpu)
    if is_exploit(cfg):
        assert not gpu.all()
    else:
        assert gpu.all()
