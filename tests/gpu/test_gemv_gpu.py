"""HIP GEMVs against the oracle, bit for bit (the reference's tests/gpu/test_gemv_cuda.py and
tests/gpu/test_gemv_fp8.py cases, plus the Llama-3-8B decode shapes, every thread count, every
launch shape of the coalesced kernel, and grouped launches)."""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st
from numpy.typing import NDArray

from oracle.checker import BlockedChecker
from oracle.cmodel import gemv_coalesced_c, gemv_naive_c
from oracle.gemv import e4m3_values, emulate_gemv, emulate_gemv_coalesced, reference_gemv
from pck.cuda import gemv_coalesced, gemv_fp8, gemv_group, gemv_naive, quantize_fp8
from pck.cuda._lib import lib
from pck.fp import bf16, gamma, tree_height
from tests.strategies import Problem, gemv_problems

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

Array = NDArray[np.float32]


@dataclass(frozen=True)
class Kernel:
    name: str
    run: Callable[[torch.Tensor, torch.Tensor, int], torch.Tensor]
    model: Callable[[Array, Array, int], Array]
    vec: int


KERNELS = [
    Kernel("naive", gemv_naive, emulate_gemv, vec=1),
    Kernel("coalesced", gemv_coalesced, emulate_gemv_coalesced, vec=8),
]
kernels = pytest.mark.parametrize("kernel", KERNELS, ids=lambda k: k.name)


def to_gpu(a: Array) -> torch.Tensor:
    """BF16-valued FP32 array -> BF16 GPU tensor (exact)."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).cuda()


def run(kernel: Kernel, W: Array, x: Array, threads: int) -> Array:
    y = kernel.run(to_gpu(W), to_gpu(x), threads)
    assert y.dtype == torch.float32
    return y.cpu().numpy()


def assert_bits(got: Array, want: Array) -> None:
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def random_problem(m: int, n: int, seed: int) -> tuple[Array, Array]:
    rng = np.random.default_rng(seed)
    return bf16(rng.standard_normal((m, n)) * 0.02), bf16(rng.standard_normal(n))


SHAPES = [
    (1, 1, 32),
    (3, 5, 64),
    (7, 100, 32),
    (64, 1000, 32),
    (5, 17, 1024),
    (33, 4096, 128),
    (256, 4096, 256),
    (256, 4100, 256),
    (16, 14336, 512),
]


@kernels
@pytest.mark.parametrize(("m", "n", "threads"), SHAPES)
def test_bit_exact_with_model(kernel: Kernel, m: int, n: int, threads: int) -> None:
    W, x = random_problem(m, n, seed=m * n + threads)
    assert_bits(run(kernel, W, x, threads), kernel.model(W, x, threads))


@pytest.mark.parametrize("threads", [1, 2, 4, 8, 16])
def test_naive_small_thread_counts(threads: int) -> None:
    W, x = random_problem(9, 77, seed=threads)
    assert_bits(run(KERNELS[0], W, x, threads), emulate_gemv(W, x, threads))


# (m, n, threads): chunks of whole 16-byte vectors (every level inside one wave, across 2, 4,
# 8 and 16 waves) and chunks that are not (element loads), with n ragged or not.
NAIVE_PATHS = [(6, 256, 8), (6, 2048, 32), (5, 512, 64), (4, 1024, 128), (3, 8192, 1024),
               (7, 8200, 1024), (9, 4104, 64), (4, 4096, 512), (2, 65, 64)]  # fmt: skip


@pytest.mark.parametrize(("m", "n", "threads"), NAIVE_PATHS)
def test_naive_vector_and_element_paths(m: int, n: int, threads: int) -> None:
    W, x = random_problem(m, n, seed=n + threads)
    assert_bits(run(KERNELS[0], W, x, threads), emulate_gemv(W, x, threads))


@pytest.mark.parametrize(("m", "n"), [(1024, 4096), (4096, 14336)])
def test_naive_llama_shapes_bit_exact(m: int, n: int) -> None:
    """The naive tree at T = 256 on decode shapes (chunks of 16 and 56 columns) against the
    C model of the same order."""
    g = torch.Generator().manual_seed(1)
    W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(n, generator=g).to(torch.bfloat16)
    y = gemv_naive(W.cuda(), x.cuda(), 256).cpu().numpy()
    assert_bits(y, gemv_naive_c(W.float().numpy(), x.float().numpy(), 256))


@kernels
@settings(max_examples=30, deadline=None)
@given(gemv_problems(max_rows=32, max_cols=600), st.sampled_from([32, 64, 128, 256]))
def test_bit_exact_with_model_random(kernel: Kernel, p: Problem, threads: int) -> None:
    assert_bits(run(kernel, p.W, p.x, threads), kernel.model(p.W, p.x, threads))


LLAMA = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize(("m", "n"), LLAMA)
def test_llama_shapes_bit_exact(m: int, n: int) -> None:
    """The BASELINE decode shapes with the reference's generator (torch CPU, seed 0)."""
    g = torch.Generator().manual_seed(0)
    W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(n, generator=g).to(torch.bfloat16)
    y = gemv_coalesced(W.cuda(), x.cuda(), 256).cpu().numpy()
    want = gemv_coalesced_c(W.float().numpy(), x.float().numpy(), 256)
    assert_bits(y, want)
    err = np.abs(y.astype(np.float64) - reference_gemv(W.float().numpy(), x.float().numpy()))
    bound = gamma(tree_height(n, 256, 8)) * (np.abs(W.float().numpy()).astype(np.float64) @ np.abs(x.float().numpy()))
    assert np.all(err <= bound)


SHAPE_KNOBS = [(0, 0, 0)] + [(r, u, nt) for r in (1, 2, 4) for u in (1, 2, 4) for nt in (0, 1)]
# Thread counts other than 256 have a single launch shape, the built-in one.
LAUNCHES = [(256, shape) for shape in SHAPE_KNOBS] + [(t, (0, 0, 0)) for t in (32, 64, 128, 512, 1024)]


@pytest.mark.parametrize(("threads", "shape"), LAUNCHES, ids=str)
def test_every_launch_shape_gives_the_same_bits(threads: int, shape: tuple[int, int, int]) -> None:
    """rows per wave, loads ahead and non-temporal loads change only speed ((0, 0, 0) = the
    built-in choice)."""
    W, x = random_problem(77, 3000 + threads, seed=threads)
    want = gemv_coalesced_c(W, x, threads)
    try:
        assert lib().pck_gemv_set_shape(*shape) == 0
        assert_bits(run(KERNELS[1], W, x, threads), want)
        W2, x2 = random_problem(40, 4096, seed=threads + 1)  # no padding vectors at T <= 512
        assert_bits(run(KERNELS[1], W2, x2, threads), gemv_coalesced_c(W2, x2, threads))
    finally:
        lib().pck_gemv_set_shape(0, 0, 0)


def test_group_launch_equals_single_launches() -> None:
    pairs_np = [random_problem(m, n, seed=i) for i, (m, n) in enumerate([(4096, 4096), (1024, 4096), (1024, 4096), (33, 100)])]
    pairs = [(to_gpu(W), to_gpu(x)) for W, x in pairs_np]
    outs = gemv_group(pairs, 256)
    for (W, x), y in zip(pairs, outs):
        assert torch.equal(y.view(torch.int32), gemv_coalesced(W, x, 256).view(torch.int32))


def test_group_launch_fp8() -> None:
    g = torch.Generator().manual_seed(3)
    Ws = [(torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda() for m, n in [(512, 4096), (64, 14336)]]
    xs = [torch.randn(W.shape[1], generator=g).to(torch.bfloat16).cuda() for W in Ws]
    Qs = [quantize_fp8(W)[0] for W in Ws]
    outs = gemv_group(list(zip(Qs, xs)), 256)
    for Q, x, z in zip(Qs, xs, outs):
        assert torch.equal(z.view(torch.int32), gemv_fp8(Q, x, 256).view(torch.int32))


def test_coalesced_unaligned_pointer_uses_element_loads() -> None:
    m, n, threads = 8, 4096, 128
    W, x = random_problem(m, n, seed=3)
    flat = torch.zeros(m * n + 1, dtype=torch.bfloat16, device="cuda")
    flat[1:] = to_gpu(W).flatten()
    W_view = flat[1:].view(m, n)
    assert W_view.is_contiguous() and W_view.data_ptr() % 16 != 0
    y = gemv_coalesced(W_view, to_gpu(x), threads).cpu().numpy()
    assert_bits(y, emulate_gemv_coalesced(W, x, threads))


@kernels
def test_signed_zero_matches_model(kernel: Kernel) -> None:
    W = np.zeros((2, 64), dtype=np.float32)
    x = -np.ones(64, dtype=np.float32)
    for threads in (32, 64):
        assert_bits(run(kernel, W, x, threads), kernel.model(W, x, threads))
    W = np.zeros((3, 4096), dtype=np.float32)  # no padding: the sum of -0 products stays -0
    x = -np.ones(4096, dtype=np.float32)
    assert_bits(run(KERNELS[1], W, x, 256), emulate_gemv_coalesced(W, x, 256))


@kernels
def test_checker_passes_gpu_output(kernel: Kernel) -> None:
    m, n, threads = 512, 4100, 256
    W, x = random_problem(m, n, seed=7)
    checker = BlockedChecker(W, x, 64, tree_height(n, threads, kernel.vec))
    assert checker.verdict(run(kernel, W, x, threads), np.random.default_rng(0), checks=8).all()


@kernels
def test_empty_output(kernel: Kernel) -> None:
    W = torch.zeros((0, 8), dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(8, dtype=torch.bfloat16, device="cuda")
    assert kernel.run(W, x, 32).shape == (0,)


@kernels
@pytest.mark.parametrize(
    ("make", "match"),
    [
        (lambda W, x: (W.float(), x.float(), 32), "bfloat16"),
        (lambda W, x: (W.t(), x[:4], 32), "contiguous"),
        (lambda W, x: (W, x[:3], 32), "shape"),
        (lambda W, x: (W, x, 48), "power of two"),
        (lambda W, x: (W, x, 2048), "power of two"),
        (lambda W, x: (W.cpu(), x.cpu(), 32), "CUDA tensors"),
    ],
)
def test_rejects_bad_inputs(kernel: Kernel, make: Callable[..., Any], match: str) -> None:
    W = torch.ones((4, 8), dtype=torch.bfloat16, device="cuda")
    x = torch.ones(8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match=match):
        kernel.run(*make(W, x))


def test_coalesced_rejects_fewer_than_a_warp() -> None:
    W = torch.ones((4, 8), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match=r"\[32, 1024\]"):
        gemv_coalesced(W, torch.ones(8, dtype=torch.bfloat16, device="cuda"), 16)


# ---- FP8 (E4M3FN) ----------------------------------------------------------------------------

VEC = 16


def fp8_problem(m: int, n: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(m, n, generator=g) * 0.02).bfloat16().cuda()
    x = torch.randn(n, generator=g).bfloat16().cuda()
    return W, x


def fp8_model(Q: torch.Tensor, x: torch.Tensor, threads: int) -> Array:
    """The oracle's own E4M3 decode (not torch's cast) feeds the model."""
    codes = Q.view(torch.uint8).cpu().numpy()
    return emulate_gemv_coalesced(e4m3_values()[codes], x.float().cpu().numpy(), threads, vec=VEC)


def assert_fp8_bits(Q: torch.Tensor, x: torch.Tensor, threads: int) -> None:
    assert_bits(gemv_fp8(Q, x, threads).cpu().numpy(), fp8_model(Q, x, threads))


@pytest.mark.parametrize(
    ("m", "n", "threads"),
    [(1, 1, 32), (3, 5, 64), (7, 100, 32), (5, 17, 1024), (33, 4096, 128), (256, 4100, 256)],
)
def test_fp8_bit_exact_with_model(m: int, n: int, threads: int) -> None:
    W, x = fp8_problem(m, n, seed=m * n + threads)
    assert_fp8_bits(quantize_fp8(W)[0], x, threads)


@pytest.mark.parametrize(("m", "n"), LLAMA)
def test_fp8_llama_shapes_bit_exact(m: int, n: int) -> None:
    W, x = fp8_problem(m, n, seed=1)
    Q = quantize_fp8(W)[0]
    codes = Q.view(torch.uint8).cpu().numpy()
    want = gemv_coalesced_c(e4m3_values()[codes], x.float().cpu().numpy(), 256, VEC)
    assert_bits(gemv_fp8(Q, x, 256).cpu().numpy(), want)


def test_every_fp8_code_decodes_exactly() -> None:
    """Each of the 254 finite E4M3FN codes times x = 1 (one column per row) gives the code's
    value, subnormals included: the hardware decode matches the format's definition."""
    codes = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F], dtype=torch.uint8)
    Q = codes.view(torch.float8_e4m3fn).reshape(-1, 1).cuda()
    x = torch.ones(1, dtype=torch.bfloat16, device="cuda")
    z = gemv_fp8(Q, x, 32).cpu().numpy()
    assert_bits(z, e4m3_values()[codes.numpy()].astype(np.float32) + np.float32(0))


@settings(max_examples=30, deadline=None)
@given(st.integers(1, 32), st.integers(1, 600), st.sampled_from([32, 64, 128, 256]), st.integers(0, 2**31 - 1))
def test_every_fp8_value_bit_exact(m: int, n: int, threads: int, seed: int) -> None:
    """Raw E4M3 bit patterns (every finite value, subnormals included) against wide-range x."""
    g = torch.Generator().manual_seed(seed)
    bits = torch.randint(0, 256, (m, n), generator=g, dtype=torch.uint8)
    bits[(bits & 0x7F) == 0x7F] = 0  # E4M3 NaN
    Q = bits.view(torch.float8_e4m3fn).cuda()
    x = torch.randn(n, generator=g) * 2.0 ** torch.randint(-8, 8, (n,), generator=g)
    assert_fp8_bits(Q, x.bfloat16().cuda(), threads)


def test_fp8_unaligned_pointer_uses_element_loads() -> None:
    m, n, threads = 8, 4096, 128
    W, x = fp8_problem(m, n, seed=3)
    Q = quantize_fp8(W)[0]
    flat = torch.zeros(m * n + 1, dtype=torch.uint8, device="cuda")
    flat[1:] = Q.view(torch.uint8).flatten()
    view = flat[1:].view(torch.float8_e4m3fn).view(m, n)
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    assert torch.equal(gemv_fp8(view, x, threads), gemv_fp8(Q, x, threads))


def test_quantize_fp8_scales_rows() -> None:
    W, _ = fp8_problem(16, 300, seed=1)
    W[3] = 0
    Q, s = quantize_fp8(W)
    assert Q.dtype == torch.float8_e4m3fn and s.shape == (16,)
    assert s[3] == 1 and not Q[3].float().any()
    assert torch.allclose(Q.float().abs().amax(dim=1)[s != 1], torch.tensor(448.0).cuda())
    rel = (s[:, None] * Q.float() - W.float()).norm() / W.float().norm()
    assert rel < 0.05


def nearest_e4m3_codes(v: NDArray[np.float32]) -> NDArray[np.uint8]:
    """Brute force over the 254 finite codes of `oracle.gemv.e4m3_values`: the code nearest to
    each FP32 value (|v| <= 448), ties to the code with an even mantissa, zeros keeping the
    sign of v."""
    table = e4m3_values().astype(np.float64)
    codes = np.array([c for c in range(256) if np.isfinite(table[c])])
    dist = np.abs(v.astype(np.float64)[:, None] - table[codes][None, :])
    best = dist.min(axis=1, keepdims=True)
    tied = dist == best
    even = (codes & 1) == 0
    sign_match = ((codes & 0x80) != 0)[None, :] == np.signbit(v)[:, None]
    score = tied * (4 + 2 * even[None, :] + sign_match)  # nearest first, then even, then sign
    return codes[score.argmax(axis=1)].astype(np.uint8)


def test_quantize_fp8_codes_are_the_nearest_e4m3() -> None:
    """Q's bits against a brute-force nearest-E4M3 (ties to even) of W / s, with
    s = max|w| * fl(1 / 448) and W / s IEEE FP32 operations: row 0 (max 448, so s = 1) holds every finite E4M3 value, every
    midpoint between neighbours (exact ties, including the subnormal range and 0), and the
    BF16 values just beside each midpoint; the other rows are seeded at several scales."""
    table = e4m3_values()
    pos = np.unique(table[np.isfinite(table) & (table >= 0)])
    mids = (pos[:-1] + pos[1:]) / 2  # 4 significant bits: BF16-exact
    beside = np.concatenate([np.nextafter(mids, 0), np.nextafter(mids, 1)])
    special = np.concatenate([pos, mids, bf16(beside), [2.0**-11, 2.0**-10, 3 * 2.0**-11]])
    special = np.concatenate([special, -special])
    n = special.size + (-special.size) % 16
    rng = np.random.default_rng(4)
    rows = [np.concatenate([special, np.zeros(n - special.size)])]
    for scale in (1e-6, 0.02, 1.0, 300.0, 2.0**40, 2.0**-100):
        for _ in range(3):
            rows.append(rng.standard_normal(n) * scale)
    W = bf16(np.stack(rows)).astype(np.float32)
    assert np.abs(W[0]).max() == 448.0
    Q, s = quantize_fp8(torch.from_numpy(W).to(torch.bfloat16).cuda())
    amax = np.abs(W).max(axis=1)
    # torch divides a tensor by a Python scalar as a product with the FP32 reciprocal
    inv = np.float32(1.0) / np.float32(448.0)
    s_ref = np.where(amax > 0, amax * inv, np.float32(1.0)).astype(np.float32)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    v = np.clip(W / s_ref[:, None], -448.0, 448.0).astype(np.float32)
    want = nearest_e4m3_codes(v.ravel()).reshape(v.shape)
    got = Q.view(torch.uint8).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    assert (v[0] != 0).sum() > 1000 and len(np.unique(got[0])) == 254


@pytest.mark.parametrize(("m", "n"), [(4096, 4096), (4096, 14336), (37, 1000)])
def test_fp8_scaled_epilogue(m: int, n: int) -> None:
    """The dequantising launch writes z with exactly gemv_fp8's bits and y = s z with exactly
    the bits of torch's s * z (one FP32 multiply), on the vector path and on the element path
    (n = 1000 is not a multiple of 16)."""
    from pck.cuda import gemv_fp8_scaled

    g = torch.Generator().manual_seed(m + n)
    W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
    x = torch.randn(n, generator=g).to(torch.bfloat16).cuda()
    Q, s = quantize_fp8(W)
    z, y = gemv_fp8_scaled(Q, x, s)
    assert torch.equal(z.view(torch.int32), gemv_fp8(Q, x).view(torch.int32))
    assert torch.equal(y.view(torch.int32), (s * z).view(torch.int32))


def test_fp8_scaled_group_carries_checks() -> None:
    """q, k, v in one dequantising launch that also carries the checks of earlier outputs:
    every z and y as in single launches, and the check results bit-identical to check_many."""
    from pck.cuda import GpuBlockedChecker, check_many, gemv_group_fp8_scaled

    g = torch.Generator().manual_seed(2)
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096)]
    triples, checks = [], []
    for m, n in shapes:
        W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
        Q, s = quantize_fp8(W)
        x = torch.randn(n, generator=g).to(torch.bfloat16).cuda()
        triples.append((Q, x, s))
        checker = GpuBlockedChecker(Q.to(torch.bfloat16), 128, tree_height(n, 256, 16),
                                    generator=torch.Generator().manual_seed(m))  # fmt: skip
        checks.append((checker, x, gemv_fp8(Q, x)))
    zs, ys, results = gemv_group_fp8_scaled(triples, checks)
    want = check_many(checks)
    for (Q, x, s), z, y in zip(triples, zs, ys, strict=True):
        assert torch.equal(z.view(torch.int32), gemv_fp8(Q, x).view(torch.int32))
        assert torch.equal(y.view(torch.int32), (s * z).view(torch.int32))
    for got, ref in zip(results, want, strict=True):
        assert torch.equal(got.passed, ref.passed) and bool(got.passed.all())
        assert torch.equal(got.rho.view(torch.int64), ref.rho.view(torch.int64))
        assert torch.equal(got.tau.view(torch.int64), ref.tau.view(torch.int64))
    with pytest.raises(RuntimeError, match="float32"):
        gemv_group_fp8_scaled([(triples[0][0], triples[0][1], triples[0][2].double())])


def test_fp8_rejects_bf16_weights() -> None:
    W, x = fp8_problem(4, 32, seed=0)
    with pytest.raises(RuntimeError, match="Float8_e4m3fn"):
        gemv_fp8(W, x)
