"""The HIP blocked checker against the oracle: verdicts equal to the CPU reference checker on the
same (W, x, y, r); rho within the kernel's own proven rounding of the exact value; tau never
below the exact threshold formula (every operation rounded up) and tight above it; planted
shortcuts, bit flips and non-finite outputs caught; the reference's GPU checker, check_many and
side-stream cases (tests/gpu/test_checker_cuda.py, test_check_many.py, test_side_stream.py)."""

from __future__ import annotations

import math
from fractions import Fraction
from typing import Any

import numpy as np
import pytest
import torch
from numpy.typing import NDArray

from oracle.checker import BlockedChecker, gpu_rho_exact, gpu_threshold_exact
from oracle.gemv import emulate_gemv
from pck.cuda import GpuBlockedChecker, SideStreamChecker, check_many, gemv_coalesced, gemv_naive
from pck.cuda.checker import blocked_check
from pck.fp import U32, bf16, gamma, tree_height

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

M, N, THREADS = 512, 4100, 256
HEIGHT = tree_height(N, THREADS, vec=8)


def problem(m: int = M, n: int = N, seed: int = 0):  # type: ignore[no-untyped-def]
    rng = np.random.default_rng(seed)
    W, x = bf16(rng.standard_normal((m, n)) * 0.02), bf16(rng.standard_normal(n))
    return W, x, torch.from_numpy(W).to(torch.bfloat16).cuda(), torch.from_numpy(x).to(torch.bfloat16).cuda()


def make(Wt: torch.Tensor, block: int = 64, checks: int = 8, seed: int = 0) -> GpuBlockedChecker:
    return GpuBlockedChecker(Wt, block, HEIGHT, checks=checks, generator=torch.Generator().manual_seed(seed))


def as_gpu(y: NDArray[np.float32]) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32)).cuda()


@pytest.mark.parametrize("block", [1, 8, 64, 128, 512])
def test_legit_gpu_output_passes(block: int) -> None:
    _, _, Wt, xt = problem()
    checker = make(Wt, block)
    for y in (gemv_coalesced(Wt, xt, THREADS), gemv_naive(Wt, xt, THREADS)):
        result = checker.check(xt, y)
        assert result.passed.all()
        assert (result.rho.abs() <= result.tau).all()


def test_rho_and_tau_against_exact_arithmetic() -> None:
    """tau >= the exact threshold formula (T3's round-up hypothesis) and at most 2^-40 above it
    (s = a.|x| and the rest are FP64 round-up sums, so only FP64 round-up slack remains); rho
    within geps (sum |c x| + sum |y|) of exact rho."""
    _, x, Wt, xt = problem(m=64, n=1000, seed=1)
    checker = GpuBlockedChecker(Wt, 32, HEIGHT, checks=2, generator=torch.Generator().manual_seed(1))
    y = gemv_coalesced(Wt, xt, 128)
    res = checker.check(xt, y)
    a = checker.a.float().cpu().numpy()
    yn = y.cpu().numpy()
    tau_exact = gpu_threshold_exact(a, x, yn, 32, checker.coef, checker.geps, checker.tau_floor)
    tau = res.tau.cpu().numpy()
    for k in range(2):
        for beta, te in enumerate(tau_exact):
            assert Fraction(float(tau[k, beta])) >= te
            assert Fraction(float(tau[k, beta])) <= te * (1 + Fraction(1, 2**40))
    c = checker.c.cpu().numpy()
    r = checker.r.cpu().numpy()
    rho_exact = gpu_rho_exact(c, r, x, yn)
    mags = np.abs(c.astype(np.float64)) @ np.abs(x.astype(np.float64)) + np.abs(yn.astype(np.float64)).reshape(-1, 32).sum(1)
    assert np.all(np.abs(res.rho.cpu().numpy() - rho_exact) <= checker.geps * mags * 1.01 + 1e-300)


def cpu_verdict(W, x, y, checker: GpuBlockedChecker, height: int) -> NDArray[np.bool_]:  # type: ignore[no-untyped-def]
    cpu = BlockedChecker(W, x, checker.block, height)
    return cpu.verdict_with_signs(y, checker.r.cpu().numpy().astype(np.float64))[0].all(0)


@pytest.mark.parametrize("exploit", ["legit", "skip_tail", "acc_bf16", "partial_bf16", "bf16_output"])
def test_verdicts_equal_the_cpu_reference_on_the_same_signs(exploit: str) -> None:
    W, x, Wt, xt = problem(m=512, n=2048, seed=2)
    height = tree_height(2048, 128)
    checker = GpuBlockedChecker(Wt, 64, height, checks=8, generator=torch.Generator().manual_seed(2))
    legit = emulate_gemv(W, x, 128)
    y = {
        "legit": lambda: legit,
        "skip_tail": lambda: emulate_gemv(W, x, 128, drop_tail=4),
        "acc_bf16": lambda: emulate_gemv(W, x, 128, acc_bf16=True),
        "partial_bf16": lambda: emulate_gemv(W, x, 128, partial_bf16=True),
        "bf16_output": lambda: bf16(legit),
    }[exploit]()
    gpu = checker.verdict(xt, as_gpu(y)).cpu().numpy()
    np.testing.assert_array_equal(gpu, cpu_verdict(W, x, y, checker, height))
    assert gpu.all() == (exploit == "legit")


@pytest.mark.parametrize("bit", [23, 27, 30, 31])
def test_bit_flips_match_the_cpu_reference(bit: int) -> None:
    """One flip per block (rows drawn from a seeded generator): the GPU flags exactly the blocks
    the CPU reference flags with the same signs."""
    W, x, Wt, xt = problem(m=1024, n=4096, seed=3)
    checker = GpuBlockedChecker(Wt, 128, tree_height(4096, 256, 8), generator=torch.Generator().manual_seed(3))
    y = gemv_coalesced(Wt, xt, 256).cpu().numpy()
    rng = np.random.default_rng(bit)
    rows = np.arange(0, 1024, 128) + rng.integers(0, 128, 8)
    bits = y.view(np.uint32).copy()
    bits[rows] ^= np.uint32(1 << bit)
    flipped = bits.view(np.float32)
    gpu = checker.verdict(xt, as_gpu(flipped)).cpu().numpy()
    np.testing.assert_array_equal(gpu, cpu_verdict(W, x, flipped, checker, tree_height(4096, 256, 8)))
    if bit >= 27:
        assert not gpu.any()


@pytest.mark.parametrize("bad", [math.nan, math.inf, -math.inf])
def test_non_finite_output_fails_its_block_only(bad: float) -> None:
    _, _, Wt, xt = problem()
    checker = make(Wt, 64, checks=2)
    y = gemv_coalesced(Wt, xt, THREADS)
    y[130] = bad
    expected = np.ones(M // 64, dtype=bool)
    expected[130 // 64] = False
    np.testing.assert_array_equal(checker.verdict(xt, y).cpu().numpy(), expected)


def test_large_single_error_always_caught() -> None:
    _, _, Wt, xt = problem(seed=4)
    checker = make(Wt, 64, checks=8, seed=4)
    y = gemv_coalesced(Wt, xt, THREADS)
    tau = checker.check(xt, y).tau.min(dim=0).values
    for i in (torch.arange(0, M, 64 + 3) % M).tolist():
        bad = y.clone()
        bad[i] += 2.5 * float(tau[i // 64])
        verdict = checker.verdict(xt, bad)
        assert not verdict[i // 64] and verdict.sum() == M // 64 - 1


def test_no_false_alarms_over_many_draws() -> None:
    _, _, Wt, xt = problem(seed=5)
    y = gemv_coalesced(Wt, xt, THREADS)
    for seed in range(50):
        assert make(Wt, 64, checks=8, seed=seed).verdict(xt, y).all()


@pytest.mark.parametrize(
    ("kwargs", "match"),
    [({"block": 7}, "divide"), ({"block": 0}, "positive"), ({"block": 64, "checks": 0}, "checks")],
)
def test_rejects_bad_configuration(kwargs: dict[str, Any], match: str) -> None:
    _, _, Wt, _ = problem(m=64, n=16)
    with pytest.raises(ValueError, match=match):
        GpuBlockedChecker(Wt, height=4, **kwargs)


def test_rejects_non_bf16_weights() -> None:
    with pytest.raises(ValueError, match="bfloat16"):
        GpuBlockedChecker(torch.ones((8, 8), device="cuda"), 4, 4)


@pytest.mark.parametrize(
    ("which", "match"),
    [("y_dtype", "y must be"), ("y_shape", "shape"), ("x_dtype", "x must be"), ("y_cpu", "CUDA")],
)
def test_rejects_bad_check_inputs(which: str, match: str) -> None:
    _, _, Wt, xt = problem(m=64, n=16)
    checker = GpuBlockedChecker(Wt, 16, 4)
    y = torch.zeros(64, device="cuda")
    args = {
        "y_dtype": (xt, y.double()),
        "y_shape": (xt, y[:32]),
        "x_dtype": (xt.float(), y),
        "y_cpu": (xt, y.cpu()),
    }[which]
    with pytest.raises(RuntimeError, match=match):
        checker.check(*args)


@pytest.mark.parametrize("segments", [1, 2, 3, 7, 64, 1000])
def test_segment_count_does_not_change_result(segments: int) -> None:
    _, x, Wt, xt = problem(m=256, n=1000, seed=6)
    y = gemv_coalesced(Wt, xt, 128)

    def checker(segs: int) -> GpuBlockedChecker:
        return GpuBlockedChecker(Wt, 32, HEIGHT, checks=4, generator=torch.Generator().manual_seed(6), segments=segs)

    ref = checker(1).check(xt, y)
    split_checker = checker(segments)
    split = split_checker.check(xt, y)
    assert torch.equal(split.passed, ref.passed)
    assert bool(((split.rho - ref.rho).abs() <= 1e-4 * ref.tau).all())
    torch.testing.assert_close(split.tau, ref.tau, rtol=(1000 + 1) * 2.0**-24, atol=0)
    a = split_checker.a.float().cpu().numpy().astype(np.float64)
    s_exact = a @ np.abs(x.astype(np.float64))
    assert np.all(split.tau.cpu().numpy() >= (gamma(HEIGHT) + U32) * s_exact * (1 - 1e-12))


def test_repeated_calls_reuse_scratch_correctly() -> None:
    _, _, Wt, xt = problem(seed=7)
    checker = make(Wt, 64, checks=2)
    y = gemv_coalesced(Wt, xt, THREADS)
    bad = y.clone()
    bad[5] = math.nan
    first = checker.check(xt, y)
    for _ in range(20):
        assert torch.equal(checker.verdict(xt, bad)[1:], first.verdict[1:])
        assert not checker.verdict(xt, bad)[0]
        again = checker.check(xt, y)
        assert torch.equal(again.passed, first.passed)
        assert torch.equal(again.rho, first.rho)
        assert torch.equal(again.tau, first.tau)
    assert int(checker._counters.abs().sum()) == 0  # tickets are left at zero


@pytest.mark.parametrize("segments", [0, 1001])
def test_rejects_bad_segment_count(segments: int) -> None:
    _, _, Wt, _ = problem(m=64, n=1000)
    with pytest.raises(ValueError, match="segments"):
        GpuBlockedChecker(Wt, 16, 4, segments=segments)


def test_a_is_bf16_rounded_up_from_exact() -> None:
    W, _, Wt, _ = problem(m=256, n=1000, seed=8)
    checker = GpuBlockedChecker(Wt, 32, HEIGHT)
    a = checker.a.float().cpu().numpy().astype(np.float64)
    exact = np.abs(W.astype(np.float64)).reshape(256 // 32, 32, 1000).sum(axis=1)
    assert checker.a.dtype == torch.bfloat16
    assert np.all(a >= exact) and np.all(a <= exact * (1 + 2.0**-7))


def test_c_is_the_rounded_exact_checksum() -> None:
    W, _, Wt, _ = problem(m=256, n=600, seed=10)
    checker = GpuBlockedChecker(Wt, 64, HEIGHT, checks=2, generator=torch.Generator().manual_seed(10))
    r = checker.r.cpu().numpy().astype(np.float64)
    Wb = W.astype(np.float64).reshape(4, 64, 600)
    exact = np.einsum("kbi,bin->kbn", r, Wb)  # exact: 64 BF16 terms of small spread in FP64
    np.testing.assert_array_equal(checker.c.cpu().numpy(), exact.astype(np.float32))


@pytest.mark.parametrize("scale_exp", [-100, -120, 60])
def test_legit_output_passes_at_extreme_scales(scale_exp: int) -> None:
    rng = np.random.default_rng(9)
    W = bf16(rng.standard_normal((256, 2048)) * 0.02)
    x = bf16(rng.standard_normal(2048) * 2.0**scale_exp)
    Wt = torch.from_numpy(W).to(torch.bfloat16).cuda()
    xt = torch.from_numpy(x).to(torch.bfloat16).cuda()
    checker = GpuBlockedChecker(Wt, 64, tree_height(2048, 128, vec=8), checks=8, generator=torch.Generator().manual_seed(9))
    y = gemv_coalesced(Wt, xt, 128)
    assert torch.isfinite(y).all()
    assert checker.verdict(xt, y).all()


def test_an_overflowing_threshold_fails_closed() -> None:
    m, n = 128, 4096
    signs = torch.where(torch.arange(n) % 2 == 0, 1.0, -1.0)
    Wt = (signs * 2.0**100).repeat(m, 1).to(torch.bfloat16).cuda()
    xt = torch.full((n,), 2.0**24).to(torch.bfloat16).cuda()
    checker = make(Wt, 64, checks=2)
    res = checker.check(xt, torch.full((m,), 1e30, device="cuda"))
    assert not res.passed.any()


# ---- check_many -------------------------------------------------------------------------------

CONFIGS = [
    (512, 4096, 64, 1, None),
    (1024, 512, 32, 2, 1),
    (256, 14336, 128, 4, 7),
    (64, 1000, 8, 1, 3),
    (2048, 4096, 256, 2, None),
]


def make_item(m: int, n: int, block: int, checks: int, segments: int | None, seed: int):  # type: ignore[no-untyped-def]
    gen = torch.Generator().manual_seed(seed)
    W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
    checker = GpuBlockedChecker(W, block, tree_height(n, 128, vec=8), checks=checks, generator=gen, segments=segments)
    return checker, x, gemv_coalesced(W, x, 128)


def test_batch_matches_individual_checks() -> None:
    items = [make_item(*cfg, seed=i) for i, cfg in enumerate(CONFIGS)]
    for (checker, x, y), res in zip(items, check_many(items), strict=True):
        alone = checker.check(x, y)
        assert torch.equal(res.passed, alone.passed)
        assert torch.equal(res.rho, alone.rho)
        assert torch.equal(res.tau, alone.tau)
        assert res.verdict.all()


def test_a_launch_with_more_pairs_than_cus_keeps_every_result() -> None:
    # 128 + 128 + 32 + 16 (check, block) pairs over uneven row lengths: more than the GPU's
    # compute units, so the launch deals the longest rows in another order.
    shapes = [(16384, 512), (16384, 512), (4096, 2048), (2048, 512)]
    gen = torch.Generator().manual_seed(21)
    items = []
    for m, n in shapes:
        W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
        ch = GpuBlockedChecker(W, 128, tree_height(n, THREADS, vec=8), generator=gen)
        items.append((ch, x, gemv_coalesced(W, x, THREADS)))
    pairs = sum(ch.num_blocks * ch.checks for ch, _, _ in items)
    assert pairs > torch.cuda.get_device_properties(0).multi_processor_count
    y_bad = items[2][2].clone()
    y_bad[5] += 1.0  # one block of the longest rows fails, and only that one
    items[2] = (items[2][0], items[2][1], y_bad)
    for (checker, x, y), res in zip(items, check_many(items), strict=True):
        alone = checker.check(x, y)  # one descriptor: launched in its own order
        assert torch.equal(res.passed, alone.passed)
        assert torch.equal(res.rho, alone.rho)
        assert torch.equal(res.tau, alone.tau)
    verdicts = [r.verdict for r in check_many(items)]
    assert all(bool(v.all()) for i, v in enumerate(verdicts) if i != 2)
    assert verdicts[2].tolist() == [False] + [True] * (len(verdicts[2]) - 1)


def test_more_than_one_launch_and_fault_isolation() -> None:
    items = [make_item(*CONFIGS[i % len(CONFIGS)], seed=10 + i) for i in range(11)]
    checker, x, y = items[9]
    bad = y.clone()
    bad[3] = float("inf")
    items[9] = (checker, x, bad)
    results = check_many(items)
    assert len(results) == 11
    for i, res in enumerate(results):
        if i == 9:
            assert not res.verdict[0] and res.verdict[1:].all()
        else:
            assert res.verdict.all()


def test_rejects_same_checker_twice() -> None:
    item = make_item(*CONFIGS[0], seed=0)
    with pytest.raises(ValueError, match="once"):
        check_many([item, item])


def test_native_entry_rejects_bad_batches() -> None:
    """The launch entry with the reference's pybind argument lists (bindings.cpp:221-256)."""
    checker, x, y = make_item(*CONFIGS[0], seed=0)
    args = [checker.c, checker.a, checker.r, x, y, checker._partial_cx, checker._partial_s,
            checker._counters, checker.coef, checker.geps, checker.tau_floor]  # fmt: skip
    with pytest.raises(RuntimeError, match="batch size"):
        blocked_check(*([] for _ in args))
    with pytest.raises(RuntimeError, match="batch size"):
        blocked_check(*([a] * 9 for a in args))
    lists = [[a] for a in args]
    lists[4] = [y, y]
    with pytest.raises(RuntimeError, match="same length"):
        blocked_check(*lists)


# ---- side stream ------------------------------------------------------------------------------


def side_setup(m: int, n: int, seed: int):  # type: ignore[no-untyped-def]
    gen = torch.Generator().manual_seed(seed)
    W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
    return W, x, GpuBlockedChecker(W, 64, tree_height(n, 256, vec=8), checks=2, generator=gen)


def test_side_stream_matches_same_stream() -> None:
    W, x, checker = side_setup(512, 4096, seed=0)
    y = gemv_coalesced(W, x, 256)
    serial = checker.check(x, y)
    result = SideStreamChecker().submit(checker, x, y).wait()
    assert torch.equal(result.passed, serial.passed)
    assert torch.equal(result.rho, serial.rho)
    assert torch.equal(result.tau, serial.tau)
    assert result.verdict.all()


def test_check_sees_output_even_if_freed_and_overwritten() -> None:
    W, x, checker = side_setup(1024, 4096, seed=1)
    side = SideStreamChecker()
    pending = []
    for _ in range(20):
        y = gemv_coalesced(W, x, 256)
        pending.append(side.submit(checker, x, y))
        del y
        garbage = torch.full((1024,), float("nan"), device="cuda")
        garbage.add_(1)
    for p in pending:
        assert p.wait().verdict.all()


def test_many_layers_overlap_and_detect_a_fault() -> None:
    side = SideStreamChecker()
    layers = [side_setup(m, n, seed=s) for s, (m, n) in enumerate([(512, 4096), (2048, 512)] * 3)]
    pending = []
    for i, (W, x, checker) in enumerate(layers):
        y = gemv_coalesced(W, x, 256)
        if i == 3:
            y[7] += 1.0
        pending.append(side.submit(checker, x, y))
    side.wait_all()
    for i, v in enumerate(p.wait().verdict for p in pending):
        if i == 3:
            assert not v[0] and v[1:].all()
        else:
            assert v.all()


# (m, n, block, checks): quad loads (n % 4 == 0) and element loads (n % 4 != 0), block sizes
# below, at and above the 256 lanes that take the y rows, the Llama-3-8B widths.
BIT_CASES = [(512, 4096, 128, 2), (256, 14336, 128, 1), (512, 4100, 64, 3), (512, 1001, 512, 2),
             (64, 4096, 8, 4), (256, 4096, 256, 1)]  # fmt: skip


@pytest.mark.parametrize(("m", "n", "block", "checks"), BIT_CASES)
def test_passed_rho_tau_equal_the_hip_model_bit_for_bit(m: int, n: int, block: int, checks: int) -> None:
    """The kernel's (passed, rho, tau) equal `oracle.checker_orders.hip_check` bit for bit, on
    an honest output, one with a BF16-rounded tail and flipped exponent and sign bits, and one
    with a NaN and an infinity; and its tau is never above the reference CUDA kernel's
    (`reference_gpu_check`) at the segment count the reference would choose on its 30-SM GPU."""
    from oracle.checker_orders import hip_check, reference_default_segments, reference_gpu_check

    print(f"checker bits m={m} n={n} b={block} K={checks}", flush=True)
    _, x, Wt, xt = problem(m, n, seed=m + n)
    h = tree_height(n, THREADS, 8)
    ch = GpuBlockedChecker(Wt, block, h, checks=checks, generator=torch.Generator().manual_seed(n))
    y = gemv_coalesced(Wt, xt, THREADS)
    bad = y.clone()
    bad[m // 2 :] = bad[m // 2 :].bfloat16().float()
    bits = bad.view(torch.int32)
    bits[1] ^= 1 << 27
    bits[m - 2] ^= -(2**31)
    odd = y.clone()
    odd[block // 2] = float("nan")
    odd[m - 1] = float("inf")
    c, a, r = ch.c.cpu().numpy(), ch.a.float().cpu().numpy(), ch.r.cpu().numpy()
    seg = reference_default_segments(n, checks, ch.num_blocks, 30)
    for name, yy in (("honest", y), ("faulty", bad), ("non-finite", odd)):
        res = check_many([(ch, xt, yy)])[0]
        yn = yy.cpu().numpy()
        passed, rho, tau = hip_check(c, a, r, x, yn, ch.coef, ch.geps, ch.tau_floor)
        assert np.array_equal(res.passed.cpu().numpy(), passed), name
        for got, want in ((res.rho.cpu().numpy(), rho), (res.tau.cpu().numpy(), tau)):
            same = (got.view(np.uint64) == want.view(np.uint64)) | (np.isnan(got) & np.isnan(want))
            assert same.all(), (name, np.argwhere(~same)[:4])
        _, _, tau_ref = reference_gpu_check(c, a, r, x, yn, ch.coef, ch.geps, ch.tau_floor, seg)
        finite = np.isfinite(tau_ref)
        assert (res.tau.cpu().numpy()[finite] <= tau_ref[finite]).all(), name
    assert bool(check_many([(ch, xt, y)])[0].passed.all())


def test_zero_activations_give_the_model_bits() -> None:
    """x = 0 (and zero weight rows with a nonzero x) leave s = 0: tau is the threshold's floor
    terms only, with the exact zero products kept at +0 (no ulp raise), bit for bit as the
    model's general round-up product gives them."""
    from oracle.checker_orders import hip_check

    m, n, block = 256, 4096, 128
    W, x, Wt, xt = problem(m, n, seed=11)
    W[:block] = 0.0  # first block: zero rows
    Wt = torch.from_numpy(W).to(torch.bfloat16).cuda()
    ch = GpuBlockedChecker(Wt, block, tree_height(n, THREADS, 8), checks=2,
                           generator=torch.Generator().manual_seed(1))  # fmt: skip
    c, a, r = ch.c.cpu().numpy(), ch.a.float().cpu().numpy(), ch.r.cpu().numpy()
    for xv in (np.zeros_like(x), x):
        xg = torch.from_numpy(xv).to(torch.bfloat16).cuda()
        y = gemv_coalesced(Wt, xg, THREADS)
        res = check_many([(ch, xg, y)])[0]
        passed, rho, tau = hip_check(c, a, r, xv, y.cpu().numpy(), ch.coef, ch.geps, ch.tau_floor)
        assert np.array_equal(res.passed.cpu().numpy(), passed)
        assert np.array_equal(res.tau.cpu().numpy().view(np.uint64), tau.view(np.uint64))
        assert np.array_equal(res.rho.cpu().numpy().view(np.uint64), rho.view(np.uint64))
        assert bool(res.passed.all())
