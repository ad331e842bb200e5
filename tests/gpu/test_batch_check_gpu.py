"""The batched blocked checker (every column of Y = X W^T checked) against the oracle: verdicts
equal to the CPU reference checker, column by column, on the same (W, X[b], Y[b], r) for honest
and faulty outputs (for the reference's BF16-accumulator and BF16-partials shortcuts at the
down projection's full size, BF16 and FP8, except in the band just above the CPU's tau that the
BF16 rounding of the GPU bank's a opens); equal to the single-vector HIP checker; tau within [exact threshold,
exact (1 + 2^-15)] (the BF16 matrix-core bound of a . |x|) and never below the exact threshold
when X spans subnormals to large values; rho within its proven rounding; honest batched
products at Llama-3-8B shapes pass with the batched tree height."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch
from numpy.typing import NDArray

from oracle.checker import BlockedChecker, WeightBank, gpu_rho_exact, gpu_threshold_exact
from pck.cuda import (
    GpuBlockedChecker,
    batched_height,
    check_batched,
    check_many,
    gemm_batched,
    pack_batched_weights,
    quantize_fp8,
)
from pck.fp import bf16

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def problem(m: int, n: int, B: int, seed: int):  # type: ignore[no-untyped-def]
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    X = bf16(rng.standard_normal((B, n)))
    Wt = torch.from_numpy(W).to(torch.bfloat16).cuda()
    Xt = torch.from_numpy(X).to(torch.bfloat16).cuda()
    return W, X, Wt, Xt


def cpu_verdicts(W, X, Y, checker: GpuBlockedChecker, height: int) -> NDArray[np.bool_]:  # type: ignore[no-untyped-def]
    """(nb, B) verdicts of the CPU reference checker, one column at a time, with the GPU
    checker's signs."""
    bank = WeightBank(W, checker.block)
    signs = checker.r.cpu().numpy().astype(np.float64)
    cols = []
    for b in range(X.shape[0]):
        cpu = BlockedChecker(W, X[b], checker.block, height, bank=bank)
        cols.append(cpu.verdict_with_signs(Y[b], signs)[0].all(0))
    return np.stack(cols, axis=1)


def faulty(kind: str, Wt: torch.Tensor, Xt: torch.Tensor, rng: np.random.Generator) -> torch.Tensor:
    """Y with a planted fault: dropped tail columns (the product skips the last four columns
    of the reduction), BF16 outputs, or one bit flipped per (block, column): the top exponent
    bit of a random output, or the sign of the block's largest output."""
    if kind == "legit":
        return gemm_batched(Wt, Xt)
    if kind == "skip_tail":
        Wz = Wt.clone()
        Wz[:, -4:] = 0
        return gemm_batched(Wz, Xt)
    Y = gemm_batched(Wt, Xt)
    if kind == "bf16_output":
        return Y.to(torch.bfloat16).float()
    bit = {"exp_flip": 30, "sign_flip": 31}[kind]
    y = Y.cpu().numpy().copy()
    B, m = y.shape
    if kind == "sign_flip":
        # the largest output of each block: negating a value below tau / 2 is an error no
        # rounding bound can separate from rounding (the CPU reference passes it too)
        rows = np.abs(y).reshape(B, m // 64, 64).argmax(axis=2) + np.arange(0, m, 64)
    else:
        rows = rng.integers(0, 64, (B, m // 64)) + np.arange(0, m, 64)
    bits = y.view(np.uint32)
    for b in range(B):
        bits[b, rows[b]] ^= np.uint32(1 << bit)
    return torch.from_numpy(y).cuda()


@pytest.mark.parametrize("kind", ["legit", "skip_tail", "bf16_output", "exp_flip", "sign_flip"])
def test_verdicts_equal_the_cpu_reference_column_by_column(kind: str) -> None:
    m, n, B = 256, 1024, 33
    W, X, Wt, Xt = problem(m, n, B, seed=7)
    height = batched_height(n)
    checker = GpuBlockedChecker(Wt, 64, height, checks=3, generator=torch.Generator().manual_seed(7))
    Y = faulty(kind, Wt, Xt, np.random.default_rng(7))
    print(f"batch check kind={kind} m={m} n={n} B={B}", flush=True)
    res = checker.check_batched(Xt, Y)
    assert res.passed.shape == (3, m // 64, B)
    gpu = res.verdict.cpu().numpy()
    np.testing.assert_array_equal(gpu, cpu_verdicts(W, X, Y.cpu().numpy(), checker, height))
    if kind == "legit":
        assert gpu.all()
    elif kind == "bf16_output":
        assert not gpu.all()  # an error near tau per check: most cells, not every one
    else:
        assert not gpu.any()


def shortcut(kind: str, Wq: torch.Tensor, X: torch.Tensor) -> torch.Tensor:
    """A batched product with a reduced-precision shortcut, from FP32 products of the exact
    weight values: ``bf16_partials`` rounds each of the 8 K segments' sums to BF16 before
    adding them; ``bf16_accumulator`` rounds the running sum to BF16 after every 32 columns."""
    Wf = Wq.float().t().contiguous()  # (n, m), exact E4M3 / BF16 values
    Xf = X.float()
    n = Xf.size(1)
    Y = torch.zeros((Xf.size(0), Wf.size(1)), dtype=torch.float32, device=X.device)
    if kind == "bf16_partials":
        seg = -(-n // 8)
        for j in range(0, n, seg):
            Y += (Xf[:, j : j + seg] @ Wf[j : j + seg]).to(torch.bfloat16).float()
    else:
        for j in range(0, n, 32):
            Y = (Y + Xf[:, j : j + 32] @ Wf[j : j + 32]).to(torch.bfloat16).float()
    return Y


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
@pytest.mark.parametrize("kind", ["bf16_accumulator", "bf16_partials"])
def test_shortcuts_at_the_down_projection(kind: str, fp8: bool) -> None:
    """The reference's BF16-accumulator and BF16-partials shortcuts planted in batched outputs of
    Llama-3-8B's down projection (4096 x 14336), BF16 and FP8 weights, b = 128: honest outputs
    pass, and the batched checker's verdicts equal the CPU reference column by column except
    where the CPU's |rho| lies just above its own tau: the GPU bank rounds a up to BF16 (as
    the reference's GPU bank does, `cuda/checker.py:99-101`) where the CPU checker rounds it up
    to FP32, so the GPU tau may be up to 2^-8 larger and pass such a cell.  The largest
    |rho| / tau over a column's blocks is reported for the column nearest to escaping (an
    error below tau in every block is the bound's floor: T2 promises detection above 2 tau).
    """
    m, n, B = 4096, 14336, 48
    g = torch.Generator().manual_seed(1 + fp8)
    W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
    Wq = quantize_fp8(W)[0] if fp8 else W
    Wc = Wq.to(torch.bfloat16)  # the weights' exact values
    X = torch.randn(B, n, generator=g).to(torch.bfloat16).cuda()
    height = batched_height(n)
    checker = GpuBlockedChecker(Wc, 128, height, generator=torch.Generator().manual_seed(5))
    print(f"batched shortcut {kind} fp8={fp8} m={m} n={n} B={B}", flush=True)
    honest = checker.check_batched(X, gemm_batched(pack_batched_weights(Wq), X))
    assert bool(honest.verdict.all())
    Y = shortcut(kind, Wq, X)
    res = checker.check_batched(X, Y)
    gpu = res.verdict.cpu().numpy()
    W_np, X_np, Y_np = Wc.float().cpu().numpy(), X.float().cpu().numpy(), Y.cpu().numpy()
    bank = WeightBank(W_np, 128)
    signs = checker.r.cpu().numpy().astype(np.float64)
    cpu_pass, cpu_ratio = [], []
    for b in range(B):
        passed, rho, tau = BlockedChecker(W_np, X_np[b], 128, height, bank=bank).verdict_with_signs(Y_np[b], signs)
        cpu_pass.append(passed.all(0))
        cpu_ratio.append((np.abs(rho) / tau).max(0))
    cpu, cpu_r = np.stack(cpu_pass, 1), np.stack(cpu_ratio, 1)
    band = ~cpu & gpu & (cpu_r <= 1 + 2.0**-7)
    assert ((gpu == cpu) | band).all()
    print(f"  cells {gpu.size}, verdicts differing in the a-rounding band {int(band.sum())}", flush=True)
    ratio = (res.rho.abs() / res.tau).amax(dim=(0, 1))  # per column: its largest block ratio
    caught = int((~res.verdict).any(dim=0).sum())
    print(f"  K = 1: columns caught {caught}/{B}; smallest column max |rho|/tau "
          f"{float(ratio.min()):.3g}", flush=True)  # fmt: skip
    assert bool(((ratio > 1) == (~res.verdict).any(dim=0)).all())
    # The reference's protocol checks each planted kernel with 8 sign draws
    # (harness/numerics_sim.py:76): then every column must be caught.
    k8 = GpuBlockedChecker(Wc, 128, height, checks=8, generator=torch.Generator().manual_seed(6))
    assert bool(k8.check_batched(X, gemm_batched(pack_batched_weights(Wq), X)).verdict.all())
    res8 = k8.check_batched(X, Y)
    caught8 = int((~res8.verdict).any(dim=0).sum())
    ratio8 = (res8.rho.abs() / res8.tau).amax(dim=(0, 1))
    print(f"  K = 8: columns caught {caught8}/{B}; smallest column max |rho|/tau "
          f"{float(ratio8.min()):.3g}", flush=True)  # fmt: skip
    assert caught8 == B


def test_batched_equals_the_single_vector_checker() -> None:
    """Same bank, same columns: the batched launch and check_many on each column agree on every
    verdict (the bounds of s differ by at most one FP32 rounding, far from any verdict here)."""
    m, n, B = 512, 2048, 20
    _, _, Wt, Xt = problem(m, n, B, seed=8)
    checker = GpuBlockedChecker(Wt, 128, batched_height(n), checks=2, generator=torch.Generator().manual_seed(8))
    Y = gemm_batched(Wt, Xt)
    bad = Y.clone()
    bad[3, 200] += 1.0
    bad[17, 5] *= -1.0
    for out in (Y, bad):
        res = checker.check_batched(Xt, out)
        for b in range(B):
            single = check_many([(checker, Xt[b].contiguous(), out[b].contiguous())])[0]
            np.testing.assert_array_equal(res.passed[:, :, b].cpu().numpy(), single.passed.cpu().numpy())


@pytest.mark.parametrize("n,B", [(1001, 2), (1001, 19), (4100, 9)])
def test_shapes_off_the_batched_kernel_check_column_by_column(n: int, B: int) -> None:
    """n % 8 != 0 (the batched kernel's loads need n % 8 == 0): every column goes through the
    single-vector kernel, eight per launch with the same bank; results equal check_many on each
    column, faulty columns included."""
    m = 256
    _, _, Wt, Xt = problem(m, n, B, seed=n + B)
    checker = GpuBlockedChecker(Wt, 128, batched_height(n), checks=2, generator=torch.Generator().manual_seed(3))
    Y = gemm_batched(Wt, Xt)
    Y[B - 1, 130] += 5.0  # block 1 of the last column
    res = checker.check_batched(Xt, Y)
    assert res.passed.shape == (2, m // 128, B)
    for b in range(B):
        single = check_many([(checker, Xt[b].contiguous(), Y[b].contiguous())])[0]
        assert torch.equal(res.passed[:, :, b], single.passed)
        assert torch.equal(res.rho[:, :, b], single.rho) and torch.equal(res.tau[:, :, b], single.tau)
    assert res.verdict[:, : B - 1].all() and res.verdict[:, B - 1].tolist() == [True, False]


def tau_and_rho_within_bounds(X: NDArray[np.float32], Xt: torch.Tensor, Wt: torch.Tensor, n: int,
                              rel: Fraction) -> None:
    checker = GpuBlockedChecker(Wt, 32, batched_height(n), checks=2, generator=torch.Generator().manual_seed(9))
    Y = gemm_batched(Wt, Xt)
    res = checker.check_batched(Xt, Y)
    a = checker.a.float().cpu().numpy()
    c = checker.c.cpu().numpy()
    r = checker.r.cpu().numpy()
    tau = res.tau.cpu().numpy()
    rho = res.rho.cpu().numpy()
    Yn = Y.cpu().numpy()
    for b in (0, 7, 17):
        exact = gpu_threshold_exact(a, X[b], Yn[b], 32, checker.coef, checker.geps, checker.tau_floor)
        for k in range(2):
            for beta, te in enumerate(exact):
                assert Fraction(float(tau[k, beta, b])) >= te
                assert Fraction(float(tau[k, beta, b])) <= te * (1 + rel)
        rho_exact = gpu_rho_exact(c, r, X[b], Yn[b])
        mags = np.abs(c.astype(np.float64)) @ np.abs(X[b].astype(np.float64)) + np.abs(
            Yn[b].astype(np.float64)
        ).reshape(-1, 32).sum(1)
        assert np.all(np.abs(rho[:, :, b] - rho_exact) <= checker.geps * mags * 1.01 + 1e-300)


def test_tau_and_rho_against_exact_arithmetic() -> None:
    m, n, B = 64, 640, 18
    _, X, Wt, Xt = problem(m, n, B, seed=9)
    tau_and_rho_within_bounds(X, Xt, Wt, n, Fraction(1, 2**15))


@pytest.mark.parametrize("n", [776, 1032])
def test_steps_cut_by_the_row_end(n: int) -> None:
    """n % 8 == 0 but n % 32 != 0: the last K step of a row is cut inside, so lanes of one step
    are in range and the rest read zero through the offsets' out-of-range bit.  rho and tau
    stay within their proven bounds of the exact values, and a planted sign flip is caught by
    exactly the cells the CPU checker flags."""
    m, B = 64, 18
    print(f"batched check cut step n={n}", flush=True)
    W, X, Wt, Xt = problem(m, n, B, seed=n)
    tau_and_rho_within_bounds(X, Xt, Wt, n, Fraction(1, 2**15))
    height = batched_height(n)
    checker = GpuBlockedChecker(Wt, 32, height, checks=2, generator=torch.Generator().manual_seed(n))
    Y = gemm_batched(Wt, Xt)
    bad = Y.clone()
    bad[5, 40] = -bad[5, 40]
    gpu = checker.check_batched(Xt, bad).verdict.cpu().numpy()
    np.testing.assert_array_equal(gpu, cpu_verdicts(W, X, bad.cpu().numpy(), checker, height))
    assert gpu.sum() == gpu.size - 1 and not gpu[1, 5]


def test_tau_never_below_exact_for_wide_and_subnormal_x() -> None:
    """X spanning 2^-133 (BF16 subnormal) to 2^40 in one row: the matrix-core step truncates the
    small products against the large ones and may flush subnormal products; tau must still be at
    least the exact threshold (the upper bound is looser here: the n 2^-125 floor of s)."""
    m, n, B = 64, 640, 18
    rng = np.random.default_rng(12)
    _, _, Wt, _ = problem(m, n, B, seed=12)
    exps = rng.integers(-133, 41, (B, n)).astype(np.float64)
    X = bf16(np.ldexp(rng.uniform(1.0, 2.0, (B, n)), exps.astype(np.int64)) * rng.choice([-1.0, 1.0], (B, n)))
    X[:, ::7] = bf16(np.ldexp(1.0, -133) * rng.integers(1, 128, (B, len(range(0, n, 7)))))  # subnormals
    Xt = torch.from_numpy(X).to(torch.bfloat16).cuda()
    assert np.array_equal(Xt.float().cpu().numpy(), X)
    tau_and_rho_within_bounds(X, Xt, Wt, n, Fraction(1, 2**10))


@pytest.mark.parametrize("bad", [math.nan, math.inf])
def test_non_finite_output_fails_its_block_and_column_only(bad: float) -> None:
    m, n, B = 256, 512, 40
    _, _, Wt, Xt = problem(m, n, B, seed=10)
    checker = GpuBlockedChecker(Wt, 64, batched_height(n), generator=torch.Generator().manual_seed(10))
    Y = gemm_batched(Wt, Xt)
    Y[29, 130] = bad
    expected = np.ones((m // 64, B), dtype=bool)
    expected[130 // 64, 29] = False
    np.testing.assert_array_equal(checker.check_batched(Xt, Y).verdict.cpu().numpy(), expected)


@pytest.mark.parametrize("B", [128, 256])
def test_honest_llama_layer_passes(B: int) -> None:
    """All seven Llama-3-8B projections (q/k/v fused, gate/up fused), packed route, BF16 and
    FP8 weights, one checker launch for the layer; 0 false alarms."""
    g = torch.Generator().manual_seed(B)
    shapes = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]
    for fp8 in (False, True):
        items = []
        for m, n in shapes:
            W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
            if fp8:
                W, _ = quantize_fp8(W)  # the check is against the E4M3 values themselves
            Wc = W.to(torch.bfloat16)
            X = torch.randn(B, n, generator=g).to(torch.bfloat16).cuda()
            Y = gemm_batched(pack_batched_weights(W), X)
            checker = GpuBlockedChecker(Wc, 128, batched_height(n), generator=torch.Generator().manual_seed(m))
            items.append((checker, X, Y))
        print(f"batch check llama B={B} fp8={fp8}", flush=True)
        for res in check_batched(items):
            assert bool(res.passed.all())
            assert bool((res.rho.abs() <= res.tau).all())


def test_two_layers_in_one_call_give_the_verdicts_of_two_calls() -> None:
    """The two-layer schedule: eight outputs (two Llama-3-8B layers, B = 128) in one call plan
    a longer K segment than four do, which moves only the rounding of rho and tau.  Verdicts
    equal those of one call per layer: every honest column passes, and columns with a flipped
    exponent bit in some outputs (layer 2's o and down) fail in both."""
    g = torch.Generator().manual_seed(2)
    shapes = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]
    B = 128
    items = []
    for layer in range(2):
        for m, n in shapes:
            W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
            X = torch.randn(B, n, generator=g).to(torch.bfloat16).cuda()
            Y = gemm_batched(pack_batched_weights(W), X)
            if layer == 1 and m == 4096:  # o and down: flip bit 30 of one output in 5 columns
                cols = torch.tensor([0, 17, 64, 101, 127], device="cuda")
                rows = torch.randint(0, m, (5,), generator=g).cuda()
                Yi = Y.view(torch.int32)
                Yi[cols, rows] ^= 1 << 30
            checker = GpuBlockedChecker(W, 128, batched_height(n), generator=torch.Generator().manual_seed(m + layer))
            items.append((checker, X, Y))
    print("batch check two layers in one call B=128", flush=True)
    together = check_batched(items)
    apart = check_batched(items[:4]) + check_batched(items[4:])
    for i, (one, two) in enumerate(zip(together, apart)):
        assert torch.equal(one.passed, two.passed), i
        ok = one.passed  # finite rho there; the flipped outputs can make rho infinite
        assert bool(((one.rho - two.rho).abs() <= 1e-6 * one.tau)[ok].all()), i
    failing = [int((~r.verdict).any(dim=0).sum()) for r in together]
    assert failing == [0, 0, 0, 0, 0, 5, 0, 5]


def test_validation_messages() -> None:
    _, _, Wt, Xt = problem(128, 256, 4, seed=11)
    checker = GpuBlockedChecker(Wt, 64, batched_height(256), generator=torch.Generator().manual_seed(11))
    Y = gemm_batched(Wt, Xt)
    with pytest.raises(RuntimeError, match="X must be"):
        checker.check_batched(Xt.float(), Y)
    with pytest.raises(RuntimeError, match="shape"):
        checker.check_batched(Xt[:, :128].contiguous(), Y)
    with pytest.raises(RuntimeError, match="shape"):
        checker.check_batched(Xt, Y[:3].contiguous())
    with pytest.raises(RuntimeError, match="CUDA"):
        checker.check_batched(Xt, Y.cpu())
    # an empty batch is validated like any other and gives empty results, as gemm_batched
    # gives an empty product
    X0 = Xt[:0].contiguous()
    Y0 = gemm_batched(Wt, X0)
    res = checker.check_batched(X0, Y0)
    assert res.passed.shape == (1, 2, 0) and res.rho.shape == res.tau.shape == (1, 2, 0)
    with pytest.raises(RuntimeError, match="X must be"):
        checker.check_batched(X0.float(), Y0)
    with pytest.raises(RuntimeError, match="shape"):
        checker.check_batched(X0, Y[:0, :64].contiguous())
