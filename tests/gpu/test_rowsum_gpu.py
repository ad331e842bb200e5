"""In-pass checksums (pck_gemv_group_rowsums, pck_rowsum_check) against the oracle.

- the in-pass launch keeps y's bits (those of pck_gemv_group) and writes row sums equal, bit for
  bit, to `oracle.rowsum.row_sums` for BF16 and FP8 weights, every thread count, vector and
  element loads, padded chains and the Llama-3-8B shapes;
- the row-sum check (standalone, and carried in a later in-pass launch) gives passed, rho and
  tau equal bit for bit to `oracle.rowsum.rowsum_check_with_signs`;
- its verdicts equal the bank checker's (GpuBlockedChecker, same signs) on honest outputs and
  on the planted faults of the reference's campaign (dropped tail, BF16 accumulator, partials
  and output, exponent and sign flips), except where |rho| falls between the two thresholds;
  its tau is never more than 2^-14 above the bank checker's (the bank's BF16 column sums are
  up to 2^-8 above the exact ones);
- non-finite outputs and weights fail closed; bad arguments raise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.gemv import e4m3_values, emulate_gemv, emulate_gemv_coalesced
from oracle.rowsum import row_sums, rowsum_check_with_signs
from pck.cuda import (
    GpuBlockedChecker,
    RowSumChecker,
    check_many,
    gemv_group,
    gemv_group_rowsums,
    quantize_fp8,
    rowsum_check_many,
)
from pck.faults import flip_bit
from pck.fp import bf16, tree_height

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def weights(m: int, n: int, seed: int, fp8: bool):  # type: ignore[no-untyped-def]
    """(device W or Q, device x, W values as float32 on the host, x values)."""
    gen = torch.Generator().manual_seed(seed)
    W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn(n, generator=gen).to(torch.bfloat16)
    Wd, xd = W.cuda(), x.cuda()
    if fp8:
        Q = quantize_fp8(Wd)[0]
        vals = e4m3_values()[Q.view(torch.uint8).cpu().numpy()]
        return Q, xd, vals, x.float().numpy()
    return Wd, xd, W.float().numpy(), x.float().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    a = t.detach().cpu().numpy()
    return a.view(np.uint64 if a.dtype == np.float64 else np.uint32)


SHAPES = [(256, 4096), (128, 14336), (96, 4100), (64, 40), (3, 8)]


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("m,n", SHAPES)
@pytest.mark.parametrize("threads", [32, 64, 256, 1024])
def test_row_sums_bits_equal_model(fp8: bool, m: int, n: int, threads: int) -> None:
    print(f"row sums fp8={fp8} m={m} n={n} threads={threads}", flush=True)
    W, x, Wv, xv = weights(m, n, seed=m + n + threads, fp8=fp8)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), threads)
    plain = gemv_group([(W, x)], threads)[0]
    assert np.array_equal(bits(ys[0]), bits(plain)), "in-pass y differs from the plain tree"
    want = row_sums(Wv, xv, threads, 16 if fp8 else 8)
    assert np.array_equal(bits(sums[0]), want.view(np.uint64))


@pytest.mark.parametrize("fp8", [False, True])
def test_row_sums_llama_shapes_grouped(fp8: bool) -> None:
    shapes = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
    made = [weights(m, n, seed=i, fp8=fp8) for i, (m, n) in enumerate(shapes)]
    # grouped launch: q/k/v-like (shared n) and the down shape on its own
    ys, sums, _ = gemv_group_rowsums([(W, x) for W, x, _, _ in made[:3]], (), 256)
    y4, s4, _ = gemv_group_rowsums([(made[3][0], made[3][1])], (), 256)
    vec = 16 if fp8 else 8
    for (W, x, Wv, xv), y, s in zip(made, ys + y4, sums + s4):
        print(f"llama row sums fp8={fp8} shape={tuple(W.shape)}", flush=True)
        assert np.array_equal(bits(y), emulate_gemv_coalesced(Wv, xv, 256, vec).view(np.uint32))
        assert np.array_equal(bits(s), row_sums(Wv, xv, 256, vec).view(np.uint64))


def rowsum_checker(m: int, n: int, block: int, seed: int, checks: int = 1, vec: int = 8):  # type: ignore[no-untyped-def]
    gen = torch.Generator().manual_seed(seed)
    return RowSumChecker(m, n, block, tree_height(n, 256, vec), checks, generator=gen)


def model_check(ch: RowSumChecker, sums: torch.Tensor, y: torch.Tensor):  # type: ignore[no-untyped-def]
    return rowsum_check_with_signs(
        sums.cpu().numpy(), y.cpu().numpy(), ch.r.cpu().numpy(), ch.block, ch.coef, ch.geps,
        ch.tau_floor, ch.s_factor,
    )  # fmt: skip


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("block,checks", [(128, 1), (256, 1), (96, 3), (64, 2)])
def test_rowsum_check_bits_equal_model(fp8: bool, block: int, checks: int) -> None:
    print(f"row-sum check fp8={fp8} block={block} checks={checks}", flush=True)
    m, n = 768, 4096
    W, x, Wv, xv = weights(m, n, seed=block, fp8=fp8)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), 256)
    ch = rowsum_checker(m, n, block, seed=7, checks=checks, vec=16 if fp8 else 8)
    y_bad = ys[0].clone()
    y_bad[5] += 0.5 * float(ys[0].abs().max())  # one faulty block (FP8 outputs are unscaled)
    for y in (ys[0], y_bad):
        res = ch.check(sums[0], y)
        passed, rho, tau = model_check(ch, sums[0], y)
        assert np.array_equal(res.passed.cpu().numpy(), passed)
        assert np.array_equal(bits(res.rho), rho.view(np.uint64))
        assert np.array_equal(bits(res.tau), tau.view(np.uint64))
    assert bool(ch.verdict(sums[0], ys[0]).all())
    assert not bool(ch.verdict(sums[0], y_bad)[0])


@pytest.mark.parametrize("fp8", [False, True])
def test_carried_rowsum_checks_equal_standalone(fp8: bool) -> None:
    shapes = [(1024, 4096), (512, 14336), (256, 4096)]
    made = [weights(m, n, seed=20 + i, fp8=fp8) for i, (m, n) in enumerate(shapes)]
    produced = [gemv_group_rowsums([(W, x)], (), 256) for W, x, _, _ in made]
    vec = 16 if fp8 else 8
    items = [
        (rowsum_checker(W.size(0), W.size(1), 128, seed=30 + i, vec=vec), s[0], y[0])
        for i, ((W, x, _, _), (y, s, _)) in enumerate(zip(made, produced))
    ]
    alone = rowsum_check_many(items)
    Wc, xc, Wcv, xcv = weights(2048, 4096, seed=40, fp8=fp8)
    outs, sums, riding = gemv_group_rowsums([(Wc, xc)], items, 256)
    for a, b in zip(riding, alone):
        assert torch.equal(a.passed, b.passed) and torch.equal(a.rho, b.rho)
        assert torch.equal(a.tau, b.tau) and bool(a.verdict.all())
    assert np.array_equal(bits(sums[0]), row_sums(Wcv, xcv, 256, vec).view(np.uint64))
    assert np.array_equal(bits(outs[0]), bits(gemv_group([(Wc, xc)], 256)[0]))


def planted(Wv: np.ndarray, xv: np.ndarray, y: np.ndarray, seed: int) -> dict[str, np.ndarray]:
    """The reference campaign's faults (harness/campaign.py:56-135): shortcuts through the
    naive-kernel model and one random exponent- or sign-bit flip per block."""
    rng = np.random.default_rng(seed)
    out = {
        "drop_tail": emulate_gemv(Wv, xv, 256, drop_tail=4),
        "bf16_accumulator": emulate_gemv(Wv, xv, 256, acc_bf16=True),
        "bf16_partials": emulate_gemv(Wv, xv, 256, partial_bf16=True),
        "bf16_output": bf16(y).astype(np.float32),
    }
    for kind, choices in (("exp_flip", range(23, 31)), ("sign_flip", [31])):
        z = y.copy()
        for beta in range(len(y) // 128):
            z = flip_bit(z, beta * 128 + int(rng.integers(128)), int(rng.choice(list(choices))))
        out[kind] = z
    return out


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("m,n", [(4096, 4096), (4096, 14336)])
def test_verdicts_equal_bank_checker(fp8: bool, m: int, n: int) -> None:
    print(f"verdict parity with the bank checker fp8={fp8} m={m} n={n}", flush=True)
    W, x, Wv, xv = weights(m, n, seed=m + n, fp8=fp8)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), 256)
    vec = 16 if fp8 else 8
    h = tree_height(n, 256, vec)
    bank = GpuBlockedChecker(W.to(torch.bfloat16), 128, h, generator=torch.Generator().manual_seed(5))
    rs = RowSumChecker(m, n, 128, h, generator=torch.Generator().manual_seed(5))
    assert torch.equal(bank.r, rs.r), "the same generator state gives the same signs"
    y = ys[0].cpu().numpy()
    cases = {"honest": y} | planted(Wv, xv, y, seed=n)
    in_window = 0
    for name, yy in cases.items():
        yt = torch.from_numpy(np.ascontiguousarray(yy, dtype=np.float32)).cuda()
        a = check_many([(bank, x, yt)])[0]
        b = rs.check(sums[0], yt)
        tau_bank, tau_rs = a.tau.cpu().numpy(), b.tau.cpu().numpy()
        finite = np.isfinite(tau_bank) & np.isfinite(tau_rs)
        # the bank's a is BF16 rounded up (up to 2^-8 over the exact column sums), the row sums'
        # s at most 2^-14 over the exact S
        assert (tau_rs[finite] <= tau_bank[finite] * (1 + 2.0**-14)).all(), name
        assert np.array_equal(np.isfinite(tau_bank), np.isfinite(tau_rs)), name
        rho = np.abs(a.rho.cpu().numpy())
        clear = (rho < 0.99 * tau_rs) | (rho > 1.01 * tau_bank)
        va, vb = a.passed.cpu().numpy(), b.passed.cpu().numpy()
        assert np.array_equal(va[clear], vb[clear]), name
        in_window += int((~clear).sum())
        if name == "honest":
            assert va.all() and vb.all()
    print(f"blocks between the two thresholds: {in_window}", flush=True)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("m,n", [(4096, 4096), (4096, 14336)])
def test_every_planted_fault_caught_at_eight_draws(fp8: bool, m: int, n: int) -> None:
    """The reference's protocol for planted shortcuts (8 sign draws, harness/numerics_sim.py:76):
    with y faulty after the products (the campaign's faults against the honest launch's row
    sums), both the row-sum and the bank check catch every kind at b = 128."""
    print(f"planted faults at K = 8 fp8={fp8} m={m} n={n}", flush=True)
    W, x, Wv, xv = weights(m, n, seed=m + n + 1, fp8=fp8)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), 256)
    h = tree_height(n, 256, 16 if fp8 else 8)
    bank = GpuBlockedChecker(W.to(torch.bfloat16), 128, h, checks=8, generator=torch.Generator().manual_seed(7))
    rs = RowSumChecker(m, n, 128, h, checks=8, generator=torch.Generator().manual_seed(7))
    y = ys[0].cpu().numpy()
    for name, yy in planted(Wv, xv, y, seed=n + 1).items():
        yt = torch.from_numpy(np.ascontiguousarray(yy, dtype=np.float32)).cuda()
        assert not bool(check_many([(bank, x, yt)])[0].verdict.all()), f"bank: {name} not caught"
        assert not bool(rs.check(sums[0], yt).verdict.all()), f"row sums: {name} not caught"


@pytest.mark.parametrize("fp8", [False, True])
def test_faults_inside_the_producing_launch(fp8: bool) -> None:
    """The row-sum check's trust model.  A shortcut inside the producing launch moves y and its
    row sums together: the in-pass launch run on W with its last 4 columns zeroed (a dropped
    tail) or on another x (a wrong activation vector) writes y and (d, s) that agree with each
    other, so the row-sum check passes them, as it passes honest outputs; the bank checker,
    whose checksums come from the weights and x themselves, rejects them.  Faults after the
    products (reductions, partials, output, flips) are the row-sum check's domain."""
    m, n = 4096, 4096
    W, x, _, _ = weights(m, n, seed=21, fp8=fp8)
    h = tree_height(n, 256, 16 if fp8 else 8)
    bank = GpuBlockedChecker(W.to(torch.bfloat16), 128, h, generator=torch.Generator().manual_seed(9))
    rs = RowSumChecker(m, n, 128, h, generator=torch.Generator().manual_seed(9))
    Wz = W.clone()
    Wz.view(torch.uint8 if fp8 else torch.int16)[:, -4:] = 0
    x2 = torch.randn(n, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16).cuda()
    (yz, y2), (sz, s2), _ = gemv_group_rowsums([(Wz, x), (W, x2)], (), 256)
    for name, yy, ss in (("drop_tail", yz, sz), ("wrong_x", y2, s2)):
        assert bool(rs.check(ss, yy).verdict.all()), f"row sums from the faulty launch: {name}"
        assert not bool(check_many([(bank, x, yy)])[0].verdict.all()), f"bank: {name} not caught"


def test_non_finite_fails_closed() -> None:
    W, x, _, _ = weights(256, 4096, seed=3, fp8=False)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), 256)
    ch = rowsum_checker(256, 4096, 128, seed=1)
    y = ys[0].clone()
    y[3] = float("nan")
    y[200] = float("inf")
    assert not bool(ch.verdict(sums[0], y).any())
    W2 = W.clone()
    W2[130, 7] = float("inf")  # an infinite weight: s and tau non-finite in its block
    ys2, sums2, _ = gemv_group_rowsums([(W2, x)], (), 256)
    assert ch.verdict(sums2[0], ys2[0]).tolist() == [True, False]


def test_bad_arguments_raise() -> None:
    W, x, _, _ = weights(256, 4096, seed=4, fp8=False)
    ys, sums, _ = gemv_group_rowsums([(W, x)], (), 256)
    ch = rowsum_checker(256, 4096, 128, seed=1)
    with pytest.raises(RuntimeError, match="sums must have shape"):
        ch.check(sums[0][:128], ys[0])
    with pytest.raises(RuntimeError, match="y must have shape"):
        ch.check(sums[0], ys[0][:128])
    with pytest.raises(RuntimeError, match="Double"):
        ch.check(sums[0].float(), ys[0])
    with pytest.raises(ValueError, match="divide m"):
        RowSumChecker(100, 4096, 128, 23)
