"""The bit-level models of the reference's CUDA checker and of this build's HIP checker
(`oracle/checker_orders.py`), pinned and compared.

- Small-integer inputs: every operation is exact, so both models give the exact rho, and
  their tau is the exact s and sum |y| carried through tau's round-up steps.
- The reference's own GPU-test criterion (`tests/gpu/test_checker_cuda.py:54-80`): tau is at
  or above the exact threshold and within n 2^-24 (reference) or 2^-40 (this build) above it;
  rho is within the threshold's own allowance of the exact value.
- Hand-traced cases in which the reference's FP32 round-up chain rounds and this build's FP64
  sum does not, and in which its Dot2 chain keeps a term that a plain FP32 sum would drop.
- The ordering: on decode-shaped inputs, for every segment count the reference can choose, this
  build's tau is never above the reference GPU checker's, and the two give the same verdicts
  on honest outputs and on the planted shortcuts.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle.checker import gpu_threshold_exact
from oracle.checker_orders import hip_check, reference_default_segments, reference_gpu_check
from oracle.gemv import emulate_gemv, emulate_gemv_coalesced
from pck.fp import U32, bf16, gamma, next_up, tree_height


def ru(q: Fraction) -> float:
    f = float(q)
    return math.nextafter(f, math.inf) if Fraction(f) < q else f


def bank(W: np.ndarray, r: np.ndarray, block: int) -> tuple[np.ndarray, np.ndarray]:
    """c = r^T W_beta rounded to FP32 and a = sum |W| over the block rounded up to BF16 (the
    GPU bank's rules)."""
    m, n = W.shape
    Wb = W.reshape(m // block, block, n).astype(np.float64)
    c = np.einsum("kbi,bin->kbn", r.astype(np.float64), Wb).astype(np.float32)
    col = np.abs(Wb).sum(axis=1)
    a32 = col.astype(np.float32)
    a32 = np.where(a32.astype(np.float64) < col, np.nextafter(a32, np.float32(np.inf)), a32)
    bits = a32.view(np.uint32)
    bits = np.where(bits & 0xFFFF, (bits + 0x10000) & 0xFFFF0000, bits).astype(np.uint32)
    return c, bits.view(np.float32)


def constants(n: int, h: int) -> tuple[float, float, float]:
    return next_up(gamma(h) + U32, 2), next_up(gamma(n + 129, 2.0**-53) * 1.0001, 2), next_up(n * 2.0**-148, 2)


MODELS = {"reference": lambda *a: reference_gpu_check(*a, segments=3), "hip": hip_check}


@pytest.mark.parametrize("model", MODELS)
def test_small_integers_are_exact(model: str) -> None:
    rng = np.random.default_rng(1)
    K, nb, b, n = 2, 3, 8, 700
    c = rng.integers(-5, 6, (K, nb, n)).astype(np.float32)
    a = rng.integers(0, 6, (nb, n)).astype(np.float32)
    x = rng.integers(-3, 4, n).astype(np.float32)
    r = rng.choice([-1, 1], (K, nb, b)).astype(np.int8)
    y = rng.integers(-50, 51, nb * b).astype(np.float32)
    coef, geps, tf = 0.25, 2.0**-40, 2.0**-100
    passed, rho, tau = MODELS[model](c, a, r, x, y, coef, geps, tf)
    for k in range(K):
        for beta in range(nb):
            yb = y[beta * b : (beta + 1) * b].astype(np.int64)
            want_rho = int(c[k, beta].astype(np.int64) @ x.astype(np.int64) - r[k, beta].astype(np.int64) @ yb)
            s = Fraction(int(a[beta].astype(np.int64) @ np.abs(x).astype(np.int64)))
            ya = Fraction(int(np.abs(yb).sum()))
            cabs = ru(Fraction(1.0 + 2.0**-24) * s)
            eps = ru(Fraction(geps) * Fraction(ru(Fraction(cabs) + ya)))
            want_tau = ru(Fraction(ru(Fraction(ru(Fraction(coef) * s)) + Fraction(eps))) + Fraction(tf))
            assert rho[k, beta] == want_rho and tau[k, beta] == want_tau
            assert passed[k, beta] == (abs(want_rho) <= want_tau)


def decode_block(n: int, seed: int, m: int = 256, K: int = 2, block: int = 128):  # type: ignore[no-untyped-def]
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    r = rng.choice([-1, 1], (K, m // block, block)).astype(np.int8)
    c, a = bank(W, r, block)
    return W, x, r, c, a


@pytest.mark.parametrize("model", MODELS)
@pytest.mark.parametrize("n", [1000, 4096])
def test_the_reference_tests_criterion(model: str, n: int) -> None:
    W, x, r, c, a = decode_block(n, seed=n)
    y = emulate_gemv_coalesced(W, x, 256)
    coef, geps, tf = constants(n, tree_height(n, 256, 8))
    passed, rho, tau = MODELS[model](c, a, r, x, y, coef, geps, tf)
    exact = gpu_threshold_exact(a, x, y, 128, coef, geps, tf)
    slack = n * 2.0**-24 if model == "reference" else 2.0**-40
    for beta, t in enumerate(exact):
        assert (tau[:, beta] >= float(t)).all() and (tau[:, beta] <= float(t) * (1 + slack)).all()
    rho_exact = c.astype(np.float64) @ x.astype(np.float64) - np.einsum(
        "kbi,bi->kb", r.astype(np.float64), y.astype(np.float64).reshape(-1, 128))
    allowance = geps * ((1 + U32) * (a.astype(np.float64) @ np.abs(x.astype(np.float64)))
                        + np.abs(y.astype(np.float64)).reshape(-1, 128).sum(1))  # fmt: skip
    assert (np.abs(rho - rho_exact) <= allowance).all()
    assert passed.all()


def test_hand_traced_chains() -> None:
    """Thread 0 holds columns 0 and 256 of one segment: a.|x| terms 1 and 2^-30.  The
    reference's FP32 round-up chain gives 1 + 2^-23, this build's FP64 sum 1 + 2^-30; with
    coef = 1 and geps = tau_floor = 0, tau is s.  The c . x terms 1 and 2^-30, which a plain
    FP32 sum would round to 1, survive in the reference's Dot2 chain: rho = 1 + 2^-30 in both."""
    n = 512
    a = np.zeros((1, n), np.float32)
    x = np.zeros(n, np.float32)
    c = np.zeros((1, 1, n), np.float32)
    a[0, 0], x[0], a[0, 256], x[256] = 1.0, 1.0, 2.0**-15, 2.0**-15
    c[0, 0, 0], c[0, 0, 256] = 1.0, 2.0**-15
    r = np.ones((1, 1, 1), np.int8)
    y = np.zeros(1, np.float32)
    _, rho_ref, tau_ref = reference_gpu_check(c, a, r, x, y, 1.0, 0.0, 0.0, segments=1)
    _, rho_hip, tau_hip = hip_check(c, a, r, x, y, 1.0, 0.0, 0.0)
    assert tau_ref[0, 0] == 1 + 2.0**-23 and tau_hip[0, 0] == 1 + 2.0**-30
    assert rho_ref[0, 0] == rho_hip[0, 0] == 1 + 2.0**-30
    # Two segments: the terms meet only in the FP64 sum of the partials, which is exact.
    _, _, tau_two = reference_gpu_check(c, a, r, x, y, 1.0, 0.0, 0.0, segments=2)
    assert tau_two[0, 0] == 1 + 2.0**-30


@pytest.mark.parametrize("n", [4096, 14336])
def test_hip_tau_is_never_above_the_reference_gpu_checkers(n: int) -> None:
    """Decode-shaped blocks (W ~ N(0, 0.02) BF16, x ~ N(0, 1)), honest and with the planted
    shortcuts: for every segment count the reference's default rule picks (its 30-SM RTX 5060
    and a 256-CU MI355X, K = 1 and 8 over a Llama layer's blocks) and for 1 .. 16, this build's
    tau is at most the reference's in every block, and the verdicts are equal."""
    W, x, r, c, a = decode_block(n, seed=n + 1)
    coef, geps, tf = constants(n, tree_height(n, 256, 8))
    legit = emulate_gemv_coalesced(W, x, 256)
    outputs = {
        "legit": legit,
        "drop_tail": emulate_gemv(W, x, 256, drop_tail=4),
        "bf16_accumulator": emulate_gemv(W, x, 256, acc_bf16=True),
        "bf16_output": bf16(legit).astype(np.float32),
    }
    layer_blocks = 43008 // 128
    segments = {reference_default_segments(n, k, layer_blocks // 4, sms) for k in (1, 8) for sms in (30, 256)}
    segments |= {1, 2, 3, 4, 8, 16}
    for name, y in outputs.items():
        passed_hip, rho_hip, tau_hip = hip_check(c, a, r, x, y, coef, geps, tf)
        for seg in sorted(segments):
            passed_ref, rho_ref, tau_ref = reference_gpu_check(c, a, r, x, y, coef, geps, tf, seg)
            assert (tau_hip <= tau_ref).all(), (name, seg, float((tau_hip / tau_ref).max()))
            assert np.array_equal(passed_hip, passed_ref), (name, seg)
            assert (np.abs(rho_hip - rho_ref) <= 2.0**-40 * tau_ref).all()
        if name in ("legit", "drop_tail", "bf16_accumulator"):
            assert passed_hip.all() == (name == "legit"), name
