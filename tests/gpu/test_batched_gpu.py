"""Batched decode product Y = X W^T (B >= 16 path): bit-exact against the oracle's model of the
kernel's order, within the proven bound of the exact product, and the wrapper's validation."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.batched import batched_height as oracle_height
from oracle.batched import emulate_batched
from oracle.gemv import e4m3_values
from pck.cuda import batched_height, gemm_batched, pack_batched_weights, quantize_fp8
from pck.fp import bf16, gamma

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf16_tensor(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(DEV)


def _family(rng: np.random.Generator, shape: tuple[int, ...], kind: str) -> np.ndarray:
    if kind == "real_w":
        return bf16(rng.standard_normal(shape) * 0.02)
    if kind == "real_x":
        return bf16(rng.standard_normal(shape))
    if kind == "wide":
        v = (1 + rng.integers(0, 128, shape) / 128.0) * np.exp2(rng.integers(-20, 21, shape))
        v *= rng.choice([-1.0, 1.0], shape)
        v[rng.random(shape) < 0.1] = 0
        return bf16(v)
    if kind == "cancel":
        v = rng.choice([-1.0, 1.0], shape) * np.exp2(rng.integers(-4, 13, shape))
        small = rng.random(shape) < 0.5
        v[small] = bf16(rng.standard_normal(shape) * 1e-4)[small]
        return bf16(v)
    if kind == "tiny":
        v = (1 + rng.integers(0, 128, shape) / 128.0) * np.exp2(rng.integers(-70, -60, shape))
        return bf16(v * rng.choice([-1.0, 1.0], shape))
    raise ValueError(kind)


def _run(W: np.ndarray, X: np.ndarray, packed: bool = False) -> np.ndarray:
    Wt = _bf16_tensor(W)
    Y = gemm_batched(pack_batched_weights(Wt) if packed else Wt, _bf16_tensor(X))
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def _run_codes(codes: np.ndarray, X: np.ndarray, packed: bool) -> np.ndarray:
    Q = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(DEV)
    Y = gemm_batched(pack_batched_weights(Q) if packed else Q, _bf16_tensor(X))
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


SHAPES = [
    (32, 8, 32),     # one chunk: the raw matrix-core step
    (64, 64, 16),
    (33, 24, 7),     # ragged rows, batch below one tile
    (96, 1000, 40),  # n % 8 != 0: element loads
    (128, 4096, 128),
    (64, 512, 256),  # eight batch tiles in one pass
    (40, 136, 300),  # two batch passes
    (1, 4104, 1),
]


@pytest.mark.parametrize(("m", "n", "B"), SHAPES)
@pytest.mark.parametrize("fam", ["real", "wide", "cancel"])
def test_batched_bits_match_model(m: int, n: int, B: int, fam: str) -> None:
    rng = np.random.default_rng(m * 7919 + n * 31 + B)
    W = _family(rng, (m, n), "real_w" if fam == "real" else fam)
    X = _family(rng, (B, n), "real_x" if fam == "real" else fam)
    print(f"batched m={m} n={n} B={B} fam={fam}", flush=True)
    want = emulate_batched(W, X)
    assert _same_bits(_run(W, X), want)
    assert _same_bits(_run(W, X, packed=True), want)


# (m, n, B), all with a packed route (n % 128 == 0, m % 4 == 0): rows past m in the last tile
# (m = 36, 100), segments of an odd number of step pairs shorter than one ring pass (n = 384:
# 3 pairs per wave), one ring pass plus a partial one (n = 1152: 9 pairs), several passes
# (n = 4096), batch tails and several batch passes.
TILE_SHAPES = [(36, 384, 33), (64, 1152, 100), (32, 4096, 300), (100, 2048, 5)]


@pytest.mark.parametrize("shape", [(1, 1), (1, 2), (1, 4), (2, 2), (3, 1)], ids=str)
@pytest.mark.parametrize(("m", "n", "B"), TILE_SHAPES)
def test_every_tile_setting_gives_the_model_bits(shape: tuple[int, int], m: int, n: int, B: int) -> None:
    """Weight and batch tiles per workgroup change only speed: BF16 and FP8 weights, every
    setting (a last row group with one weight tile when two are asked for: m = 36, 100)."""
    from pck.cuda._lib import lib

    rng = np.random.default_rng(m + n + B + 10 * shape[0] + shape[1])
    W = _family(rng, (m, n), "wide")
    X = _family(rng, (B, n), "real_x")
    codes = rng.integers(0, 256, (m, n), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    print(f"batched shape={shape} m={m} n={n} B={B}", flush=True)
    assert pack_batched_weights(_bf16_tensor(W)).packed is not None
    try:
        assert lib().pck_bgemm_set_shape(*shape) == 0
        assert _same_bits(_run(W, X, packed=True), emulate_batched(W, X))
        Qv = e4m3_values()[codes].astype(np.float32)
        assert _same_bits(_run_codes(codes, X, packed=True), emulate_batched(Qv, X))
    finally:
        lib().pck_bgemm_set_shape(0, 0)


# Far more items (R x T tiles) than the GPU holds workgroups, so each workgroup loops over
# several: segments of a whole number of ring passes (the next item's first pairs are loaded
# during the current one's last pass: n = 512 at two tiles, n = 1024 at three), of a partial
# pass (n = 384: the ring is refilled at each item's start), several batch passes with the
# row groups a multiple of 8 (m = 9728: the passes of a row group are items 8 apart), and a
# ragged last row group and batch pass (m = 19252: 602 row tiles, the last group of two).
LOOP_SHAPES = [((2, 2), 19200, 512, 33), ((2, 2), 19200, 384, 64), ((1, 2), 9600, 1024, 100),
               ((1, 4), 9728, 512, 300), ((1, 1), 9612, 512, 70),
               ((3, 1), 19252, 512, 100)]  # fmt: skip


@pytest.mark.parametrize(("shape", "m", "n", "B"), LOOP_SHAPES, ids=str)
def test_workgroups_looping_over_items_give_the_model_bits(shape: tuple[int, int], m: int, n: int,
                                                           B: int) -> None:  # fmt: skip
    """Every output equals the element kernel's (one K-step per load, no item loop, itself
    bit-exact against the model) and a sample (three row tiles by 24 batch rows, an output
    depending only on its own row and batch row) equals the model, BF16 and FP8."""
    from pck.cuda._lib import lib

    rng = np.random.default_rng(m + n + B)
    W = _family(rng, (m, n), "wide")
    X = _family(rng, (B, n), "real_x")
    codes = rng.integers(0, 256, (m, n), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    Qv = e4m3_values()[codes].astype(np.float32)
    tiles = (m + 31) // 32
    sample = sorted({0, tiles // 2 + 1, tiles - 1})
    rows = np.concatenate([np.arange(32 * t, min(32 * t + 32, m)) for t in sample])
    bs = np.unique(np.concatenate([np.arange(8), np.arange(B // 2, B // 2 + 8), np.arange(B - 8, B)]))
    print(f"batched items shape={shape} m={m} n={n} B={B}", flush=True)
    try:
        assert lib().pck_bgemm_set_shape(*shape) == 0
        got = _run(W, X, packed=True)
        got8 = _run_codes(codes, X, packed=True)
    finally:
        lib().pck_bgemm_set_shape(0, 0)
    assert _same_bits(got, _run(W, X))
    assert _same_bits(got8, _run_codes(codes, X, packed=False))
    assert _same_bits(got[np.ix_(bs, rows)], emulate_batched(W[rows], X[bs]))
    assert _same_bits(got8[np.ix_(bs, rows)], emulate_batched(Qv[rows], X[bs]))


@pytest.mark.parametrize("B", [128, 100])
def test_uneven_item_counts_split_into_two_launches_keep_the_bits(B: int) -> None:
    """896 row tiles at four batch tiles (gate/up's shape at B = 128) give 896 looping items
    for 256 workgroups: the built-in shape runs the first 768 row tiles and (1, 2) items the
    last 128, in a second launch writing the same output.  Every output equals the element
    kernel's, and a sample on both sides of the split equals the model, BF16 and FP8."""
    m, n = 28672, 512
    rng = np.random.default_rng(B)
    W = _family(rng, (m, n), "wide")
    X = _family(rng, (B, n), "real_x")
    codes = rng.integers(0, 256, (m, n), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    Qv = e4m3_values()[codes].astype(np.float32)
    print(f"batched split m={m} n={n} B={B}", flush=True)
    got = _run(W, X, packed=True)
    got8 = _run_codes(codes, X, packed=True)
    assert _same_bits(got, _run(W, X))
    assert _same_bits(got8, _run_codes(codes, X, packed=False))
    rows = np.concatenate([np.arange(32 * 767, 32 * 769), np.arange(m - 32, m)])
    bs = np.unique(np.concatenate([np.arange(4), np.arange(B - 4, B)]))
    assert _same_bits(got[np.ix_(bs, rows)], emulate_batched(W[rows], X[bs]))
    assert _same_bits(got8[np.ix_(bs, rows)], emulate_batched(Qv[rows], X[bs]))


@pytest.mark.parametrize(("m", "n", "B"), [(64, 64, 32), (32, 8, 64)])
def test_batched_tiny_magnitudes_match_model(m: int, n: int, B: int) -> None:
    """Products in the FP32 subnormal range; the results stay normal here (exactness of a
    subnormal result is covered by the threshold's floor, not by this model)."""
    rng = np.random.default_rng(5)
    W = _family(rng, (m, n), "tiny")
    X = bf16(rng.standard_normal((B, n)) * 2.0**20)
    assert _same_bits(_run(W, X), emulate_batched(W, X))


@pytest.mark.parametrize(("m", "n", "B"), [(128, 4096, 128), (64, 14336, 16)])
def test_batched_fp8_bits_match_model(m: int, n: int, B: int) -> None:
    gen = torch.Generator().manual_seed(m + n + B)
    Wf = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16)
    Q, _ = quantize_fp8(Wf)
    X = torch.randn(B, n, generator=gen).to(torch.bfloat16)
    print(f"batched fp8 m={m} n={n} B={B}", flush=True)
    Qv = e4m3_values()[Q.view(torch.uint8).numpy()].astype(np.float32)
    want = emulate_batched(Qv, X.float().numpy())
    for packed in (False, True):
        Wq = pack_batched_weights(Q.to(DEV)) if packed else Q.to(DEV)
        Y = gemm_batched(Wq, X.to(DEV))
        torch.cuda.synchronize()
        assert _same_bits(Y.cpu().numpy(), want)


def test_batched_every_fp8_code() -> None:
    """All 256 E4M3FN codes as weights against a few activations (NaN codes give NaN)."""
    codes = np.arange(256, dtype=np.uint8).reshape(32, 8)
    Q = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    X = bf16(np.random.default_rng(1).standard_normal((16, 8)))
    Y = gemm_batched(Q.to(DEV), _bf16_tensor(X))
    torch.cuda.synchronize()
    Qv = e4m3_values()[codes].astype(np.float32)
    assert _same_bits(Y.cpu().numpy(), emulate_batched(Qv, X))


def test_batched_special_values() -> None:
    W = np.zeros((32, 16), np.float32)
    W[0, 0] = np.inf
    W[1, 0], W[1, 1] = np.inf, -np.inf
    W[2, 3] = np.nan
    W[3, :] = bf16(np.float32(3.0e38))
    W[4:, :] = bf16(np.random.default_rng(2).standard_normal((28, 16)))
    X = np.ones((16, 16), np.float32)
    X[5, :] = 2.0
    assert _same_bits(_run(W, X), emulate_batched(W, X))


def test_batched_within_proven_bound() -> None:
    """|Y - X W^T| <= gamma_h sum |w x| with h = batched_height(n), against exact rationals."""
    rng = np.random.default_rng(9)
    m, n, B = 8, 4096, 16
    W = _family(rng, (m, n), "real_w")
    X = _family(rng, (B, n), "real_x")
    Y = _run(W, X)
    h = batched_height(n)
    g = gamma(h)
    for b in range(0, B, 5):
        for i in range(m):
            exact = sum(Fraction(float(W[i, j])) * Fraction(float(X[b, j])) for j in range(n))
            absum = float(np.sum(np.abs(W[i].astype(np.float64) * X[b].astype(np.float64))))
            assert abs(Fraction(float(Y[b, i])) - exact) <= Fraction(g * absum)


def test_batched_height_formula() -> None:
    assert batched_height(8) == 9 + 1 + 1 + 3  # one chunk: one group of one
    assert batched_height(4096) == 9 + 16 + 4 + 3  # 64 chunks per segment: 4 groups of 16
    assert batched_height(14336) == 9 + 16 + 14 + 3  # 224 chunks per segment
    for n in range(1, 40000, 97):
        assert batched_height(n) == oracle_height(n)


def test_batched_writes_into_a_given_output() -> None:
    """gemm_batched(..., out=Y) writes the product's bits into Y and returns it, on both
    routes; a wrong shape, dtype or layout is refused."""
    rng = np.random.default_rng(5)
    W = _family(rng, (96, 512), "real_w")
    X = _family(rng, (40, 512), "real_x")
    Wt, Xt = _bf16_tensor(W), _bf16_tensor(X)
    for w in (Wt, pack_batched_weights(Wt)):
        Y = torch.full((40, 96), float("nan"), dtype=torch.float32, device=DEV)
        got = gemm_batched(w, Xt, out=Y)
        torch.cuda.synchronize()
        assert got is Y
        assert _same_bits(Y.cpu().numpy(), emulate_batched(W, X))
        for bad in (torch.empty(40, 95, device=DEV), torch.empty(40, 96, dtype=torch.float64, device=DEV),
                    torch.empty(96, 40, device=DEV).t()):  # fmt: skip
            with pytest.raises(RuntimeError, match="out must be"):
                gemm_batched(w, Xt, out=bad)


def test_batched_validation_messages() -> None:
    W = torch.zeros(4, 8, dtype=torch.bfloat16, device=DEV)
    X = torch.zeros(2, 8, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        gemm_batched(W.cpu(), X)
    with pytest.raises(RuntimeError, match="bfloat16"):
        gemm_batched(W.float(), X)
    with pytest.raises(RuntimeError, match="shape"):
        gemm_batched(W, X[:, :4].contiguous())
    with pytest.raises(RuntimeError, match="contiguous"):
        gemm_batched(torch.zeros(8, 4, dtype=torch.bfloat16, device=DEV).t(), X)
    assert gemm_batched(W[:0], X).shape == (2, 0)


def test_packed_route_validation_and_fallback() -> None:
    """Shapes without a packed route (n % 128 != 0, m % 4 != 0) keep the plain weights and give
    the model's bits through the element kernel; bad arguments raise."""
    rng = np.random.default_rng(3)
    for m, n in ((33, 128), (32, 60), (32, 320)):
        W = _family(rng, (m, n), "real_w")
        X = _family(rng, (20, n), "real_x")
        bw = pack_batched_weights(_bf16_tensor(W))
        assert bw.packed is None and bw.raw is not None
        assert _same_bits(_run(W, X, packed=True), emulate_batched(W, X))
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        pack_batched_weights(torch.zeros(4, 8, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="BFloat16"):
        pack_batched_weights(torch.zeros(4, 8, device=DEV))
    bw = pack_batched_weights(torch.zeros(4, 8, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(RuntimeError, match="shape"):
        gemm_batched(bw, torch.zeros(2, 16, dtype=torch.bfloat16, device=DEV))


def _packed_layout(bits: np.ndarray) -> np.ndarray:
    """The step-pair layout of `pck_bgemm_pack` restated on the host from (rows, n) BF16 bit
    patterns: tile t, pair p, lane L = 32 h + l holds row 32 t + l, columns 16 p + 4 h .. + 3
    then 16 p + 8 + 4 h .. + 3; rows past the end are zero."""
    rows, n = bits.shape
    tiles, pairs = (rows + 31) // 32, n // 16
    padded = np.zeros((tiles * 32, n), dtype=np.uint16)
    padded[:rows] = bits
    out = np.zeros((tiles, pairs, 64, 8), dtype=np.uint16)
    for h in range(2):
        lanes = slice(32 * h, 32 * h + 32)
        for p in range(pairs):
            block = padded.reshape(tiles, 32, n)
            out[:, p, lanes, 0:4] = block[:, :, 16 * p + 4 * h : 16 * p + 4 * h + 4]
            out[:, p, lanes, 4:8] = block[:, :, 16 * p + 8 + 4 * h : 16 * p + 12 + 4 * h]
    return out.reshape(-1)


@pytest.mark.parametrize("rows,n", [(33, 384), (100, 1024), (128, 4096), (256, 14336)])
def test_activation_pack_layout_aligned_and_8_byte_aligned(rows: int, n: int) -> None:
    """Both BF16 pack routes (16-byte aligned sources go through LDS, 8-byte aligned ones piece
    by piece) write exactly the documented layout, including the zero rows of a ragged tile."""
    from pck.cuda._lib import check, lib, stream_handle

    rng = np.random.default_rng(rows * 7 + n)
    bits = rng.integers(0, 1 << 16, (rows, n), dtype=np.uint16)
    want = _packed_layout(bits)
    flat = torch.from_numpy(bits.view(np.int16).reshape(-1).copy()).to(DEV)
    # the same rows at a 16-byte aligned address and at one 8 bytes past it
    holder = torch.zeros(rows * n + 4, dtype=torch.int16, device=DEV)
    holder[4:] = flat
    for src in (flat, holder[4:]):
        dst = torch.full((want.size,), 0x5555, dtype=torch.int16, device=DEV)
        check(lib().pck_bgemm_pack(0, src.data_ptr(), dst.data_ptr(), rows, n,
                                   stream_handle(torch.device(DEV))), "pack")  # fmt: skip
        got = dst.cpu().numpy().view(np.uint16)
        assert src.data_ptr() % 16 == (0 if src is flat else 8)
        assert np.array_equal(got, want)
