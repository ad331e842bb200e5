"""Pins the template oracle (oracle/template.py) before the HIP templates are compared with it.

Mirrors the reference's tests/agent/test_config.py (default knobs = the coalesced tree,
rows_per_block and unroll change nothing, each exploit changes y as described, the worked
column layout, INT8 groups) and adds closed forms a plausible slip would fail: the two-term
chains of the BF16 accumulator, the halving of BF16-rounded chain sums, exact small-integer
sums, the proven bound gamma_h * sum |w x| at the height each config reports, and hand-made
INT8 groups (ties to even, the clip, an all-zero group, a partial last group).
"""

from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given
from hypothesis import strategies as st

from oracle.gemv import (
    WARP,
    abs_row_sums,
    chain_sums_coalesced,
    emulate_gemv_coalesced,
    halving_sum,
    reference_gemv,
)
from oracle.template import dequantize_rows, emulate, emulate_column, quantize_rows
from pck.agent.column import ColumnConfig, column_space
from pck.agent.config import (
    GROUP,
    THREADS,
    VECS,
    KernelConfig,
    config_index,
    config_space,
    depends_on_x,
    int8_space,
    is_exploit,
    make_config,
    row_space,
    template_flags,
)
from pck.fp import bf16, gamma, tree_height


def problem(m: int, n: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    return bf16(rng.standard_normal((m, n)) * 0.02), bf16(rng.standard_normal(n))


@given(st.sampled_from(THREADS), st.sampled_from(VECS), st.integers(1, 700), st.integers(0, 99))
def test_default_knobs_are_the_coalesced_tree(threads: int, vec: int, n: int, seed: int) -> None:
    W, x = problem(4, n, seed)
    got = emulate(KernelConfig(threads=threads, vec=vec), W, x)
    np.testing.assert_array_equal(got, emulate_gemv_coalesced(W, x, threads, vec))


def test_rows_per_block_splits_the_lanes_and_unroll_changes_nothing() -> None:
    W, x = problem(8, 1000, 0)
    base = emulate(KernelConfig(threads=128), W, x)
    np.testing.assert_array_equal(emulate(KernelConfig(threads=256, rows_per_block=2), W, x), base)
    np.testing.assert_array_equal(emulate(KernelConfig(threads=512, rows_per_block=4), W, x), base)
    np.testing.assert_array_equal(emulate(KernelConfig(threads=128, unroll=4), W, x), base)
    cfg = KernelConfig(threads=512, vec=4, rows_per_block=4)
    assert cfg.threads_per_row == 128 and cfg.tree_height(1000) == tree_height(1000, 128, 4)


def test_bf16_output_and_skipped_tail_are_their_closed_forms() -> None:
    W, x = problem(8, 1000, 1)
    honest = emulate(KernelConfig(), W, x)
    np.testing.assert_array_equal(emulate(KernelConfig(out="bf16"), W, x), bf16(honest))
    # 64 lanes x 8 columns: one full tile of 512 columns, the other 488 are dropped
    Wt = W.copy()
    Wt[:, 512:] = 0
    np.testing.assert_array_equal(
        emulate(KernelConfig(threads=64, skip_tail=True), W, x), emulate(KernelConfig(threads=64), Wt, x)
    )
    # 256 lanes x 8 = 2048 > 1000: no full tile, everything is dropped
    assert not emulate(KernelConfig(skip_tail=True), W, x).any()


def test_bf16_partials_are_the_halving_of_rounded_chain_sums() -> None:
    W, x = problem(6, 900, 2)
    for tpr, vec in ((64, 8), (128, 2), (32, 1)):
        chains = bf16(chain_sums_coalesced(W, x, tpr, vec))
        want = halving_sum(halving_sum(chains.reshape(6, tpr // WARP, WARP)))
        cfg = KernelConfig(threads=tpr * 2, rows_per_block=2, vec=vec, partials="bf16")
        np.testing.assert_array_equal(emulate(cfg, W, x), want)


def test_bf16_accumulator_rounds_after_each_add_but_not_the_first_term() -> None:
    """32 lanes, vec 1, n = 40: lane t adds columns t and t + 32 (columns past 40 are +0), so
    its chain is bf16(p_t + p_{t+32}) exactly, and y halves the 32 chains."""
    rng = np.random.default_rng(3)
    W = bf16(rng.standard_normal((5, 40)))
    x = bf16(rng.standard_normal(40))
    p = np.zeros((5, 64), np.float32)
    p[:, :40] = (W * x).astype(np.float32)
    chains = bf16((p[:, :32] + p[:, 32:]).astype(np.float32))
    want = halving_sum(chains)
    cfg = KernelConfig(threads=64, rows_per_block=2, vec=1, acc="bf16")
    np.testing.assert_array_equal(emulate(cfg, W, x), want)
    # rounding the first term too would differ on these inputs
    wrong = halving_sum(bf16((bf16(p[:, :32]) + p[:, 32:]).astype(np.float32)))
    assert not np.array_equal(wrong, want)


@given(st.sampled_from(row_space()[::7]), st.integers(1, 600), st.integers(0, 99))
def test_honest_variants_meet_the_bound_and_small_integers_are_exact(
    cfg: KernelConfig, n: int, seed: int
) -> None:
    W, x = problem(3, n, seed)
    y = emulate(cfg, W, x)
    if template_flags(cfg) == 0:
        bound = gamma(cfg.tree_height(n)) * abs_row_sums(W, x)
        assert np.all(np.abs(y.astype(np.float64) - reference_gemv(W, x)) <= bound)
    rng = np.random.default_rng(seed)
    Wi = rng.integers(-8, 9, (3, n)).astype(np.float32)
    xi = rng.integers(-8, 9, n).astype(np.float32)
    # Integer sums below 2^24 are exact in FP32; the BF16 roundings are exact below 2^8.
    if not cfg.skip_tail and (template_flags(cfg) == 0 or n * 64 < 256):
        np.testing.assert_array_equal(emulate(cfg, Wi, xi), (Wi @ xi).astype(np.float32))


def test_int8_variant_is_the_fp32_template_on_the_dequantized_weights() -> None:
    rng = np.random.default_rng(5)
    m, n = 7, GROUP + 40
    W = bf16(rng.standard_normal((m, n)).astype(np.float32))
    x = bf16(rng.standard_normal(n).astype(np.float32))
    deq = dequantize_rows(*quantize_rows(W))
    for vec in (1, 4, 8):
        q = KernelConfig(threads=64, vec=vec, weights="int8")
        np.testing.assert_array_equal(emulate(q, W, x), emulate(KernelConfig(threads=64, vec=vec), deq, x))
    y16 = emulate(KernelConfig(threads=64, vec=16, weights="int8"), W, x)
    h = tree_height(n, 64, 16)
    # the products fl(w' x) are not exact: one more rounding per term than the sum's height
    bound = gamma(h + 1) * abs_row_sums(deq, x)
    assert np.all(np.abs(y16.astype(np.float64) - reference_gemv(deq, x)) <= bound)


def test_quantize_rows_on_hand_made_groups() -> None:
    W = np.zeros((3, GROUP + 3), np.float32)
    # row 0: max 127 -> scale 1; halves round to even, negatives too
    W[0, :6] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5]
    # row 1: all zero in group 0 -> scale 1, q = 0; partial group 1 has max 254 -> scale 2
    W[1, GROUP:] = [254.0, -5.0, 1.0]
    # row 2: max |w| = 0.3 -> scale fl(0.3 / 127); w = -0.3 -> -127 exactly
    W[2, 0] = -0.3
    W[2, 1] = 0.15
    Wq, S = quantize_rows(W)
    assert Wq.shape == W.shape and Wq.dtype == np.int8 and S.shape == (3, 2) and S.dtype == np.float32
    assert list(Wq[0, :6]) == [127, 2, 4, -2, -4, 0] and S[0, 0] == 1 and S[0, 1] == 1
    assert S[1, 0] == 1 and not Wq[1, :GROUP].any()
    assert S[1, 1] == 2 and list(Wq[1, GROUP:]) == [127, -2, 0]  # -2.5 -> -2, 0.5 -> 0
    s = np.float32(np.float32(0.3) / np.float32(127))
    assert S[2, 0] == s and Wq[2, 0] == -127
    assert Wq[2, 1] == int(np.rint(np.float32(np.float32(0.15) / s)))
    assert np.abs(Wq).max() <= 127
    deq = dequantize_rows(Wq, S)
    step = np.repeat(S, GROUP, axis=1)[:, : W.shape[1]]
    assert np.all(np.abs(deq - W) <= step / 2 + np.abs(W) * 2.0**-23)


@given(st.sampled_from(column_space()), st.integers(1, 3000), st.integers(0, 99))
def test_column_template_meets_its_bound_unless_it_skips(cfg: ColumnConfig, n: int, seed: int) -> None:
    W, x = problem(4, n, seed)
    y = emulate(cfg, W, x)
    kept = np.where(np.abs(x) < np.float32(cfg.skip_below), 0, x).astype(np.float32)
    bound = gamma(cfg.tree_height(n)) * abs_row_sums(W, kept)
    # skipping a column is zeroing its activation; the rest is within gamma_h
    assert np.all(np.abs(y.astype(np.float64) - reference_gemv(W, kept)) <= bound)


def test_column_tree_follows_the_split_layout() -> None:
    """threads 64 (K = 2 warps) x 4 grid splits over n = 1000: split s owns columns
    [250 s, 250 (s + 1)), warp k every other one of them, summed in order from +0."""
    W, x = problem(8, 1000, 3)
    cfg = ColumnConfig(threads=64, splits=4)
    assert cfg.num_splits == 8 and cfg.tree_height(1000) == 124 + 3
    prod = (W * x).astype(np.float32)
    acc = np.zeros((8, 4, 2), np.float32)
    for j in range(1000):
        s, k = j // 250, (j % 250) % 2
        acc[:, s, k] = (acc[:, s, k] + prod[:, j]).astype(np.float32)
    warps = (acc[:, :, 0] + acc[:, :, 1]).astype(np.float32)
    halves = (warps[:, :2] + warps[:, 2:]).astype(np.float32)
    want = (halves[:, 0] + halves[:, 1]).astype(np.float32)
    np.testing.assert_array_equal(emulate_column(cfg, W, x), want)


def test_column_template_on_small_integers_is_exact_and_skipping_zeroes_columns() -> None:
    rng = np.random.default_rng(4)
    Wi = rng.integers(-8, 9, (16, 777)).astype(np.float32)
    xi = rng.integers(-8, 9, 777).astype(np.float32)
    for cfg in (ColumnConfig(), ColumnConfig(threads=32, vec=2, splits=1), ColumnConfig(splits=64)):
        np.testing.assert_array_equal(emulate_column(cfg, Wi, xi), (Wi @ xi).astype(np.float32))
    xs = xi * np.float32(0.01)  # |x| = 0, 0.01, 0.02, ... : skip_below 0.03 drops 0, +-1, +-2
    skip = ColumnConfig(skip_below=0.03)
    kept = np.where(np.abs(xs) < np.float32(0.03), 0, xs).astype(np.float32)
    np.testing.assert_array_equal(emulate_column(skip, Wi, xs), emulate_column(ColumnConfig(), Wi, kept))


@pytest.mark.parametrize(
    ("kwargs", "match"),
    [
        ({"threads": 100}, "threads"),
        ({"vec": 3}, "vec"),
        ({"vec": 16}, "vec"),
        ({"acc": "fp16"}, "acc"),
        ({"skip_tail": 1}, "skip_tail"),
        ({"threads": 64, "rows_per_block": 4}, "warp"),
        ({"acc": "bf16", "weights": "int8"}, "int8 weights need"),
        ({"weights": "fp8"}, "weights"),
    ],
)
def test_invalid_row_configs_are_rejected(kwargs: dict[str, object], match: str) -> None:
    with pytest.raises(ValueError, match=match):
        KernelConfig(**kwargs)  # type: ignore[arg-type]


def test_config_space_and_helpers() -> None:
    space = config_space()
    assert len(space) == len(set(space)) == 2112 + 672 + 165
    assert len(row_space()) == 2112 and len(column_space()) == 672 and len(int8_space()) == 165
    assert all(config_index(c) == i for i, c in enumerate(space))
    assert KernelConfig().as_dict()["layout"] == "row"
    assert make_config(ColumnConfig().as_dict()) == ColumnConfig()
    assert make_config({"layout": "row", "vec": 4}) == KernelConfig(vec=4)
    assert is_exploit(KernelConfig(skip_tail=True)) and is_exploit(ColumnConfig(skip_below=0.1))
    assert is_exploit(KernelConfig(weights="int8")) and not depends_on_x(KernelConfig(weights="int8"))
    assert not is_exploit(KernelConfig()) and not is_exploit(ColumnConfig())
    assert template_flags(KernelConfig(acc="bf16", out="bf16", skip_tail=True)) == 1 | 4 | 8
    assert KernelConfig(vec=16, weights="int8").tree_height(4096) == tree_height(4096, 256, 16)
    with pytest.raises(ValueError, match="splits"):
        ColumnConfig(splits=3)
    with pytest.raises(ValueError, match="skip_below"):
        ColumnConfig(skip_below=0.5)


def test_models_reject_a_wrong_x_shape() -> None:
    W, x = problem(4, 10, 0)
    with pytest.raises(ValueError, match="shape"):
        emulate(KernelConfig(), W, x[:5])
    with pytest.raises(ValueError, match="shape"):
        emulate_column(ColumnConfig(), W, np.ones(3, np.float32))
