"""`pck.faults`: the output bit flips and the approximate (sharded) top-k the campaigns plant.

flip_bit is checked against the IEEE-754 layout directly (each exponent bit scales by
2^(+-2^(bit-23)), the sign bit negates, mantissa bits move the value by a multiple of its ulp),
for every bit of several values, and is an involution that never touches its input.
sharded_topk is checked against brute force: exact whenever each shard keeps at least k, a
subset of the true candidates otherwise, and wrong on a clustered example.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from pck.faults import flip_bit, sharded_topk


@pytest.mark.parametrize("value", [1.5, -3.25, 1e-20, 6.5e4, 2.0**-126])
def test_every_bit_against_the_ieee_layout(value: float) -> None:
    y = np.array([0.0, value, 7.0], dtype=np.float32)
    v = float(y[1])
    exp = (int(y.view(np.uint32)[1]) >> 23) & 0xFF
    ulp = math.ldexp(1.0, max(exp, 1) - 127 - 23)
    for bit in range(32):
        z = flip_bit(y, 1, bit)
        assert z[0] == 0.0 and z[2] == 7.0 and float(y[1]) == v  # others and the input untouched
        w = float(z[1])
        if bit == 31:
            assert w == -v
        elif bit >= 23:
            delta = 1 << (bit - 23)
            new_exp = exp ^ delta
            if new_exp not in (0, 255) and exp != 0:
                assert w == v * 2.0 ** (new_exp - exp)
        else:
            assert abs(w - v) == math.ldexp(ulp, bit)
        assert flip_bit(z, 1, bit).tobytes() == y.tobytes()


def test_flip_argument_errors() -> None:
    with pytest.raises(TypeError, match="float32"):
        flip_bit(np.ones(2), 0, 3)
    with pytest.raises(ValueError, match="bit"):
        flip_bit(np.ones(2, np.float32), 0, -1)
    with pytest.raises(ValueError, match="bit"):
        flip_bit(np.ones(2, np.float32), 0, 32)


def brute_topk(a: np.ndarray, k: int) -> set[int]:
    return set(sorted(range(a.size), key=lambda i: (-float(a[i]), i))[:k])


@pytest.mark.parametrize("seed", range(5))
def test_sharded_topk_is_exact_with_enough_per_shard(seed: int) -> None:
    rng = np.random.default_rng(seed)
    a = rng.integers(-20, 20, 97).astype(np.float32)  # many ties: the lower index wins
    for k in (1, 5, 17):
        for shards in (1, 3, 8):
            got = sharded_topk(a, k, shards, k)
            assert set(got.tolist()) == brute_topk(a, k) and got.size == k


def test_sharded_topk_misses_a_cluster() -> None:
    a = np.zeros(40, dtype=np.float32)
    a[:6] = [9, 8, 7, 6, 5, 4]  # the top 6 all sit in the first of 4 shards
    got = sharded_topk(a, 6, 4, 2)
    assert set(got.tolist()) != brute_topk(a, 6)
    assert {0, 1} <= set(got.tolist()) and got.size == 6


def test_sharded_topk_argument_errors() -> None:
    a = np.arange(10, dtype=np.float32)
    for k, shards, per in ((0, 1, 1), (11, 1, 1), (3, 0, 1), (3, 2, 0)):
        with pytest.raises(ValueError):
            sharded_topk(a, k, shards, per)
