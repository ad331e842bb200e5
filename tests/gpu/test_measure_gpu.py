"""The read-stream kernel behind the HBM read ceiling (`pck_read_stream`): it reads every word of
its buffer exactly once, whatever the split into workgroups, so the time it reports is the time
of reading those bytes."""

from __future__ import annotations

import ctypes
import functools

import pytest
import torch

from pck.cuda._lib import lib, stream_handle

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def xor_words(words: torch.Tensor) -> int:
    return functools.reduce(lambda a, b: a ^ b, words.cpu().view(torch.int32).tolist(), 0) & 0xFFFFFFFF


@pytest.mark.parametrize(
    ("words", "groups"),
    [(4, 1), (4 * 1000, 1), (4 * 1000, 7), (4 * 4099, 3), (4 * 100, 300), (1 << 20, 16), (1 << 20, 1)],
)
def test_every_word_is_read_once(words: int, groups: int) -> None:
    gen = torch.Generator().manual_seed(words + groups)
    src = torch.randint(-(2**31), 2**31 - 1, (words,), dtype=torch.int32, generator=gen).cuda()
    sink = torch.full((4 * groups,), -1, dtype=torch.int32, device="cuda")  # one word per wave
    err = lib().pck_read_stream(src.data_ptr(), 4 * words, sink.data_ptr(), groups, stream_handle(src.device))
    assert err == 0
    torch.cuda.synchronize()
    assert xor_words(sink) == xor_words(src)


def test_bad_arguments_are_refused() -> None:
    src = torch.zeros(64, dtype=torch.int32, device="cuda")
    sink = torch.zeros(16, dtype=torch.int32, device="cuda")
    stream = stream_handle(src.device)
    call = lib().pck_read_stream
    assert call(src.data_ptr(), 24, sink.data_ptr(), 4, stream) != 0  # not a multiple of 16
    assert call(src.data_ptr() + 4, 64, sink.data_ptr(), 4, stream) != 0  # misaligned
    assert call(src.data_ptr(), 64, sink.data_ptr(), 0, stream) != 0  # no workgroups
    assert call(ctypes.c_void_p(None), 64, sink.data_ptr(), 4, stream) != 0


def test_cold_timer_times_the_function_not_the_flush() -> None:
    """ColdL2Timer: the flush buffer spans twice L2 plus the MALL; a spin kernel of 2N cycles
    times about twice one of N (the flush before each rep is outside the timed events); the
    reported quantiles are ordered; a 1 GiB device copy runs at a plausible rate."""
    from pck.cuda.timing import ColdL2Timer, cache_bytes, copy_bandwidth_gbps

    timer = ColdL2Timer(warmup=2, reps=12)
    assert timer.flush.numel() >= 2 * cache_bytes() >= 2 * (256 << 20)
    short = timer(lambda: torch.cuda._sleep(2_000_000))
    long = timer(lambda: torch.cuda._sleep(4_000_000))
    for t in (short, long):
        assert 0 < t.p10_ms <= t.median_ms <= t.p90_ms
    assert 1.7 < long.median_ms / short.median_ms < 2.3
    gbps = copy_bandwidth_gbps(ColdL2Timer(1, 5))
    assert 500 < gbps < 16_000
