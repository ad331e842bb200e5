"""pck.cuda.CarriedChecker: the reference's call pattern (GEMVs, then check_many of their
outputs) with the checks carried in later GEMV launches.  Every result is bit-identical to
check_many on the same items; small launches carry nothing; a checker queued twice rides in two
launches; the last checks are flushed; results are refused before a launch took them and
across streams; graph replays reproduce the eager results."""

from __future__ import annotations

import pytest
import torch

from pck.cuda import CarriedChecker, GpuBlockedChecker, check_many, gemv_group, quantize_fp8
from pck.fp import tree_height

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

SHAPES = [(1024, 4096), (512, 14336), (256, 4100)]  # outputs checked each "layer"
CARRIER = (4096, 4096)  # the large launch that carries them


def weights(shapes, seed, fp8=False):  # type: ignore[no-untyped-def]
    gen = torch.Generator().manual_seed(seed)
    out = []
    for m, n in shapes:
        W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
        if fp8:
            W = quantize_fp8(W)[0]
        checker = GpuBlockedChecker(W.to(torch.bfloat16), 128, tree_height(n, 256, 16 if fp8 else 8), generator=gen)
        out.append((W, x, checker))
    return out


def same(a, b) -> None:  # type: ignore[no-untyped-def]
    assert torch.equal(a.passed, b.passed)
    assert torch.equal(a.rho, b.rho)
    assert torch.equal(a.tau, b.tau)


def run_pass(carrier: CarriedChecker, produced, big, layers: int):  # type: ignore[no-untyped-def]
    """``layers`` rounds of: the small GEMVs, the large one, check_many of the small outputs."""
    handles, items = [], []
    for _ in range(layers):
        ys = [carrier.gemv_group([(W, x)])[0] for W, x, _ in produced]
        carrier.gemv_group([(big[0], big[1])])
        step = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
        items.append(step)
        handles.append(carrier.check_many(step))
    return handles, items


@pytest.mark.parametrize("fp8", [False, True])
def test_results_equal_check_many(fp8: bool) -> None:
    produced = weights(SHAPES, seed=1, fp8=fp8)
    big = weights([CARRIER], seed=2, fp8=fp8)[0]
    carrier = CarriedChecker(min_rows=4096)
    handles, items = run_pass(carrier, produced, big, layers=3)
    # the small launches (fewer than min_rows rows) carry nothing; layer i's checks ride in
    # layer i + 1's large launch, and the last layer's are still queued
    assert carrier.pending == len(SHAPES)
    assert all(h.launched for h in handles[0] + handles[1])
    assert not any(h.launched for h in handles[2])
    with pytest.raises(RuntimeError, match="not been launched"):
        handles[2][0].result()
    carrier.flush()
    assert carrier.pending == 0
    for hs, step in zip(handles, items):
        for h, alone in zip(hs, check_many(step)):
            same(h.result(), alone)
            assert h.result().verdict.all()


def test_small_launches_carry_nothing() -> None:
    produced = weights(SHAPES, seed=3)
    carrier = CarriedChecker()  # default min_rows 16384: none of these launches qualifies
    ys = [carrier.gemv_group([(W, x)])[0] for W, x, _ in produced]
    hs = carrier.check_many([(ch, x, y) for (W, x, ch), y in zip(produced, ys)])
    carrier.gemv_group([(W, x) for W, x, _ in produced])
    assert carrier.pending == len(SHAPES) and not any(h.launched for h in hs)
    carrier.flush()
    for h, alone in zip(hs, check_many([(ch, x, y) for (W, x, ch), y in zip(produced, ys)])):
        same(h.result(), alone)


def test_a_checker_queued_twice_rides_in_two_launches() -> None:
    (W, x, ch), = weights([(1024, 4096)], seed=4)
    big = weights([CARRIER], seed=5)[0]
    carrier = CarriedChecker(min_rows=4096)
    y1 = gemv_group([(W, x)])[0]
    x2 = torch.randn(4096, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).cuda()
    y2 = gemv_group([(W, x2)])[0]
    h1, h2 = carrier.check_many([(ch, x, y1), (ch, x2, y2)])
    carrier.gemv_group([(big[0], big[1])])
    assert h1.launched and not h2.launched and carrier.pending == 1
    carrier.gemv_group([(big[0], big[1])])
    assert h2.launched and carrier.pending == 0
    same(h1.result(), check_many([(ch, x, y1)])[0])
    same(h2.result(), check_many([(ch, x2, y2)])[0])


def test_checks_are_not_carried_across_streams() -> None:
    (W, x, ch), = weights([(1024, 4096)], seed=7)
    big = weights([CARRIER], seed=8)[0]
    carrier = CarriedChecker(min_rows=4096)
    y = gemv_group([(W, x)])[0]
    carrier.submit(ch, x, y)
    other = torch.cuda.Stream()
    other.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(other), pytest.raises(RuntimeError, match="another stream"):
        carrier.gemv_group([(big[0], big[1])])
    torch.cuda.current_stream().wait_stream(other)
    carrier.flush()
    with pytest.raises(RuntimeError, match="x must have shape"):
        carrier.submit(ch, x[:100].contiguous(), y)


def test_fp8_scaled_launches_carry_checks() -> None:
    produced = weights(SHAPES, seed=9, fp8=True)
    gen = torch.Generator().manual_seed(10)
    Wb = (torch.randn(*CARRIER, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    Q, s = quantize_fp8(Wb)
    xb = torch.randn(CARRIER[1], generator=gen).to(torch.bfloat16).cuda()
    carrier = CarriedChecker(min_rows=4096)
    ys = [gemv_group([(W, x)])[0] for W, x, _ in produced]
    items = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
    hs = carrier.check_many(items)
    z, y = carrier.gemv_group_fp8_scaled([(Q, xb, s)])
    assert all(h.launched for h in hs)
    for h, alone in zip(hs, check_many(items)):
        same(h.result(), alone)
    assert torch.equal(z[0].view(torch.int32), gemv_group([(Q, xb)])[0].view(torch.int32))


def test_carried_checker_in_a_graph() -> None:
    produced = weights(SHAPES, seed=11)
    big = weights([CARRIER], seed=12)[0]

    def body():  # type: ignore[no-untyped-def]
        carrier = CarriedChecker(min_rows=4096)
        handles, items = run_pass(carrier, produced, big, layers=2)
        carrier.flush()
        return [h.result() for hs in handles for h in hs], items

    eager, eager_items = body()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured, _ = body()
    for _ in range(3):
        for r in captured:
            r.rho.fill_(float("nan"))
            r.tau.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, eager):
            same(a, b)
            assert a.verdict.all()


def test_other_thread_counts_run_the_checks_before_the_gemvs() -> None:
    # At threads != 256 the carried checks run as their own launch just before the GEMVs
    # (same results); the carrying GEMVs keep their own bits at that thread count.
    produced = weights(SHAPES, seed=13)
    big = weights([CARRIER], seed=14)[0]
    carrier = CarriedChecker(threads=128, min_rows=4096)
    ys = [gemv_group([(W, x)])[0] for W, x, _ in produced]
    items = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
    hs = carrier.check_many(items)
    out = carrier.gemv_group([(big[0], big[1])])[0]
    for h, alone in zip(hs, check_many(items)):
        same(h.result(), alone)
    assert torch.equal(out.view(torch.int32), gemv_group([(big[0], big[1])], 128)[0].view(torch.int32))
