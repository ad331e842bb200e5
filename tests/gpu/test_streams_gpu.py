"""Concurrent use from two streams (default priority): the kernels keep no state between
calls, so GEMVs with their checks, batched products with the batched checker, and the
membership check enqueued on two streams at once give the bits of the same calls run one after
the other."""

from __future__ import annotations

import pytest
import torch

from pck.cuda import (
    GpuBlockedChecker,
    batched_height,
    check_batched,
    check_many,
    gemm_batched,
    gemv_coalesced,
    pack_batched_weights,
)
from pck.fp import tree_height
from pck.member import check_members

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def _bits(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.float64:
        return t.view(torch.int64)
    return t.view(torch.int32) if t.dtype == torch.float32 else t


def _work(seed: int):  # type: ignore[no-untyped-def]
    """One stream's work: two GEMVs checked at b = 128, a batched product (B = 64) checked
    column by column, and a membership check; returns a function that enqueues it on the
    current stream and returns every output."""
    g = torch.Generator().manual_seed(seed)
    W1 = (torch.randn(4096, 4096, generator=g) * 0.02).to(torch.bfloat16).cuda()
    W2 = (torch.randn(1024, 14336, generator=g) * 0.02).to(torch.bfloat16).cuda()
    x1 = torch.randn(4096, generator=g).to(torch.bfloat16).cuda()
    x2 = torch.randn(14336, generator=g).to(torch.bfloat16).cuda()
    c1 = GpuBlockedChecker(W1, 128, tree_height(4096, 256, 8), generator=g)
    c2 = GpuBlockedChecker(W2, 128, tree_height(14336, 256, 8), generator=g)
    Wb = (torch.randn(2048, 4096, generator=g) * 0.02).to(torch.bfloat16).cuda()
    Wp = pack_batched_weights(Wb)
    X = torch.randn(64, 4096, generator=g).to(torch.bfloat16).cuda()
    cb = GpuBlockedChecker(Wb, 128, batched_height(4096), generator=g)
    logits = (torch.randn(32, 151936, generator=g) * 3).cuda()
    tokens = logits.argmax(dim=1)
    top_k = torch.full((32,), 40, device="cuda")
    top_p = torch.full((32,), 0.9, device="cuda", dtype=torch.float64)
    host_k = top_k.cpu().numpy()

    def run() -> list[torch.Tensor]:
        y1, y2 = gemv_coalesced(W1, x1), gemv_coalesced(W2, x2)
        r1, r2 = check_many([(c1, x1, y1), (c2, x2, y2)])
        Y = gemm_batched(Wp, X)
        (rb,) = check_batched([(cb, X, Y)])
        m = check_members(logits, tokens, top_k=top_k, top_p=top_p, top_k_host=host_k)
        outs = [y1, y2, Y, m["ok"], m["above"], m["mass_above"]]
        for r in (r1, r2, rb):
            outs += [r.passed, r.rho, r.tau]
        return outs

    return run


def test_two_streams_at_once_give_the_serial_bits() -> None:
    runs = [_work(21), _work(22)]
    print("two streams: serial reference", flush=True)
    serial = [run() for run in runs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        print(f"two streams: concurrent round {rep}", flush=True)
        got = []
        for s, run in zip(streams, runs):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                got.append(run())
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for a_list, b_list in zip(got, serial):
            for i, (a, b) in enumerate(zip(a_list, b_list)):
                assert torch.equal(_bits(a), _bits(b)), (rep, i)
    for outs in serial:  # every check passed and every token was a member
        assert bool(outs[3].all())
        assert all(bool(outs[k].all()) for k in (6, 9, 12))
