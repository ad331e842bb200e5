"""Detection campaign on one MI355X: the reference's protocol for false alarms, bit-flip
detection and planted shortcuts (`harness/campaign.py:1-16`, `harness/numerics_sim.py:48-110`),
run through this build's HIP GEMVs and checkers.

1. False alarms (`false_alarms`, reference `harness/campaign.py:56-110`).  One fused
   Llama-3-8B decode layer (q/k/v 6144 x 4096, o 4096 x 4096, gate/up 28672 x 4096, down
   4096 x 14336, W ~ N(0, 0.02) BF16) is run with fresh activations every trial through the
   coalesced tree and the naive tree (T = 256), and every output block is checked by the
   blocked checker with K sign draws (K = 8), the signs redrawn every ``redraw`` trials.
   Activations cycle through four families: Gaussian, Student-t with 3 degrees of freedom,
   mixed-scale (N(0, 1) times 2^k, k uniform in -20 .. 20) and outliers (1% of channels times
   100).  A block check is one (sign draw, block) pair; reported per block size and kernel:
   block checks, alarms, and the largest |rho| / tau seen, overall and per family.
2. Bit flips (`bit_flips`, reference `harness/campaign.py:112-145`).  A 4096 x 4096 GEMV; each
   trial draws a fresh x, flips one bit of one random output of every block, and counts the
   blocks the checker rejects; per block size (64, 128), family (Gaussian, Student-t,
   outliers), K (1, 4) and bit (mantissa 12 .. 22, exponent 23, 27, 30, sign 31).
3. Shortcuts at K = 8 (`shortcuts_b1`, `shortcuts_batched`; reference
   `harness/numerics_sim.py:58-80`, which checks each planted kernel with 8 sign draws).  The
   reference's planted shortcuts -- a dropped reduction tail of 4 columns, a BF16 running
   accumulator, BF16 partial sums before the tree, a BF16 output -- and one exponent or sign
   flip per block, for every projection of a batch-1 layer (BF16 and FP8 weights) and for the
   batched down projection (B = 128 and 256), checked at K = 8 for b = 64, 128 and 256.
   An output (a batched column) counts as caught when any of its blocks is rejected; every
   escape is reported with its largest |rho| / tau.

Activations and weights are drawn on the GPU from seeded generators (the signs from a seeded
CPU generator, as `GpuBlockedChecker` draws them), so a run is repeatable.  Everything here
calls the library through `pck.cuda`; nothing reads the oracle.

Run: python campaign.py [--quick] [--target 10000000] [--seed 0]
"""

from __future__ import annotations

import argparse
import json
import math
import sys
import time
from pathlib import Path
from typing import Any

ROOT = Path(__file__).resolve().parent
if str(ROOT / "proof-carrying-kernels_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "proof-carrying-kernels_amd"))

THREADS = 256
FUSED_LAYER = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096),
               ("down", 4096, 14336)]  # fmt: skip
SPLIT_LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
               ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]  # fmt: skip
FAMILIES = ("gauss", "student-t", "mixed-scale", "outliers")
BITS = (12, 14, 16, 18, 20, 22, 23, 27, 30, 31)
SHORTCUTS = ("drop_tail_4", "bf16_accumulator", "bf16_partials", "bf16_output")
FLIPS = ("exponent_flip", "sign_flip")


def activations(family: str, count: int, n: int, gen: Any) -> Any:
    """``count`` activation vectors of length n (BF16, on the GPU) from one family.

    Student-t(3) is Z / sqrt(chi2_3 / 3) with chi2_3 a sum of three squared normals; the
    outlier channels of a row are its n // 100 smallest keys of a uniform draw."""
    import torch

    dev = torch.device("cuda")
    z = torch.randn(count, n, generator=gen, device=dev)
    if family == "student-t":
        chi2 = torch.randn(count, n, 3, generator=gen, device=dev).square().sum(dim=2)
        z = z / torch.sqrt(chi2 / 3.0)
    elif family == "mixed-scale":
        k = torch.randint(-20, 21, (count, n), generator=gen, device=dev)
        z = z * torch.exp2(k.float())
    elif family == "outliers":
        keys = torch.rand(count, n, generator=gen, device=dev)
        idx = keys.argsort(dim=1)[:, : max(1, n // 100)]
        z.scatter_(1, idx, z.gather(1, idx) * 100.0)
    elif family != "gauss":
        raise ValueError(f"unknown activation family {family!r}")
    return z.to(torch.bfloat16).contiguous()


def _kernels() -> dict[str, tuple[Any, int]]:
    from pck.cuda import gemv_coalesced, gemv_naive

    return {"coalesced": (gemv_coalesced, 8), "naive": (gemv_naive, 1)}


def false_alarms(block: int, checks: int, target: int, redraw: int, seed: int,
                 kernels: tuple[str, ...] = ("coalesced", "naive")) -> dict[str, Any]:  # fmt: skip
    """Part 1: at least ``target`` block checks per kernel on honest outputs."""
    import torch

    from pck.cuda import GpuBlockedChecker, check_many, gemv_group
    from pck.fp import tree_height

    gen = torch.Generator(device="cuda").manual_seed(seed)
    signs = torch.Generator().manual_seed(seed)
    weights = [(torch.randn(m, n, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
               for _, m, n in FUSED_LAYER]  # fmt: skip
    per_trial = checks * sum(m // block for _, m, _ in FUSED_LAYER)
    trials = max(1, math.ceil(target / per_trial))
    redraw = max(len(FAMILIES), redraw - redraw % len(FAMILIES))
    out: dict[str, Any] = {}
    for kname in kernels:
        gemv, vec = _kernels()[kname]
        alarms = torch.zeros((), dtype=torch.int64, device="cuda")
        worst = torch.zeros(len(FAMILIES), dtype=torch.float64, device="cuda")
        t0 = time.time()
        done = 0
        while done < trials:
            span = min(redraw, trials - done)
            checkers = [GpuBlockedChecker(W, block, tree_height(W.shape[1], THREADS, vec),
                                          checks=checks, generator=signs) for W in weights]  # fmt: skip
            per_family = -(-span // len(FAMILIES))
            xs = {f: [activations(f, per_family, W.shape[1], gen) for W in weights] for f in FAMILIES}
            for t in range(span):
                f = (done + t) % len(FAMILIES)
                xt = [X[t // len(FAMILIES)] for X in xs[FAMILIES[f]]]
                if kname == "coalesced":
                    ys = gemv_group(list(zip(weights, xt)), THREADS)
                else:
                    ys = [gemv(W, x, THREADS) for W, x in zip(weights, xt)]
                for res in check_many(list(zip(checkers, xt, ys))):
                    alarms += (~res.passed).sum()
                    worst[f] = torch.maximum(worst[f], (res.rho.abs() / res.tau).max())
            done += span
            del checkers, xs
        torch.cuda.synchronize()
        w = worst.tolist()
        out[kname] = {
            "block_checks": trials * per_trial,
            "alarms": int(alarms),
            "max_rho_over_tau": float(f"{max(w):.3e}"),
            "by_family": {f: float(f"{v:.3e}") for f, v in zip(FAMILIES, w)},
            "seconds": round(time.time() - t0, 1),
        }
    return out


def bit_flips(trials: int, seed: int, blocks=(64, 128), families=("gauss", "student-t", "outliers"),
              checks_list=(1, 4)) -> dict[str, Any]:  # type: ignore[no-untyped-def]  # fmt: skip
    """Part 2: share of single-bit flips caught, per block size, family, K and bit.  The
    ``trials`` outputs of a cell are computed by grouped launches of the coalesced tree (eight
    GEMVs a launch, the bits of `gemv_coalesced`), flipped, and checked eight outputs a launch
    by the single-vector checker kernel (the verdicts of `check_many`)."""
    import torch

    from pck.cuda import GpuBlockedChecker, gemv_group
    from pck.cuda.checker import _check_columns
    from pck.fp import tree_height

    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    signs = torch.Generator().manual_seed(seed + 1)
    m = n = 4096
    W = (torch.randn(m, n, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    height = tree_height(n, THREADS, 8)
    out: dict[str, Any] = {}
    for block in blocks:
        nb = m // block
        base = torch.arange(0, m, block, device="cuda")
        for family in families:
            cell: dict[str, list[float]] = {}
            for checks in checks_list:
                checker = GpuBlockedChecker(W, block, height, checks=checks, generator=signs)
                rates = []
                for bit in BITS:
                    X = activations(family, trials, n, gen)
                    Y = torch.stack([y for t in range(0, trials, 8)
                                     for y in gemv_group([(W, X[i]) for i in range(t, min(t + 8, trials))],
                                                         THREADS)])  # fmt: skip
                    rows = base + torch.randint(0, block, (trials, nb), generator=gen, device="cuda")
                    mask = -(2**31) if bit == 31 else 1 << bit
                    Yi = Y.view(torch.int32)
                    Yi.scatter_(1, rows, Yi.gather(1, rows) ^ mask)
                    v = _check_columns(checker, X, Y).verdict  # (nb, trials)
                    rates.append(round(int((~v).sum()) / (trials * nb), 4))
                cell[f"K{checks}"] = rates
            out.setdefault(f"b{block}", {})[family] = cell
    return {"bits": list(BITS), "trials_per_cell": trials, "shape": [m, n], "rates": out}


def naive_shortcut(W, x, acc_bf16: bool = False, partial_bf16: bool = False):  # type: ignore[no-untyped-def]
    """y = W x in the naive tree's order (T = 256 lanes, lane t sums the contiguous chunk
    [t c, (t + 1) c), then neighbour pairs) with one of the reference's planted shortcuts
    (`src/pck/gemv.py:14-57`): the running sum rounded to BF16 after every add, or each lane's
    chain sum rounded to BF16 before the tree.  Torch ops on the GPU (a fault generator)."""
    import torch

    m, n = W.shape
    lanes = 256
    chunk = -(-n // lanes)
    p = torch.zeros(m, lanes * chunk, device=W.device)
    p[:, :n] = W.float() * x.float()
    p = p.view(m, lanes, chunk)
    acc = p[:, :, 0].clone()
    for j in range(1, chunk):
        acc = acc + p[:, :, j]
        if acc_bf16:
            acc = acc.bfloat16().float()
    if partial_bf16:
        acc = acc.bfloat16().float()
    while acc.size(1) > 1:
        acc = acc[:, 0::2] + acc[:, 1::2]
    return acc[:, 0].contiguous()


def planted_faults(W, x, y, gen, block: int):  # type: ignore[no-untyped-def]
    """The planted faults for one GEMV output y = W x (reference `harness/numerics_sim.py:58-64`,
    `harness/campaign.py:131-135`): a dropped reduction tail of 4 columns (the honest kernel on
    W with them zeroed), the BF16 accumulator and BF16 partials shortcuts, the BF16-rounded
    output, and one flip per block of a random exponent bit (23-30) or of the sign bit of a
    random output.  ``gen`` is a CPU generator."""
    import torch

    from pck.cuda import gemv_group

    Wz = W.clone()
    Wz.view(torch.uint8 if W.element_size() == 1 else torch.int16)[:, -4:] = 0
    out = {
        "drop_tail_4": gemv_group([(Wz, x)], THREADS)[0],
        "bf16_accumulator": naive_shortcut(W, x, acc_bf16=True),
        "bf16_partials": naive_shortcut(W, x, partial_bf16=True),
        "bf16_output": y.bfloat16().float(),
    }
    blocks = y.numel() // block
    base = torch.arange(0, y.numel(), block, device=y.device)
    for kind, lo, hi in (("exponent_flip", 23, 31), ("sign_flip", 31, 32)):
        rows = base + torch.randint(0, block, (blocks,), generator=gen).to(y.device)
        bit = torch.randint(lo, hi, (blocks,), generator=gen).to(y.device)
        z = y.clone()
        zi = z.view(torch.int32)
        zi[rows] ^= torch.bitwise_left_shift(torch.ones_like(bit, dtype=torch.int32), bit.int())
        out[kind] = z
    return out


def _tally(stats: dict, kind: str, res: Any, columns: bool = False) -> None:  # type: ignore[type-arg]
    """Adds one checked output (or, with ``columns``, every column of a batched output) to
    the per-kind counts: outputs caught (some block rejected) of outputs, and for each escape
    its largest |rho| / tau over checks and blocks."""
    import torch

    v = res.verdict  # (nb,) or (nb, B)
    ratio = res.rho.abs() / res.tau
    if columns:
        caught = (~v).any(dim=0)
        worst = ratio.amax(dim=(0, 1))
    else:
        caught = (~v).any().reshape(1)
        worst = ratio.amax().reshape(1)
    c = stats.setdefault(kind, {"outputs": 0, "caught": 0, "escaped_max_rho_over_tau": []})
    c["outputs"] += int(caught.numel())
    c["caught"] += int(caught.sum())
    missed = worst[~caught]
    if missed.numel():
        c["escaped_max_rho_over_tau"].extend(round(float(r), 4) for r in missed.tolist())


def shortcuts_b1(seed: int, blocks=(64, 128, 256), checks: int = 8) -> dict[str, Any]:  # type: ignore[no-untyped-def]
    """Part 3, batch 1: every projection of one Llama-3-8B layer (BF16 and FP8 weights), the
    planted faults of `planted_faults`, checked at K = ``checks`` for each block size; also the
    honest outputs (false alarms).  Per weight type and block size: {"by_kind", "false_alarms"}."""
    import torch

    from pck.cuda import GpuBlockedChecker, gemv_group, quantize_fp8
    from pck.fp import tree_height

    gen = torch.Generator(device="cuda").manual_seed(seed + 2)
    cpu = torch.Generator().manual_seed(seed + 2)
    out: dict[str, Any] = {}
    for fp8 in (False, True):
        entry = {f"b{b}": {"by_kind": {}, "false_alarms": 0} for b in blocks}
        for _, m, n in SPLIT_LAYER:
            W = (torch.randn(m, n, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
            x = torch.randn(n, generator=gen, device="cuda").to(torch.bfloat16)
            if fp8:
                W = quantize_fp8(W)[0]
            y = gemv_group([(W, x)], THREADS)[0]
            checked = W.to(torch.bfloat16) if fp8 else W
            h = tree_height(n, THREADS, 16 if fp8 else 8)
            for b in blocks:
                ch = GpuBlockedChecker(checked, b, h, checks=checks, generator=cpu)
                entry[f"b{b}"]["false_alarms"] += int((~ch.check(x, y).passed).sum())
                for kind, yy in planted_faults(W, x, y, cpu, b).items():
                    _tally(entry[f"b{b}"]["by_kind"], kind, ch.check(x, yy))
                del ch
        out["fp8" if fp8 else "bf16"] = entry
    return out


def batched_faults(Wq, X, Y, fp8: bool, block: int, rng):  # type: ignore[no-untyped-def]
    """The planted faults of one batched product Y = X Wq^T (B, m): BF16 outputs, the top
    exponent bit of a random output and the sign of the largest output of every (block,
    column), a product that drops the last 4 columns of every reduction, BF16 partial sums
    of the 8 K segments, and a BF16 accumulator rounded after every 32 columns.  ``rng`` is a
    NumPy generator."""
    import torch

    from pck.cuda import gemm_batched

    B, m = Y.shape
    n = X.size(1)
    out = {"bf16_output": Y.to(torch.bfloat16).float()}
    for bit, kind in ((30, "exponent_flip"), (31, "sign_flip")):
        y = Y.clone()
        blocks = m // block
        if bit == 31:
            sel = y.abs().view(B, blocks, block).argmax(dim=2)
        else:
            sel = torch.from_numpy(rng.integers(0, block, (B, blocks))).cuda()
        rows = sel + torch.arange(0, m, block, device=y.device)
        bits = y.view(torch.int32)
        bits.scatter_(1, rows, bits.gather(1, rows) ^ (1 << bit))
        out[kind] = y
    Wf = Wq.float().t()  # (n, m) exact values of the BF16 or E4M3 weights
    Xf = X.float()
    Wz = Wq.clone()
    Wz.view(torch.uint8 if fp8 else torch.int16)[:, -4:] = 0
    out["drop_tail_4"] = gemm_batched(Wz, X)
    seg = -(-n // 8)
    yp = torch.zeros_like(Y)
    for j in range(0, n, seg):
        yp += (Xf[:, j : j + seg] @ Wf[j : j + seg]).to(torch.bfloat16).float()
    out["bf16_partials"] = yp
    ya = torch.zeros_like(Y)
    for j in range(0, n, 32):
        ya = (ya + Xf[:, j : j + 32] @ Wf[j : j + 32]).to(torch.bfloat16).float()
    out["bf16_accumulator"] = ya
    return out


def shortcuts_batched(seed: int, batches=(128, 256), blocks=(64, 128), checks: int = 8) -> dict[str, Any]:  # type: ignore[no-untyped-def]
    """Part 3, batched: the down projection (4096 x 14336) on the matrix cores at batch B, BF16
    and FP8 weights, the planted faults of `batched_faults`, every column checked at K =
    ``checks``.  Per batch, weight type and block size: {"by_kind", "false_alarms"}."""
    import numpy as np
    import torch

    from pck.cuda import GpuBlockedChecker, batched_height, check_batched, gemm_batched, quantize_fp8

    gen = torch.Generator(device="cuda").manual_seed(seed + 3)
    cpu = torch.Generator().manual_seed(seed + 3)
    rng = np.random.default_rng(seed + 3)
    m, n = 4096, 14336
    W = (torch.randn(m, n, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    Q = quantize_fp8(W)[0]
    out: dict[str, Any] = {}
    for B in batches:
        X = torch.randn(B, n, generator=gen, device="cuda").to(torch.bfloat16)
        for fp8, Wq in ((False, W), (True, Q)):
            Y = gemm_batched(Wq, X)
            entry: dict[str, Any] = {}
            for b in blocks:
                ch = GpuBlockedChecker(Wq.to(torch.bfloat16), b, batched_height(n), checks=checks,
                                       generator=cpu)  # fmt: skip
                stats: dict = {}  # type: ignore[type-arg]
                honest = check_batched([(ch, X, Y)])[0]
                for kind, yy in batched_faults(Wq, X, Y, fp8, b, rng).items():
                    _tally(stats, kind, check_batched([(ch, X, yy)])[0], columns=True)
                entry[f"b{b}"] = {"by_kind": stats, "false_alarms": int((~honest.passed).sum())}
                del ch
            out[f"B{B}_{'fp8' if fp8 else 'bf16'}"] = entry
    return out


def summarize_shortcuts(part: dict[str, Any]) -> dict[str, Any]:
    """Compact per-kind figures of a shortcut part: "caught/outputs" per kind, the escapes'
    largest |rho| / tau per kind, and the false alarms on the honest outputs."""
    out: dict[str, Any] = {}
    for key, entry in part.items():
        for bkey, cell in entry.items():
            kinds = cell["by_kind"]
            row: dict[str, Any] = {k: f"{c['caught']}/{c['outputs']}" for k, c in kinds.items()}
            row["escapes"] = {k: c["escaped_max_rho_over_tau"] for k, c in kinds.items()
                              if c["escaped_max_rho_over_tau"]}  # fmt: skip
            row["false_alarms"] = cell["false_alarms"]
            out.setdefault(key, {})[bkey] = row
    return out


def contract_summary(res: dict[str, Any]) -> dict[str, Any]:
    """The campaign's figures for one line: per block size and kernel, block checks, alarms and
    the largest |rho| / tau (overall and per family); the bit-flip detection rates; and per
    shortcut case and block size, the caught outputs per kind with every escape's |rho| / tau."""
    fa = {bkey: {k: {"block_checks": v["block_checks"], "alarms": v["alarms"],
                     "max_rho_over_tau": v["max_rho_over_tau"], "by_family": v["by_family"]}
                 for k, v in per.items()}
          for bkey, per in res["false_alarms"].items()}  # fmt: skip
    flips = res["bit_flips"]
    return {
        "checks": res["checks"],
        "false_alarms": fa,
        "bit_flips": {"bits": flips["bits"], "trials_per_cell": flips["trials_per_cell"]} | flips["rates"],
        "shortcuts_b1": summarize_shortcuts(res["shortcuts_b1"]),
        "shortcuts_batched_down": summarize_shortcuts(res["shortcuts_batched_down"]),
        "seconds": res["seconds"],
    }


def run(target: int = 10_000_000, redraw: int = 100, flip_trials: int = 200, seed: int = 0,
        checks: int = 8, quick: bool = False) -> dict[str, Any]:  # fmt: skip
    """All three parts; ``quick`` shrinks them to a smoke run."""
    if quick:
        target, redraw, flip_trials = 20_000, 4, 5
    t0 = time.time()
    res: dict[str, Any] = {"checks": checks, "seed": seed}
    res["false_alarms"] = {f"b{b}": false_alarms(b, checks, target, redraw, seed) for b in (128, 64)}
    print(f"[campaign] false alarms done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["bit_flips"] = bit_flips(flip_trials, seed)
    print(f"[campaign] bit flips done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["shortcuts_b1"] = shortcuts_b1(seed, checks=checks)
    res["shortcuts_batched_down"] = shortcuts_batched(seed, checks=checks)
    res["seconds"] = round(time.time() - t0, 1)
    print(f"[campaign] shortcuts done ({res['seconds']:.0f} s)", file=sys.stderr, flush=True)
    return res


def main() -> None:
    ap = argparse.ArgumentParser(description="False-alarm, bit-flip and shortcut campaign.")
    ap.add_argument("--target", type=int, default=10_000_000, help="block checks per kernel")
    ap.add_argument("--checks", type=int, default=8, help="K for the false-alarm and shortcut parts")
    ap.add_argument("--redraw", type=int, default=100, help="trials between sign redraws")
    ap.add_argument("--flip-trials", type=int, default=200)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--quick", action="store_true", help="small smoke run")
    args = ap.parse_args()
    res = run(args.target, args.redraw, args.flip_trials, args.seed, args.checks, args.quick)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
