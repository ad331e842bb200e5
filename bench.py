"""Benchmark of the decode hot path on one MI355X (BASELINE.json's metric and configs).

A step is one Llama-3-8B decode layer at batch 1 through the hot path: the seven projections
(q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down 4096x14336) as four launches (q, k, v
grouped; o; gate, up grouped; down), with all seven outputs checked by the trusted blocked
checker at block b = 128, K = 1.  Weights are random (the reference's generator:
N(0, 0.02) BF16, x ~ N(0, 1) BF16) and rotate over several distinct layer copies whose total
exceeds L2 + MALL, so every step streams its weights from HBM, as decoding through a model does.

A 32-layer decode pass (the depth of Llama-3-8B) cycling over the layer copies is captured once
in a HIP graph per mode and replayed, as a decode loop replays its captured model.  The modes
are replayed in alternating rounds, max(7, steps / 32) rounds whatever --steps is (3 with
--quick), and each figure is the median round.  Modes (BF16 and FP8 layers):
  gemv_only          the four launches, nothing checked
  carried (b = 128, 256)  every output checked by the bank checker inside the next layer's
                     gate/up launch (pck_gemv_group_check, bit-identical to a standalone check);
                     the pass ends with one standalone check of the last gate, up and down
  carried_check_many (b = 128)  the reference's call pattern (GEMVs, then check_many of the
                     layer's outputs) through pck.cuda.CarriedChecker, which carries each
                     layer's checks in the next gate/up launch
  inpass (b = 128, 256)   the GEMVs also write per-row checksums in the same pass
                     (pck_gemv_group_rowsums) and the row-sum checks ride as above
  serial, side_stream     one standalone check per layer, inline or on a second stream
The headline `value` is the carried mode at b = 128.  A B = 1 fault campaign plants the
reference's shortcuts (dropped tail, BF16 accumulator / partials / output) and per-block
exponent and sign flips in every output of one layer and reports caught outputs and false
alarms for the bank and row-sum checks at b = 128 and 256, K = 1, plus two faults planted
inside the producing in-pass launch.  The detection campaign of `campaign.py` (the reference's
protocol at K = 8: >= 10^7 honest block checks per kernel and block size, per-bit flip rates,
every shortcut at batch 1 and on the batched down projection) runs in the default section too.

Printed: one compact JSON line on stdout (the contract line) and the full per-section figures
as one `[bench detail]` JSON line on stderr.  The contract line holds:
  value          GEMV algorithmic bytes per step / time per replayed step, checker included
  checker_overhead_pct, fp8_checker_overhead_pct   every mode above against gemv_only
  faults_b1      the K = 1 campaign's caught outputs, false alarms and each escape's
                 |rho| / tau; `inlaunch`: faults planted inside the producing launch
  detection_k8   the K = 8 campaign: alarms and the largest |rho| / tau per activation family,
                 per-bit flip detection rates, caught shortcut outputs with every escape
  membership     the top-k / top-p membership check, 256 x 151,936 logits
  vllm_plugin    the plugin wrapper's cost per step at the same size, beside the check alone
  batched        B = 128 and 256: products, checker overhead (one checker call per layer, and
                 one per two layers), caught faulty columns (with the largest |rho| / tau of
                 any column that escaped), hipBLASLt's time
  roofline       the dominant kernel (the BF16 tree GEMV instance used by q/k/v, o, gate/up):
                 algorithmic bytes per launch / its mean launch duration, from HIP events on
                 the launch stream around a graph that replays those launches back to back
                 over every layer copy, against 8 TB/s; traffic = its HBM bytes per launch
                 from two rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE), as recorded in
                 the committed summary named by traffic_source
  cpu_baseline   the oracle's CPU model of the same work (coalesced-tree GEMV + CPU blocked
                 checker) timed on this host on a bounded sample, one core (the all-core C
                 model in cpu_baseline_all_cores_gbps, the FP8 layer in fp8_cpu_baseline_gbps)
The detail line adds the set-sampling checker, the agent's GEMV templates over the same layer
and the read-only stream ceilings: the long stream (hbm_read_ceiling_gbps) and one launch over
each GEMV launch's bytes (size_matched_read_us; pct_of_size_matched_read is their sum over the
layer's time).

Run: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--quick]
                     [--section all|b1|templates|members|batched|campaign]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Any

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "proof-carrying-kernels_amd"))

HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth
TRAFFIC_PROFILE = ROOT / "profiles" / "gemv_tree_llama3_8b_decode_layer_hbm_traffic.md"


def recorded_traffic() -> int | None:
    """HBM bytes per launch of the dominant kernel, as recorded from the two counter passes
    (FETCH_SIZE, WRITE_SIZE, calibrated against a 2 GiB read and fill) in the committed
    rocprofv3 summary; None if that summary is absent."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    for line in text.splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None
LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]  # fmt: skip
LAUNCHES = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",))]
THREADS = 256
BLOCK = 128


def gemv_bytes(m: int, n: int, weight_bytes: int) -> int:
    """Algorithmic bytes of one GEMV: weights, x (BF16) and y (FP32), the reference's formula
    (harness/bench_gemv.py:74, harness/bench_fp8.py:56)."""
    return weight_bytes * m * n + 2 * n + 4 * m


BLOCKS = (128, 256)  # checker block sizes measured (rows per checksum)


def build_layers(copies: int, fp8: bool, gen):  # type: ignore[no-untyped-def]
    """``copies`` layer copies; layer[name] = {"W", "x", "s", "bank": {b: GpuBlockedChecker},
    "rows": {b: RowSumChecker}} for each projection and checker block b (FP8: W holds the
    E4M3 codes Q and s the row scales of `quantize_fp8`; BF16: s is None)."""
    import torch

    from pck.cuda import GpuBlockedChecker, RowSumChecker, quantize_fp8
    from pck.fp import tree_height

    vec = 16 if fp8 else 8
    layers = []
    for _ in range(copies):
        layer = {}
        for name, m, n in LAYER:
            W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
            x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
            s = None
            if fp8:
                W, s = quantize_fp8(W)
            h = tree_height(n, THREADS, vec)
            checked = W.to(torch.bfloat16) if fp8 else W  # FP8: the bound is on Q itself
            layer[name] = {
                "W": W,
                "x": x,
                "s": s,
                "bank": {b: GpuBlockedChecker(checked, b, h, generator=gen) for b in BLOCKS},
                "rows": {b: RowSumChecker(m, n, b, h, generator=gen) for b in BLOCKS},
            }
            del checked
        layers.append(layer)
    return layers


def pairs(layer, names):  # type: ignore[no-untyped-def]
    return [(layer[n]["W"], layer[n]["x"]) for n in names]


def run_step(layer, with_check: bool, events=None):  # type: ignore[no-untyped-def]
    """One decode layer; with ``with_check`` the seven outputs are checked by one standalone
    bank-checker launch (b = 128); with ``events`` a list receiving (launch, start, end)."""
    import torch

    from pck.cuda import check_many, gemv_group

    outs = {}
    for launch, names in LAUNCHES:
        if events is not None:
            start = torch.cuda.Event(enable_timing=True)
            start.record()
        ys = gemv_group(pairs(layer, names), THREADS)
        if events is not None:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            events.append((launch, start, end))
        outs.update(zip(names, ys))
    if with_check:
        if events is not None:
            start = torch.cuda.Event(enable_timing=True)
            start.record()
        results = check_many([(layer[n]["bank"][BLOCK], layer[n]["x"], outs[n]) for n, _, _ in LAYER])
        if events is not None:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            events.append(("check", start, end))
        return outs, results
    return outs, None


# Modes of the batch-1 pass.  gemv: the GEMVs alone.  serial / side_stream: one standalone
# bank-checker launch per layer after its GEMVs, on the same stream / on a side stream
# overlapping the next layer (the reference's modes).  carried: the bank checks ride in later
# GEMV launches.  carried_api: the reference's call pattern (the layer's GEMVs, then
# check_many of its seven outputs) through pck.cuda.CarriedChecker, which carries each layer's
# checks in the next gate/up launch and flushes the last layer's at the end.  inpass: the GEMVs
# compute their row sums in the same pass and the row-sum checks ride in later launches (no
# bank read).  inpass_sums: the in-pass GEMVs with no checks (the cost of the sums alone).  A
# _b256 suffix: checker block b = 256 instead of 128.
MODES = ("gemv", "serial", "side_stream", "carried", "carried_api", "carried_b256", "inpass",
         "inpass_b256", "inpass_sums")  # fmt: skip
# FP8 only, with the row scales applied (y = s z).  gemv_scale_after: the GEMVs, then one
# elementwise multiply per output (the reference's order).  gemv_scaled: the GEMVs with the
# multiply in their epilogue (pck_gemv_group_fp8_scaled).  carried_scaled: the carried checks
# riding in the scaled launches.
FP8_MODES = MODES + ("gemv_scale_after", "gemv_scaled", "carried_scaled")

# In the carried and in-pass modes the gate_up launch of layer L also checks every output
# finished since the previous gate_up: the previous layer's gate, up and down and this layer's
# q, k, v and o; the other launches carry nothing, and the pass ends with one standalone check
# of the last layer's gate, up and down.  ("prev", name) refers to the previous layer's output.
# gate_up is the launch with many more workgroups than the GPU holds at once (3,584 at
# threads 256), so the dispatcher fills the CUs that finish early and the carried checks add
# about their bytes; in a launch that fits in one round (down: 512), each CU that hosts a
# check finishes last and the launch waits for it.
CARRIES = {
    "qkv": (),
    "o": (),
    "gate_up": (("prev", "gate"), ("prev", "up"), ("prev", "down"), ("this", "q"), ("this", "k"),
                ("this", "v"), ("this", "o")),
    "down": (),
}
LAST_CHECKED = ("gate", "up", "down")  # the pass's final standalone check


def carried_pass(layers, depth: int, block: int, inpass: bool, checks: bool = True,  # type: ignore[no-untyped-def]
                 scaled: bool = False):  # fmt: skip
    """One decode pass of ``depth`` layers whose checks ride in later launches: bank checks
    (pck_gemv_group_check; with ``scaled``, FP8 launches that also write y = s z,
    pck_gemv_group_fp8_scaled) or, with ``inpass``, row-sum checks of in-pass GEMVs
    (pck_gemv_group_rowsums).  Returns every check result."""
    from pck.cuda import (check_many, gemv_group_check, gemv_group_fp8_scaled, gemv_group_rowsums,
                          rowsum_check_many)  # fmt: skip

    results = []
    prev = None  # (layer, outputs, sums) of the previous layer
    for i in range(depth):
        layer = layers[i % len(layers)]
        outs, sums = {}, {}
        for launch, names in LAUNCHES:
            items = []
            for which, name in CARRIES[launch] if checks else ():
                src = prev if which == "prev" else (layer, outs, sums)
                if src is not None:
                    owner, produced, produced_sums = src
                    if inpass:
                        items.append((owner[name]["rows"][block], produced_sums[name], produced[name]))
                    else:
                        items.append((owner[name]["bank"][block], owner[name]["x"], produced[name]))
            if inpass:
                ys, ss, res = gemv_group_rowsums(pairs(layer, names), items, THREADS)
                sums.update(zip(names, ss))
            elif scaled:
                triples = [(layer[n]["W"], layer[n]["x"], layer[n]["s"]) for n in names]
                ys, _, res = gemv_group_fp8_scaled(triples, items, THREADS)
            else:
                ys, res = gemv_group_check(pairs(layer, names), items, THREADS)
            results.extend(res)
            outs.update(zip(names, ys))
        prev = (layer, outs, sums)
    if checks:
        owner, produced, produced_sums = prev
        if inpass:
            results.extend(rowsum_check_many([(owner[n]["rows"][block], produced_sums[n], produced[n])
                                              for n in LAST_CHECKED]))  # fmt: skip
        else:
            results.extend(check_many([(owner[n]["bank"][block], owner[n]["x"], produced[n])
                                       for n in LAST_CHECKED]))  # fmt: skip
    return results


def capture(layers, mode: str, depth: int):  # type: ignore[no-untyped-def]
    """One HIP graph holding a decode pass of ``depth`` layers (cycling over the layer copies)
    in ``mode`` (see MODES and FP8_MODES).  Only this library's kernels are captured, and in
    gemv_scale_after torch's elementwise multiply (no memset, no library reduction).  Returns (graph, the pass's check results and outputs)."""
    import torch

    from pck.cuda import CarriedChecker, check_many, gemv_group, gemv_group_fp8_scaled

    def body():  # type: ignore[no-untyped-def]
        if mode == "carried_api":
            carrier = CarriedChecker(THREADS)
            handles = []
            for i in range(depth):
                layer = layers[i % len(layers)]
                outs = {}
                for _, names in LAUNCHES:
                    outs.update(zip(names, carrier.gemv_group(pairs(layer, names))))
                handles.extend(carrier.check_many([(layer[n]["bank"][BLOCK], layer[n]["x"], outs[n])
                                                   for n, _, _ in LAYER]))  # fmt: skip
            carrier.flush()
            return [h.result() for h in handles]
        if mode.startswith(("carried", "inpass")):
            block = 256 if mode.endswith("_b256") else BLOCK
            return carried_pass(layers, depth, block, mode.startswith("inpass"), mode != "inpass_sums",
                                mode == "carried_scaled")  # fmt: skip
        keep = []
        if mode in ("gemv_scale_after", "gemv_scaled"):
            for i in range(depth):
                layer = layers[i % len(layers)]
                for _, names in LAUNCHES:
                    if mode == "gemv_scaled":
                        triples = [(layer[n]["W"], layer[n]["x"], layer[n]["s"]) for n in names]
                        keep.extend(gemv_group_fp8_scaled(triples, (), THREADS)[1])
                    else:
                        zs = gemv_group(pairs(layer, names), THREADS)
                        keep.extend(torch.mul(layer[n]["s"], z) for n, z in zip(names, zs))
            return keep
        cap = torch.cuda.current_stream()
        for i in range(depth):
            layer = layers[i % len(layers)]
            outs, res = run_step(layer, mode == "serial")
            keep.append(outs)
            if res is not None:
                keep.extend(res)
            if mode == "side_stream":
                ready = torch.cuda.Event()
                ready.record(cap)
                side.wait_event(ready)
                with torch.cuda.stream(side):
                    keep.extend(check_many([(layer[n]["bank"][BLOCK], layer[n]["x"], outs[n]) for n, _, _ in LAYER]))
        if mode == "side_stream":
            done = torch.cuda.Event()
            done.record(side)
            cap.wait_event(done)
        return keep

    side = torch.cuda.Stream()
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        body()  # warm the allocator outside capture
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        keep = body()
    torch.cuda.synchronize()
    return graph, keep


def timed_modes(graphs: dict, depth: int, rounds: int) -> dict:  # type: ignore[type-arg]
    """ms per layer of each captured pass: one warm replay each, then ``rounds`` rounds that
    replay every pass once in turn; the median round per pass.  Alternating the passes gives
    each the same clocks and cache state."""
    import torch

    for graph in graphs.values():
        graph.replay()
    torch.cuda.synchronize()
    times: dict = {mode: [] for mode in graphs}  # type: ignore[type-arg]
    for _ in range(rounds):
        for mode, graph in graphs.items():
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            times[mode].append(start.elapsed_time(end) / depth)
    return {mode: statistics.median(t) for mode, t in times.items()}


def honest_verdicts(keep) -> tuple[int, int]:  # type: ignore[no-untyped-def]
    """(blocks checked, blocks rejected) over the CheckResults among ``keep``."""
    from pck.cuda import CheckResult

    results = [r for r in keep if isinstance(r, CheckResult)]
    checked = sum(int(r.passed.numel()) for r in results)
    rejected = sum(int((~r.passed).sum()) for r in results)
    return checked, rejected


def b1_modes(layers, depth: int, rounds: int, modes=MODES) -> tuple[dict, dict]:  # type: ignore[no-untyped-def]
    """ms per layer of every mode in ``modes`` (alternating rounds) and the honest-run verdict
    counts."""
    captured = {mode: capture(layers, mode, depth) for mode in modes}
    ms = timed_modes({mode: graph for mode, (graph, _) in captured.items()}, depth, rounds)
    verdicts = {}
    for mode, (_, keep) in captured.items():
        checked, rejected = honest_verdicts(keep)
        expect = 0 if mode.startswith("gemv") or mode == "inpass_sums" else 7 * depth
        n_results = sum(1 for r in keep if hasattr(r, "passed"))
        assert n_results == expect, (mode, n_results)
        assert rejected == 0, f"{mode}: the checker rejected {rejected} honest blocks"
        verdicts[mode] = checked
    del captured
    return ms, verdicts


def dominant_launch_ms(layers, reps: int, inpass: bool = False) -> tuple[float, int]:  # type: ignore[no-untyped-def]
    """Mean duration of the dominant kernel's launches (the q/k/v, o and gate/up groups; with
    ``inpass`` the in-pass kernel, row sums included) replayed back to back from one graph over
    every layer copy, timed with HIP events on the stream the launches run on (each replay on
    its own; the median replay, so that one disturbed replay does not move the figure), and
    their mean algorithmic bytes."""
    import torch

    from pck.cuda import gemv_group, gemv_group_rowsums

    dom = [launch for launch in LAUNCHES if launch[0] != "down"]

    def launches() -> None:
        for layer in layers:
            for _, names in dom:
                if inpass:
                    gemv_group_rowsums(pairs(layer, names), (), THREADS)
                else:
                    gemv_group(pairs(layer, names), THREADS)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launches()
    nbytes = sum(gemv_bytes(m, n, 2) for name, m, n in LAYER for _, names in dom if name in names)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]  # fmt: skip
    for start, end in events:
        start.record()
        g.replay()
        end.record()
    torch.cuda.synchronize()
    per_replay = statistics.median(start.elapsed_time(end) for start, end in events)
    return per_replay / (len(dom) * len(layers)), nbytes // len(dom)


def timed(layers, steps: int, warmup: int, with_check: bool, per_kernel: bool):  # type: ignore[no-untyped-def]
    """(ms per step, {launch: [ms per launch]}) over ``steps`` steps after ``warmup``."""
    import torch

    for i in range(warmup):
        run_step(layers[i % len(layers)], with_check)
    events: list = [] if per_kernel else None  # type: ignore[assignment]
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        run_step(layers[i % len(layers)], with_check, events)
    end.record()
    torch.cuda.synchronize()
    per_launch: dict[str, list[float]] = {}
    for name, s, e in events or []:
        per_launch.setdefault(name, []).append(s.elapsed_time(e))
    return start.elapsed_time(end) / steps, per_launch


def fault_campaign_b1(layer, seed: int) -> dict:  # type: ignore[no-untyped-def]
    """BASELINE config 4, reference-parity reading (batch 1), on one layer copy: each of the
    seven outputs, honest and with every planted fault of `campaign.planted_faults`, checked
    by the bank checker and by the row-sum checker of the in-pass path, at b = 128 and 256,
    K = 1 (the production setting; the K = 8 protocol is `campaign.py`'s).  Per checker and
    kind: outputs caught (some block rejected) of outputs, faulty blocks caught, false alarms
    (honest blocks rejected), and each escaped output's largest |rho| / tau.

    The planted outputs are checked against the honest launch's row sums, so they test the
    row-sum check on faults that arise after the products (reductions, partials, output).
    Two further kinds plant the fault inside the producing in-pass launch, so that y and its
    row sums come from the same faulty launch: a dropped tail of 4 columns (the launch run on
    W with those columns zeroed) and a wrong activation vector (the launch run on another x).
    These are reported apart, under ``inlaunch``: the bank check must catch them; the row-sum
    check cannot, since d moves with y."""
    import torch

    from campaign import planted_faults
    from pck.cuda import check_many, gemv_group_rowsums, rowsum_check_many

    gen = torch.Generator().manual_seed(seed)
    stats: dict = {}
    inlaunch: dict = {}
    honest_blocks = 0

    def count(c: dict, res, faulty=None) -> None:  # type: ignore[no-untyped-def]
        v = res.verdict
        c["outputs"] += 1
        if faulty is None:  # honest output
            c["false_alarms"] += int((~v).sum())
            return
        caught = bool((~v).any())
        c["outputs_caught"] += int(caught)
        c["faulty_blocks"] += int(faulty.sum())
        c["faulty_blocks_caught"] += int((faulty & ~v).sum())
        c["false_alarms"] += int((~faulty & ~v).sum())
        if not caught:
            c["escaped"].append(round(float((res.rho.abs() / res.tau).max()), 4))

    def cell(d: dict, *keys: str) -> dict:  # type: ignore[type-arg]
        for k in keys[:-1]:
            d = d.setdefault(k, {})
        return d.setdefault(keys[-1], {"outputs": 0, "outputs_caught": 0, "faulty_blocks": 0,
                                       "faulty_blocks_caught": 0, "false_alarms": 0, "escaped": []})  # fmt: skip

    for name, _, n in LAYER:
        ent = layer[name]
        W, x = ent["W"], ent["x"]
        (y,), (sums,), _ = gemv_group_rowsums([(W, x)], (), THREADS)
        Wz = W.clone()
        Wz.view(torch.uint8 if W.element_size() == 1 else torch.int16)[:, -4:] = 0
        x2 = torch.randn(n, generator=gen).to(torch.bfloat16).to(x.device)
        (yz, y2), (sz, s2), _ = gemv_group_rowsums([(Wz, x), (W, x2)], (), THREADS)
        for b in BLOCKS:
            bank, rows = ent["bank"][b], ent["rows"][b]
            cases = {"honest": y} | planted_faults(W, x, y, gen, b)
            for kind, yy in cases.items():
                faulty = None if kind == "honest" else (yy.view(-1, b) != y.view(-1, b)).any(dim=1)
                if kind == "honest" and b == BLOCK:
                    honest_blocks += y.numel() // b
                count(cell(stats, f"b{b}", "bank", kind), check_many([(bank, x, yy)])[0], faulty)
                count(cell(stats, f"b{b}", "rowsum", kind), rowsum_check_many([(rows, sums, yy)])[0], faulty)
            for kind, yy, ss in (("drop_tail_4", yz, sz), ("wrong_x", y2, s2)):
                faulty = (yy.view(-1, b) != y.view(-1, b)).any(dim=1)
                count(cell(inlaunch, f"b{b}", "bank", kind), check_many([(bank, x, yy)])[0], faulty)
                count(cell(inlaunch, f"b{b}", "rowsum", kind), rowsum_check_many([(rows, ss, yy)])[0], faulty)

    def summarize(per_block: dict, honest: bool) -> dict:  # type: ignore[type-arg]
        out = {}
        for bkey, per in per_block.items():
            for checker, kinds in per.items():
                planted = {k: v for k, v in kinds.items() if k != "honest"}
                out[f"{checker}_{bkey}"] = {
                    "outputs_caught": f"{sum(v['outputs_caught'] for v in planted.values())}/"
                                      f"{sum(v['outputs'] for v in planted.values())}",
                    "escapes": {k: v["escaped"] for k, v in planted.items() if v["escaped"]},
                    "false_alarms": sum(v["false_alarms"] for v in kinds.values()),
                } if honest else {k: f"{v['outputs_caught']}/{v['outputs']}" for k, v in planted.items()}
        return out

    return {"summary": summarize(stats, True), "inlaunch": summarize(inlaunch, False),
            "by_kind": stats, "inlaunch_by_kind": inlaunch, "honest_blocks_b128": honest_blocks}


def membership(copies: int = 4, reps: int = 20) -> dict:
    """The membership check on BASELINE config 5: 256 x 151,936 FP32 logits ~ N(0, 3) with 8 hot
    tokens per row at +10..+20, top-k 50, top-p 0.9, 1% of rows given an out-of-set token.  The
    kernel is launched with prepared arguments over ``copies`` logits buffers (more than the
    MALL holds), timed with events; the verdicts are checked (planted rows flagged, no false
    alarm).  GB/s counts the logits read once (155.6 MB per launch)."""
    import numpy as np
    import torch

    from pck.cuda._lib import check, lib, stream_handle
    from pck.fp import next_up
    from pck.member import member_eps32

    rows, vocab = 256, 151_936
    g = torch.Generator(device="cuda").manual_seed(0)
    dev = torch.device("cuda")
    bufs = []
    for _ in range(copies):
        lv = torch.randn(rows, vocab, generator=g, device=dev) * 3
        hot = torch.randint(0, vocab, (rows, 8), generator=g, device=dev)
        lv.scatter_add_(1, hot, 10 + 10 * torch.rand(rows, 8, generator=g, device=dev))
        bufs.append(lv)
    top = bufs[0].topk(60, dim=1)
    tokens = top.indices[:, 0].clone()  # the argmax: in every top-k / top-p set
    planted = torch.zeros(rows, dtype=torch.bool, device=dev)
    planted[:: rows // (rows // 100)][: rows // 100] = True  # 1% of rows
    tokens = torch.where(planted, top.indices[:, 55], tokens)  # 55 larger logits: outside top-50
    k = torch.full((rows,), 50, dtype=torch.long, device=dev)
    p = torch.full((rows,), 0.9, dtype=torch.float64, device=dev)
    ok = torch.empty(rows, dtype=torch.bool, device=dev)
    above = torch.empty(rows, dtype=torch.long, device=dev)
    mass = torch.empty(rows, dtype=torch.float64, device=dev)
    slack = next_up(1e-4 + member_eps32(vocab))
    stream = stream_handle(dev)

    def launch(buf: torch.Tensor) -> None:
        check(lib().pck_check_members(buf.data_ptr(), rows, vocab, tokens.data_ptr(), k.data_ptr(),
                                      p.data_ptr(), None, slack, 50, 1, ok.data_ptr(),
                                      above.data_ptr(), mass.data_ptr(), stream), "members")  # fmt: skip

    launch(bufs[0])
    torch.cuda.synchronize()
    flagged = ~ok
    assert bool((flagged == planted).all()), "membership verdicts differ from the planted faults"
    for i in range(3):
        launch(bufs[i % copies])
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(reps):
        launch(bufs[i % copies])
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    nbytes = rows * vocab * 4
    # CPU baseline: the oracle's FP64 per-row reference on 8 rows, scaled to the same metric
    from oracle.member import check_member

    host = bufs[0][:8].cpu().numpy()
    toks = tokens[:8].cpu().numpy()
    t0 = time.perf_counter()
    for i in range(8):
        check_member(host[i], int(toks[i]), 50, 0.9)
    cpu_s = (time.perf_counter() - t0) / 8 * rows
    return {
        "workload": "256 x 151936 fp32 logits, top-k 50, top-p 0.9, 1% planted out-of-set tokens",
        "ms": round(ms, 5),
        "gbps": round(nbytes / (ms / 1e3) / 1e9, 1),
        "pct_of_peak": round(100 * nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 2),
        "planted_caught": int(planted.sum()),
        "false_alarms": int((flagged & ~planted).sum()),
        "cpu_baseline": {
            "value": round(nbytes / cpu_s / 1e9, 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": "oracle check_member (FP64, NumPy) on 8 of the 256 rows, scaled to 256",
        },
    }


def plugin_step(reps: int = 50) -> dict:
    """Per-step cost of the vLLM plugin's wrapper (`pck.vllm_plugin.install`) at B = 256,
    V = 151,936 (config 5).  A scripted stand-in with vLLM 0.33's ``_sample_random`` signature
    returns fixed tokens (the argmax of each row), so the difference between the wrapped and
    the bare method is the wrapper: the copy of the logits, one membership launch that adds
    into the device totals, and the host bookkeeping.  Times are wall clock over ``reps``
    back-to-back steps (host issue and device work together), plus the host time to issue
    them and event times of the copy and of the membership launch alone.  The reference
    measured its wrapper inside a real vLLM decode step: 22.1% of the step, about 0.9 ms of
    dispatch (harness/bench_vllm_checker_out.txt:4-5); vLLM is not installed here."""
    import json as _json
    import tempfile
    from types import SimpleNamespace

    import numpy as np
    import torch

    from pck.member import launch_check, new_totals
    from pck.vllm_plugin import install

    rows, vocab = 256, 151_936
    dev = torch.device("cuda")
    g = torch.Generator(device="cuda").manual_seed(1)
    logits = torch.randn(rows, vocab, generator=g, device=dev) * 3
    tokens = logits.argmax(dim=1)
    top_k = torch.full((rows,), 50, dtype=torch.long, device=dev)
    top_p = torch.full((rows,), 0.9, dtype=torch.float32, device=dev)
    temperature = torch.ones(rows, dtype=torch.float32, device=dev)
    idx = torch.arange(rows, device=dev)
    idx_np = np.arange(rows)

    class Scripted:
        sampling_states = SimpleNamespace(temperature=SimpleNamespace(gpu=temperature),
                                          top_k=SimpleNamespace(np=np.full(rows, 50)))  # fmt: skip

        def _sample_random(self, lg, ix, ix_np, pos, tk, tp, topp_only, fused):  # type: ignore[no-untyped-def]
            return tokens, lg

    log = Path(tempfile.mkdtemp()) / "pck_sampling_check.jsonl"
    wrapped_cls = type("Wrapped", (Scripted,), {})
    stats = install(wrapped_cls, log, every=16)

    def steps(sampler, n: int) -> tuple[float, float]:  # type: ignore[no-untyped-def]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            sampler._sample_random(logits, idx, idx_np, idx, top_k, top_p, False, False)
        issued = time.perf_counter() - t0
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3, issued / n * 1e3

    def events(fn, n: int) -> float:  # type: ignore[no-untyped-def]
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    bare, wrapped = Scripted(), wrapped_cls()
    steps(bare, 5)
    steps(wrapped, 5)
    bare_ms = statistics.median(steps(bare, reps)[0] for _ in range(5))
    runs = [steps(wrapped, reps) for _ in range(5)]
    wrapped_ms = statistics.median(r[0] for r in runs)
    issue_ms = statistics.median(r[1] for r in runs)
    totals = new_totals(dev)
    check_ms = events(lambda: launch_check(logits, tokens, top_k, top_p, None, 1e-4, np.full(rows, 50),
                                           temperature=temperature, temperature_index=idx,
                                           totals=totals, outputs=False), reps)  # fmt: skip
    clone_ms = events(lambda: logits.clone(), reps)
    stats.flush()
    last = _json.loads(log.read_text().splitlines()[-1])
    assert last["rows"] == stats.steps * rows and last["rejected"] == 0, last
    return {
        "workload": "vLLM 0.33 _sample_random stand-in, 256 x 151936 fp32 logits, top-k 50, top-p 0.9",
        "wrapper_ms_per_step": round(wrapped_ms - bare_ms, 5),
        "wrapped_step_ms": round(wrapped_ms, 5),
        "bare_step_ms": round(bare_ms, 5),
        "host_issue_ms_per_step": round(issue_ms, 5),
        "check_members_ms": round(check_ms, 5),
        "logits_copy_ms": round(clone_ms, 5),
        "steps_logged": last["steps"],
        "reference": "22.1% of a vLLM decode step, ~0.9 ms dispatch (harness/bench_vllm_checker_out.txt:4-5)",
    }


SAMPLING_REFERENCE_MS = {  # harness/bench_sampling_out.txt:6-13 (RTX 5060, cold L2, median)
    "B1": {"topk_checker": 0.0253, "topp_checker": 0.0666},
    "B8": {"topk_checker": 0.0378, "topp_checker": 0.1649},
}


def sampling_checker(reps: int = 200) -> dict:
    """The set-sampling checker as the reference's harness/bench_sampling.py times it: V =
    151,936, k = 50, p = 0.9, logits ~ N(0, 3) at batch 1 and 8, each call timed on a cold L2
    and MALL (median of ``reps``), the whole Python call included (scratch allocation and the
    three launches), next to the untrusted samplers it checks.  A selection with one wrong
    index must fail."""
    import torch

    from pck.cuda import check_topk_gpu, check_topp_gpu, topk_sample, topp_select
    from pck.cuda.timing import ColdL2Timer

    vocab, k, p = 151_936, 50, 0.9
    timer = ColdL2Timer(20, reps)
    gen = torch.Generator(device="cuda").manual_seed(5)
    out: dict = {"workload": f"V = {vocab}, top-k {k}, top-p {p}, logits ~ N(0, 3), cold L2 + MALL"}
    for batch in (1, 8):
        logits = torch.randn(batch, vocab, generator=gen, device="cuda") * 3
        selected, _ = topk_sample(logits, k)
        nucleus, lengths = topp_select(logits, p)
        assert check_topk_gpu(logits, selected, k).passed.all(), "top-k checker false alarm"
        assert check_topp_gpu(logits, nucleus, lengths, p, tol=1e-5).passed.all(), "top-p checker false alarm"
        bad = selected.clone()
        bad[:, 0] = nucleus[:, -1]  # the smallest logit of each row instead of a top-k one
        assert not check_topk_gpu(logits, bad, k).passed.any(), "planted top-k fault missed"
        times = {
            "topk_checker": timer(lambda: check_topk_gpu(logits, selected, k)),  # noqa: B023
            "topp_checker": timer(lambda: check_topp_gpu(logits, nucleus, lengths, p)),  # noqa: B023
            "topk_sampler": timer(lambda: topk_sample(logits, k)),  # noqa: B023
            "topp_selection": timer(lambda: topp_select(logits, p)),  # noqa: B023
        }
        out[f"B{batch}"] = {name: round(t.median_ms, 4) for name, t in times.items()}
        out[f"B{batch}"]["mean_nucleus"] = round(float(lengths.double().mean()), 1)
    out["reference_rtx5060_ms"] = SAMPLING_REFERENCE_MS
    return out


BATCHED_LAUNCHES = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]  # fmt: skip
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense BF16 matrix peak


def batched_layer(batches=(128, 256), copies: int = 2, depth: int = 32, reps: int = 7) -> dict:
    """BASELINE config 4 read literally: a Llama-3-8B decode layer at batch B = 128 and 256 on
    the matrix cores (four packed launches: q/k/v, o, gate/up, down; BF16 and FP8 weights),
    every column of every output checked by one batched checker call per layer (b = 128,
    K = 1, the batched product's tree height), or by one call per two layers (their eight
    outputs).  32-layer passes over ``copies`` layer copies (more than the MALL holds) are
    captured in a HIP graph and replayed.  Reported per B and weight type: ms per layer with
    and without the checker, TFLOP/s (2 B sum(m n) per layer),
    hipBLASLt's time for the same products (torch.mm, not bit-reproducible) and a fault
    campaign per kind (BF16 outputs, exponent and sign flips, a dropped reduction tail, BF16
    partial sums, a BF16 accumulator): planted faults caught and false alarms."""
    import numpy as np
    import torch

    from campaign import batched_faults
    from pck.cuda import GpuBlockedChecker, batched_height, check_batched, gemm_batched
    from pck.cuda import pack_batched_weights, quantize_fp8

    gen = torch.Generator().manual_seed(1)
    flops_per_row = 2 * sum(m * n for _, m, n in BATCHED_LAUNCHES)
    raw, layers = [], {False: [], True: []}
    for _ in range(copies):
        raw_layer, l16, l8 = [], [], []
        for _, m, n in BATCHED_LAUNCHES:
            W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
            Q, _ = quantize_fp8(W)
            h = batched_height(n)
            l16.append((pack_batched_weights(W), GpuBlockedChecker(W, BLOCK, h, generator=gen)))
            l8.append((pack_batched_weights(Q),
                       GpuBlockedChecker(Q.to(torch.bfloat16), BLOCK, h, generator=gen)))  # fmt: skip
            raw_layer.append(W)
        raw.append(raw_layer)
        layers[False].append(l16)
        layers[True].append(l8)

    def run_layer(layer, xs, with_check: bool, side=None):  # type: ignore[no-untyped-def]
        """One layer; with ``side`` its check runs on that stream after the layer's products
        (an event orders it), overlapping the next layer's products, as the reference's
        SideStreamChecker overlaps checks (src/pck/cuda/checker.py:174-215)."""
        ys = [gemm_batched(Wp, X) for (Wp, _), X in zip(layer, xs)]
        if not with_check:
            return ys, None
        if side is None:
            return ys, check_batched([(ch, X, Y) for (_, ch), X, Y in zip(layer, xs, ys)])
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            res = check_batched([(ch, X, Y) for (_, ch), X, Y in zip(layer, xs, ys)])
        return ys, res

    def side_pass(ls, xs, side):  # type: ignore[no-untyped-def]
        out = [run_layer(ls[i % copies], xs, True, side) for i in range(depth)]
        torch.cuda.current_stream().wait_stream(side)  # the pass ends after its last check
        return out

    def pair_pass(ls, xs):  # type: ignore[no-untyped-def]
        """Every output checked, two layers' eight outputs per checker call (after the second
        layer's products): the same checks, each launch pair spread over twice the work."""
        out, held = [], []
        for i in range(depth):  # depth is even
            layer = ls[i % copies]
            ys = [gemm_batched(Wp, X) for (Wp, _), X in zip(layer, xs)]
            held += [(ch, X, Y) for (_, ch), X, Y in zip(layer, xs, ys)]
            if i % 2 == 1:
                out.append(check_batched(held))
                held = []
        return out

    def capture_pass(fn):  # type: ignore[no-untyped-def]
        warm = torch.cuda.Stream()
        warm.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(warm):
            fn()
        torch.cuda.current_stream().wait_stream(warm)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        return g

    def time_passes(graphs: list) -> list[float]:  # type: ignore[type-arg]
        """ms per layer of each captured pass: the passes replayed in turn, ``reps`` rounds,
        the median per pass (so a drift of the clocks does not favour either)."""
        times: list[list[float]] = [[] for _ in graphs]
        for _ in range(reps):
            for i, g in enumerate(graphs):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                g.replay()
                b.record()
                torch.cuda.synchronize()
                times[i].append(a.elapsed_time(b) / depth)
        return [statistics.median(t) for t in times]

    out = {}
    for B in batches:
        xs = [torch.randn(B, n, generator=gen).to(torch.bfloat16).cuda() for _, _, n in BATCHED_LAUNCHES]
        entry = {"batch": B}
        for fp8 in (False, True):
            ls = layers[fp8]
            ys, res = run_layer(ls[0], xs, True)
            assert all(bool(r.passed.all()) for r in res), "batched checker rejected an honest output"
            side = torch.cuda.Stream()
            g_gemm = capture_pass(lambda: [run_layer(ls[i % copies], xs, False) for i in range(depth)])
            g_chk = capture_pass(lambda: [run_layer(ls[i % copies], xs, True) for i in range(depth)])
            g_side = capture_pass(lambda: side_pass(ls, xs, side))  # noqa: B023
            g_pair = capture_pass(lambda: pair_pass(ls, xs))  # noqa: B023
            ms_gemm, ms_chk, ms_side, ms_pair = time_passes([g_gemm, g_chk, g_side, g_pair])
            del g_gemm, g_chk, g_side, g_pair
            # fault campaign on copy 0: every (block, column) cell of every output, per kind
            # (reference fault set, harness/numerics_sim.py:58-64 and harness/campaign.py:8-13)
            rng = np.random.default_rng(B + fp8)
            kinds: dict[str, list[int]] = {}
            false_alarms = cells = 0

            by_launch: dict[str, list[int]] = {}

            escaped: dict[str, list[float]] = {}

            def tally(kind: str, res: Any) -> None:
                # verdicts (num_blocks, B); a column (one GEMV output, the reference's unit in
                # harness/real_activations.py:144-165) is caught if any of its blocks fails.
                # An escaped column's largest |rho| / tau over its blocks says how far below
                # the threshold its error stayed.
                v = res.verdict
                c = kinds.setdefault(kind, [0, 0, 0, 0])
                c[0] += int((~v).sum())
                c[1] += v.numel()
                c[2] += int((~v).any(dim=0).sum())
                c[3] += v.size(1)
                by_launch.setdefault(kind, []).append(int((~v).any(dim=0).sum()))
                missed = ~(~v).any(dim=0)
                if bool(missed.any()):
                    ratio = (res.rho.abs() / res.tau).amax(dim=(0, 1))[missed]
                    escaped.setdefault(kind, []).extend(round(float(r), 4) for r in ratio.tolist())

            for idx, ((_, ch), X, Y) in enumerate(zip(ls[0], xs, ys)):
                honest = ch.check_batched(X, Y).verdict
                false_alarms += int((~honest).sum())
                cells += honest.numel()
                Wq = quantize_fp8(raw[0][idx])[0] if fp8 else raw[0][idx]
                for kind, yy in batched_faults(Wq, X, Y, fp8, BLOCK, rng).items():
                    tally(kind, ch.check_batched(X, yy))
            planted = sum(c[3] for c in kinds.values())
            caught = sum(c[2] for c in kinds.values())
            key = "fp8" if fp8 else "bf16"
            entry[key] = {
                "ms_per_layer": round(ms_chk, 5),
                "gemm_only_ms": round(ms_gemm, 5),
                "tflops": round(B * flops_per_row / (ms_chk / 1e3) / 1e12, 1),
                "gemm_only_tflops": round(B * flops_per_row / (ms_gemm / 1e3) / 1e12, 1),
                "mfma_peak_frac": round(B * flops_per_row / (ms_gemm / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "checker_overhead_pct": round(100 * (ms_chk / ms_gemm - 1), 2),
                "checker_overhead_side_stream_pct": round(100 * (ms_side / ms_gemm - 1), 2),
                "checker_overhead_two_layers_pct": round(100 * (ms_pair / ms_gemm - 1), 2),
                "faulty_columns": planted,  # per kind and launch: every column has the fault
                "faulty_columns_caught": caught,
                "faults_by_kind": {
                    k: {"cells_caught": c, "cells": p, "columns_caught": cc, "columns": cp,
                        "columns_caught_per_launch": dict(zip([x[0] for x in BATCHED_LAUNCHES], by_launch[k]))}
                    for k, (c, p, cc, cp) in kinds.items()
                },
                "escaped_columns_max_rho_over_tau": escaped,
                "false_alarms": false_alarms,
                "honest_cells": cells,
            }
        g_blas = capture_pass(lambda: [[torch.mm(X, W.t()) for W, X in zip(raw[i % copies], xs)] for i in range(depth)])
        (ms_blas,) = time_passes([g_blas])
        del g_blas
        entry["hipblaslt_ms_per_layer"] = round(ms_blas, 5)
        out[f"B{B}"] = entry
    return out


def templates_layer(copies: int = 4, depth: int = 32, reps: int = 7) -> dict:
    """The agent's GEMV templates over the Llama-3-8B decode layer at batch 1: the seven
    projections as seven launches (a column-major launch with grid splits adds its merge
    launch), 32-layer passes over ``copies`` layer copies replayed from a HIP graph.  Per config:
    us per layer, algorithmic GB/s (weights + x + y, plus the scales for INT8) and the share of
    a size-matched read (one read launch of each projection's bytes).  The default row-major
    config is the coalesced tree at T = 256 and must equal the trusted gemv_coalesced bit for bit
    (checked here before timing)."""
    import torch

    from pck.agent.column import ColumnConfig
    from pck.agent.config import KernelConfig, is_exploit
    from pck.cuda import gemv_coalesced, gemv_column, gemv_template, row_q8
    from pck.cuda.timing import read_stream_ms

    gen = torch.Generator(device="cuda").manual_seed(2)
    layers = []
    for _ in range(copies):
        layer = {}
        for name, m, n in LAYER:
            W = (torch.randn(m, n, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            x = torch.randn(n, device="cuda", generator=gen).to(torch.bfloat16)
            layer[name] = (W, x, W.t().contiguous(), row_q8(W))
        layers.append(layer)
    W, x = layers[0]["down"][:2]
    assert torch.equal(gemv_template(W, x, KernelConfig()), gemv_coalesced(W, x, 256))

    def q8_bytes(m: int, n: int) -> int:
        return gemv_bytes(m, n, 1) + 4 * m * (-(-n // 128))

    sizes = {"bf16": [gemv_bytes(m, n, 2) for _, m, n in LAYER],
             "int8": [q8_bytes(m, n) for _, m, n in LAYER]}  # fmt: skip
    matched = {k: sum(read_stream_ms(v)) for k, v in sizes.items()}
    configs = {
        "row_default": KernelConfig(),
        "row_t256_v8_u2": KernelConfig(unroll=2),
        "row_t512_r2_v4_u4": KernelConfig(threads=512, rows_per_block=2, vec=4, unroll=4),
        "int8_t256_r4_v16": KernelConfig(threads=256, rows_per_block=4, vec=16, weights="int8"),
        "column_default": ColumnConfig(),
        "column_t256_v4_s32": ColumnConfig(threads=256, vec=4, splits=32),
        "column_t128_v8_s1": ColumnConfig(splits=1),
        # the activation-sparsity exploit: |x| < 0.3 is 23.6% of N(0, 1) activations, whose
        # weights it never reads
        "column_default_skip_0.3": ColumnConfig(skip_below=0.3),
    }

    def run(cfg, layer):  # type: ignore[no-untyped-def]
        for name, _, _ in LAYER:
            W, x, WT, q8 = layer[name]
            if isinstance(cfg, ColumnConfig):
                gemv_column(WT, x, cfg)
            else:
                gemv_template(W, x, cfg, q8 if cfg.weights == "int8" else None)

    out = {"workload": "Llama-3-8B decode layer, batch 1, 7 launches (+ merges), 32-layer graph passes",
           "size_matched_read_us": {k: round(1e3 * v, 2) for k, v in matched.items()}}  # fmt: skip
    for key, cfg in configs.items():
        run(cfg, layers[0])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(depth):
                run(cfg, layers[i % copies])
        graph.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            times.append(start.elapsed_time(end) / depth)
        ms = statistics.median(times)
        kind = "int8" if getattr(cfg, "weights", "bf16") == "int8" else "bf16"
        out[key] = {
            "config": {k: v for k, v in vars(cfg).items() if k != "layout"},
            "exploit": is_exploit(cfg),
            "us_per_layer": round(1e3 * ms, 2),
            "gbps": round(sum(sizes[kind]) / (ms / 1e3) / 1e9, 1),
            "pct_of_size_matched_read": round(100 * matched[kind] / ms, 2),
        }
        del graph
    del layers
    torch.cuda.empty_cache()
    return out


def host_cpu() -> str:
    """The host CPU's model name, as /proc/cpuinfo gives it."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float = 10.0, fp8: bool = False, all_cores: bool = False) -> dict:
    """The oracle on this host: the coalesced-tree CPU model of every projection of the decode
    layer (T = 256) plus the CPU blocked checker at b = 128, K = 1, repeated over whole layers
    until ``budget_s`` seconds have run; GB/s of the same metric (GEMV algorithmic bytes /
    time).  One core: the NumPy model with BLAS held to one thread.  All cores: the scalar C
    model (OpenMP over rows) with BLAS on every thread.  FP8: E4M3 weights quantized per row
    by torch on the CPU (the GPU path's quantizer), the model with 16-byte vectors of 16
    codes, the checker on the E4M3 values."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle.checker import BlockedChecker
    from oracle.cmodel import gemv_coalesced_c
    from oracle.gemv import emulate_gemv_coalesced
    from pck.cuda.gemv import quantize_fp8
    from pck.fp import bf16, tree_height

    vec = 16 if fp8 else 8
    rng = np.random.default_rng(0)
    layer = []
    for _, m, n in LAYER:
        W = bf16(rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.02))
        if fp8:
            W = quantize_fp8(torch.from_numpy(W))[0].float().numpy()
        layer.append((W, bf16(rng.standard_normal(n, dtype=np.float32))))
    nbytes = sum(gemv_bytes(m, n, 1 if fp8 else 2) for _, m, n in LAYER)
    blas = max((info.get("num_threads", 1) for info in threadpool_info()), default=1)
    passes, elapsed = 0, 0.0
    with threadpool_limits(limits=None if all_cores else 1):
        while elapsed < budget_s:
            t0 = time.perf_counter()
            for W, x in layer:
                m, n = W.shape
                y = gemv_coalesced_c(W, x, THREADS, vec) if all_cores else emulate_gemv_coalesced(W, x, THREADS, vec)
                ok = BlockedChecker(W, x, BLOCK, tree_height(n, THREADS, vec)).verdict(y, rng, checks=1)
                assert ok.all()
            elapsed += time.perf_counter() - t0
            passes += 1
    cores = os.cpu_count() or 1
    model = "scalar C model (OpenMP over rows)" if all_cores else "NumPy emulate_gemv_coalesced"
    return {
        "value": round(passes * nbytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": cores if all_cores else 1,
        "kind": "port",
        "sample": f"oracle {model} + BlockedChecker.verdict (K=1, b=128) over the 7 "
        f"{'FP8' if fp8 else 'BF16'} projections of the layer, {passes} layer passes in "
        f"{elapsed:.1f} s, {'all threads' if all_cores else 'one thread'} (BLAS "
        f"{blas if all_cores else 1} of {blas} threads); host: {cores} CPUs, {host_cpu()}",
    }


def b1_section(fp8: bool, copies: int, depth: int, rounds: int, quick: bool, steps: int,
               warmup: int, matched_ms: float) -> dict:  # fmt: skip
    """The batch-1 decode layer for one weight type: every mode of MODES in alternating rounds,
    the dominant kernels' launch durations (BF16), the eager per-launch times and the fault
    campaign."""
    import torch

    gen = torch.Generator().manual_seed(1 if fp8 else 0)
    kind = "FP8" if fp8 else "BF16"
    print(f"[bench] building {copies} {kind} layer copies", file=sys.stderr, flush=True)
    layers = build_layers(copies, fp8, gen)
    nbytes = sum(gemv_bytes(m, n, 1 if fp8 else 2) for _, m, n in LAYER)
    modes = FP8_MODES if fp8 else MODES
    print(f"[bench] timing {kind} passes ({len(modes)} modes, {rounds} rounds)", file=sys.stderr, flush=True)
    ms, checked = b1_modes(layers, depth, rounds, modes)
    base = ms["gemv"]
    out: dict = {
        "gemv_only_gbps": round(nbytes / (base / 1e3) / 1e9, 1),
        "gemv_only_ms": round(base, 5),
        "modes_ms": {m: round(v, 5) for m, v in ms.items()},
        "overhead_pct": {m: round(100 * (v / base - 1), 2) for m, v in ms.items() if m != "gemv"},
        "honest_blocks_checked_per_pass": checked,
        "gemv_only_pct_of_size_matched_read": round(100 * matched_ms / base, 2),
    }
    if not fp8:
        reps = max(21, steps // 10)
        out["dominant"] = dominant_launch_ms(layers, reps)
        out["dominant_inpass"] = dominant_launch_ms(layers, reps, inpass=True)
        if not quick:
            ms_eager, per_launch = timed(layers, steps, warmup, True, per_kernel=True)
            out["eager_ms_per_step"] = round(ms_eager, 5)
            out["eager_launch_ms"] = {k: round(statistics.mean(v), 5) for k, v in per_launch.items()}
    print(f"[bench] {kind} fault campaign (batch 1)", file=sys.stderr, flush=True)
    out["faults"] = fault_campaign_b1(layers[0], seed=11 if fp8 else 10)
    del layers
    torch.cuda.empty_cache()
    return out


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--copies", type=int, default=4, help="distinct layer copies (> MALL)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument(
        "--quick", action="store_true",
        help="fewest rounds, no eager timing, no CPU baseline (for counter collection)",
    )  # fmt: skip
    parser.add_argument(
        "--section", choices=("all", "b1", "templates", "members", "batched", "campaign"),
        default="all",
        help="b1: only the batch-1 layer (BF16 and FP8); templates: only the agent's templates; "
             "members: only the membership check and the vLLM plugin's step; batched: only the "
             "batched layer (B = 128, 256); campaign: only the detection campaign (K = 8)",
    )  # fmt: skip
    args = parser.parse_args()
    if args.quick:
        args.warmup, args.no_cpu_baseline = 1, True
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the decode hot path "
              "here has no multi-GPU step", file=sys.stderr)  # fmt: skip
        sys.exit(2)

    import torch

    import campaign
    from campaign import contract_summary
    from pck.cuda.timing import read_bandwidth_gbps, read_stream_ms

    if args.section == "templates":
        print(json.dumps({"templates": templates_layer()}), flush=True)
        return
    if args.section == "members":
        print(json.dumps({"membership": membership(), "vllm_plugin": plugin_step()}), flush=True)
        return
    if args.section == "batched":
        print(json.dumps({"batched": batched_layer(reps=3 if args.quick else 7)}), flush=True)
        return
    if args.section == "campaign":
        print(json.dumps({"detection_k8": contract_summary(campaign.run(quick=args.quick))}), flush=True)
        return
    depth = 32  # a Llama-3-8B decode pass
    # At least 7 alternating rounds whatever --steps is; each round replays one 32-layer pass
    # of every mode, so the medians never rest on one sample.
    rounds = 3 if args.quick else max(7, args.steps // depth)
    bytes_bf16 = sum(gemv_bytes(m, n, 2) for _, m, n in LAYER)
    bytes_fp8 = sum(gemv_bytes(m, n, 1) for _, m, n in LAYER)
    # Read-only streams first, in a fresh address space like the layers' own: the long-stream
    # ceiling, and each launch's bytes read by one launch (what a launch of that size can reach).
    print("[bench] timing read-only streams", file=sys.stderr, flush=True)
    read_ceiling = read_bandwidth_gbps()
    sizes = {w: {launch: sum(gemv_bytes(m, n, w) for name, m, n in LAYER if name in names)
                 for launch, names in LAUNCHES} for w in (1, 2)}  # fmt: skip
    matched = {w: dict(zip(sizes[w], read_stream_ms(list(sizes[w].values())), strict=True)) for w in (1, 2)}
    torch.cuda.empty_cache()

    common = dict(copies=args.copies, depth=depth, rounds=rounds, quick=args.quick,
                  steps=args.steps, warmup=args.warmup)  # fmt: skip
    b16 = b1_section(False, matched_ms=sum(matched[2].values()), **common)
    b8 = b1_section(True, matched_ms=sum(matched[1].values()), **common)
    detail: dict = {
        "b1_bf16": b16,
        "b1_fp8": b8,
        "size_matched_read_us": {
            kind: {k: round(1e3 * v, 2) for k, v in matched[w].items()}
            for kind, w in (("bf16", 2), ("fp8", 1))
        },
    }
    member = plugin = sampling = batched = templates = detection = None
    if args.section == "all":
        print("[bench] running the detection campaign (K = 8)", file=sys.stderr, flush=True)
        detection = campaign.run(quick=args.quick)
        detail["detection_k8"] = detection
        print("[bench] timing the membership check", file=sys.stderr, flush=True)
        member = membership()
        print("[bench] timing the vLLM plugin's wrapper per step", file=sys.stderr, flush=True)
        plugin = plugin_step()
        print("[bench] timing the set-sampling checker", file=sys.stderr, flush=True)
        sampling = sampling_checker(50 if args.quick else 200)
        print("[bench] timing the batched layer (B = 128, 256)", file=sys.stderr, flush=True)
        batched = batched_layer()
        print("[bench] timing the agent's GEMV templates", file=sys.stderr, flush=True)
        templates = templates_layer()
        detail |= {"membership": member, "vllm_plugin": plugin, "sampling": sampling, "batched": batched,
                   "templates": templates}  # fmt: skip

    # The headline: the batch-1 BF16 layer with every output checked, in the fastest checked
    # mode (bank checks carried in later GEMV launches, b = 128).
    ms_checked = b16["modes_ms"]["carried"]
    value = bytes_bf16 / (ms_checked / 1e3) / 1e9
    dom_ms, dom_bytes = b16["dominant"]
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9

    def ovh(sec: dict) -> dict:
        o = sec["overhead_pct"]
        return {"inpass_b128": o["inpass"], "inpass_b256": o["inpass_b256"],
                "bank_carried_b128": o["carried"], "bank_carried_b256": o["carried_b256"],
                "bank_carried_check_many_b128": o["carried_api"],
                "bank_serial_b128": o["serial"], "bank_side_stream_b128": o["side_stream"],
                "inpass_sums_only": o["inpass_sums"]}  # fmt: skip

    line: dict = {
        "metric": "GEMV HBM GB/s (% of peak), BF16/FP8, Llama-3-8B shapes; checker overhead %",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_checked, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x bf16 -> fp32 (checker fp64)",
        "data": "synthetic: reference generator, W ~ N(0, 0.02) bf16, x ~ N(0, 1) bf16",
        "config": {
            "workload": "Llama-3-8B decode layer, batch 1: 7 BF16 GEMVs (4 launches), every "
            "output checked by the blocked checker (b=128, K=1, T=256) in a later launch of the "
            "pass; 32-layer passes replayed from a HIP graph",
            "layer_copies": args.copies,
            "rounds": rounds,
            "gemv_bytes_per_step": bytes_bf16,
        },
        "pct_of_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "gemv_only_gbps": b16["gemv_only_gbps"],
        "pct_of_read_ceiling": round(100 * value / read_ceiling, 2),
        "hbm_read_ceiling_gbps": round(read_ceiling, 1),
        "pct_of_size_matched_read": round(100 * sum(matched[2].values()) / ms_checked, 2),
        "fp8": {
            "value_gbps": round(bytes_fp8 / (b8["modes_ms"]["carried"] / 1e3) / 1e9, 1),
            "gemv_only_gbps": b8["gemv_only_gbps"],
            "ms_per_step": b8["modes_ms"]["carried"],
            "pct_of_size_matched_read": round(100 * sum(matched[1].values()) / b8["modes_ms"]["carried"], 2),
            # y = s z: a separate multiply after the GEMVs against the multiply in their epilogue
            "dequant_ms": {k: b8["modes_ms"][k] for k in ("gemv_scale_after", "gemv_scaled", "carried_scaled")},
        },
        "checker_overhead_pct": ovh(b16),
        "fp8_checker_overhead_pct": ovh(b8),
        "faults_b1": {"bf16": b16["faults"]["summary"], "fp8": b8["faults"]["summary"],
                      "inlaunch": {"bf16": b16["faults"]["inlaunch"], "fp8": b8["faults"]["inlaunch"]}},
    }
    if detection is not None:
        line["detection_k8"] = contract_summary(detection)
    if member is not None:
        line["membership"] = {k: member[k] for k in ("ms", "gbps", "pct_of_peak", "planted_caught", "false_alarms")}
    if plugin is not None:
        line["vllm_plugin"] = {k: plugin[k] for k in ("wrapper_ms_per_step", "host_issue_ms_per_step",
                                                      "check_members_ms", "logits_copy_ms")}  # fmt: skip
    if batched is not None:
        line["batched"] = {
            key: {w: {"products_ms": e[w]["gemm_only_ms"], "checker_overhead_pct": e[w]["checker_overhead_pct"],
                      "checker_overhead_two_layers_pct": e[w]["checker_overhead_two_layers_pct"],
                      "mfma_peak_frac": e[w]["mfma_peak_frac"],
                      "faulty_columns_caught": f"{e[w]['faulty_columns_caught']}/{e[w]['faulty_columns']}",
                      "escaped_max_rho_over_tau": e[w]["escaped_columns_max_rho_over_tau"],
                      "false_alarms": e[w]["false_alarms"]} for w in ("bf16", "fp8")}
                 | {"hipblaslt_ms": e["hipblaslt_ms_per_layer"]}
            for key, e in batched.items()
        }  # fmt: skip
    line["roofline"] = {
        "bound": "hbm",
        "kernel": "gemv_tree_kernel<256,1,2,bf16,nt> (q/k/v, o, gate/up launches)",
        "launch_ms": round(dom_ms, 5),
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": recorded_traffic(),
        "traffic_source": TRAFFIC_PROFILE.relative_to(ROOT).as_posix(),
        "inpass_kernel_launch_ms": round(b16["dominant_inpass"][0], 5),
        "inpass_kernel_frac": round(dom_bytes / (b16["dominant_inpass"][0] / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
    }
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU baselines", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline()
        detail["cpu_baseline_all_cores"] = cpu_baseline(all_cores=True)
        detail["fp8_cpu_baseline"] = cpu_baseline(fp8=True)
        line["cpu_baseline_all_cores_gbps"] = detail["cpu_baseline_all_cores"]["value"]
        line["fp8_cpu_baseline_gbps"] = detail["fp8_cpu_baseline"]["value"]
        if member is not None:
            line["membership"]["cpu_baseline_gbps"] = member["cpu_baseline"]["value"]
    # the full per-section figures go to stderr (one JSON line), the contract line to stdout
    print("[bench detail] " + json.dumps(detail), file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
