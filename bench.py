#!/usr/bin/env python
"""Routed-expert hot path on one MI355X: decode GEMV, dequant producer, prefill GEMM.

Headline (the JSON line's ``value``): IQ2_KS routed decode of one token over
256 experts, top-6 -- one step is the gate+up dispatch (12 matrices of
[2048, 4096] from a 512-expert stack) plus the down dispatch (6 matrices of
[4096, 2048]) -- as weight-stream bytes per second, the reference's own
convention (bench/price.py:146).  Inputs are resident in HBM; the K timed
steps replay as one captured HIP graph between two synchronisations.

Also reported, outside the timed region: every member's decode against its
own deleted-decode floor (IQ2_KS and IQ1_S_R4 at 1 token, IQ2_K at 8 tokens)
and against a pure byte stream of the same size (IQ1_S_R4 also against the
floor that keeps its grid lookups, the reference's IQ1 floor),
the dequant producer against its floor and its row-range form, the Zipf(1.1)
mixed-member prefill (producer GB/s, grouped-GEMM and fused-GEMM TFLOP/s and
MFMA utilisation), the sorted and union decode forms on uniform multi-token
routing, the GPU wire ingest (pack), the host quantizers, and the
reference's CPU dequantizer + float32 matmul on a bounded sample of the
headline step.

Protocol (reference: bench/price.py): validation before timing; decode and
floor arms alternated with the order reversed each round, each arm's round
the best of four replays of its graph, medians over five rounds; each arm is a
captured graph of back-to-back dispatches whose routing variants are disjoint
chunks of expert permutations, so an expert's bytes are re-read only after
more than 1 GB of other traffic (beyond the 256 MB MALL).  The stream arm
reads the same byte count per dispatch from windows that walk a 2 GiB buffer.
The prefill cell times each of its kernels over four back-to-back dispatches,
three rounds alternating the routes.

Gates per cell, as the reference's (bench/price.py:458-470): the floor
streams inside the band [2000, 8000] GB/s (a quarter of HBM peak up to the
peak: a floor above it would read fewer bytes than it claims);
no_deleted_load_signature -- the decode is not faster than its own floor by
more than the two arms' spread; within_bar -- decode / floor <= 1.15 (the
producer: <= 1.05).  The JSON line carries every cell's ratios and gates;
``--json-out`` also writes the full results.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "mlx-iqk_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
FLOOR_BAND_GBS = (2000.0, HBM_PEAK_GBS)
DECODE_BAR, PRODUCER_BAR = 1.15, 1.05
STREAM_BUFFER_BYTES = 2 << 30
EXPERTS, TOP_K = 256, 6
PROBE_COPY_BYTES = 64 << 20
GU = (2048, 4096)   # gate/up: out, in
DN = (4096, 2048)   # down


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed headline steps")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rounds", type=int, default=5, help="alternated decode/floor rounds per cell")
    ap.add_argument("--block", type=int, default=200, help="dispatches per captured graph in a cell")
    ap.add_argument("--blocks", type=int, default=4, help="graph replays per arm and round; the best one counts")
    ap.add_argument("--distinct", type=int, default=2, help="distinct quantized experts per projection")
    ap.add_argument("--cells", default="iq2_ks,module,iq2_k,iq1_s_r4,dequant,prefill,pack,verify,quantize",
                    help="cells after the headline ('headline' alone: the IQ2_KS cell and the headline only)")
    ap.add_argument("--cpu-seconds", type=float, default=30.0,
                    help="CPU baseline sample budget over its four workloads (each half on one thread, half on "
                         "every core)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--json-out", default=None)
    ap.add_argument("--probe", type=int, default=0, metavar="K",
                    help="counter-probe mode: K eager dispatches of --probe-kernel, then K copies of "
                         f"{PROBE_COPY_BYTES >> 20} MiB (the HBM-byte calibration), and exit")
    ap.add_argument("--probe-kernel", default="decode:iq2_ks:1:gate_up",
                    help="decode|floor|floor_grid:<member>:<tokens>:gate_up|down, or fused|producer|gemm:<member>:"
                         "gate|down (the 2048-token Zipf prefill), or pairs|sorted|union:<member>:<tokens>:<pool> "
                         "(the verify shape: every token's top-6 from a pool of experts, gate geometry)")
    return ap.parse_args()


# --------------------------------------------------------------------- timing ---


class Arm:
    """A captured graph of `count` dispatches; time() replays it once.  The
    eager warm-up before capture runs `warm` (default: the first four
    launches)."""

    def __init__(self, torch, launches, label, warm=None):
        self.torch, self.label, self.count = torch, label, len(launches)
        for fn in (launches[: min(4, len(launches))] if warm is None else warm):
            fn()  # eager warm-up outside capture
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for fn in launches:
                fn()
        torch.cuda.synchronize()

    def time(self) -> float:
        """Average microseconds per dispatch over one replay (HIP events)."""
        torch = self.torch
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        self.graph.replay()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) * 1e3 / self.count


def alternate(arms: dict, rounds: int, blocks: int) -> dict:
    """Each round times every arm as the best of `blocks` graph replays, the
    arms in turn, the order reversed on odd rounds (bench/price.py:263-273,
    312-340: best of 4 blocks a round, median over the rounds)."""
    names = list(arms)
    for a in arms.values():
        a.time()  # one untimed replay each
    runs = {n: [] for n in names}
    every = {n: [] for n in names}  # every replay, for per-launch averages
    for r in range(rounds):
        for n in (names if r % 2 == 0 else names[::-1]):
            t = [arms[n].time() for _ in range(blocks)]
            every[n] += t
            runs[n].append(min(t))
    return {n: {"median_us": round(statistics.median(v), 3), "min_us": round(min(v), 3),
                "max_us": round(max(v), 3), "runs_us": [round(x, 3) for x in v],
                "all_replays_median_us": round(statistics.median(every[n]), 3)} for n, v in runs.items()}


def disjoint_selections(rng, count: int, tokens: int) -> list[np.ndarray]:
    """`count` routing draws [tokens, TOP_K]; each token's experts are distinct and
    consecutive draws walk disjoint chunks of fresh permutations."""
    out, pool = [], []
    for _ in range(count):
        sel = np.empty((tokens, TOP_K), dtype=np.int64)
        for t in range(tokens):
            if len(pool) < TOP_K:
                pool = list(rng.permutation(EXPERTS))
            sel[t] = [pool.pop() for _ in range(TOP_K)]
        out.append(sel)
    return out


# ---------------------------------------------------------------- decode cells ---


class StreamWindows:
    """The stream arm's source: windows of one dispatch's byte count walking a
    2 GiB device buffer, so a window is re-read only after > 1 GiB of others."""

    def __init__(self, torch, device):
        self.buf = torch.zeros(STREAM_BUFFER_BYTES, dtype=torch.uint8, device=device)
        self.out = torch.empty(STREAM_BUFFER_BYTES // 4096, dtype=torch.int32, device=device)

    # the forms of the stream: (KiB in flight a wavefront, wavefront cap: 0 =
    # one wavefront a chunk; 2048 = eight a CU, striding over the span)
    FORMS = {"stream": (4, 0), "stream_w8": (8, 0), "stream_w16": (16, 0), "stream_gs": (16, 2048)}

    def launcher(self, nbytes: int, i: int, form: str = "stream"):
        from mlx_iqk_amd import kernels
        loads, max_waves = self.FORMS[form]
        span = (nbytes + 16383) // 16384 * 16384
        slots = max(1, STREAM_BUFFER_BYTES // span)
        view = self.buf[(i % slots) * span:]
        return lambda: kernels.stream_floor(view, nbytes, out=self.out, loads=loads, max_waves=max_waves)


def gate_cell(res: dict, bar: float) -> dict:
    """The reference's three gates for one cell (bench/price.py:458-470)."""
    spread = (res["decode"]["max_us"] - res["decode"]["min_us"]) + (res["floor"]["max_us"] - res["floor"]["min_us"])
    return {"floor_in_band": bool(FLOOR_BAND_GBS[0] <= res["floor"]["gb_per_s"] <= FLOOR_BAND_GBS[1]),
            "no_deleted_load_signature": bool(res["floor"]["median_us"] - res["decode"]["median_us"] <= spread),
            "within_bar": bool(res["x_floor"] <= bar)}


def decode_cell(torch, device, member: str, tokens: int, args, seed: int, want_steps: bool = False,
                launchers_only: bool = False, windows: StreamWindows | None = None):
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels, synth

    log(f"[decode {member} x{tokens}] building 256-expert stacks")
    t0 = time.time()
    gu = synth.expert_stack(member, 2 * EXPERTS, GU[0], GU[1], seed, device, args.distinct, "gate_up")
    dn = synth.expert_stack(member, EXPERTS, DN[0], DN[1], seed, device, args.distinct, "down")
    log(f"  stacks ready in {time.time() - t0:.1f}s")
    rng = np.random.default_rng(seed)
    variants = 42  # 42 x 6 = 252 experts: one pass over a permutation per 42 dispatches
    sels = disjoint_selections(rng, variants, tokens)
    gu_mats, dn_mats = 2 * tokens * TOP_K, tokens * TOP_K
    V = []
    for s in sels:
        flat = s.reshape(-1)
        V.append({
            "gu_sel": torch.from_numpy(np.concatenate([flat, flat + EXPERTS]).astype(np.int32)).to(device),
            "dn_sel": torch.from_numpy(flat.astype(np.int32)).to(device),
            "gu_x": torch.randn(2 * tokens, GU[1], device=device).to(torch.float16),
            "dn_x": torch.randn(dn_mats, DN[1], device=device).to(torch.float16),
            "gu_y": torch.empty(gu_mats, GU[0], dtype=torch.float16, device=device),
            "dn_y": torch.empty(dn_mats, DN[0], dtype=torch.float16, device=device),
        })

    def gu_launch(i, floor: bool | str = False):
        v = V[i % variants]
        return lambda: kernels.gemv(member, v["gu_x"], gu, v["gu_sel"], TOP_K, 2 * EXPERTS, GU[0],
                                    floor=floor, out=v["gu_y"])

    def dn_launch(i, floor: bool | str = False):
        v = V[i % variants]
        return lambda: kernels.gemv(member, v["dn_x"], dn, v["dn_sel"], 1, EXPERTS, DN[0], floor=floor,
                                    out=v["dn_y"])

    # validation before timing: sampled rows of variant 0 against float64
    validation = {}
    for name, launch, stacks, (out, n), mats, ppr in (("gate_up", gu_launch, gu, GU, gu_mats, TOP_K),
                                                      ("down", dn_launch, dn, DN, dn_mats, 1)):
        launch(0)()
        torch.cuda.synchronize()
        v = V[0]
        sel = (v["gu_sel"] if name == "gate_up" else v["dn_sel"]).cpu().numpy()
        x = (v["gu_x"] if name == "gate_up" else v["dn_x"]).cpu().numpy().astype(np.float64)
        y = (v["gu_y"] if name == "gate_up" else v["dn_y"]).float().cpu().numpy().astype(np.float64)
        rows = np.random.default_rng(99).choice(out, 32, replace=False)
        worst = mag = 0.0
        for m, e in enumerate(sel):
            part = {k: t[int(e)].cpu().numpy()[rows] for k, t in zip(fmt.component_shapes(member, 1, 1, n), stacks)}
            w = fmt.decode(member, part, n).astype(np.float64)
            ref = w @ x[m // ppr]
            worst = max(worst, float(np.max(np.abs(y[m, rows] - ref))))
            mag = max(mag, float(np.max(np.abs(ref))))
        validation[name] = {"rel_dev": worst / mag, "ok": bool(worst / mag < 1.5e-3)}
        if not validation[name]["ok"]:
            raise SystemExit(f"{member} {name} failed validation ({worst / mag:.3e}); no timing taken")
    log(f"  validated: " + ", ".join(f"{k} rel {v['rel_dev']:.2e}" for k, v in validation.items()))
    if launchers_only:
        return gu_launch, dn_launch

    rb_gu, rb_dn = fmt.ik_row_bytes(member, GU[1]), fmt.ik_row_bytes(member, DN[1])
    bytes_gu, bytes_dn = gu_mats * GU[0] * rb_gu, dn_mats * DN[0] * rb_dn
    B = args.block
    cells = {}
    for name, launch, nbytes in (("gate_up", gu_launch, bytes_gu), ("down", dn_launch, bytes_dn)):
        arms = {"decode": Arm(torch, [launch(i) for i in range(B)], "decode"),
                "floor": Arm(torch, [launch(i, True) for i in range(B)], "floor")}
        if windows is not None:
            for form in windows.FORMS:
                arms[form] = Arm(torch, [windows.launcher(nbytes, i, form) for i in range(B)], form)
        if member == "iq1_s_r4":
            arms["floor_grid"] = Arm(torch, [launch(i, "grid") for i in range(B)], "floor_grid")
        res = alternate(arms, args.rounds, args.blocks)
        res["bytes_per_dispatch"] = nbytes
        for arm in arms:
            res[arm]["gb_per_s"] = round(nbytes / (res[arm]["median_us"] * 1e-6) / 1e9, 1)
            res[arm]["frac_of_8tbps"] = round(res[arm]["gb_per_s"] / HBM_PEAK_GBS, 4)
        res["x_floor"] = round(res["decode"]["median_us"] / res["floor"]["median_us"], 4)
        if "stream" in arms:
            # against the fastest form of the byte stream at this size
            best = min(StreamWindows.FORMS, key=lambda f: res[f]["median_us"])
            res["stream_best"] = best
            res["x_stream"] = round(res["decode"]["median_us"] / res[best]["median_us"], 4)
            res["x_stream_4k"] = round(res["decode"]["median_us"] / res["stream"]["median_us"], 4)
        if "floor_grid" in arms:
            res["x_floor_grid"] = round(res["decode"]["median_us"] / res["floor_grid"]["median_us"], 4)
        res["ideal_us_at_8tbps"] = round(nbytes / HBM_PEAK_GBS / 1e3, 3)
        res["gates"] = gate_cell(res, DECODE_BAR)
        if "floor_grid" in arms:  # the reference's IQ1_S_R4 floor keeps the grid lookups (bench/floors.py:14-17)
            res["within_bar_vs_grid_floor"] = bool(res["x_floor_grid"] <= DECODE_BAR)
        cells[name] = res
        log(f"  {name:8s} decode {res['decode']['median_us']:8.2f} us ({res['decode']['gb_per_s']:7.1f} GB/s)"
            f"  floor {res['floor']['median_us']:8.2f} us  x{res['x_floor']:.3f}"
            + (f"  stream " + "/".join(f"{res[f]['median_us']:.2f}" for f in StreamWindows.FORMS)
               + f" us x{res['x_stream']:.3f}" if "stream" in res else "")
            + (f"  grid floor {res['floor_grid']['median_us']:.2f} us x{res['x_floor_grid']:.3f}"
               if "floor_grid" in res else ""))
        del arms
    out = {"member": member, "tokens": tokens, "top_k": TOP_K, "experts": EXPERTS, "validation": validation,
           "cells": cells}
    if want_steps:
        out["_step"] = (gu_launch, dn_launch, bytes_gu + bytes_dn)
    return out


def headline(torch, step, steps: int, warmup: int):
    """The timed region: K steps (gate/up + down) replayed as one graph.  The
    W warm-up steps run the routing variants of the region's last W steps,
    never its first ones, so the region starts with experts that no recent
    launch has read (out of the 256 MB MALL)."""
    gu_launch, dn_launch, nbytes = step
    warm = []
    for i in range(steps - warmup, steps):
        warm += [gu_launch(i), dn_launch(i)]
    launches = []
    for i in range(steps):
        launches += [gu_launch(i), dn_launch(i)]
    arm = Arm(torch, launches, "headline", warm=warm)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    us_per_launch = arm.time()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = us_per_launch * 2 / 1e3
    return {"ms_per_step": ms_per_step, "wall_s": wall, "gb_per_s": nbytes / (ms_per_step * 1e-3) / 1e9,
            "bytes_per_step": nbytes}


def module_cell(torch, device, args, seed: int):
    """The decode dispatches the switch module itself issues at 1 token (the
    reference's SwitchGLU calls gate, up and down projections separately):
    IqkSwitchLinear gate [2048 x 4096] alone (6 pairs: 384 workgroups of 32
    rows, against the 768 of the bench's combined gate+up dispatch) and down
    [4096 x 2048] (6 pairs, 768 workgroups), each as a graph of 200 module
    calls on disjoint routings, timed as the decode cells are; plus the host
    time of an eager module call."""
    from mlx_iqk_amd import synth
    from mlx_iqk_amd.format import ik_row_bytes
    from mlx_iqk_amd.nn import IqkSwitchLinear

    member, B = "iq2_ks", args.block
    rng = np.random.default_rng(seed)
    sels = disjoint_selections(rng, 42, 1)
    res = {"member": member, "tokens": 1, "top_k": TOP_K}
    arms = {}
    # every tensor a captured graph reads stays referenced here until the
    # graphs are gone: the modules' streams, the activations and the ids
    keep = []
    for name, (out, n) in (("gate", GU), ("down", DN)):
        mod = IqkSwitchLinear(member, EXPERTS, out, n, device=device)
        for k, t in zip(mod.stream_names(), synth.expert_stack(member, EXPERTS, out, n, seed, device,
                                                                 args.distinct, f"module-{name}")):
            setattr(mod, k, t)
        ids = [torch.from_numpy(s_.astype(np.int32)).to(device) for s_ in sels]
        shape = (1, 1, 1, n) if name == "gate" else (1, TOP_K, 1, n)
        xs = [torch.randn(shape, device=device).to(torch.float16) for _ in sels]
        keep.append((mod, ids, xs))
        call = lambda i, mod=mod, ids=ids, xs=xs: (lambda: mod(xs[i % len(xs)], ids[i % len(ids)]))  # noqa: E731
        arms[name] = Arm(torch, [call(i) for i in range(B)], name)
        # host time of an eager call (the launch path: shape checks, the cached stream record, one launch)
        for i in range(20):
            call(i)()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(B):
            call(i)()
        host = (time.perf_counter() - t0) * 1e6 / B
        torch.cuda.synchronize()
        res[name] = {"bytes_per_call": TOP_K * out * ik_row_bytes(member, n), "host_us_per_eager_call": round(host, 2),
                     "workgroups": TOP_K * out // 32}
    r = alternate(arms, args.rounds, args.blocks)
    del arms  # the graphs first, then the tensors they read
    torch.cuda.synchronize()
    keep.clear()
    for name in ("gate", "down"):
        res[name].update(r[name])
        res[name]["gb_per_s"] = round(res[name]["bytes_per_call"] / (r[name]["median_us"] * 1e-6) / 1e9, 1)
    log(f"[module {member} x1] gate alone {res['gate']['median_us']:.2f} us ({res['gate']['gb_per_s']} GB/s), "
        f"down {res['down']['median_us']:.2f} us; eager host {res['gate']['host_us_per_eager_call']:.1f} us a call")
    return res


# ---------------------------------------------------------------- producer cell ---


def dequant_cell(torch, device, member: str, args, seed: int):
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels, synth

    res = {}
    chunk = 16  # experts per dispatch; 16 chunks walk the 256-stack before any re-read
    for name, (out, n) in (("gate_up", GU), ("down", DN)):
        log(f"[dequant {member} {name}]")
        st = synth.expert_stack(member, EXPERTS, out, n, seed, device, args.distinct, f"dq-{name}")
        w = torch.empty((chunk, out, n), dtype=torch.float16, device=device)
        parts = [[t[c * chunk:(c + 1) * chunk] for t in st] for c in range(EXPERTS // chunk)]
        # validation: chunk 0 against the CPU decode, bit for bit (sampled rows)
        kernels.dequant(member, parts[0], chunk, out, n, out=w)
        rows = np.random.default_rng(3).choice(out, 8, replace=False)
        for e in (0, chunk - 1):
            part = {k: t[e].cpu().numpy()[rows] for k, t in zip(fmt.component_shapes(member, 1, 1, n), parts[0])}
            want = fmt.decode(member, part, n).astype(np.float16)
            got = w[e][rows].cpu().numpy()
            if not np.array_equal(got.view(np.uint16), want.view(np.uint16)):
                raise SystemExit(f"dequant {member} {name} is not bit-exact; no timing taken")
        B = max(8, args.block // 8)

        def launch(i, floor=False):
            return lambda: kernels.dequant(member, parts[i % len(parts)], chunk, out, n, floor=floor, out=w)
        # the row-range form: the middle half of each expert's rows
        r0, nr = out // 4, out // 2
        wr = torch.empty((chunk, nr, n), dtype=torch.float16, device=device)

        def launch_range(i):
            return lambda: kernels.dequant(member, parts[i % len(parts)], chunk, out, n, row_start=r0, rows=nr, out=wr)
        arms = {"decode": Arm(torch, [launch(i) for i in range(B)], "decode"),
                "floor": Arm(torch, [launch(i, True) for i in range(B)], "floor"),
                "range": Arm(torch, [launch_range(i) for i in range(B)], "range")}
        r = alternate(arms, args.rounds, args.blocks)
        read = chunk * out * fmt.ik_row_bytes(member, n)
        written = chunk * out * n * 2
        r["range"]["rows"] = [r0, r0 + nr]
        r["range"]["gb_per_s"] = round((read + written) / 2 / (r["range"]["median_us"] * 1e-6) / 1e9, 1)
        r.update({"experts": chunk, "read_bytes": read, "written_bytes": written,
                  "x_floor": round(r["decode"]["median_us"] / r["floor"]["median_us"], 4)})
        for arm in ("decode", "floor"):
            r[arm]["gb_per_s"] = round((read + written) / (r[arm]["median_us"] * 1e-6) / 1e9, 1)
            r[arm]["frac_of_8tbps"] = round(r[arm]["gb_per_s"] / HBM_PEAK_GBS, 4)
        r["gates"] = gate_cell(r, PRODUCER_BAR)
        res[name] = r
        log(f"  decode {r['decode']['median_us']:9.2f} us ({r['decode']['gb_per_s']:7.1f} GB/s)  floor "
            f"{r['floor']['median_us']:9.2f} us  x{r['x_floor']:.3f}  half-range {r['range']['median_us']:.2f} us "
            f"({r['range']['gb_per_s']} GB/s)")
        del arms, st, parts, w, wr
        torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------------- prefill cell ---


def prefill_cell(torch, device, args, seed: int):
    """2048 tokens, Zipf(1.1) top-6 sorted routing; gate/up IQ2_KS, down IQ2_K (the
    totals), and the gate projection once more as IQ1_S_R4 and as IQ2_K (reported
    beside them)."""
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels, synth
    from mlx_iqk_amd.nn import IqkSwitchLinear

    tokens = 2048
    idx = synth.zipf_routing(tokens, EXPERTS, TOP_K, 1.1, seed)
    flat = np.sort(idx.reshape(-1))
    counts = np.bincount(flat, minlength=EXPERTS)
    log(f"[prefill] {flat.size} pairs over {int((counts > 0).sum())} experts, max {counts.max()} "
        f"median {int(np.median(counts[counts > 0]))} min {counts[counts > 0].min()}")
    x = torch.randn(flat.size, 1, GU[1], device=device).to(torch.float16)
    h = torch.randn(flat.size, 1, DN[1], device=device).to(torch.float16)
    ids = torch.from_numpy(flat.astype(np.int32)).to(device)
    projections = (("gate", "iq2_ks", GU, x), ("up", "iq2_ks", GU, x), ("down", "iq2_k", DN, h),
                   ("gate_iq1_s_r4", "iq1_s_r4", GU, x), ("gate_iq2_k", "iq2_k", GU, x))
    res = {"tokens": tokens, "pairs": int(flat.size), "experts_routed": int((counts > 0).sum()),
           "max_pairs_per_expert": int(counts.max()), "projections": {}}
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    tot_prod = tot_gemm = tot_fused = 0.0
    tot_bytes = tot_flop = 0
    for name, member, (out, n), xin in projections:
        mod = IqkSwitchLinear(member, EXPERTS, out, n, device=device)
        for k, t in zip(mod.stream_names(), synth.expert_stack(member, EXPERTS, out, n, seed, device,
                                                                 args.distinct, f"pf-{name}")):
            setattr(mod, k, t)
        y = mod(xin, ids, sorted_indices=True)  # warm-up + shapes
        torch.cuda.synchronize()
        # the two kernels of the route, timed separately with the module's own operands
        present = torch.zeros(EXPERTS, dtype=torch.int32, device=device).index_fill_(0, ids.long(), 1)
        slot = torch.where(present > 0, torch.cumsum(present, 0, dtype=torch.int32) - 1,
                           torch.full_like(present, -1))
        n_slots = EXPERTS
        routed = int(present.sum().item())
        offs = torch.zeros(n_slots + 1, dtype=torch.int32, device=device)
        offs[1:] = torch.cumsum(torch.zeros(n_slots, dtype=torch.int64, device=device).index_add_(
            0, slot[ids.long()].long(), torch.ones_like(ids, dtype=torch.int64)), 0).to(torch.int32)
        rows = torch.arange(flat.size, dtype=torch.int32, device=device)
        w = torch.empty((n_slots, out, n), dtype=torch.float16, device=device)
        # the fused route's operands: experts as groups, pairs already sorted
        offs_e = torch.zeros(EXPERTS + 1, dtype=torch.int32, device=device)
        offs_e[1:] = torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(device)
        yf = torch.empty((flat.size, out), dtype=torch.float16, device=device)
        yg = torch.empty((rows.numel(), out), dtype=torch.float16, device=device)
        # each kernel timed over `burst` back-to-back dispatches (steady state, as
        # a prefill's projections run), rounds alternating the routes
        reps, burst = 3, 4
        # the route is a kernel of a few microseconds: timed from a captured
        # graph of `burst` calls, so the figure is the kernel's, not the
        # launches' host time
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            kernels.route(ids, EXPERTS, 1, 1, flat.size)
        torch.cuda.current_stream().wait_stream(side)
        route_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(route_graph):
            for _ in range(burst):
                kernels.route(ids, EXPERTS, 1, 1, flat.size)
        times = {"producer": [], "floor": [], "gemm": [], "fused": [], "route": []}
        for _ in range(reps):
            for key in ("producer", "floor", "gemm", "fused", "route"):
                a, b = ev(), ev()
                a.record()
                for _ in range(1 if key == "route" else burst):
                    if key == "gemm":
                        kernels.grouped_gemm(xin.reshape(-1, n), w, offs, rows, out=yg)
                    elif key == "route":
                        route_graph.replay()
                    elif key == "fused":
                        kernels.fused_matmul(member, xin.reshape(-1, n), mod._streams(), EXPERTS, out, offs_e, rows,
                                             out=yf)
                    else:
                        kernels.dequant(member, mod._streams(), EXPERTS, out, n, slot_of_expert=slot,
                                        n_slots=n_slots, out=w, floor=(key == "floor"))
                b.record()
                b.synchronize()
                times[key].append(a.elapsed_time(b) * 1e3 / burst)
        med = {k: statistics.median(v) for k, v in times.items()}
        # the whole module call (the route's device-side bookkeeping + the fused kernel): GPU time
        # from events around `burst` calls, host time per call from the wall clock
        mod_gpu, mod_host = [], []
        for _ in range(reps):
            a, b = ev(), ev()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            a.record()
            for _ in range(burst):
                mod(xin, ids, sorted_indices=True)
            b.record()
            t1 = time.perf_counter()
            b.synchronize()
            mod_gpu.append(a.elapsed_time(b) * 1e3 / burst)
            mod_host.append((t1 - t0) * 1e6 / burst)
        med["module"], med["module_host"] = statistics.median(mod_gpu), statistics.median(mod_host)
        kernels.dequant(member, mod._streams(), EXPERTS, out, n, slot_of_expert=slot, n_slots=n_slots, out=w)
        yp = kernels.grouped_gemm(xin.reshape(-1, n), w, offs, rows).float()  # the producer route's output
        fused_dev = ((yf.float() - yp).abs().max() / yp.abs().max()).item()
        nbytes = routed * out * (fmt.ik_row_bytes(member, n) + 2 * n)
        flop = 2 * flat.size * out * n
        r = {"member": member, "experts_reconstructed": routed,
             "producer_us": round(med["producer"], 2), "producer_floor_us": round(med["floor"], 2),
             "producer_bytes": nbytes,
             "producer_gb_per_s": round(nbytes / (med["producer"] * 1e-6) / 1e9, 1),
             "producer_x_floor": round(med["producer"] / med["floor"], 4),
             "gemm_us": round(med["gemm"], 2), "gemm_flop": flop,
             "gemm_tflops": round(flop / (med["gemm"] * 1e-6) / 1e12, 2)}
        r["mfma_utilisation"] = round(r["gemm_tflops"] / MFMA_F16_PEAK_TFLOPS, 4)
        r.update({"route_us": round(med["route"], 2),
                  "module_forward_us": round(med["module"], 2), "module_forward_host_us": round(med["module_host"], 2),
                  "fused_us": round(med["fused"], 2), "fused_tflops": round(flop / (med["fused"] * 1e-6) / 1e12, 2),
                  "fused_speedup_over_producer_route": round((med["producer"] + med["gemm"]) / med["fused"], 2),
                  "fused_max_dev_vs_producer_route": round(fused_dev, 6)})
        r["fused_mfma_utilisation"] = round(r["fused_tflops"] / MFMA_F16_PEAK_TFLOPS, 4)
        res["projections"][name] = r
        log(f"  {name}: producer {med['producer']:.1f} us ({r['producer_gb_per_s']} GB/s, x{r['producer_x_floor']})"
            f"  gemm {med['gemm']:.1f} us ({r['gemm_tflops']} TFLOP/s)"
            f"  fused {med['fused']:.1f} us ({r['fused_tflops']} TFLOP/s, dev {fused_dev:.2e})"
            f"  route {med['route']:.1f} us  module forward {med['module']:.1f} us GPU, {med['module_host']:.1f} us host")
        del mod, w, y, yf, yp
        torch.cuda.empty_cache()
        if name.startswith("gate_"):  # outside the prefill configuration's totals
            continue
        tot_fused += med["fused"]
        tot_prod += med["producer"]
        tot_gemm += med["gemm"]
        tot_bytes += nbytes
        tot_flop += flop
    res["producer_gb_per_s"] = round(tot_bytes / (tot_prod * 1e-6) / 1e9, 1)
    res["gemm_tflops"] = round(tot_flop / (tot_gemm * 1e-6) / 1e12, 2)
    res["mfma_utilisation"] = round(res["gemm_tflops"] / MFMA_F16_PEAK_TFLOPS, 4)
    res["fused_tflops"] = round(tot_flop / (tot_fused * 1e-6) / 1e12, 2)
    res["fused_mfma_utilisation"] = round(res["fused_tflops"] / MFMA_F16_PEAK_TFLOPS, 4)
    return res


def verify_cell(torch, device, args, seed: int):
    """Multi-token decode with uniform top-6 routing per token (experts repeat
    across tokens): the pair GEMV against the expert-sorted and the union forms
    (one read of each distinct expert per run), IQ2_K on the gate geometry
    [2048x4096] of a 256-expert stack.  GB/s counts each distinct expert once."""
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels, synth

    member, (out, n) = "iq2_k", GU
    stack = synth.expert_stack(member, EXPERTS, out, n, seed, device, args.distinct, "verify")
    rb = fmt.ik_row_bytes(member, n)
    rng = np.random.default_rng(seed)
    res = {"member": member, "geometry": [out, n]}
    for tokens, pool in ((8, None), (32, None), (8, 9)):
        variants = 16
        V = []
        for _ in range(variants):
            # uniform top-6 per token, or (pool) every token's top-6 from the same few experts: the
            # speculative-verify shape, where runs of one expert are long
            src = rng.choice(EXPERTS, pool, replace=False) if pool else np.arange(EXPERTS)
            idx = np.stack([rng.choice(src, TOP_K, replace=False) for _ in range(tokens)]).astype(np.int32)
            flat = idx.reshape(-1)
            order = np.argsort(flat, kind="stable")
            V.append({"x": torch.randn(tokens, n, device=device).to(torch.float16),
                      "sel": torch.from_numpy(flat).to(device),
                      "sorted": torch.from_numpy(flat[order]).to(device),
                      "toks": torch.from_numpy((order // TOP_K).astype(np.int32)).to(device),
                      "distinct": int(np.unique(flat).size),
                      "y": torch.empty(flat.size, out, dtype=torch.float16, device=device)})
        # the three forms agree bit for bit (sorted/union rows are the pair rows, reordered)
        v = V[0]
        yp = kernels.gemv(member, v["x"], stack, v["sel"], TOP_K, EXPERTS, out).cpu().numpy()
        order = np.argsort(v["sel"].cpu().numpy(), kind="stable")
        for union in (False, True):
            ys = kernels.gemv_sorted(member, v["x"], stack, v["sorted"], v["toks"], EXPERTS, out,
                                     union=union).cpu().numpy()
            if not np.array_equal(ys.view(np.uint16), yp[order].view(np.uint16)):
                raise SystemExit(f"verify cell: the {'union' if union else 'sorted'} form differs from the pair form")

        def launch(i, mode):
            v = V[i % variants]
            if mode in ("pairs", "floor"):
                return lambda: kernels.gemv(member, v["x"], stack, v["sel"], TOP_K, EXPERTS, out,
                                            floor=mode == "floor", out=v["y"])
            return lambda: kernels.gemv_sorted(member, v["x"], stack, v["sorted"], v["toks"], EXPERTS, out,
                                               union=mode == "union", out=v["y"])
        # Sorted and union are one dispatch.  The arm that runs right after the
        # floor (no decode, so less power drawn) starts at a higher clock:
        # in the order pairs, floor, sorted, union, sorted followed the floor
        # and union measured 3-4% slower; with sorted, pairs, floor, union it
        # was the other way round.  Here the floor sits between the two, so
        # each follows it once every two rounds (the order reverses).
        arms = {mode: Arm(torch, [launch(i, mode) for i in range(variants)], mode)
                for mode in ("pairs", "sorted", "floor", "union")}
        r = alternate(arms, args.rounds, args.blocks)
        distinct = statistics.mean(v["distinct"] for v in V)
        nbytes = distinct * out * rb
        cell = {"pairs": tokens * TOP_K, "distinct_experts_mean": round(distinct, 1),
                "distinct_bytes": round(nbytes)}
        for mode in ("pairs", "floor", "sorted", "union"):
            cell[mode] = {"median_us": r[mode]["median_us"],
                          "gb_per_s_distinct": round(nbytes / (r[mode]["median_us"] * 1e-6) / 1e9, 1)}
        cell["union_speedup_over_pairs"] = round(r["pairs"]["median_us"] / r["union"]["median_us"], 3)
        res[f"tokens_{tokens}" + (f"_pool_{pool}" if pool else "")] = cell
        log(f"[verify {member} x{tokens}{' pool ' + str(pool) if pool else ''}] {tokens * TOP_K} pairs, {distinct:.1f} distinct experts: "
            + "  ".join(f"{m} {r[m]['median_us']:.1f} us" for m in ("pairs", "floor", "sorted", "union")))
        del arms, V
        torch.cuda.empty_cache()
    del stack
    torch.cuda.empty_cache()
    return res


def quantize_cell(args, seed: int):
    """The package codec's quantizers on the host: rows of 4096 from N(0, 0.02) with a
    U(0.1, 1) imatrix, at the default worker count and on one thread (a bounded
    sample; the IQ1_S_R4 grid-neighbour tables are built before timing)."""
    from mlx_iqk_amd import codec
    from mlx_iqk_amd import format as fmt

    rng = np.random.default_rng(seed)
    n = GU[1]
    w = rng.normal(0.0, 0.02, (256, n)).astype(np.float32)
    im = rng.uniform(0.1, 1.0, n).astype(np.float32)
    res = {"in_features": n, "threads_default": codec.threads()}
    for member in ("iq2_ks", "iq2_k", "iq1_s_r4"):
        codec.quantize(member, w[:4], im)  # warm-up (tables)
        cell = {}
        for label, threads in (("default", 0), ("one_thread", 1)):
            codec.set_threads(threads)
            rows = 256 if threads == 0 else 64
            t0 = time.perf_counter()
            codec.quantize(member, w[:rows], im)
            dt = time.perf_counter() - t0
            cell[label] = {"rows": rows, "rows_per_s": round(rows / dt, 1),
                           "wire_mb_per_s": round(rows * fmt.ik_row_bytes(member, n) / dt / 1e6, 2)}
        codec.set_threads(0)
        res[member] = cell
        log(f"[quantize {member}] {cell['default']['rows_per_s']} rows/s on {res['threads_default']} threads, "
            f"{cell['one_thread']['rows_per_s']} on one")
    return res


def pack_cell(torch, device, args, seed: int):
    """ik wire -> relayout on the GPU for a 256-expert gate/up stack per member (the
    on-box ingest of wire already in device memory); GB/s counts bytes read + written."""
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels

    res = {}
    out, n = GU
    rows = EXPERTS * out
    for member in ("iq2_ks", "iq2_k", "iq1_s_r4"):
        rb = fmt.ik_row_bytes(member, n)
        g = torch.Generator(device=device).manual_seed(seed)
        wire = torch.randint(0, 256, (rows, rb), dtype=torch.uint8, device=device, generator=g)
        planes = kernels.pack(member, wire, n)  # warm-up; outputs reused below
        times = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            kernels.pack(member, wire, n, out=planes)
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b) * 1e3)
        us = statistics.median(times)
        nbytes = 2 * rows * rb
        res[member] = {"rows": rows, "wire_bytes": rows * rb, "us": round(us, 1),
                       "gb_per_s": round(nbytes / (us * 1e-6) / 1e9, 1)}
        log(f"[pack {member}] {rows} rows: {us:.1f} us, {res[member]['gb_per_s']} GB/s (read + written)")
        del wire, planes
        torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------ CPU baseline ---


def _cpu_model() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


class _CpuPath:
    """The reference's CPU path for one workload: its CPU dequantizer on ik
    wire, then numpy float32 matmuls, on the experts a routing selects.
    ``job`` gives one job (one expert matrix); a job returns its seconds of
    dequantization and of matmul."""

    _local = None

    def __init__(self, deq, member: str, tiles: dict):
        import threading
        if _CpuPath._local is None:
            _CpuPath._local = threading.local()  # a worker's float32 weight buffers, reused across its jobs
        self.deq, self.member, self.tiles = deq, member, tiles

    @staticmethod
    def buffers() -> dict:
        """This worker's buffers for both geometries, allocated and resident."""
        bufs = getattr(_CpuPath._local, "bufs", None)
        if bufs is None:
            bufs = _CpuPath._local.bufs = {}
            for shape in (GU, DN):
                bufs[shape] = np.ones(shape, dtype=np.float32)
        return bufs

    def job(self, geometry: str, e: int, x: np.ndarray):
        def run():
            wire = self.tiles[geometry][e % len(self.tiles[geometry])]
            buf = self.buffers()[(wire.shape[0], x.shape[-1])]
            t0 = time.perf_counter()
            w = self.deq(self.member, wire, x.shape[-1], out=buf)
            t1 = time.perf_counter()
            _ = w @ x.T if x.ndim == 2 else w @ x
            return t1 - t0, time.perf_counter() - t1
        return run


def _cpu_run(jobs_fn, threads: int, budget: float) -> dict:
    """Whole steps of jobs on `threads` workers (numpy held to one thread a
    worker; the compiled dequantizer releases the GIL) until `budget` seconds
    have passed.  Untimed first: every worker allocates its buffers (all
    workers at once, by a barrier) and one step runs."""
    import threading
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    with threadpool_limits(limits=1), ThreadPoolExecutor(max_workers=threads) as pool:
        barrier = threading.Barrier(threads)
        list(pool.map(lambda _: (_CpuPath.buffers(), barrier.wait()), range(threads)))
        list(pool.map(lambda f: f(), jobs_fn()))
        done, dq, mm, t0 = 0, 0.0, 0.0, time.perf_counter()
        while True:
            for a, b in pool.map(lambda f: f(), jobs_fn()):
                dq, mm = dq + a, mm + b
            done += 1
            if time.perf_counter() - t0 >= budget:
                break
    return {"steps": done, "seconds": time.perf_counter() - t0, "dequant_s": dq, "matmul_s": mm}


def cpu_baseline(seconds: float, distinct: int, seed: int) -> dict:
    """The reference's CPU path -- its CPU dequantizer (compiled from its own
    sources, else the oracle's restatement) + numpy float32 matmul -- beside
    each GPU workload, each on a bounded sample, once on one thread and once
    on every host core:

    * IQ2_KS 1 token (the headline step: 6 x gate, up, down GEMVs) -- the
      reported ``value``, in the headline's unit;
    * IQ2_K 8 tokens (48 pairs: each distinct expert dequantized once and
      contracted with the tokens routed to it) and IQ1_S_R4 1 token, in the
      same bytes-per-step convention as their GPU cells;
    * the 2048-token Zipf(1.1) prefill (IQ2_KS gate/up, IQ2_K down): a
      sample of the routed experts (each dequantized, then its slots
      contracted), from which the time of the whole prefill's three
      projections is extrapolated (dequantization per expert, matmul by
      flops).
    """
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import synth
    from oracle import oracle

    kind = "reference" if oracle.ref_available() else "port"
    deq = oracle.ref_dequantize if kind == "reference" else oracle.dequantize
    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(seed)
    tile_cache = {}

    def tiles(member):
        if member not in tile_cache:
            tile_cache[member] = {
                name: [synth.quantized_rows(member, out, n, synth.seed_for(seed, name, member, out, n, t),
                                            imatrix_seed=synth.seed_for(seed, name, "imatrix", n))
                       for t in range(distinct)] for name, (out, n) in (("gate_up", GU), ("down", DN))}
        return tile_cache[member]

    def decode_jobs(member: str, tokens: int):
        """One routed decode step: gate and up (one activation row a token),
        down (one row a pair); per distinct expert one dequantization."""
        path = _CpuPath(deq, member, tiles(member))
        xg = rng.standard_normal((tokens, GU[1])).astype(np.float16).astype(np.float32)
        xd = rng.standard_normal((tokens * TOP_K, DN[1])).astype(np.float16).astype(np.float32)

        def jobs():
            sel = np.stack([rng.choice(EXPERTS, TOP_K, replace=False) for _ in range(tokens)])
            out = []
            for e in np.unique(sel):
                toks = np.nonzero((sel == e).any(axis=1))[0]
                pairs = np.flatnonzero(sel.reshape(-1) == e)
                xt = xg[toks] if tokens > 1 else xg[0]
                for p in range(2):  # gate, up
                    out.append(path.job("gate_up", int(e) + p, xt))
                out.append(path.job("down", int(e), xd[pairs] if tokens > 1 else xd[pairs[0]]))
            return out
        nbytes = tokens * TOP_K * (2 * GU[0] * fmt.ik_row_bytes(member, GU[1]) + DN[0] * fmt.ik_row_bytes(member, DN[1]))
        return jobs, nbytes

    def decode_entry(member, tokens, budget):
        jobs, nbytes = decode_jobs(member, tokens)
        jobs()[0]()  # untimed: loads the dequantizer library before any worker starts
        one, every = _cpu_run(jobs, 1, budget / 2), _cpu_run(jobs, cores, budget / 2)
        rate = lambda r: round(r["steps"] * nbytes / r["seconds"] / 1e9, 3)  # noqa: E731
        return {"value": rate(every), "unit": "GB/s", "cores": cores, "single_thread": rate(one),
                "ms_per_step": round(every["seconds"] / every["steps"] * 1e3, 2),
                "sample": f"{every['steps']} + {one['steps']} steps of {tokens} token(s) x top-{TOP_K} "
                          f"({member}; {cores} threads, then 1)"}

    def prefill_entry(budget):
        """The Zipf prefill's three projections, extrapolated from a sample of
        routed experts (gate/up IQ2_KS, down IQ2_K), one expert a job."""
        idx = synth.zipf_routing(2048, EXPERTS, TOP_K, 1.1, 23)
        counts = np.bincount(idx.reshape(-1), minlength=EXPERTS)
        routed = np.flatnonzero(counts)
        x = {"gate_up": rng.standard_normal((int(counts.max()), GU[1])).astype(np.float16).astype(np.float32),
             "down": rng.standard_normal((int(counts.max()), DN[1])).astype(np.float16).astype(np.float32)}
        paths = {"iq2_ks": _CpuPath(deq, "iq2_ks", tiles("iq2_ks")), "iq2_k": _CpuPath(deq, "iq2_k", tiles("iq2_k"))}
        projections = (("gate_up", "iq2_ks", GU), ("gate_up", "iq2_ks", GU), ("down", "iq2_k", DN))
        total_flop = sum(2 * int(counts.sum()) * out * n for _, _, (out, n) in projections)
        total_experts = len(projections) * routed.size
        order = rng.permutation(routed)
        state = {"k": 0}

        def take(count):  # the next `count` (expert, projection) jobs of the shuffled order
            out = []
            for _ in range(count):
                i = state["k"]
                state["k"] += 1
                e = int(order[i % order.size])
                geo, member, _ = projections[i % 3]
                out.append(paths[member].job(geo, e, x[geo][:int(counts[e])]))
            return out

        def entry(threads, share):
            state["k"] = 0
            r = _cpu_run(lambda: take(threads), threads, share)
            n = state["k"]
            picked = [(int(order[i % order.size]), projections[i % 3][2]) for i in range(n)]
            flop = sum(2 * int(counts[e]) * out * k for e, (out, k) in picked)
            # per-expert dequantization and flop-proportional matmul, scaled to the whole prefill
            work = r["dequant_s"] * total_experts / n + r["matmul_s"] * total_flop / flop
            return work * r["seconds"] / (r["dequant_s"] + r["matmul_s"]), n, r

        take(1)[0]()
        t1, n1, _ = entry(1, budget / 2)
        tc, nc, rc = entry(cores, budget / 2)
        return {"value": round(tc * 1e3, 1), "unit": "ms per prefill (gate+up+down, extrapolated)", "cores": cores,
                "single_thread": round(t1 * 1e3, 1),
                "matmul_gflop_per_s": round(total_flop / (tc * rc["matmul_s"] / (rc["dequant_s"] + rc["matmul_s"])) / 1e9, 1),
                "sample": f"{nc} + {n1} expert projections of the 2048-token Zipf(1.1) top-{TOP_K} prefill "
                          f"({routed.size} experts routed, {int(counts.sum())} pairs; {cores} threads, then 1)"}

    budget = seconds / 5
    head = decode_entry("iq2_ks", 1, 2 * budget)
    configs = {"iq2_ks_1_token": head, "iq2_k_8_tokens": decode_entry("iq2_k", 8, budget),
               "iq1_s_r4_1_token": decode_entry("iq1_s_r4", 1, budget), "zipf_prefill_2048": prefill_entry(budget)}
    return {"value": head["value"], "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": head["sample"], "single_thread": head["single_thread"], "cpu_model": _cpu_model(),
            "configs": configs}


def prefill_launcher(torch, device, member: str, projection: str, kind: str, args, seed: int = 23):
    """One kernel of the 2048-token Zipf(1.1) top-6 prefill (sorted pairs), as a
    launch closure, with its algorithmic bytes and flops per dispatch."""
    from mlx_iqk_amd import format as fmt
    from mlx_iqk_amd import kernels, synth

    out, n = GU if projection == "gate" else DN
    idx = synth.zipf_routing(2048, EXPERTS, TOP_K, 1.1, seed)
    flat = np.sort(idx.reshape(-1))
    counts = np.bincount(flat, minlength=EXPERTS)
    st = synth.expert_stack(member, EXPERTS, out, n, seed, device, args.distinct, f"pf-{projection}")
    x = torch.randn(flat.size, n, device=device).to(torch.float16)
    rows = torch.arange(flat.size, dtype=torch.int32, device=device)
    offs = torch.zeros(EXPERTS + 1, dtype=torch.int32, device=device)
    offs[1:] = torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(device)
    y = torch.empty((flat.size, out), dtype=torch.float16, device=device)
    routed = int((counts > 0).sum())
    info = {"pairs": int(flat.size), "experts_routed": routed, "flop": 2 * flat.size * out * n,
            "stream_bytes": routed * out * fmt.ik_row_bytes(member, n)}
    if kind == "fused":
        return (lambda: kernels.fused_matmul(member, x, st, EXPERTS, out, offs, rows, out=y)), info
    slot = torch.arange(EXPERTS, dtype=torch.int32, device=device)
    w = torch.empty((EXPERTS, out, n), dtype=torch.float16, device=device)
    kernels.dequant(member, st, EXPERTS, out, n, slot_of_expert=slot, n_slots=EXPERTS, out=w)
    info["fp16_weight_bytes"] = routed * out * n * 2
    if kind == "producer":
        return (lambda: kernels.dequant(member, st, EXPERTS, out, n, slot_of_expert=slot, n_slots=EXPERTS,
                                        out=w)), info
    return (lambda: kernels.grouped_gemm(x, w, offs, rows, out=y)), info


def probe(torch, device, args) -> int:
    """Eager dispatches for hardware-counter passes (rocprofv3 --pmc): K
    dispatches of one kernel (a decode cell's dispatch on its disjoint routing
    variants, or one kernel of the Zipf prefill), then a plain device copy of
    known size whose counters calibrate HBM bytes."""
    from mlx_iqk_amd.format import ik_row_bytes

    kind, member, *rest = args.probe_kernel.split(":")
    info = {"probe": args.probe, "kernel": args.probe_kernel}
    if kind in ("pairs", "sorted", "union"):
        from mlx_iqk_amd import kernels, synth
        tokens, pool = int(rest[0]), int(rest[1])
        out, n = GU
        stack = synth.expert_stack(member, EXPERTS, out, n, 31, device, args.distinct, "verify")
        rng = np.random.default_rng(31)
        distinct = []
        for _ in range(args.probe):
            src = rng.choice(EXPERTS, pool, replace=False)
            idx = np.stack([rng.choice(src, TOP_K, replace=False) for _ in range(tokens)]).astype(np.int32)
            flat = idx.reshape(-1)
            order = np.argsort(flat, kind="stable")
            x = torch.randn(tokens, n, device=device).to(torch.float16)
            distinct.append(int(np.unique(flat).size))
            if kind == "pairs":
                kernels.gemv(member, x, stack, torch.from_numpy(flat).to(device), TOP_K, EXPERTS, out)
            else:
                kernels.gemv_sorted(member, x, stack, torch.from_numpy(flat[order]).to(device),
                                    torch.from_numpy((order // TOP_K).astype(np.int32)).to(device), EXPERTS, out,
                                    union=kind == "union")
        info["pair_bytes_per_dispatch"] = tokens * TOP_K * out * ik_row_bytes(member, n)
        info["distinct_bytes_per_dispatch_mean"] = statistics.mean(distinct) * out * ik_row_bytes(member, n)
    elif kind in ("decode", "floor", "floor_grid"):
        tokens, which = int(rest[0]), rest[1]
        gu_launch, dn_launch = decode_cell(torch, device, member, tokens, args, seed=11, launchers_only=True)
        launch = gu_launch if which == "gate_up" else dn_launch
        floor = {"decode": False, "floor": True, "floor_grid": "grid"}[kind]
        out, n = GU if which == "gate_up" else DN
        mats = (2 if which == "gate_up" else 1) * tokens * TOP_K
        info["bytes_per_dispatch"] = mats * out * ik_row_bytes(member, n)
        for i in range(args.probe):
            launch(i, floor)()
    else:
        fn, extra = prefill_launcher(torch, device, member, rest[0], kind, args)
        info.update(extra)
        for _ in range(args.probe):
            fn()
    src = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device=device).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(args.probe):
        dst.copy_(src)
    torch.cuda.synchronize()
    info["copy_bytes"] = PROBE_COPY_BYTES
    print(json.dumps(info), flush=True)
    return 0


# ------------------------------------------------------------------------- main ---


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X: the routed-expert path here runs on a single GPU and has no "
              f"multi-GPU mode (asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        return 2
    import torch

    device = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(device)
    log(f"device {props.name} {props.gcnArchName} CUs {props.multi_processor_count}")
    if args.probe:
        return probe(torch, device, args)
    cells = [c for c in args.cells.split(",") if c]
    results = {}
    t_start = time.time()
    windows = StreamWindows(torch, device)
    # the headline member always runs: its gate/up kernel is the roofline kernel
    results["iq2_ks"] = decode_cell(torch, device, "iq2_ks", 1, args, seed=11, want_steps=True, windows=windows)
    step = results["iq2_ks"].pop("_step")
    head = headline(torch, step, args.steps, args.warmup)
    log(f"[headline] {args.steps} steps: {head['ms_per_step'] * 1e3:.2f} us/step, {head['gb_per_s']:.1f} GB/s")
    if "module" in cells:
        results["module"] = module_cell(torch, device, args, seed=41)
    if "iq2_k" in cells:
        results["iq2_k"] = decode_cell(torch, device, "iq2_k", 8, args, seed=13, windows=windows)
    if "iq1_s_r4" in cells:
        results["iq1_s_r4"] = decode_cell(torch, device, "iq1_s_r4", 1, args, seed=17, windows=windows)
    del windows
    torch.cuda.empty_cache()
    if cells == ["headline"]:
        cells = []
    if "dequant" in cells:
        results["dequant"] = {m: dequant_cell(torch, device, m, args, seed=19) for m in ("iq2_ks", "iq2_k", "iq1_s_r4")}
    if "prefill" in cells:
        results["prefill"] = prefill_cell(torch, device, args, seed=23)
    if "pack" in cells:
        results["pack"] = pack_cell(torch, device, args, seed=29)
    if "verify" in cells:
        results["verify"] = verify_cell(torch, device, args, seed=31)
    if "quantize" in cells:
        results["quantize"] = quantize_cell(args, seed=37)
    base = None if args.no_cpu else cpu_baseline(args.cpu_seconds, args.distinct, seed=11)

    gu = results["iq2_ks"]["cells"]["gate_up"]
    traffic_file = ROOT / "profiles" / "gemv_mfma_iq2_ks_gate_up_traffic.json"
    traffic = json.loads(traffic_file.read_text())["traffic_bytes"] if traffic_file.is_file() else None
    # the kernel's per-launch time over every timed replay of its graph (not the best
    # replay a round that the x-floor ratios use), as a kernel trace averages it
    per_launch = gu["decode"]["all_replays_median_us"]
    achieved = round(gu["bytes_per_dispatch"] / (per_launch * 1e-6) / 1e9, 1)
    roofline = {"bound": "hbm", "kernel": "gemv_mfma_kernel<IQ2_KS,4096> (gate/up dispatch)",
                "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "per_launch_us": per_launch, "bytes_per_launch": gu["bytes_per_dispatch"],
                # HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE passes over `--probe`,
                # each calibrated on a plain copy of known size
                "traffic": traffic, "traffic_source": traffic_file.name if traffic else None,
                "trace": "profiles/gemv_mfma_iq2_ks_routed_decode.md"}
    # every priced cell: its ratios and the reference's gates (kept short, so the whole line
    # survives a tail of the output; `--json-out` has every figure)
    summary, gates = {}, {}
    for m, r in results.items():
        for c, cell in (r.get("cells") or {}).items():
            key = f"{m}_{c}" + (f"_x{r['tokens']}" if r.get("tokens", 1) != 1 else "")
            summary[key] = {k: round(cell[k], 3) for k in ("x_floor", "x_stream", "x_floor_grid") if k in cell}
            if "stream_best" in cell:
                summary[key]["stream_best"] = cell["stream_best"]
            summary[key]["us"] = round(cell["decode"]["median_us"], 2)
            gates[key] = dict(cell["gates"])
            if "within_bar_vs_grid_floor" in cell:
                gates[key]["within_bar_vs_grid_floor"] = cell["within_bar_vs_grid_floor"]
    for m, r in (results.get("dequant") or {}).items():
        for c, cell in r.items():
            key = f"producer_{m}_{c}"
            summary[key] = {"x_floor": round(cell["x_floor"], 3), "us": round(cell["decode"]["median_us"], 2)}
            gates[key] = cell["gates"]
    if "module" in results:
        summary["module_iq2_ks_x1"] = {k: results["module"][k]["median_us"] for k in ("gate", "down")}
    if "verify" in results:
        summary["verify"] = {k: {m: v[m]["median_us"] for m in ("pairs", "sorted", "union")}
                             for k, v in results["verify"].items() if k.startswith("tokens_")}
    if "prefill" in results:
        pf = results["prefill"]
        summary["prefill"] = {"producer_gb_per_s": pf["producer_gb_per_s"], "gemm_tflops": pf["gemm_tflops"],
                              "fused_tflops": pf["fused_tflops"], "fused_mfma_utilisation": pf["fused_mfma_utilisation"],
                              "gemm_mfma_utilisation": pf["mfma_utilisation"]}
    line = {
        "metric": "routed decode achieved HBM GB/s (IQ2_KS, 256 experts, top-6, 1 token: gate+up and down)",
        "value": round(head["gb_per_s"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8x3/int32",
        "arithmetic": "fp16 activations as three exact int8 byte planes per 32-element block (20-bit fixed "
                      "point), int8 weights, int32 MFMA sums, f32 scale folds, fp16 out",
        "data": "synthetic: N(0,0.02) rows, U(0.1,1) imatrix, quantized by the package codec "
                f"({args.distinct} distinct experts per projection, row-rotated to 256 distinct stacks)",
        "config": {"workload": "IQ2_KS routed decode, 256 experts, top-6, 1 token, gate/up [2048x4096] x2 "
                               "+ down [4096x2048]", "experts": EXPERTS, "top_k": TOP_K, "tokens": 1,
                   "bytes_per_step": head["bytes_per_step"]},
        "roofline": roofline,
        "cpu_baseline": base,
        "bars": {"decode_vs_own_floor": DECODE_BAR, "producer_vs_own_floor": PRODUCER_BAR,
                 "floor_band_gb_s": list(FLOOR_BAND_GBS)},
        "cells": summary,
        # the gates each cell fails (floor_in_band, no_deleted_load_signature, within_bar,
        # within_bar_vs_grid_floor); a cell that passes all of them is not listed
        "gates_checked": len(gates),
        "gates_failed": {k: [n for n, ok in g.items() if not ok] for k, g in gates.items() if not all(g.values())},
        "all_gates_pass": all(all(g.values()) for g in gates.values()),
        "elapsed_s": round(time.time() - t_start, 1),
    }
    full = dict(line, results=results)
    if args.json_out:
        Path(args.json_out).write_text(json.dumps(full, indent=2) + "\n")
    else:
        log("results: " + json.dumps(results))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
