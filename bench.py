"""
Benchmark: nanoSpeaker MoE block on one MI355X (tokens/s, fwd and fwd+bwd, at T = 8192 bf16).

A step is one forward + backward of the MoE block over one batch of synthetic tokens
(the training-shape workload: T = 8192, bf16, train mode, loss = (out * g).sum() + aux_loss):
router GEMM, the HIP route / dispatch / grouped-expert / combine kernels, and the HIP
backward producing dX, dW for all 78 experts and the router gradient.  Inputs and
weights are resident in HBM before the timed region.

Prints ONE JSON line.  `value` is forward+backward tokens/s with the step captured once in
a HIP graph and replayed (every kernel of the step runs on every replay; `--eager`
reports the eagerly issued step instead, which is always reported beside it as
`eager_tokens_per_s`); the forward-only rate (train mode, no_grad) is reported too.  `roofline` covers the step's dominant
kernel, timed live with HIP events recorded by the library on the stream it launches
on.  `cpu_baseline` times the CPU restatement of the reference's eager bf16 path
(oracle/moe_ref.py, pinned bit-exact to the reference by tests/golden) on this host's
cores over a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --calibrate-copy ...      (under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)
       python bench.py --pmc-summary FETCH_CSV WRITE_CSV   (-> profiles/hbm_traffic_T8192.md)
       python bench.py --stats-summary KERNEL_STATS_CSV    (-> profiles/*_kernel_stats.md)
       python bench.py --prefill-legs KERNEL_TRACE_CSV     (-> profiles/prefill_B4x8192_kernel_stats.md)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
COPY_BYTES = 256 << 20      # the calibration copy: bytes read and bytes written
# The library's named launch stages (its HIP-event timers), in step order.
KERNEL_NAMES = ("route_fwd", "dispatch", "place_pack", "pack", "expert_fwd", "combine",
                "route_bwd", "expert_bwd", "expert_dx", "dw_in", "dw_out", "dw",
                "combine_dx", "router_dw", "norm_bwd")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="time only the headline workload (T=8192 fwd+bwd)")
    ap.add_argument("--only", metavar="NAMES",
                    help="run only these comma-separated configurations (c1_T2048_fwd, "
                         "c3_T64_eval, c4_T16384_skew_fwd_bwd, c5_prefill, "
                         "c5_head_cross_entropy) and print their JSON, no headline line")
    ap.add_argument("--single-stream", action="store_true",
                    help="keep every kernel on one stream (the library's default: the "
                         "side_stream option off), so that profiled kernels never overlap")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("MOPS_CSV", "MFMAUTIL_CSV"),
                    help="print the MFMA table from two rocprofv3 --pmc runs "
                         "(SQ_INSTS_VALU_MFMA_MOPS_BF16, MfmaUtil) and a --stats run's "
                         "kernel_stats.csv (--stats-csv), and exit")
    ap.add_argument("--stats-csv", help="kernel_stats.csv for --mfma-summary")
    ap.add_argument("--eager", action="store_true",
                    help="report the eagerly issued step as `value` (default: HIP-graph replay)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one plain 256 MiB copy kernel, the HBM-counter yardstick")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="print a rocprofv3 --stats kernel table as markdown, and exit")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the HBM-traffic table from two rocprofv3 --pmc runs "
                         "(FETCH_SIZE, WRITE_SIZE) of `bench.py --calibrate-copy`, and exit")
    ap.add_argument("--prefill-legs", metavar="KERNEL_TRACE_CSV",
                    help="print per-leg kernel tables of a rocprofv3 --kernel-trace run of "
                         "`bench.py --only c5_prefill,c5_head_cross_entropy`, and exit")
    return ap.parse_args()


def build_block(T: int, seed: int = 0):
    """Seed 0, params in the reference's draw order x 0.02 (moe.py:131-165), bf16; then x, g."""
    from nanospeaker_amd import MoEBlock

    torch.manual_seed(seed)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(torch.bfloat16).train()
    x = torch.randn(T, 576).to(torch.bfloat16)
    g = torch.randn(T, 576).to(torch.bfloat16)
    return m, x, g


def kernel_units(name: str, T: int, k: int, S: int, d: int, H: int, E: int):
    """(algorithmic units per launch, bound, unit) for the roofline of kernel `name`."""
    rows = T * k + S * T  # routed pairs + shared rows
    if name == "expert_fwd":        # GEMM1 + GEMM2 per row
        return rows * (2 * d * 2 * H + 2 * H * d), "mfma", "TFLOP/s"
    if name == "expert_bwd":        # G = dout W_out^T per row (a1 saved by the forward)
        return rows * (2 * d * H), "mfma", "TFLOP/s"
    if name == "expert_dx":         # dX rows = dA1 W_in^T
        return rows * (2 * 2 * H * d), "mfma", "TFLOP/s"
    if name == "dw_in":
        return rows * (2 * d * 2 * H), "mfma", "TFLOP/s"
    if name == "dw_out":
        return rows * (2 * H * d), "mfma", "TFLOP/s"
    if name == "dw":                # dW_in and dW_out in one launch
        return rows * (2 * d * 2 * H + 2 * H * d), "mfma", "TFLOP/s"
    if name == "combine":           # read k + S rows, write one, per token (+ inv)
        return T * ((k + S) * d * 2 + d * 2 + k * 4), "hbm", "GB/s"
    if name == "route_fwd":         # x in; bf16 logits, fp32 probs, ids + gates out
        return T * (d * 2 + E * 2 + E * 4 + k * 8 + k * 2), "hbm", "GB/s"
    if name == "dispatch":          # ids read once (histograms come from the router),
        return T * k * (8 + 4 + 4), "hbm", "GB/s"  # sorted ids + inverse written
    if name == "combine_dx":        # expert dX rows + d(logits) in, dx out, per token
        return T * ((k + S) * d * 2 + (E + 7) // 8 * 8 * 2 + d * 2 + k * 4), "hbm", "GB/s"
    if name == "router_dw":         # x and d(logits) read once
        return T * (d * 2 + (E + 7) // 8 * 8 * 2), "hbm", "GB/s"
    if name == "route_bwd":         # bf16 logits, fp32 probs, ids, gate grads in; d(logits) out
        return T * (E * 2 + E * 4 + k * 8 + k * 2 + (E + 7) // 8 * 8 * 2), "hbm", "GB/s"
    if name == "pack":              # W_in and W_out (routed + shared) read and written once
        return (E + S) * (d * 2 * H + H * d) * 2 * 2, "hbm", "GB/s"
    return None


def kernel_bytes(name: str, T: int, k: int, S: int, d: int, H: int, E: int):
    """Algorithmic HBM bytes per launch of the grouped-GEMM kernels (each input read once,
    each output written once; gathered token rows counted once), or None."""
    rows = T * k + S * T
    w_in, w_out = (E + S) * d * 2 * H * 2, (E + S) * H * d * 2
    if name == "expert_fwd":        # x, both weights in; rows out, saved a1 out
        return T * d * 2 + w_in + w_out + rows * d * 2 + rows * 2 * H * 2
    if name == "expert_bwd":        # dout, a1, W_out in; dA1, w h out
        return T * d * 2 + rows * 2 * H * 2 + w_out + rows * 2 * H * 2 + rows * H * 2
    if name == "expert_dx":         # dA1, W_in in; dX rows out
        return rows * 2 * H * 2 + w_in + rows * d * 2
    if name == "dw":                # x, dout, dA1, w h in; dW_in, dW_out out
        return 2 * T * d * 2 + rows * 2 * H * 2 + rows * H * 2 + w_in + w_out
    return None


def roofline_of(name: str, T: int, k: int, S: int, d: int, H: int, E: int):
    """(units, bound, unit, extra) for kernel `name`: the grouped GEMMs are rated against
    the MFMA peak, the dense-contraction roof the measurement plan names for them; `extra`
    adds their algorithmic bytes, which at these shapes sit below the ridge point
    (2.5 PFLOP/s / 8 TB/s = 312 FLOP/B), so the HBM roof is reported beside it."""
    units, bound, unit = kernel_units(name, T, k, S, d, H, E)
    nbytes = kernel_bytes(name, T, k, S, d, H, E)
    extra = {"bytes_per_launch": nbytes} if bound == "mfma" and nbytes is not None else {}
    return units, bound, unit, extra


def time_gpu(m, x, g, steps: int, warmup: int):
    """Eager fwd+bwd step time, its host enqueue time, per-kernel launch times and the
    eager forward (no_grad, weights unchanged, so the forward reuses the cached packs)."""
    from nanospeaker_amd import _native as nat
    from nanospeaker_amd import moe_kernel as mk

    params = [p for p in m.parameters()]
    xg = x.detach().requires_grad_(True)
    one = torch.ones((), dtype=torch.float32, device=x.device)

    def step():
        # Every gradient of the block (input, router, experts) is computed and returned;
        # none is accumulated into a .grad buffer.  A training step's weights are new each
        # step, so the weight-pack cache is emptied first: every step packs.
        mk.PACKS.clear()
        out = m(xg)
        return torch.autograd.grad([out, m.aux_loss], [xg] + params, [g, one])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # fwd + bwd, timed, as the library issues it (eager calls overlap the weight pack and
    # the dW stage with the rest on a second stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    host_ms = (time.perf_counter() - t0) * 1e3 / steps   # enqueue time, before the wait
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps

    # Per-kernel launch times, from the library's HIP-event pairs on the launch stream, in a
    # pass of its own on one stream, so that no other kernel shares the GPU with the one
    # being timed.
    prev = nat.get_option("side_stream")
    nat.set_option("side_stream", 0)
    try:
        step()
        torch.cuda.synchronize()
        nat.timing_enable(64 * steps + 64)
        torch.cuda.synchronize()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        kernels = {}
        for name in KERNEL_NAMES:
            tot, n = nat.timing_read(name)
            if n:
                kernels[name] = (tot / n, n // steps)
        nat.timing_enable(0)
    finally:
        nat.set_option("side_stream", prev)

    # forward only (train mode, no autograd)
    with torch.no_grad():
        for _ in range(warmup):
            m(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            m(x)
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t0) * 1e3 / steps
    return ms, fwd_ms, kernels, host_ms


# bench.py kernel name -> the symbol prefix of the HIP kernel(s) it times.
KERNEL_SYMBOLS = {
    "expert_fwd": ("nsmoe::expert_fwd_reg_kernel", "nsmoe::expert_fwd_async_kernel",
                   "nsmoe::expert_fwd_kernel"),
    "expert_bwd": ("nsmoe::expert_bwd_reg_kernel", "nsmoe::expert_bwd_async_kernel",
                   "nsmoe::expert_bwd_kernel"),
    "expert_dx": ("nsmoe::expert_dx_res_kernel", "nsmoe::expert_dx_reg_kernel",
                  "nsmoe::expert_dx_async_kernel"),
    "dw": ("nsmoe::dw_pair_kernel",),
    "dw_in": ("nsmoe::dw_kernel<0, 0",),
    "dw_out": ("nsmoe::dw_kernel<0, 1",),
    "route_fwd": ("nsmoe::router_fwd_kernel", "nsmoe::route_fwd_kernel"),
    "combine": ("nsmoe::combine_kernel",),
    "combine_dx": ("nsmoe::combine_dx_kernel",),
    "pack": ("nsmoe::pack_pair_kernel", "nsmoe::pack_kernel", "nsmoe::pack_ks_kernel"),
    "dispatch": ("nsmoe::dispatch_hist_kernel", "nsmoe::dispatch_place_kernel"),
    "place_pack": ("nsmoe::dispatch_place_pack_kernel",),
    "router_dw": ("nsmoe::router_dw_kernel",),
    "route_bwd": ("nsmoe::route_bwd_kernel",),
}
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "hbm_traffic_T8192.md")
COPY_SYMBOL = "neg_kernel_cuda"


def _pmc_per_kernel(path):
    """{short kernel name: (dispatches, mean counter value)} from a counter_collection.csv."""
    import csv

    acc = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"].replace("void ", "").split("(")[0]
            n, s = acc.get(name, (0, 0.0))
            acc[name] = (n + 1, s + float(r["Counter_Value"]))
    return {k: (n, s / n) for k, (n, s) in acc.items()}


def pmc_summary(fetch_csv, write_csv):
    """Markdown table of HBM bytes per launch: FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by what the same counter reads for the calibration copy
    (COPY_BYTES read and written) -- the factor that turns the counter into bytes."""
    fetch, write = _pmc_per_kernel(fetch_csv), _pmc_per_kernel(write_csv)

    def copy_factor(tab):
        hits = [v for k, v in tab.items() if COPY_SYMBOL in k]
        if not hits:
            raise SystemExit("no calibration copy in " + str(tab.keys()))
        return COPY_BYTES / (hits[0][1] * 1024.0)

    ff, fw = copy_factor(fetch), copy_factor(write)
    lines = [
        f"Calibration: the {COPY_BYTES >> 20} MiB copy reads {next(v[1] for k, v in fetch.items() if COPY_SYMBOL in k):.1f} KiB"
        f" by FETCH_SIZE and {next(v[1] for k, v in write.items() if COPY_SYMBOL in k):.1f} KiB by WRITE_SIZE:"
        f" bytes = FETCH_SIZE x 1024 x {ff:.4f} and WRITE_SIZE x 1024 x {fw:.4f}.",
        "",
        "| bench kernel | HIP kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes / launch |",
        "|---|---|---|---|---|---|",
    ]
    for bname, prefixes in KERNEL_SYMBOLS.items():
        for sym, (n, fv) in fetch.items():
            if sym.startswith(prefixes) and sym in write:
                wv = write[sym][1]
                tb = fv * 1024 * ff + wv * 1024 * fw
                lines.append(f"| {bname} | `{sym}` | {n} | {fv:.1f} | {wv:.1f} | {tb:.0f} |")
    return "\n".join(lines)


def prefill_legs(path, top=14):
    """Markdown tables of a --kernel-trace run of the prefill configurations, one per leg
    in the order bench.py runs them: the prefills with the HIP attention (up to the first
    dispatch of torch SDPA's `attn_fwd`), the prefills with torch attention (up to the last
    MoE-library or SDPA kernel before the first `ce_rows_kernel`), then the head's
    cross-entropy calls; with the hip leg's `attn_fwd_kernel` launches split into global
    (> 300 us) and windowed layers."""
    import csv
    from collections import defaultdict

    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    names = [r["Kernel_Name"] for r in rows]
    first_sdpa = names.index("attn_fwd")
    first_ce = next(i for i, n in enumerate(names) if n.startswith("void nsmoe::ce_rows"))
    last_body = max(i for i in range(first_ce) if "nsmoe::" in names[i] or names[i] == "attn_fwd")
    legs = {"hip": rows[:first_sdpa], "sdpa": rows[first_sdpa:last_body + 1],
            "head": rows[last_body + 1:]}

    def us(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

    out = []
    for leg, rs in legs.items():
        agg = defaultdict(list)
        for r in rs:
            agg[r["Kernel_Name"]].append(us(r))
        tot = sum(sum(v) for v in agg.values())
        wall = (int(rs[-1]["End_Timestamp"]) - int(rs[0]["Start_Timestamp"])) / 1e6
        out += [f"\n## {leg}: {len(rs)} dispatches, {tot / 1e3:.2f} ms of kernel time "
                f"({wall:.2f} ms from first start to last end)",
                "| kernel | calls | avg us | total ms | % |", "|---|---|---|---|---|"]
        for n, v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:top]:
            out.append(f"| {n[:80]} | {len(v)} | {sum(v) / len(v):.2f} | {sum(v) / 1e3:.2f} | "
                       f"{100 * sum(v) / tot:.1f} |")
    att = [us(r) for r in legs["hip"] if r["Kernel_Name"].startswith("void nsmoe::attn_fwd_kernel")]
    glob = [t for t in att if t > 300.0]
    win = [t for t in att if t <= 300.0]
    if glob and win:
        out.append(f"\nhip leg `attn_fwd_kernel`: {len(glob)} global launches, avg "
                   f"{sum(glob) / len(glob):.1f} us; {len(win)} windowed, avg "
                   f"{sum(win) / len(win):.1f} us")
    return "\n".join(out)


def stats_summary(path, top=30):
    """Markdown table of a rocprofv3 `*_kernel_stats.csv`, longest total first."""
    import csv

    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: -float(r["TotalDurationNs"]))
    out = ["| kernel | calls | avg us | min us | max us | total ms | % |",
           "|---|---|---|---|---|---|---|"]
    for r in rows[:top]:
        out.append(f"| {r['Name'][:80]} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    return "\n".join(out)


# FLOPs per row the MFMA kernels issue (bf16, H = 128, d = 576).  With the forward's
# pre-activations saved (the block's training default) the GLU-backward kernel runs
# G = dout W_out^T (2 d H) alone; recomputing them would add a1 = x W_in (2 d 2H).
ISSUED_FLOPS_PER_ROW = {
    "expert_fwd": 2 * 576 * 256 + 2 * 128 * 576,
    "expert_bwd": 2 * 576 * 128,  # G only: a1 comes saved from the forward
    "expert_dx": 2 * 256 * 576,
    "dw": 2 * 576 * 256 + 2 * 128 * 576,
}


def mfma_summary(mops_csv, util_csv, stats_csv, T=8192, rows=8192 * 8):
    """Markdown table per MFMA kernel: the MFMA work it issued (SQ_INSTS_VALU_MFMA_MOPS_BF16
    x 512 FLOPs) against the algorithmic and the issued count (ISSUED_FLOPS_PER_ROW), the
    achieved rate from its average duration in the --stats run, and rocprofv3's derived
    MfmaUtil (MFMA-busy share of the kernel's GPU cycles)."""
    import csv

    mops, util = _pmc_per_kernel(mops_csv), _pmc_per_kernel(util_csv)
    dur = {}
    with open(stats_csv) as f:
        for r in csv.DictReader(f):
            dur[r["Name"].replace("void ", "").split("(")[0]] = float(r["AverageNs"]) / 1e3
    lines = ["| bench kernel | HIP kernel | avg us | MOPS x 512 (GFLOP) | algorithmic GFLOP | "
             "issued GFLOP | achieved TFLOP/s (MOPS) | % of 2500 | "
             "MfmaUtil % |",
             "|---|---|---|---|---|---|---|---|---|"]
    for bname, prefixes in KERNEL_SYMBOLS.items():
        if bname not in ISSUED_FLOPS_PER_ROW:
            continue
        for sym, (n, mv) in sorted(mops.items()):
            if not sym.startswith(prefixes):
                continue
            flops = mv * 512
            alg = kernel_units(bname, T, 6, 2, 576, 128, 76)[0]
            issued = ISSUED_FLOPS_PER_ROW[bname] * rows
            us = dur.get(sym, float("nan"))
            rate = flops / (us * 1e-6) / 1e12
            u = util.get(sym, (0, float("nan")))[1]
            lines.append(f"| {bname} | `{sym}` | {us:.2f} | {flops / 1e9:.2f} | "
                         f"{alg / 1e9:.2f} | {issued / 1e9:.2f} | {rate:.0f} | "
                         f"{100 * rate / PEAK_BF16_TFLOPS:.1f} | {u:.1f} |")
    return "\n".join(lines)


def committed_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter table, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 6 and cells[0] == kernel:
                    return int(cells[5])
    except (OSError, ValueError):
        return None
    return None


def calibrate_copy():
    """One dispatch of torch's elementwise negation over 256 MiB of bf16: it reads and
    writes exactly COPY_BYTES each, so under `rocprofv3 --pmc FETCH_SIZE` (or WRITE_SIZE)
    its counter value fixes the KiB-to-bytes factor applied to the other kernels."""
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst




def graph_time(fn, steps: int, warmup: int) -> float:
    """Milliseconds per replay of `fn` captured once in a HIP graph (torch's recipe:
    warm-up on a side stream, then capture).  Every replay runs every kernel `fn`
    issues; the weight packs are captured too (the pack cache is bypassed under
    capture), so each replay re-packs the weights."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 2)):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    del graph
    return ms


def eager_time(fn, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def train_step_fn(m, x, g, logit_bias=None):
    """One fwd+bwd of the block returning every gradient (input, router, experts)."""
    from nanospeaker_amd import moe_kernel as mk

    params = list(m.parameters())
    xg = x.detach().requires_grad_(True)
    one = torch.ones((), dtype=torch.float32, device=x.device)

    def step():
        if logit_bias is None:
            out, aux = m(xg), m.aux_loss
        else:  # the skewed workload: the router offset enters through the op's hook
            out, aux, _, _, _ = mk.block_forward(
                xg, m.router.W, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, None, None, None,
                None, 6, True, True, "silu", 1e-2, logit_bias=logit_bias)
        return torch.autograd.grad([out, aux], [xg] + params, [g, one])

    return step


def zipf_bias():
    import numpy as np

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden",
                        "zipf_logit_bias.npy")
    return torch.from_numpy(np.load(path, allow_pickle=False)).float()


def config1(steps, warmup):
    """T = 2048 forward (train mode, no autograd)."""
    m, x, _ = build_block(2048)
    m, x = m.cuda(), x.cuda()
    with torch.no_grad():
        g_ms = graph_time(lambda: m(x), steps, warmup)
        e_ms = eager_time(lambda: m(x), steps, warmup)
    return {"workload": "T=2048 forward, train mode, bf16",
            "tokens_per_s": round(2048 / (g_ms / 1e3), 1), "ms": round(g_ms, 4),
            "eager_tokens_per_s": round(2048 / (e_ms / 1e3), 1), "eager_ms": round(e_ms, 4)}


def config3(steps, warmup):
    """T = 64 decode call (eval branch): microseconds per call, graph-replayed with the
    cached packs shared into the graph (PackCache.share_with_graphs: a decode loop whose
    weights do not change), graph-replayed with the pack inside the graph, and eagerly
    issued with the packs cached and re-packing every call (those two interleaved in
    rounds, median of the rounds, so host drift affects both alike)."""
    from nanospeaker_amd import moe_kernel as mk

    m, x, _ = build_block(64)
    m, x = m.cuda().eval(), x.cuda()
    reps = max(steps, 50)
    with torch.no_grad():
        def repack():
            mk.PACKS.clear()
            m(x)

        cached, fresh = [], []
        for _ in range(7):
            cached.append(eager_time(lambda: m(x), reps, warmup))
            fresh.append(eager_time(repack, reps, warmup))
        cached.sort()
        fresh.sort()
        g_ms = graph_time(lambda: m(x), reps, warmup)
        mk.PACKS.clear()
        mk.PACKS.share_with_graphs = True
        try:
            m(x)  # files the pack the graph will read
            torch.cuda.synchronize()
            g_cached = graph_time(lambda: m(x), reps, warmup)
        finally:
            mk.PACKS.share_with_graphs = False
            mk.PACKS.clear()
        m(x)
    empty = int((m.expert_counts == 0).sum())
    return {"workload": "T=64 decode call, eval branch, bf16",
            "us_per_call": round(g_cached * 1e3, 2),
            "us_per_call_is": "HIP graph replay reading the cached packs (share_with_graphs)",
            "graph_us_per_call_repacking": round(g_ms * 1e3, 2),
            "eager_us_per_call_cached_packs": round(cached[3] * 1e3, 2),
            "eager_us_per_call_repacking": round(fresh[3] * 1e3, 2),
            "eager_rounds": 7,
            "empty_experts": empty}


def config4(steps, warmup):
    """T = 16384 fwd+bwd with the Zipf(1.2) router offset, through the block op."""
    m, x, g = build_block(16384)
    m, x, g = m.cuda(), x.cuda(), g.cuda()
    bias = zipf_bias().cuda()
    g_ms = graph_time(train_step_fn(m, x, g, bias), steps, warmup)
    from nanospeaker_amd import moe_kernel as mk

    with torch.no_grad():
        _, _, counts, _, _ = mk.block_forward(
            x, m.router.W, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, None, None, None, None, 6,
            True, True, "silu", 1e-2, logit_bias=bias)
    share = float(counts.max()) / float(counts.sum())
    return {"workload": "T=16384 fwd+bwd, Zipf(1.2) router offset, train, bf16",
            "tokens_per_s": round(16384 / (g_ms / 1e3), 1), "ms": round(g_ms, 4),
            "hot_expert_share": round(share, 4)}


def routing_flips(sizes=(2048, 8192, 32768)):
    """How the block's routing compares with routing on the CPU's own router GEMM, as the
    reference computes it ((x @ W).float() in bf16, router.py:69, then torch.topk on the
    CPU, the eval branch): per size, the tokens whose top-6 expert list differs and the
    share of logits that differ (the two GEMMs sum in fp32 in different orders and round
    once)."""
    out = {}
    for T in sizes:
        m, x, _ = build_block(T)
        W = m.router.W.detach().clone()
        m, xd = m.cuda().eval(), x.cuda()
        with torch.no_grad():
            m(xd)
        torch.cuda.synchronize()
        gpu_logits, gpu_idx = m._logits.cpu(), m._routing.cpu()
        cpu_logits = (x @ W).float()
        cpu_idx = cpu_logits.topk(6, dim=-1).indices
        flips = int((cpu_idx != gpu_idx).any(1).sum())
        out[f"T{T}"] = {"tokens": T, "tokens_routed_differently": flips,
                        "logits_differ": round(float((gpu_logits.float() != cpu_logits)
                                                     .float().mean()), 6)}
        del m, xd
    return out


def build_decoder(n_layers=20, seed=0):
    from nanospeaker_amd.decoder import Decoder, DecoderConfig

    torch.manual_seed(seed)
    model = Decoder(DecoderConfig(n_layers=n_layers)).to(torch.bfloat16).eval()
    idx = torch.randint(0, 32768, (4, 8192))
    return model, idx


def attention_flops(B: int, T: int, H: int, window, dh: int = 64) -> float:
    """Useful FLOPs of one attention layer over a prefill: per (head, query), the keys it
    sees (min(q + 1, window) under a window, q + 1 without) times 2 dh for Q K^T and 2 dh
    for P V; masked scores count nothing."""
    if window is None or window >= T:
        keys = T * (T + 1) // 2
    else:
        keys = window * (window + 1) // 2 + (T - window) * window
    return float(B * H * keys * 4 * dh)


def config5(steps, warmup):
    """The 20-layer prefill (batch 4 x 8192, eval, bf16; window 512 with every fourth layer
    global): tokens/s with the HIP attention (nsmoe_attn_prefill) and the HIP MoE in every
    layer, the shares of the attention sublayers and of the MoE sublayers from HIP events
    around each call, and the same prefill with the attention on torch SDPA (the reference's
    path) for comparison."""
    model, idx = build_decoder()
    model, idx = model.cuda(), idx.cuda()
    pairs = {"attn": [], "moe": []}

    def timed(kind, fn):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        y = fn()
        b.record()
        pairs[kind].append((a, b))
        return y

    def hook(blk, h):
        # The FFN half: x + moe(norm_ffn(x)), norm and residual inside the MoE kernels.
        return timed("moe", lambda: blk.ffn.forward_residual(h, blk.norm_ffn))

    # the attention sublayer, x + attn(norm_attn(x)) minus the norm: the trunk calls
    # forward_residual (the residual is the W_O GEMM's addend on the kernel path)
    originals = [blk.attn.forward_residual for blk in model.blocks]
    reps = max(2, min(steps, 3))

    def run_timed(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            model(idx)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    with torch.no_grad():
        assert model.blocks[1].attn.use_kernel(model.embed(idx[:, :1]))
        for _ in range(max(1, min(warmup, 2))):
            model(idx)
        ms = run_timed(reps)
        for blk, fwd in zip(model.blocks, originals):
            blk.attn.forward_residual = (
                lambda x, z, fwd=fwd, **kw: timed("attn", lambda: fwd(x, z, **kw)))
        model(idx, ffn_hook=hook)
        torch.cuda.synchronize()
        for v in pairs.values():
            v.clear()
        t0 = time.perf_counter()
        model(idx, ffn_hook=hook)
        torch.cuda.synchronize()
        hooked_ms = (time.perf_counter() - t0) * 1e3
        moe_ms = sum(a.elapsed_time(b) for a, b in pairs["moe"])
        attn_ms = sum(a.elapsed_time(b) for a, b in pairs["attn"])
        for blk, fwd in zip(model.blocks, originals):
            blk.attn.forward_residual = fwd
        # the attention kernels alone, from the library's event pairs (one prefill)
        from nanospeaker_amd import _native as nat
        nat.timing_enable(4096)
        model(idx)
        torch.cuda.synchronize()
        fwd_ms, n_fwd = nat.timing_read("attn_fwd")
        prep_ms, _ = nat.timing_read("attn_k_prep")
        nat.timing_enable(0)
        B, T = idx.shape
        flops = sum(attention_flops(B, T, blk.attn.h, blk.attn.window) for blk in model.blocks)
        # the same prefill with the attention on torch SDPA
        for blk in model.blocks:
            blk.attn.kernel = False
        model(idx)
        sdpa_ms = run_timed(max(1, reps - 1))
        for blk in model.blocks:
            blk.attn.kernel = True
    n = idx.numel()
    return {"workload": "20-layer decoder prefill, batch 4 x 8192, eval, bf16; HIP attention "
                        "(QK-norm, RoPE, window 512, global_every 4) and HIP MoE with its "
                        "RMSNorm and residual in every layer",
            "tokens_per_s": round(n / (ms / 1e3), 1), "ms": round(ms, 3),
            "attn_ms": round(attn_ms, 3), "attn_share": round(attn_ms / hooked_ms, 4),
            "moe_ms": round(moe_ms, 3), "moe_share": round(moe_ms / hooked_ms, 4),
            "moe_calls": len(pairs["moe"]), "moe_tokens_per_call": n,
            "attn_fwd_kernel_ms": round(fwd_ms, 3), "attn_k_prep_ms": round(prep_ms, 3),
            "attn_fwd_launches": n_fwd,
            "attn_fwd_tflops": round(flops / (fwd_ms * 1e-3) / 1e12, 1),
            "attn_fwd_mfma_frac": round(flops / (fwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "attn_useful_tflop_per_prefill": round(flops / 1e12, 3),
            "sdpa_attention_ms": round(sdpa_ms, 3),
            "sdpa_attention_tokens_per_s": round(n / (sdpa_ms / 1e3), 1)}


def config5_head(steps, warmup):
    """The tied head with the next-token cross-entropy at the prefill batch (4 x 8192
    tokens: 32764 rows, vocabulary 32768, d 576), loss and both gradients (the training
    form, nanospeaker.py:241-250): milliseconds per call, and the HIP cross-entropy
    kernel's own time and HBM rate (each logit read once and its gradient written once)."""
    from nanospeaker_amd import _native as nat
    from nanospeaker_amd.head import linear_cross_entropy

    g = torch.Generator().manual_seed(0)
    n, V, d = 4 * 8191, 32768, 576
    h = torch.randn(n, d, generator=g).to(torch.bfloat16).cuda().requires_grad_(True)
    W = (torch.randn(V, d, generator=g) * 0.02).to(torch.bfloat16).cuda().requires_grad_(True)
    y = torch.randint(0, V, (n,), generator=g).cuda()

    def call():
        h.grad = W.grad = None
        linear_cross_entropy(h, W, y).backward()

    reps = max(3, min(steps, 10))
    ms = eager_time(call, reps, max(1, min(warmup, 3)))
    nat.timing_enable(16)
    call()
    torch.cuda.synchronize()
    ce_ms, nce = nat.timing_read("ce_rows")
    nat.timing_enable(0)
    ce_us = ce_ms * 1e3 / max(nce, 1)
    gbs = n * V * 4 / (ce_us * 1e-6) / 1e9
    gemm_tflop = 3 * 2 * n * V * d / 1e12
    return {"workload": "tied head + next-token cross-entropy, loss and dh, dW, 4 x 8191 "
                        "rows, vocab 32768, d 576, bf16 (logits in one chunk)",
            "ms": round(ms, 3), "tokens_per_s": round(n / (ms / 1e3), 1),
            "ce_rows_us": round(ce_us, 2), "ce_rows_hbm_gbs": round(gbs, 1),
            "ce_rows_hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "gemm_tflop_per_call": round(gemm_tflop, 3)}


def cpu_info():
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return {"cpu": model, "amx_bf16": "amx_bf16" in flags, "avx512_bf16": "avx512_bf16" in flags}


def cpu_threads() -> int:
    """The threads the CPU baseline uses: every core of this process's affinity, capped at
    OMP_NUM_THREADS where the launcher sets it (the GPU pool gives a one-GPU job a share
    of 16 host cores and sets OMP_NUM_THREADS=16 to match)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else n


def _median_time(fn, reps, budget_s, spread=False):
    times = []
    t_start = time.perf_counter()
    while len(times) < reps and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    if spread:
        return times[len(times) // 2], len(times), times[0], times[-1]
    return times[len(times) // 2], len(times)


def cpu_baseline(seconds: float, configs: bool):
    """The reference's eager bf16 CPU path (restated op for op in oracle/moe_ref.py,
    pinned bit-exact to the reference by tests/golden), on this host's cores."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import moe_ref as R

    cores = cpu_threads()
    torch.set_num_threads(cores)
    c = R.nanospeaker_config()
    p = R.make_params(0, c["d"], c["E"], c["d_ff"], n_shared=c["n_shared"]).to(dtype=torch.bfloat16)

    def data(T):
        return torch.randn(T, c["d"]).to(torch.bfloat16), torch.randn(T, c["d"]).to(torch.bfloat16)

    x, g = data(8192)
    R.block(x[:512], p, 6, grad_out=g[:512])  # warm-up on a slice
    med, n = _median_time(lambda: R.block(x, p, 6, grad_out=g), 5, seconds)
    out = {"value": round(8192 / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"{n} fwd+bwd steps of the eager bf16 block at T=8192 (median "
                     f"{med * 1e3:.0f} ms; oracle/moe_ref.py, torch CPU)", **cpu_info()}
    if not configs:
        return out
    per = {}
    x1, _ = data(2048)
    with torch.no_grad():
        R.block(x1, p, 6)  # warm-up at the measured size
        med, n, lo, hi = _median_time(lambda: R.block(x1, p, 6), 7, seconds / 3, spread=True)
    per["c1_T2048_fwd"] = {"tokens_per_s": round(2048 / med, 1), "runs": n,
                           "run_ms": [round(lo * 1e3, 1), round(med * 1e3, 1),
                                      round(hi * 1e3, 1)],
                           "run_ms_is": "min, median, max after one warm-up run"}
    x3, _ = data(64)
    with torch.no_grad():
        R.block(x3, p, 6, train=False)
        med, n = _median_time(lambda: R.block(x3, p, 6, train=False), 21, seconds / 3)
    per["c3_T64_eval"] = {"us_per_call": round(med * 1e6, 1), "runs": n}
    x4, g4 = data(16384)
    bias = zipf_bias()
    med, n = _median_time(lambda: R.block(x4, p, 6, grad_out=g4, logit_bias=bias), 3, seconds)
    per["c4_T16384_skew_fwd_bwd"] = {"tokens_per_s": round(16384 / med, 1), "runs": n}
    # config 5: a 4-layer stack in the 20-layer pattern (1 global + 3 windowed layers) at
    # the full batch, on the block's eager path, scaled to 20 layers; the tied head once.
    model, idx = build_decoder(n_layers=4)
    with torch.no_grad():
        def stack():
            x5, _ = model.trunk(idx)
            return x5

        t0 = time.perf_counter()
        h5 = stack()
        t_stack = time.perf_counter() - t0
        t0 = time.perf_counter()
        h5 @ model.embed.weight.t()
        t_head = time.perf_counter() - t0
    est = 5 * t_stack + t_head
    per["c5_prefill"] = {"tokens_per_s": round(idx.numel() / est, 1),
                         "sample": f"one pass of a 4-layer stack (1 global + 3 windowed) at "
                                   f"batch 4 x 8192 ({t_stack:.1f} s) x 5 + the tied head "
                                   f"({t_head:.1f} s)"}
    out["configs"] = per
    return out


def main():
    a = parse()
    if a.pmc_summary:
        print(pmc_summary(*a.pmc_summary))
        return
    if a.stats_summary:
        print(stats_summary(a.stats_summary))
        return
    if a.prefill_legs:
        print(prefill_legs(a.prefill_legs))
        return
    if a.mfma_summary:
        print(mfma_summary(*a.mfma_summary, a.stats_csv))
        return
    if a.single_stream:
        from nanospeaker_amd import _native as nat

        nat.set_option("side_stream", 0)
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is "
                                   "design-only, so --gpus must be 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if a.only:
        fns = {"c1_T2048_fwd": config1, "c3_T64_eval": config3,
               "c4_T16384_skew_fwd_bwd": config4, "c5_prefill": config5,
               "c5_head_cross_entropy": config5_head}
        out = {}
        for name in a.only.split(","):
            print(f"[bench] {name}", file=sys.stderr, flush=True)
            out[name] = fns[name](a.steps, a.warmup)
        print(json.dumps({"configs": out}), flush=True)
        return
    T = a.tokens
    if a.calibrate_copy:
        calibrate_copy()
    graph_ms = graph_fwd_ms = None
    if not a.eager:  # captured before any eager use of the module (torch's recipe)
        print(f"[bench] T={T} fwd+bwd, HIP graph", file=sys.stderr, flush=True)
        m, x, g = (t.cuda() for t in build_block(T))
        graph_ms = graph_time(train_step_fn(m, x, g), a.steps, a.warmup)
        with torch.no_grad():
            graph_fwd_ms = graph_time(lambda: m(x), a.steps, a.warmup)
        del m, x, g
    # The eager timing on a fresh copy of the block (same seed, same weights): the graph
    # recipe's side-stream warm-up leaves the parameters' gradient-accumulation nodes on
    # that stream, and later eager steps of the same module would pay a cross-stream
    # synchronisation per parameter.
    print(f"[bench] T={T} eager and per-kernel timing", file=sys.stderr, flush=True)
    m, x, g = (t.cuda() for t in build_block(T))
    ms, fwd_ms, kernels, host_ms = time_gpu(m, x, g, a.steps, a.warmup)
    eager_ms, eager_fwd_ms = ms, fwd_ms
    if not a.eager:
        ms, fwd_ms = graph_ms, graph_fwd_ms
    del m, x, g

    k, S, d, H, E = 6, 2, 576, 128, 76
    dom = max(kernels, key=lambda n: kernels[n][0] * kernels[n][1]) if kernels else None
    roofline = None
    if dom:
        units, bound, unit, extra = roofline_of(dom, T, k, S, d, H, E)
        avg_s = kernels[dom][0] / 1e3
        if bound == "mfma":
            achieved, peak = units / avg_s / 1e12, PEAK_BF16_TFLOPS
        else:
            achieved, peak = units / avg_s / 1e9, PEAK_HBM_GBS
        roofline = {"kernel": dom, "bound": bound, "achieved": round(achieved, 2),
                    "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
                    "traffic": committed_traffic(dom) if T == 8192 else None,
                    "traffic_source": "profiles/" + os.path.basename(TRAFFIC_FILE),
                    "avg_launch_us": round(kernels[dom][0] * 1e3, 2),
                    "algorithmic_per_launch": units}
        if extra:  # the same launch against the HBM roof, from its algorithmic bytes
            gbs = extra["bytes_per_launch"] / avg_s / 1e9
            roofline.update(algorithmic_bytes_per_launch=extra["bytes_per_launch"],
                            hbm_algorithmic_gbs=round(gbs, 1),
                            hbm_frac=round(gbs / PEAK_HBM_GBS, 4))
    rec = {
        "metric": "MoE-block tokens/s fwd & fwd+bwd at T=8192 bf16; % of MFMA / HBM peak",
        "value": round(T / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"nanoSpeaker MoE block fwd+bwd, T={T} (training shape)",
                   "n_tokens": T, "d_model": d, "n_experts": E, "n_shared": S, "top_k": k,
                   "d_hidden": H, "mode": "train, aux_loss 1e-2",
                   "issue": "eager" if a.eager else "hip_graph"},
        "fwd_tokens_per_s": round(T / (fwd_ms / 1e3), 1),
        "fwd_ms": round(fwd_ms, 4),
        "eager_tokens_per_s": round(T / (eager_ms / 1e3), 1),
        "eager_ms_per_step": round(eager_ms, 4),
        "eager_fwd_tokens_per_s": round(T / (eager_fwd_ms / 1e3), 1),
        "host_enqueue_ms_per_step": round(host_ms, 4),
        "kernels_us": {n: round(v[0] * 1e3, 2) for n, v in kernels.items()},
        "roofline": roofline,
    }
    if not a.no_configs:
        torch.cuda.empty_cache()
        confs = {}
        for name, fn in (("c1_T2048_fwd", config1), ("c3_T64_eval", config3),
                         ("c4_T16384_skew_fwd_bwd", config4), ("c5_prefill", config5),
                         ("c5_head_cross_entropy", config5_head)):
            print(f"[bench] {name}", file=sys.stderr, flush=True)
            confs[name] = fn(a.steps, a.warmup)
            torch.cuda.empty_cache()
        rec["configs"] = confs
        print("[bench] routing flips against the CPU router GEMM", file=sys.stderr, flush=True)
        rec["routing_flips"] = routing_flips()
    if not a.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        rec["cpu_baseline"] = cpu_baseline(a.cpu_seconds, not a.no_configs)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
