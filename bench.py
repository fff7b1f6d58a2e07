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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--no-cpu-baseline", action="store_true")
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
    if name == "expert_bwd":        # G = dout W_out^T per row (the a1 recompute not counted)
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
    if name == "route_fwd":         # bf16 logits in, fp32 probs out, ids + gates out
        return T * (E * 2 + E * 4 + k * 8 + k * 2), "hbm", "GB/s"
    if name == "dispatch":          # ids read twice, sorted ids + inverse written
        return T * k * (8 * 2 + 4 + 4), "hbm", "GB/s"
    if name == "combine_dx":        # expert dX rows + d(logits) in, dx out, per token
        return T * ((k + S) * d * 2 + (E + 7) // 8 * 8 * 2 + d * 2 + k * 4), "hbm", "GB/s"
    if name == "router_dw":         # x and d(logits) read once
        return T * (d * 2 + (E + 7) // 8 * 8 * 2), "hbm", "GB/s"
    if name == "pack":              # W_in (routed + shared) read once and written once
        return (E + S) * d * 2 * H * 2 * 2, "hbm", "GB/s"
    return None


def time_gpu(m, x, g, steps: int, warmup: int):
    from nanospeaker_amd import _native as nat

    params = [p for p in m.parameters()]
    xg = x.detach().requires_grad_(True)
    one = torch.ones((), dtype=torch.float32, device=x.device)

    def step():
        # Every gradient of the block (input, router, experts) is computed and returned;
        # none is accumulated into a .grad buffer.
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
    nat.set_option("single_stream", 1)
    try:
        step()
        torch.cuda.synchronize()
        nat.timing_enable(64 * steps + 64)
        torch.cuda.synchronize()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        kernels = {}
        for name in ("route_fwd", "dispatch", "pack", "expert_fwd", "combine", "expert_bwd",
                     "expert_dx", "dw_in", "dw_out", "dw", "combine_dx", "router_dw"):
            tot, n = nat.timing_read(name)
            if n:
                kernels[name] = (tot / n, n // steps)
        nat.timing_enable(0)
    finally:
        nat.set_option("single_stream", 0)

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
    "expert_dx": ("nsmoe::expert_dx_reg_kernel", "nsmoe::expert_dx_async_kernel"),
    "dw": ("nsmoe::dw_pair_kernel",),
    "dw_in": ("nsmoe::dw_async_kernel<0, 0", "nsmoe::dw_kernel<0, 0"),
    "dw_out": ("nsmoe::dw_async_kernel<0, 1", "nsmoe::dw_kernel<0, 1"),
    "route_fwd": ("nsmoe::route_fwd_kernel",),
    "combine": ("nsmoe::combine_kernel",),
    "combine_dx": ("nsmoe::combine_dx_kernel",),
    "pack": ("nsmoe::pack_kernel", "nsmoe::pack_ks_kernel"),
    "dispatch": ("nsmoe::dispatch_hist_kernel", "nsmoe::dispatch_place_kernel"),
    "router_dw": ("nsmoe::router_dw_kernel", "nsmoe::router_dw_reduce_kernel"),
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


def time_gpu_graph(m, x, g, steps: int, warmup: int):
    """The same fwd+bwd step (and the forward alone), captured once in a HIP graph and
    replayed: every replay runs every kernel of the step on the resident inputs; only the
    host-side enqueue (Python, autograd, the library's argument setup) is removed.
    torch's capture recipe: warm-up on a side stream, then capture."""
    params = [p for p in m.parameters()]
    xg = x.detach().requires_grad_(True)
    one = torch.ones((), dtype=torch.float32, device=x.device)

    def step():
        # All gradients of the block (input, router, experts) are returned by the step, in
        # the graph's own memory; no .grad buffer is zeroed or accumulated into.
        out = m(xg)
        return torch.autograd.grad([out, m.aux_loss], [xg] + params, [g, one])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 2)):
            step()
        with torch.no_grad():
            for _ in range(2):
                m(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    fwd_graph = torch.cuda.CUDAGraph()
    with torch.no_grad():
        with torch.cuda.graph(fwd_graph):
            m(x)

    def timed(gr):
        for _ in range(warmup):
            gr.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            gr.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    return timed(graph), timed(fwd_graph)


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


def cpu_baseline(seconds: float):
    """The reference's eager bf16 CPU path (restated in oracle/moe_ref.py), fwd + bwd."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import moe_ref as R

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    c = R.nanospeaker_config()
    p = R.make_params(0, c["d"], c["E"], c["d_ff"], n_shared=c["n_shared"]).to(dtype=torch.bfloat16)
    T = 8192
    x = torch.randn(T, c["d"]).to(torch.bfloat16)
    g = torch.randn(T, c["d"]).to(torch.bfloat16)
    R.block(x[:512], p, c["top_k"], grad_out=g[:512])  # warm-up on a slice
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < seconds:
        t0 = time.perf_counter()
        R.block(x, p, c["top_k"], grad_out=g)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(T / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
        "sample": f"{len(times)} fwd+bwd steps of the eager bf16 block at T=8192 "
                  f"(median {med * 1e3:.0f} ms; oracle/moe_ref.py, torch CPU)",
    }


def main():
    a = parse()
    if a.pmc_summary:
        print(pmc_summary(*a.pmc_summary))
        return
    if a.stats_summary:
        print(stats_summary(a.stats_summary))
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is "
                                   "design-only, so --gpus must be 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    T = a.tokens
    if a.calibrate_copy:
        calibrate_copy()
    m, x, g = build_block(T)
    m = m.cuda()
    x, g = x.cuda(), g.cuda()
    if not a.eager:  # captured before any eager use of the module (torch's recipe)
        graph_ms, graph_fwd_ms = time_gpu_graph(m, x, g, a.steps, a.warmup)
    ms, fwd_ms, kernels, host_ms = time_gpu(m, x, g, a.steps, a.warmup)
    eager_ms, eager_fwd_ms = ms, fwd_ms
    if not a.eager:
        ms, fwd_ms = graph_ms, graph_fwd_ms

    k, S, d, H, E = 6, 2, 576, 128, 76
    dom = max(kernels, key=lambda n: kernels[n][0] * kernels[n][1]) if kernels else None
    roofline = None
    if dom:
        units, bound, unit = kernel_units(dom, T, k, S, d, H, E)
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
    if not a.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
