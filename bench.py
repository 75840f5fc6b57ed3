#!/usr/bin/env python3
"""Benchmark of the W8A8 INT8 linear and the fused DiT norm kernels on one MI355X.

Step = one pass of the hot path over one batch of the QKV workload
(X[32768, 5120] bf16 with 0.1% of elements scaled x20, W int8 [15360, 5120],
per-channel fp32 scales, bf16 bias): per-token quantize + int8 GEMM with the
fused dequant/bias epilogue.  value = 2*M*N*K / step time (TOPS), inputs
resident in HBM.  The same run also reports:
  roofline      the GEMM kernel's own time (HIP events around each launch;
                for the small C0 linear, where an event pair around one launch
                also measures the host's submission of it, one event pair
                around 50 back-to-back launches) against the dense INT8 MFMA
                peak;
  cpu_baseline  the same linear in PyTorch eager on the host CPU cores, on a
                row sample, and whether its output equals the GPU's;
  vendor        torch._int_mm (hipBLASLt, int32 out, no epilogue) on the shape;
  norms         GB/s of norm_mod / gate_norm_mod_ / gate_ and the quantizer
                on x[32768, 5120] against the 8 TB/s HBM peak.
Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "minimax-h3-multi-dgx-spark_amd")

METRIC = "INT8 GEMM TOPS (% of MI355X INT8 peak) at H3 DiT shapes; fused-norm GB/s"
PEAK_INT8_TOPS = 5000.0    # MI355X dense INT8 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

WORKLOADS = {
    # name: (M, N, K, outlier fraction, input, seed, description)
    "qkv": (32768, 15360, 5120, 0.001, "randn", 1, "H3-like DiT fused QKV projection W8A8 (quantize + GEMM + bias)"),
    "up": (32768, 13824, 5120, 0.0, "randn", 2, "H3-like DiT MLP up projection W8A8 (quantize + GEMM + bias)"),
    "down": (32768, 5120, 13824, 0.0, "gelu", 2,
             "H3-like DiT MLP down projection W8A8 on GELU-tanh activations (quantize + GEMM + bias)"),
    "c0": (2048, 3072, 3072, 0.0, "randn", 0, "single W8A8 linear X[2048,3072] W[3072,3072] (quantize + GEMM + bias)"),
}
SHARD_M = 4096  # one GPU's rows of the QKV workload when the tokens are split over 8 GPUs


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["block", "h3"], default="qkv",
                    help="block: one H3-like DiT block forward; h3: the real H3 DiT linears (hidden 5376) and fused "
                         "norms at --tokens rows (each prints its own JSON line)")
    ap.add_argument("--tokens", type=int, default=19200, help="h3 workload: tokens per GPU (19200 or 38400)")
    ap.add_argument("--settle", type=float, default=1.0, metavar="SECONDS",
                    help="before the warm-up steps, run the step back to back for this long so the shader clock has "
                         "settled at the level the chip holds under this load (the timed steps then measure the "
                         "sustained rate, not the first milliseconds after idle); the norm, quantizer and H3 layer "
                         "timings settle for min(SECONDS, 0.25) each; 0 disables")
    ap.add_argument("--fuse-quant", action="store_true",
                    help="block workload: the norms that feed a linear also quantize h (norm_mod_q / gate_norm_mod_q_) "
                         "and the linear takes the int8 rows directly")
    ap.add_argument("--only", choices=["all", "gemm", "norms"], default="all",
                    help="gemm: skip the norm section; norms: only the norm section")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (the vendor GEMM still runs)")
    ap.add_argument("--no-mlp-block", action="store_true",
                    help="skip the MLP pair and block sections of the default line (shorter counter runs)")
    ap.add_argument("--summarize", nargs="+", metavar="DIR",
                    help="no GPU work: print a markdown summary of rocprofv3 output directories (kernel stats and "
                         "FETCH_SIZE / WRITE_SIZE counter runs of this script) and exit")
    ap.add_argument("--sustain", type=float, metavar="SECONDS",
                    help="run this library's QKV GEMM, then hipBLASLt's on the same operands, back to back for SECONDS "
                         "each with the shader clock sampled from rocm-smi; print throughput, median clock and int8 "
                         "ops per CU per clock (the MFMA's dense peak is 8192) and exit")
    ap.add_argument("--traffic-out", metavar="FILE",
                    help="with --summarize: also write the calibrated HBM bytes per launch (the file this script "
                         "reads for roofline.traffic)")
    return ap.parse_args()


def read_traffic(kernel):
    """HBM bytes per launch measured by rocprofv3 PMC runs (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 2 and parts[0] == kernel:
                try:
                    return float(parts[1])
                except ValueError:
                    return None
    return None


# Kernels named in the traffic file, matched by substring of the rocprof kernel name.
TRAFFIC_KERNELS = {
    # tag: substrings of the kernel names (any matches)
    "w8a8_gemm": ("w8a8_gemm_direct_kernel",),
    "quant_rowwise": ("quant_multi_kernel",),
    "norm_mod": ("norm_stream_kernel<256, 64, 10, false, 0>",),
    "gate_norm_mod_": ("norm_stream_kernel<256, 64, 10, true, 0>", "gate_norm_split_kernel<5, 0>"),
    "gate_": ("gate_stream_kernel<10>",),
    "norm_mod_q": ("norm_stream_kernel<256, 64, 10, false, 1>",),
    "gate_norm_mod_q_": ("norm_stream_kernel<256, 64, 10, true, 1>",),
    # the real H3 workload (--workload h3): ConvRot shapes of qkv/fc1 (K=5376), out (K=7168) and fc2 (SwiGLU),
    # the norms at hidden 5376 (11 chunks), q/k RMSNorm + RoPE
    "convrot_k5376": ("convrot_quant_kernel<3, 2, false>",),
    "convrot_k7168": ("convrot_quant_kernel<2, 4, false>",),
    "convrot_swiglu": ("convrot_quant_kernel<4, 4, true>",),
    "norm_mod_h3": ("norm_stream_kernel<256, 64, 11, false, 0>",),
    "gate_norm_mod_h3": ("norm_stream_kernel<256, 64, 11, true, 0>", "gate_norm_split_kernel<5, 1>"),
    "gate_h3": ("gate_stream_kernel<11>",),
    "rms_rope": ("rms_rope_kernel",),
    # hipBLASLt's int8 GEMM (torch._int_mm, the vendor line) on the same operands
    "hipblaslt_i8": ("Cijk_",),
}
COPY_KERNEL = "__amd_rocclr_copyBuffer"
SIMDS, XCDS = 1024, 8  # MI355X: 256 CUs x 4 SIMDs in 8 XCDs
COPY_BYTES = 2.0 * 32768 * 5120  # the device copy in the norm section: bytes read (and written) per launch


def _short(name):
    return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:110]


def _gemm_segments(items):
    """items: (order key, kernel name, grid, payload) of one run, any kernels.  Returns (segment, payload, name,
    grid) per item, where the segment of a GEMM dispatch counts how often the GEMM's (kernel, grid) changed before
    it in launch order: a resident grid has the same size for every shape, so back-to-back runs of one shape are
    told apart by their order instead (others get segment 0)."""
    pats = TRAFFIC_KERNELS["w8a8_gemm"]
    out, prev, seg = [], None, 0
    for _, name, grid, payload in sorted(items, key=lambda t: t[0]):
        sg = 0
        if any(p in name for p in pats):
            if prev is not None and prev != (name, grid):
                seg += 1
            prev = (name, grid)
            sg = seg + 1
        out.append((sg, payload, name, grid))
    return out


def summarize(dirs, traffic_out):
    """Markdown summary of rocprofv3 runs of this script: kernel statistics per (kernel, grid size) from the
    kernel trace, and per-dispatch FETCH_SIZE / WRITE_SIZE scaled so that the device copy of COPY_BYTES reads
    (writes) COPY_BYTES.  GEMM rows are further split by launch segment (see _gemm_segments), numbered in launch
    order.  The traffic file gets, per kernel, the launch group that moves the most bytes per launch: the full
    workload (the others are the 8-way shard shape and the parity-size calls)."""
    import csv
    import glob
    trace, disp = [], []
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
            rows = []
            for r in csv.DictReader(open(f)):
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                rows.append((int(r["Start_Timestamp"]), r["Kernel_Name"], grid, us))
            trace += _gemm_segments(rows)
        for f in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            per = {}
            for r in csv.DictReader(open(f)):
                e = per.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"], "grid": int(r["Grid_Size"])})
                e[r["Counter_Name"]] = float(r["Counter_Value"])
            disp += _gemm_segments([(k, e["name"], e["grid"], e) for k, e in per.items()])
    out = []

    def label(name, seg):
        return f"`{_short(name)}`" + (f" (segment {seg})" if seg else "")

    if trace:
        groups = {}
        for seg, us, name, grid in trace:
            groups.setdefault((name, grid, seg), []).append(us)
        total = sum(us for _, us, _, _ in trace)
        out += ["| kernel | grid (threads) | calls | average (us) | median (us) | min (us) | max (us) | share |",
                "|---|---|---|---|---|---|---|---|"]
        for (name, grid, seg), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"| {label(name, seg)} | {grid} | {len(v)} | {statistics.mean(v):.1f} | "
                       f"{statistics.median(v):.1f} | {min(v):.1f} | {max(v):.1f} | {100 * sum(v) / total:.1f}% |")
        out.append("")
    traffic = {}
    for cname in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = [(seg, e[cname], name, grid) for seg, e, name, grid in disp if cname in e]
        if not rows:
            continue
        big = [v for _, v, k, _ in rows if COPY_KERNEL in k and v * 1024 >= 0.5 * COPY_BYTES]
        if not big:
            out.append(f"{cname}: no device copy of {COPY_BYTES:.0f} bytes found to calibrate against")
            continue
        factor = COPY_BYTES / (statistics.mean(big) * 1024)
        out.append(f"{cname}: device copy of {COPY_BYTES / 1e6:.1f} MB reads {statistics.mean(big) * 1024 / 1e6:.1f} MB "
                   f"by the counter over {len(big)} launches: scale factor {factor:.4f}")
        out += ["", f"| kernel | grid (threads) | launches | {cname} (KiB, raw) | calibrated bytes per launch |",
                "|---|---|---|---|---|"]
        for tag, pats in TRAFFIC_KERNELS.items():
            groups = {}
            for seg, v, k, grid in rows:
                if any(p in k for p in pats):
                    groups.setdefault((k, grid, seg), []).append(v)
            if not groups:
                continue
            full = max(groups, key=lambda g: statistics.mean(groups[g]))
            for key in sorted(groups, key=lambda g: -statistics.mean(groups[g])):
                vals = groups[key]
                b = statistics.mean(vals) * 1024 * factor
                if key == full:
                    traffic[tag] = traffic.get(tag, 0.0) + b
                short = _short(key[0])
                if "DTile<" in short:  # the tile configuration is what tells the GEMM rows apart
                    short = short[short.index("DTile<"):].split(">")[0] + ">"
                short = f"`{short[:70]}`" + (f" (segment {key[2]})" if key[2] else "")
                out.append(f"| {tag}: {short} | {key[1]} | {len(vals)} | "
                           f"{statistics.mean(vals):.0f} | {b / 1e6:.1f} MB |")
        out.append("")
    mfma = [(seg, e) for seg, e, _, _ in disp if e.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) > 0 and "GRBM_GUI_ACTIVE" in e]
    if mfma:
        # SQ_VALU_MFMA_BUSY_CYCLES is summed over the SIMDs, GRBM_GUI_ACTIVE over the XCDs (one value per dispatch)
        out += [f"MFMA utilisation per dispatch (MFMA busy cycles / {SIMDS} SIMDs over GPU-active cycles / {XCDS} "
                f"XCDs):", "", "| kernel | grid (threads) | dispatches | MFMA busy per SIMD | active cycles per XCD |",
                "|---|---|---|---|---|"]
        groups = {}
        for seg, e in mfma:
            groups.setdefault((e["name"], e["grid"], seg), []).append(e)
        for (name, grid, seg), ds in sorted(groups.items(), key=lambda kv: kv[0][2]):
            util = [x["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS / (x["GRBM_GUI_ACTIVE"] / XCDS) for x in ds]
            act = [x["GRBM_GUI_ACTIVE"] / XCDS for x in ds]
            out.append(f"| {label(name, seg)} | {grid} | {len(ds)} | {100 * statistics.median(util):.1f}% | "
                       f"{statistics.median(act):.3g} |")
        out.append("")
    valu = [(seg, e) for seg, e, _, _ in disp if "SQ_ACTIVE_INST_VALU" in e and e.get("GRBM_GUI_ACTIVE", 0) > 0]
    if valu:
        # SQ_ACTIVE_INST_VALU counts issue cycles in units of 4 (a wave64 VALU instruction holds a 16-lane SIMD for
        # 4 cycles), summed over the SIMDs; SQ_INSTS_VALU is the wave-level instruction count
        out += [f"VALU utilisation per dispatch (SQ_ACTIVE_INST_VALU x 4 / {SIMDS} SIMDs over GPU-active cycles / "
                f"{XCDS} XCDs):", "", "| kernel | grid (threads) | dispatches | VALU busy per SIMD | VALU instructions "
                "(wave) | active cycles per XCD |", "|---|---|---|---|---|---|"]
        groups = {}
        for seg, e in valu:
            groups.setdefault((e["name"], e["grid"], seg), []).append(e)
        for (name, grid, seg), ds in sorted(groups.items(), key=lambda kv: -kv[1][0]["GRBM_GUI_ACTIVE"]):
            util = [4 * x["SQ_ACTIVE_INST_VALU"] / SIMDS / (x["GRBM_GUI_ACTIVE"] / XCDS) for x in ds]
            ins = statistics.median(x.get("SQ_INSTS_VALU", 0.0) for x in ds)
            act = [x["GRBM_GUI_ACTIVE"] / XCDS for x in ds]
            out.append(f"| {label(name, seg)} | {grid} | {len(ds)} | {100 * statistics.median(util):.1f}% | "
                       f"{ins:.4g} | {statistics.median(act):.3g} |")
        out.append("")
    lds = [(seg, e) for seg, e, _, _ in disp if "SQ_LDS_BANK_CONFLICT" in e and e.get("SQ_INSTS_LDS", 0) > 0]
    if lds:
        out += ["LDS bank conflicts per dispatch (SQ_LDS_BANK_CONFLICT cycles per LDS instruction, both summed "
                "over the SIMDs):", "", "| kernel | grid (threads) | dispatches | LDS instructions | conflict cycles "
                "| per instruction |", "|---|---|---|---|---|---|"]
        groups = {}
        for seg, e in lds:
            groups.setdefault((e["name"], e["grid"], seg), []).append(e)
        for (name, grid, seg), ds in sorted(groups.items(), key=lambda kv: -kv[1][0]["SQ_INSTS_LDS"]):
            ins = statistics.median(x["SQ_INSTS_LDS"] for x in ds)
            cf = statistics.median(x["SQ_LDS_BANK_CONFLICT"] for x in ds)
            out.append(f"| {label(name, seg)} | {grid} | {len(ds)} | {ins:.4g} | {cf:.4g} | {cf / ins:.4f} |")
        out.append("")
    if traffic:
        out += ["HBM bytes per launch at the full workload (per kernel the launch group that moves the most bytes; "
                "FETCH + WRITE, calibrated):", ""]
        out += [f"* {k}: {v / 1e6:.1f} MB" for k, v in traffic.items()]
        if traffic_out:
            with open(traffic_out, "w") as f:
                f.write("# kernel  HBM bytes per launch at the full workload (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                        "copy-calibrated)\n")
                for k, v in traffic.items():
                    f.write(f"{k} {v:.0f}\n")
    print("\n".join(out))


def make_linear_inputs(torch, M, N, K, outliers, seed, kind="randn"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if kind == "gelu":
        x = torch.nn.functional.gelu(x, approximate="tanh")
    if outliers > 0:  # exactly that fraction of the elements, chosen without repetition, times 20
        n_out = int(outliers * M * K)
        idx = torch.randperm(M * K, generator=g)[:n_out]
        x.view(-1)[idx] *= 20
    x = x.to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    ws = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    bias = (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16)
    return x, w, ws, bias


def settle(torch, fn, seconds):
    """Run fn back to back for about `seconds` (in batches of 10 launches), untimed."""
    if seconds <= 0:
        return
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def settled_events(torch, fn, n, seconds):
    """timed_events after running fn back to back for `seconds`: the first launches after an idle moment (the
    bench builds each section's inputs on the CPU meanwhile) run up to 10% slower than the steady state a busy
    forward pass keeps, as the GEMM lines' settle phase already allows for."""
    settle(torch, fn, seconds)
    return timed_events(torch, fn, n)


def timed_events(torch, fn, n):
    """Run fn n times back to back between one HIP event pair; mean ms per launch.  An event pair around every
    launch would add the gap between each start event and its kernel (1-4 us, a few percent of a norm kernel)."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(n):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def bench_linear(torch, h3mi, args):
    M, N, K, outl, kind, seed, desc = WORKLOADS[args.workload]
    log(f"[bench] workload {args.workload}: M={M} N={N} K={K}")
    x_cpu, w_cpu, ws_cpu, b_cpu = make_linear_inputs(torch, M, N, K, outl, seed=seed, kind=kind)
    dev = torch.device("cuda", 0)
    x, w, ws, bias = (t.to(dev) for t in (x_cpu, w_cpu, ws_cpu, b_cpu))
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M, 1), dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def quant():
        h3mi.quantize_rowwise(x, xq, xs)

    def gemm():
        h3mi.int8_mm_scaled(xq, w, xs, ws, out=out, bias=bias)

    settle(torch, lambda: (quant(), gemm()), args.settle)
    for _ in range(args.warmup):
        quant()
        gemm()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e in ev:
        e[0].record()
        quant()
        e[1].record()
        gemm()
        e[2].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    gemm_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in ev)
    quant_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in ev)
    ops = 2.0 * M * N * K
    res = {
        "M": M, "N": N, "K": K, "desc": desc,
        "ms_per_step": ms_step,
        "tops": ops / (ms_step * 1e-3) / 1e12,
        "gemm_ms": gemm_ms,
        "gemm_tops": ops / (gemm_ms * 1e-3) / 1e12,
        "quant_ms": quant_ms,
        "quant_gbs": (3.0 * M * K + 4.0 * M) / (quant_ms * 1e-3) / 1e9,
        "tile_config": h3mi.config_for(M, N, K),
    }
    log(f"[bench] step {ms_step:.3f} ms ({res['tops']:.1f} TOPS); GEMM {gemm_ms:.3f} ms ({res['gemm_tops']:.1f} TOPS); "
        f"quantizer {quant_ms:.3f} ms ({res['quant_gbs']:.0f} GB/s); tile {res['tile_config']}")
    if ops < 1e12:
        # For a kernel this short an event pair around each launch also times the host's submission of it (the GPU
        # idles until the launch arrives).  Back-to-back launches keep the queue ahead of the GPU, so one event pair
        # around them times the kernels (median of 5 batches of 50).
        b2b = sorted(timed_events(torch, gemm, 50) for _ in range(5))
        res["gemm_b2b_ms"] = b2b[2]
        res["gemm_b2b_tops"] = ops / (res["gemm_b2b_ms"] * 1e-3) / 1e12
        log(f"[bench] GEMM back to back (median of 5 x 50 launches): {res['gemm_b2b_ms'] * 1e3:.1f} us "
            f"({res['gemm_b2b_tops']:.1f} TOPS)")

    # vendor GEMM on the same operands (int32 out, no epilogue)
    wt = w.t()
    for _ in range(2):
        torch._int_mm(xq, wt)
    vend_ms = timed_events(torch, lambda: torch._int_mm(xq, wt), 5)
    res["vendor"] = {"name": "torch._int_mm (hipBLASLt), int32 out, no epilogue",
                     "ms": vend_ms, "tops": ops / (vend_ms * 1e-3) / 1e12}
    log(f"[bench] vendor torch._int_mm {vend_ms:.3f} ms ({res['vendor']['tops']:.1f} TOPS)")
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_linear(torch, x_cpu, w_cpu, ws_cpu, b_cpu, out, M, N, K)
    if args.workload == "qkv":
        # one GPU's share when the tokens are split over 8 GPUs: the same weights, M = 4096
        xq_s, xs_s, out_s = xq[:SHARD_M], xs[:SHARD_M], out[:SHARD_M]
        shard = lambda: h3mi.int8_mm_scaled(xq_s, w, xs_s, ws, out=out_s, bias=bias)
        settle(torch, shard, min(args.settle, 0.5))
        for _ in range(3):
            shard()
        sh_ms = timed_events(torch, shard, 20)
        res["shard"] = {"M": SHARD_M, "N": N, "K": K, "gemm_ms": sh_ms,
                        "tops": 2.0 * SHARD_M * N * K / (sh_ms * 1e-3) / 1e12,
                        "tile_config": h3mi.config_for(SHARD_M, N, K)}
        log(f"[bench] 8-way token shard M={SHARD_M}: GEMM {sh_ms:.3f} ms ({res['shard']['tops']:.1f} TOPS)")
    return res


def bench_mlp(torch, h3mi, args):
    """The C2 workload (the MLP pair) at its own shapes: the MLP up (32768 x 5120 -> 13824, X ~ N(0,1)) and down (32768 x 13824 ->
    5120, X = GELU-tanh of N(0,1), re-quantized per token) projections, each as per-token quantize + GEMM + bias,
    timed per kernel with HIP events; hipBLASLt (torch._int_mm) on the same operands beside each GEMM."""
    res = {}
    dev = torch.device("cuda", 0)
    n = max(5, min(args.steps, 20))
    for name in ("up", "down"):
        M, N, K, outl, kind, seed, desc = WORKLOADS[name]
        x_cpu, w_cpu, ws_cpu, b_cpu = make_linear_inputs(torch, M, N, K, outl, seed=seed, kind=kind)
        x, w, ws, bias = (t.to(dev) for t in (x_cpu, w_cpu, ws_cpu, b_cpu))
        del x_cpu
        xq = torch.empty((M, K), dtype=torch.int8, device=dev)
        xs = torch.empty((M, 1), dtype=torch.float32, device=dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        quant = lambda: h3mi.quantize_rowwise(x, xq, xs)
        gemm = lambda: h3mi.int8_mm_scaled(xq, w, xs, ws, out=out, bias=bias)
        settle(torch, lambda: (quant(), gemm()), min(args.settle, 0.5))
        for _ in range(max(2, args.warmup)):
            quant()
            gemm()
        q_ms = timed_events(torch, quant, n)
        g_ms = timed_events(torch, gemm, n)
        wt = w.t()
        torch._int_mm(xq, wt)
        v_ms = timed_events(torch, lambda: torch._int_mm(xq, wt), 5)
        ops = 2.0 * M * N * K
        qb = 3.0 * M * K + 4.0 * M
        res[name] = {"M": M, "N": N, "K": K, "input": kind, "gemm_ms": g_ms, "gemm_tops": ops / g_ms / 1e9,
                     "frac": ops / g_ms / 1e9 / PEAK_INT8_TOPS, "quant_ms": q_ms, "quant_gbs": qb / q_ms / 1e6,
                     "quant_frac": qb / q_ms / 1e6 / PEAK_HBM_GBS, "vendor_ms": v_ms, "vendor_tops": ops / v_ms / 1e9,
                     "tile_config": h3mi.config_for(M, N, K)}
        log(f"[bench] mlp {name} M={M} K={K} N={N} ({kind} input): GEMM {g_ms:.3f} ms ({ops / g_ms / 1e9:.0f} TOPS, "
            f"{100 * ops / g_ms / 1e9 / PEAK_INT8_TOPS:.1f}%), quantizer {q_ms * 1e3:.1f} us ({qb / q_ms / 1e6:.0f} GB/s); "
            f"hipBLASLt {v_ms:.3f} ms ({ops / v_ms / 1e9:.0f} TOPS)")
        del x, w, xq, out
        torch.cuda.empty_cache()
    return res


def smi_sclk():
    """Current shader clock of card 0 in MHz from rocm-smi, or None."""
    import re
    import subprocess
    try:
        out = subprocess.run(["rocm-smi", "--showclocks", "--json"], capture_output=True, text=True, timeout=10).stdout
        for card in json.loads(out[out.index("{"):]).values():
            m = re.search(r"(\d+)\s*Mhz", card.get("sclk clock speed:", ""))
            if m:
                return float(m.group(1))
    except (OSError, ValueError, subprocess.SubprocessError):
        return None
    return None


def bench_sustain(torch, h3mi, args):
    """Each GEMM back to back for args.sustain seconds on the QKV operands, the shader clock sampled
    alongside (rocm-smi, every ~0.3 s; samples of the first second are dropped).  Ops per CU per clock
    = throughput / (median clock x CUs): the share of the MFMA's peak that the kernel reaches at the clock the
    chip actually holds under it."""
    import threading
    M, N, K, outl, kind, seed, _ = WORKLOADS["qkv"]
    x_cpu, w_cpu, ws_cpu, b_cpu = make_linear_inputs(torch, M, N, K, outl, seed=seed, kind=kind)
    dev = torch.device("cuda", 0)
    x, w, ws, bias = (t.to(dev) for t in (x_cpu, w_cpu, ws_cpu, b_cpu))
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M, 1), dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    h3mi.quantize_rowwise(x, xq, xs)
    wt = w.t()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ops = 2.0 * M * N * K
    res = {"M": M, "N": N, "K": K, "seconds": args.sustain, "cus": cus, "kernels": {}}
    for name, fn in (("w8a8_gemm (this library, bf16 epilogue)",
                      lambda: h3mi.int8_mm_scaled(xq, w, xs, ws, out=out, bias=bias)),
                     ("torch._int_mm (hipBLASLt, int32 out, no epilogue)", lambda: torch._int_mm(xq, wt))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        samples, stop = [], threading.Event()

        def sample():
            while not stop.is_set():
                v = smi_sclk()
                if v is not None:
                    samples.append((time.perf_counter(), v))
                stop.wait(0.3)

        th = threading.Thread(target=sample, daemon=True)
        t0 = time.perf_counter()
        th.start()
        n = 0
        while time.perf_counter() - t0 < args.sustain:
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
            n += 20
        t1 = time.perf_counter()
        stop.set()
        th.join()
        steady = [v for t, v in samples if t - t0 > 1.0] or [v for _, v in samples]
        sclk = statistics.median(steady) if steady else None
        tops = ops * n / (t1 - t0) / 1e12
        per_clk = tops * 1e12 / (sclk * 1e6 * cus) if sclk else None
        res["kernels"][name] = {"launches": n, "tops": tops, "ms_per_launch": (t1 - t0) * 1e3 / n,
                                "sclk_mhz_median": sclk, "sclk_samples": len(steady),
                                "sclk_mhz_min": min(steady) if steady else None,
                                "sclk_mhz_max": max(steady) if steady else None,
                                "ops_per_cu_clk": per_clk, "mfma_frac_at_clock": per_clk / 8192 if per_clk else None}
        log(f"[bench] sustained {name}: {tops:.0f} TOPS over {n} launches; shader clock median "
            f"{sclk if sclk else float('nan'):.0f} MHz ({len(steady)} samples); "
            f"{per_clk if per_clk else float('nan'):.0f} int8 ops per CU per clock "
            f"({100 * per_clk / 8192 if per_clk else float('nan'):.1f}% of the MFMA peak at that clock)")
    return res


def cpu_linear(torch, x_cpu, w_cpu, ws_cpu, b_cpu, out_gpu, M, N, K, budget_s=20.0):
    """The same linear in PyTorch eager on the host cores: the whole workload, a warm-up on 64 rows, then up to 3
    timed runs (median) while the total stays within about budget_s seconds."""
    sys.path.insert(0, ROOT)
    from oracle import torch_cpu
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch_cpu.w8a8_linear(x_cpu[:64].contiguous(), w_cpu, ws_cpu, b_cpu)  # warm-up
    times, y = [], None
    while len(times) < 3 and (not times or sum(times) + times[-1] <= budget_s):
        t0 = time.perf_counter()
        y = torch_cpu.w8a8_linear(x_cpu, w_cpu, ws_cpu, b_cpu)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    ops = 2.0 * M * N * K
    match = bool(torch.equal(y, out_gpu.cpu()))
    log(f"[bench] CPU eager baseline: {M} rows in {t:.3f} s ({ops / t / 1e12:.3f} TOPS, {cores} threads, "
        f"{len(times)} runs); output equals GPU: {match}")
    return {"value": ops / t / 1e12, "unit": "TOPS", "cores": cores, "kind": "port",
            "sample": f"the whole workload ({M}x{N}x{K}): per-token quantize + torch._int_mm + epilogue + bias in "
                      f"PyTorch eager on the host CPU (oracle/torch_cpu.py), median of {len(times)} runs after a "
                      f"warm-up",
            "seconds": t, "matches_gpu": match}


def bench_norms(torch, h3mi, args):
    S, N, eps = 32768, 5120, 1e-6
    g = torch.Generator().manual_seed(3)
    x_cpu = torch.randn(S, N, generator=g).to(torch.bfloat16)
    o_cpu = torch.randn(S, N, generator=g).to(torch.bfloat16)
    shift = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    gate = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    w_cpu = (1 + 0.02 * torch.randn(N, generator=g)).to(torch.bfloat16)
    s1_cpu = (1.0 + scale).contiguous()
    dev = torch.device("cuda", 0)
    x, o, sh, s1, gt, w = (t.to(dev) for t in (x_cpu, o_cpu, shift, s1_cpu, gate, w_cpu))
    ridx = torch.zeros(S, dtype=torch.int32, device=dev)
    n = max(args.steps, 10)
    kernels = {
        "norm_mod": (lambda: h3mi.norm_mod(x, w, eps, ridx, s1, sh), 4.0 * S * N + 6.0 * N + 4.0 * S),
        "gate_": (lambda: h3mi.gate_(x, o, gt, ridx), 6.0 * S * N + 2.0 * N + 4.0 * S),
        "gate_norm_mod_": (lambda: h3mi.gate_norm_mod_(x, o, gt, w, eps, ridx, s1, sh), 8.0 * S * N + 8.0 * N + 4.0 * S),
    }
    res = {"S": S, "N": N}
    ks = min(args.settle, 0.25)
    for name, (fn, nbytes) in kernels.items():
        for _ in range(3):
            fn()
        ms = settled_events(torch, fn, n, ks)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": ms, "bytes": nbytes, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS}
        log(f"[bench] {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s)")
    # norm -> quantizer fusion: the int8 activations of h (and their scales) for the next linear, h not written,
    # against norm_mod (or gate_norm_mod_) followed by quantize_rowwise
    fused = {
        "norm_mod_q": (lambda: h3mi.norm_mod_q(x, w, eps, ridx, s1, sh), 3.0 * S * N + 4.0 * S + 6.0 * N,
                       lambda: h3mi.quantize_rowwise(h3mi.norm_mod(x, w, eps, ridx, s1, sh))),
        "gate_norm_mod_q_": (lambda: h3mi.gate_norm_mod_q_(x, o, gt, w, eps, ridx, s1, sh),
                             7.0 * S * N + 4.0 * S + 8.0 * N,
                             lambda: h3mi.quantize_rowwise(h3mi.gate_norm_mod_(x, o, gt, w, eps, ridx, s1, sh))),
    }
    for name, (fn, nbytes, unfused) in fused.items():
        for _ in range(3):
            fn()
            unfused()
        ms = settled_events(torch, fn, n, ks)
        ums = settled_events(torch, unfused, n, ks)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": ms, "bytes": nbytes, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS, "unfused_ms": ums}
        log(f"[bench] {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s); "
            f"norm then quantizer: {ums * 1e3:.1f} us")
    # copy bandwidth the box achieves (context for the fractions above)
    src = torch.empty(S * N * 2, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    ms = settled_events(torch, lambda: dst.copy_(src), n, ks)
    res["copy_gbs"] = 2.0 * src.numel() / (ms * 1e-3) / 1e9
    log(f"[bench] device copy: {res['copy_gbs']:.0f} GB/s")
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        from oracle import torch_cpu
        rows = S
        xs_ = x_cpu[:rows].clone()
        torch_cpu.norm_mod(xs_[:8], w_cpu, eps, s1_cpu[0], shift[0])
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            torch_cpu.norm_mod(xs_, w_cpu, eps, s1_cpu[0], shift[0])
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        nb = 4.0 * rows * N
        res["cpu_baseline_norm_mod"] = {"gbs": nb / t / 1e9, "cores": len(os.sched_getaffinity(0)),
                                        "sample": f"rows 0..{rows - 1}: F.rms_norm -> mul_ -> add_ in eager bf16 on CPU"}
        log(f"[bench] CPU eager norm_mod: {nb / t / 1e9:.2f} GB/s")
    return res


class DiTBlockC4:
    """One H3-like DiT block at world_size=1 (the C4 workload): 32768 video tokens (+512 text tokens for
    cross-attention), hidden 5120, 40 heads x 128.  Every linear is W8A8 (per-token quantize + int8 GEMM + bias);
    attention is torch SDPA on its flash / memory-efficient backends (never the math path).

    norms: "fused" runs the adaLN norms, gates and residuals as this library's kernels; "eager" runs the upstream
    eager sequence they replace (F.rms_norm -> mul_(1 + scale) -> add_(shift); addcmul_(o, gate)), so the two give
    the same bytes when the fused kernels are exact.  fuse_quant: the fused norms that feed a linear also quantize h
    (norm_mod_q / gate_norm_mod_q_) and the linear takes the int8 rows.  Every launch is bracketed by HIP events per
    kernel group (quantize, gemm, norm, attention, other)."""

    LINEARS = {
        # name: (K, N, input rows: "video" or "text")
        "self_qkv": (5120, 15360, "video"), "self_out": (5120, 5120, "video"),
        "cross_q": (5120, 5120, "video"), "cross_kv": (5120, 10240, "text"), "cross_out": (5120, 5120, "video"),
        "mlp_up": (5120, 13824, "video"), "mlp_down": (13824, 5120, "video"),
    }
    GROUPS = ("quantize", "gemm", "norm", "attention", "other")

    def __init__(self, torch, h3mi, norms="fused", fuse_quant=False, seed=4, S=32768, ST=512):
        assert norms in ("fused", "eager") and not (fuse_quant and norms == "eager")
        self.torch, self.h3mi, self.norms, self.fq = torch, h3mi, norms, fuse_quant
        H = 5120
        self.S, self.ST, self.H, self.NH, self.HD, self.eps = S, ST, H, 40, 128, 1e-6
        g = torch.Generator().manual_seed(seed)
        dev = torch.device("cuda", 0)
        self.x0 = torch.randn(S, H, generator=g).to(torch.bfloat16).to(dev)
        self.text = torch.randn(ST, H, generator=g).to(torch.bfloat16).to(dev)
        self.lin = {}
        for name, (K, N, _) in self.LINEARS.items():
            w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
            ws = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(dev)
            b = (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev)
            self.lin[name] = (w, ws, b)
        tab = lambda: (0.1 * torch.randn(1, H, generator=g)).to(torch.bfloat16).to(dev)
        self.nw = [(1 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev) for _ in range(3)]
        self.shift, scale, self.gate = [tab() for _ in range(3)], [tab() for _ in range(3)], [tab() for _ in range(3)]
        self.s1 = [(1.0 + sc).contiguous() for sc in scale]  # bf16 arithmetic, as the patched forward builds it
        self.ridx = torch.zeros(S, dtype=torch.int32, device=dev)
        self.spent = {k: [] for k in self.GROUPS}

    def gemm_ops(self):
        return sum(2.0 * (self.S if rows == "video" else self.ST) * self.lin[n][0].shape[0] * self.lin[n][0].shape[1]
                   for n, (_, _, rows) in self.LINEARS.items())

    def _timed(self, group, fn):
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        r = fn()
        b.record()
        self.spent[group].append((a, b))
        return r

    def _linear(self, inp, name, pre=None):
        w, ws, b = self.lin[name]
        h3mi = self.h3mi
        q, sx = pre if pre is not None else self._timed("quantize", lambda: h3mi.quantize_rowwise(inp))
        return self._timed("gemm", lambda: h3mi.int8_mm_scaled(q, w, sx, ws, bias=b))

    # the three norm steps, fused or eager
    def _norm_mod(self, x, i):
        if self.norms == "fused":
            return self.h3mi.norm_mod(x, self.nw[i], self.eps, self.ridx, self.s1[i], self.shift[i])
        h = self.torch.nn.functional.rms_norm(x, (self.H,), self.nw[i], self.eps)
        return h.mul_(self.s1[i][0]).add_(self.shift[i][0])

    def _gate_norm_mod(self, x, o, gi, i):
        if self.norms == "fused":
            return self.h3mi.gate_norm_mod_(x, o, self.gate[gi], self.nw[i], self.eps, self.ridx, self.s1[i],
                                            self.shift[i])
        x.addcmul_(o, self.gate[gi][0])
        return self._norm_mod(x, i)

    def _gate(self, x, o, gi):
        if self.norms == "fused":
            return self.h3mi.gate_(x, o, self.gate[gi], self.ridx)
        return x.addcmul_(o, self.gate[gi][0])

    def _norm_lin(self, name, plain, fused_q):
        # the norm output only feeds this linear: with fuse_quant it never leaves the norm kernel as bf16
        if self.fq:
            return self._linear(None, name, self._timed("norm", fused_q))
        return self._linear(self._timed("norm", plain), name)

    def _heads(self, t, rows):  # [rows, H] -> [1, NH, rows, HD], contiguous
        return t.view(1, rows, self.NH, self.HD).transpose(1, 2).contiguous()

    def _attention(self, q, k, v, rows):
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(q, k, v)
        return o.transpose(1, 2).reshape(rows, self.H).contiguous()

    def forward(self, x):
        """The block on x [S, H] (updated in place and returned)."""
        import torch.nn.functional as F
        h3mi, S, ST, H, eps, T = self.h3mi, self.S, self.ST, self.H, self.eps, self._timed
        qkv = self._norm_lin("self_qkv", lambda: self._norm_mod(x, 0),
                             lambda: h3mi.norm_mod_q(x, self.nw[0], eps, self.ridx, self.s1[0], self.shift[0]))
        q, k, v = T("other", lambda: [self._heads(t, S) for t in qkv.split(H, dim=1)])
        a = T("attention", lambda: self._attention(q, k, v, S))
        o = self._linear(a, "self_out")
        cq = self._norm_lin("cross_q", lambda: self._gate_norm_mod(x, o, 0, 1),
                            lambda: h3mi.gate_norm_mod_q_(x, o, self.gate[0], self.nw[1], eps, self.ridx, self.s1[1],
                                                          self.shift[1]))
        ckv = self._linear(self.text, "cross_kv")
        q, (k, v) = T("other", lambda: (self._heads(cq, S), [self._heads(t, ST) for t in ckv.split(H, dim=1)]))
        a = T("attention", lambda: self._attention(q, k, v, S))
        o = self._linear(a, "cross_out")
        u = self._norm_lin("mlp_up", lambda: self._gate_norm_mod(x, o, 1, 2),
                           lambda: h3mi.gate_norm_mod_q_(x, o, self.gate[1], self.nw[2], eps, self.ridx, self.s1[2],
                                                         self.shift[2]))
        u = T("other", lambda: F.gelu(u, approximate="tanh"))
        d = self._linear(u, "mlp_down")
        T("norm", lambda: self._gate(x, d, 2))
        return x

    def measure(self, steps):
        """Median latency over `steps` forwards (after one warm-up) and the median time per kernel group."""
        torch = self.torch
        self.forward(self.x0.clone())
        torch.cuda.synchronize()
        lat = []
        for _ in range(max(1, steps)):
            x = self.x0.clone()
            for k in self.GROUPS:
                self.spent[k].clear()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            self.forward(x)
            b.record()
            torch.cuda.synchronize()
            lat.append((a.elapsed_time(b),
                        {k: sum(e0.elapsed_time(e1) for e0, e1 in self.spent[k]) for k in self.GROUPS}))
        ms = statistics.median(t for t, _ in lat)
        share = {k: statistics.median(d[k] for _, d in lat) for k in self.GROUPS}
        return {"ms": ms, "group_ms": share, "group_share": {k: v / ms for k, v in share.items()},
                "gemm_tops": self.gemm_ops() / (share["gemm"] * 1e-3) / 1e12, "steps": len(lat)}


def bench_block(torch, h3mi, args, steps=None):
    """One H3-like DiT block forward at world_size=1 (DiTBlockC4): latency and the share of each kernel group."""
    log("[bench] block: building inputs")
    blk = DiTBlockC4(torch, h3mi, fuse_quant=getattr(args, "fuse_quant", False))
    res = blk.measure(steps if steps is not None else max(1, min(args.steps, 5)))
    ms, share = res["ms"], res["group_ms"]
    log(f"[bench] block {ms:.2f} ms: " + ", ".join(f"{k} {v:.2f} ms ({100 * v / ms:.1f}%)" for k, v in share.items()))
    del blk
    torch.cuda.empty_cache()
    return res


def bench_h3(torch, h3mi, args):
    """The real H3 DiT linears (hidden 5376, 56 x 128 heads: qkv 5376->21504, out 7168->5376, fc1 5376->28672,
    fc2 14336->5376) at args.tokens rows, each as the ConvRot quantizer (256-group Hadamard + per-row int8; fc2 takes
    the SwiGLU input [tokens, 28672], as the reference's fc2 call) + GEMM (no bias, as the reference's fast path),
    with the per-token quantizer and torch._int_mm (hipBLASLt, int32 out) on the same operands beside it; then the
    three fused norms at [tokens, 5376] and the q/k RMSNorm + RoPE on the qkv output."""
    from h3mi import h3_weights as HW
    M, dev = args.tokens, torch.device("cuda", 0)
    layers, tot_ops, tot_ms = {}, 0.0, 0.0
    for i, (name, (K, N)) in enumerate(HW.SHAPES.items()):
        g = torch.Generator().manual_seed(10 + i)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        ws = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(dev)
        xq = torch.empty((M, K), dtype=torch.int8, device=dev)
        xs = torch.empty((M, 1), dtype=torch.float32, device=dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        quant = lambda: h3mi.quantize_rowwise(x, xq, xs)
        gemm = lambda: h3mi.int8_mm_scaled(xq, w, xs, ws, out=out)
        for _ in range(max(2, args.warmup)):
            quant()
            gemm()
        ks = min(args.settle, 0.25)
        q_ms = settled_events(torch, quant, max(5, args.steps), ks)
        g_ms = settled_events(torch, gemm, max(5, args.steps), ks)
        wt = w.t()
        torch._int_mm(xq, wt)
        v_ms = settled_events(torch, lambda: torch._int_mm(xq, wt), 5, ks)
        act = "swiglu" if name == "fc2" else None
        xr = x if act is None else torch.randn(M, 2 * K, generator=g).to(torch.bfloat16).to(dev)
        conv = lambda: h3mi.quantize_rowwise_convrot(xr, act, xq=xq, xs=xs)
        for _ in range(2):
            conv()
        c_ms = settled_events(torch, conv, max(5, args.steps), ks)
        cb = 2.0 * M * xr.shape[1] + 1.0 * M * K + 4.0 * M
        ops = 2.0 * M * N * K
        layers[name] = {"K": K, "N": N, "quant_ms": q_ms, "gemm_ms": g_ms, "gemm_tops": ops / g_ms / 1e9,
                        "frac": ops / g_ms / 1e9 / PEAK_INT8_TOPS, "vendor_ms": v_ms, "vendor_tops": ops / v_ms / 1e9,
                        "tile_config": h3mi.config_for(M, N, K),
                        "convrot": {"act": act or "none", "ms": c_ms, "gbs": cb / c_ms / 1e6,
                                    "frac": cb / c_ms / 1e6 / PEAK_HBM_GBS}}
        tot_ops += ops
        tot_ms += c_ms + g_ms
        log(f"[bench] h3 {name} M={M} K={K} N={N}: GEMM {g_ms:.3f} ms ({ops / g_ms / 1e9:.0f} TOPS, "
            f"{100 * ops / g_ms / 1e9 / PEAK_INT8_TOPS:.1f}%), ConvRot quantizer ({act or 'none'}) {c_ms:.3f} ms "
            f"({cb / c_ms / 1e6:.0f} GB/s), per-token quantizer {q_ms:.3f} ms; hipBLASLt {v_ms:.3f} ms "
            f"({ops / v_ms / 1e9:.0f} TOPS)")
        del x, xr, w, xq, out
    S, Nn, eps = M, HW.HIDDEN, 1e-6
    g = torch.Generator().manual_seed(3)
    x = torch.randn(S, Nn, generator=g).to(torch.bfloat16).to(dev)
    o = torch.randn(S, Nn, generator=g).to(torch.bfloat16).to(dev)
    wn = (1 + 0.02 * torch.randn(Nn, generator=g)).to(torch.bfloat16).to(dev)
    s1 = (1.0 + (0.1 * torch.randn(1, Nn, generator=g)).to(torch.bfloat16)).to(dev)
    sh, gt = ((0.1 * torch.randn(1, Nn, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2))
    ridx = torch.zeros(S, dtype=torch.int32, device=dev)
    norms = {}
    for name, fn, nb in (("norm_mod", lambda: h3mi.norm_mod(x, wn, eps, ridx, s1, sh), 4.0 * S * Nn),
                         ("gate_", lambda: h3mi.gate_(x, o, gt, ridx), 6.0 * S * Nn),
                         ("gate_norm_mod_", lambda: h3mi.gate_norm_mod_(x, o, gt, wn, eps, ridx, s1, sh), 8.0 * S * Nn)):
        for _ in range(3):
            fn()
        ms = settled_events(torch, fn, max(10, args.steps), min(args.settle, 0.25))
        norms[name] = {"ms": ms, "gbs": nb / ms / 1e6, "frac": nb / ms / 1e6 / PEAK_HBM_GBS}
        log(f"[bench] h3 {name} [{S}, {Nn}]: {ms * 1e3:.1f} us, {nb / ms / 1e6:.0f} GB/s "
            f"({100 * nb / ms / 1e6 / PEAK_HBM_GBS:.1f}%)")
    # q/k RMSNorm + split-half RoPE in place on the qkv output [tokens, 3 * 56 * 128] (full rotation)
    H, D = HW.HEADS, HW.HEAD_DIM
    qkv = torch.randn(S, 3 * H * D, generator=g).to(torch.bfloat16).to(dev)
    qw, kw = ((1 + 0.02 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2))
    ang = torch.rand(S, D // 2, generator=g) * 6.3
    tab = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    tab = tab.to(torch.bfloat16)[None].to(dev)
    q, k = qkv[:, :H * D].view(1, S, H, D), qkv[:, H * D:2 * H * D].view(1, S, H, D)
    rope = lambda: h3mi.rms_rope_split_half_(q, k, tab, qw, kw, epsilon=eps)
    for _ in range(3):
        rope()
    ms = settled_events(torch, rope, max(10, args.steps), min(args.settle, 0.25))
    nb = 2.0 * 2 * 2 * S * H * D + tab.numel() * 2
    norms["rms_rope_split_half_"] = {"ms": ms, "gbs": nb / ms / 1e6, "frac": nb / ms / 1e6 / PEAK_HBM_GBS}
    log(f"[bench] h3 rms_rope_split_half_ q,k [{S}, {H}, {D}]: {ms * 1e3:.1f} us, {nb / ms / 1e6:.0f} GB/s "
        f"({100 * nb / ms / 1e6 / PEAK_HBM_GBS:.1f}%)")
    del qkv
    # a device copy of COPY_BYTES: the box's copy rate, and the reference launch the rocprof traffic summary
    # calibrates FETCH_SIZE / WRITE_SIZE against
    src = torch.empty(int(COPY_BYTES), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    cms = settled_events(torch, lambda: dst.copy_(src), 10, min(args.settle, 0.25))
    norms["copy_gbs"] = 2.0 * COPY_BYTES / cms / 1e6
    log(f"[bench] device copy: {norms['copy_gbs']:.0f} GB/s")
    return {"M": M, "layers": layers, "tops": tot_ops / tot_ms / 1e9, "ms": tot_ms, "norms": norms}


def main():
    args = parse()
    if args.summarize:
        summarize(args.summarize, args.traffic_out)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import h3mi
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    log(f"[bench] torch {torch.__version__} on {torch.cuda.get_device_name(0)}")
    if args.sustain:
        print(json.dumps({"sustained_gemm": bench_sustain(torch, h3mi, args)}), flush=True)
        return
    if args.workload == "block":
        blk = bench_block(torch, h3mi, args)
        print(json.dumps({
            "metric": "H3-like DiT block forward latency (W8A8 linears, fused norms, SDPA)", "value": blk["ms"],
            "unit": "ms", "n_gpus": 1, "steps": blk["steps"], "warmup": 1, "ms_per_step": blk["ms"],
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
            "data": "synthetic (seeded randn/randint, random-init weights)",
            "config": {"workload": "one H3-like DiT block at world_size=1: 32768 video + 512 text tokens, hidden 5120, "
                                   "40x128 heads, W8A8 self-QKV/out, cross-Q/KV/out, MLP 5120->13824->5120"
                                   + (", norms fused with the quantizer of the linear they feed" if args.fuse_quant
                                      else ""),
                       "group_ms": blk["group_ms"], "group_share": blk["group_share"],
                       "gemm_tops": blk["gemm_tops"]}}), flush=True)
        return
    if args.workload == "h3":
        r = bench_h3(torch, h3mi, args)
        print(json.dumps({
            "metric": METRIC, "value": r["tops"], "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": r["ms"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded randn/randint, random-init weights)",
            "config": {"workload": f"real H3 DiT linears qkv/out/fc1/fc2 (hidden 5376) at {r['M']} tokens: ConvRot "
                                   f"quantize (fc2: SwiGLU input) + GEMM each; value = all four layers' ops / their "
                                   f"summed time",
                       "layers": r["layers"], "norms": r["norms"]}}), flush=True)
        return
    line = {
        "metric": METRIC, "value": None, "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded randn/randint, random-init weights)",
    }
    if args.only in ("all", "gemm"):
        lin = bench_linear(torch, h3mi, args)
        M, N, K = lin["M"], lin["N"], lin["K"]
        line["value"] = lin["tops"]
        line["ms_per_step"] = lin["ms_per_step"]
        line["config"] = {"workload": lin["desc"], "M": M, "N": N, "K": K, "tile": lin["tile_config"],
                          "quant_ms": lin["quant_ms"], "gemm_ms": lin["gemm_ms"], "quant_gbs": lin["quant_gbs"],
                          "settle_s": args.settle}
        g_tops = lin.get("gemm_b2b_tops", lin["gemm_tops"])
        line["roofline"] = {"bound": "mfma", "kernel": "w8a8_gemm_direct_kernel", "achieved": g_tops,
                            "peak": PEAK_INT8_TOPS, "unit": "TOP/s", "frac": g_tops / PEAK_INT8_TOPS,
                            "traffic": read_traffic("w8a8_gemm") if args.workload == "qkv" else None,
                            "timing": "HIP events around 50 back-to-back launches" if "gemm_b2b_tops" in lin else
                                      "HIP events around each launch"}
        if "gemm_b2b_ms" in lin:
            line["config"]["gemm_b2b_ms"] = lin["gemm_b2b_ms"]
        line["vendor"] = lin["vendor"]
        if "cpu_baseline" in lin:
            line["cpu_baseline"] = lin["cpu_baseline"]
        if "shard" in lin:
            line["shard"] = lin["shard"]
    if args.only == "all" and args.workload == "qkv" and not args.no_mlp_block:
        line["mlp"] = bench_mlp(torch, h3mi, args)
        blk = bench_block(torch, h3mi, args, steps=3)
        line["block"] = {"workload": "one H3-like DiT block at world_size=1 (32768 video + 512 text tokens, hidden "
                                     "5120, 40x128 heads, W8A8 linears, fused norms, torch SDPA)",
                         "ms": blk["ms"], "group_ms": blk["group_ms"], "group_share": blk["group_share"],
                         "gemm_tops": blk["gemm_tops"], "steps": blk["steps"]}
    if args.only in ("all", "norms"):
        line["norms"] = bench_norms(torch, h3mi, args)
        if args.only == "norms":
            nm = line["norms"]["norm_mod"]
            line.update({"metric": METRIC, "value": nm["gbs"], "unit": "GB/s", "ms_per_step": nm["ms"],
                         "dtype": "bf16", "config": {"workload": "norm_mod x[32768,5120] bf16"},
                         "roofline": {"bound": "hbm", "kernel": "norm_stream_kernel", "achieved": nm["gbs"],
                                      "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": nm["frac"],
                                      "traffic": read_traffic("norm_mod")}})
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
