"""Measured throughput of the kernel set on one MI355X, next to the CPU path.

    python bench.py [--steps K] [--warmup W] [--report FILE] [--gemm-shapes]
    python bench.py --collect-counters OUT    (rocprofv3 counter passes -> profiles/counters.json)

Prints ONE JSON line.  The headline (``value``) is causal attention at
8 heads x 2048 x d128 bf16 in TFLOP/s, counting the exact causal FLOPs
4*H*d*S(S+1)/2.  The same line carries every other benchmark configuration,
each with its own roofline object: the fused softmax / RMSNorm / SwiGLU at
4096 x 2048 bf16 (HBM GB/s), the 1024^3 bf16 matmul, causal attention at
1 x 4096 and 32 x 16384, and the decoder block (the fp16 configuration, which
meets 1e-3 against the fp32 block, with the all-bf16 and split-operand ones
beside it).

Timing: every kernel is launched from a captured HIP graph (so host launch
overhead does not leave the GPU idle between launches), replayed at least 50
times with a HIP event recorded on the graph's stream after every replay; the
result is the median over the replays of one replay's duration over its
launches.  Each graph cycles through enough distinct input/output buffers
(at least twice the MI355X's 256 MB last-level cache) that no launch finds
its data there: every kernel is measured against HBM.  The decoder block is
the exception: one input and its ~100 MB of weights serve every launch, and
its entry says so ("llc").

CPU baseline: the oracle's NumPy restatement of the reference's flash
algorithm (the "NKI-algorithm CPU path") timed on this host, plus PyTorch CPU
SDPA, on the same seeded inputs.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nki-kernel-lab_amd"))
sys.path.insert(0, ROOT)

METRIC = "causal attn TFLOPS (8h×2048×d128 bf16) + row-kernel HBM GB/s, % of peak"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
LLC_BYTES = 256 << 20       # MI355X Infinity Cache


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


MIN_REPLAYS = 50


def capture(launches):
    """A HIP graph of `launches` (zero-arg callables, one call each).  An eager
    pass runs first on the stream the capture uses, so that per-stream scratch
    (the attention's partial states and counters) exists before capture and
    no allocation or fill is captured."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in launches:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for f in launches:
            f()
    torch.cuda.synchronize()
    return graph


def time_launches(launches, reps: int, warmup: int) -> float:
    """Seconds per launch: the median, over max(reps, 50) replays of the graph
    of `launches`, of one replay's duration (between two HIP events recorded
    on the stream the graph runs on) over its number of launches."""
    import torch

    graph = capture(launches)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    n = max(reps, MIN_REPLAYS)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    ev[0].record()
    for i in range(n):
        graph.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(ev[i].elapsed_time(ev[i + 1]) * 1e-3 / len(launches) for i in range(n))
    return per[n // 2] if n % 2 else 0.5 * (per[n // 2 - 1] + per[n // 2])


def n_sets(bytes_per_set: int) -> int:
    """Distinct buffer sets needed so a cyclic sweep overflows the LLC twice over."""
    return max(2, math.ceil(2 * LLC_BYTES / bytes_per_set))


def roofline(bound: str, achieved: float, unit: str, counters: dict | None = None) -> dict:
    """The roofline object of one workload; `counters` is its entry of
    profiles/counters.json (HBM bytes per launch from FETCH_SIZE/WRITE_SIZE,
    MFMA busy fraction from SQ_VALU_MFMA_BUSY_CYCLES), when collected."""
    peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    c = counters or {}
    out = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": c.get("bytes")}
    if bound == "mfma":
        out["mfma_busy"] = c.get("mfma_busy")
    return out


# ------------------------------------------------------------ workloads --

def bench_attention(H, S, d, reps, warmup, seed=0, sets=None):
    import torch

    from nkilab import ops, workloads

    q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, d, seed=seed))
    per_set = 4 * H * S * d * 2
    sets = sets or n_sets(per_set)
    bufs = [(q, k, v, torch.empty_like(q))] + [
        (q.clone(), k.clone(), v.clone(), torch.empty_like(q)) for _ in range(sets - 1)]
    launches = [lambda b=b: ops.attention_into(*b) for b in bufs]
    sec = time_launches(launches, reps, warmup)
    flops = workloads.causal_flops(H, S, d)
    return {"H": H, "S": S, "d": d, "us": sec * 1e6, "tflops": flops / sec / 1e12, "flops": flops,
            "bytes": per_set, "buffer_sets": sets}, bufs[0]


def bench_attention_beside_sdpa(reps, warmup):
    """This library's causal attention and torch's scaled_dot_product_attention
    (is_causal, the ROCm flash backend) on the same inputs, same harness and
    buffer rotation, at the benchmark shapes."""
    import torch
    import torch.nn.functional as F

    from nkilab import ops, workloads

    out = []
    for H, S in ((8, 2048), (1, 4096), (8, 8192), (32, 16384)):
        q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, 128))
        big = S > 8192
        sets = n_sets(4 * H * S * 128 * 2)
        bufs = [(q, k, v, torch.empty_like(q))] + [
            (q.clone(), k.clone(), v.clone(), torch.empty_like(q)) for _ in range(sets - 1)]
        r = max(3, reps // 10) if big else reps
        ours = time_launches([lambda b=b: ops.attention_into(*b) for b in bufs], r, warmup)
        sb = [tuple(t.unsqueeze(0) for t in b[:3]) for b in bufs]
        with torch.nn.attention.sdpa_kernel([torch.nn.attention.SDPBackend.FLASH_ATTENTION]):
            ref = F.scaled_dot_product_attention(*sb[0], is_causal=True)[0]
            theirs = time_launches([lambda b=b: F.scaled_dot_product_attention(*b, is_causal=True) for b in sb], r,
                                   warmup)
        mine = ops.attention_into(q, k, v, torch.empty_like(q))
        torch.cuda.synchronize()
        flops = workloads.causal_flops(H, S, 128)
        out.append({"H": H, "S": S, "nkilab_us": round(ours * 1e6, 2), "nkilab_tflops": round(flops / ours / 1e12, 1),
                    "sdpa_us": round(theirs * 1e6, 2), "sdpa_tflops": round(flops / theirs / 1e12, 1),
                    "max_abs_diff_rel": float((mine.float() - ref.float()).abs().max() / ref.float().abs().max())})
        log(f"  {H}x{S}: nkilab {out[-1]['nkilab_us']} us, torch SDPA {out[-1]['sdpa_us']} us")
        del bufs, sb
    return out


def bench_attention_sweep(reps, warmup):
    """Time per launch of the default configuration from tiny shapes up to the
    headline one (d = 128): how much of a launch does not scale with the work."""
    import torch

    from nkilab import ops, workloads

    out = []
    for H, S in ((1, 64), (1, 128), (16, 128), (2, 200), (1, 256), (1, 1024), (1, 2048), (8, 512), (8, 1024),
                 (2, 2048), (4, 2048), (8, 2048), (16, 2048), (8, 4096)):
        q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, 128))
        sets = n_sets(4 * H * S * 128 * 2)
        bufs = [(q.clone(), k.clone(), v.clone(), torch.empty_like(q)) for _ in range(sets)]
        sec = time_launches([lambda b=b: ops.attention_into(*b) for b in bufs], reps, warmup)
        flops = workloads.causal_flops(H, S, 128)
        out.append({"H": H, "S": S, "us": round(sec * 1e6, 2), "tflops": round(flops / sec / 1e12, 1)})
        log(f"  {H}x{S}: {out[-1]['us']} us")
        del bufs
    return out


def bench_rows(R, D, reps, warmup, seed=0):
    import torch

    from nkilab import ops, workloads

    x, w, gate, up = (t.cuda() for t in workloads.rows_inputs(R, D, seed=seed))
    out = {}
    eb = 2
    specs = {
        "softmax": (2 * R * D * eb, lambda xs, ys: ops.softmax_into(xs, ys)),
        "rmsnorm": (2 * R * D * eb + D * eb, lambda xs, ys: ops.rmsnorm_into(xs, w, ys, 1e-6)),
    }
    for name, (nbytes, fn) in specs.items():
        sets = n_sets(nbytes)
        bufs = [(x.clone(), torch.empty_like(x)) for _ in range(sets)]
        sec = time_launches([lambda b=b, fn=fn: fn(*b) for b in bufs], reps, warmup)
        out[name] = {"us": sec * 1e6, "GB/s": nbytes / sec / 1e9, "bytes": nbytes, "buffer_sets": sets}
        del bufs
    nbytes = 3 * R * D * eb
    sets = n_sets(nbytes)
    bufs = [(gate.clone(), up.clone(), torch.empty_like(gate)) for _ in range(sets)]
    sec = time_launches([lambda b=b: ops.swiglu_into(*b) for b in bufs], reps, warmup)
    out["swiglu"] = {"us": sec * 1e6, "GB/s": nbytes / sec / 1e9, "bytes": nbytes, "buffer_sets": sets}
    del bufs
    for r in out.values():
        r["frac"] = r["GB/s"] / PEAK_HBM_GBS
    return out


def bench_copy_ceiling(R, D, reps, warmup):
    """The HBM ceiling at the row kernels' size: nkl_stream_copy of one
    [R, D] bf16 tensor (their access pattern, no arithmetic), same harness."""
    import torch

    from nkilab import _lib
    from nkilab._tensors import stream_handle

    x = torch.empty((R, D), dtype=torch.bfloat16, device="cuda").normal_()
    nb = x.numel() * 2
    sets = n_sets(2 * nb)
    bufs = [(x.clone(), torch.empty_like(x)) for _ in range(sets)]
    sec = time_launches([lambda b=b: _lib.call("nkl_stream_copy", b[0].data_ptr(), b[1].data_ptr(), nb,
                                                stream_handle()) for b in bufs], reps, warmup)
    ok = all(torch.equal(a, b) for a, b in bufs)
    del bufs
    return {"us": sec * 1e6, "GB/s": 2 * nb / sec / 1e9, "frac": 2 * nb / sec / 1e9 / PEAK_HBM_GBS,
            "bytes": 2 * nb, "buffer_sets": sets, "copy_exact": ok}


def bench_copy_curve(reps, warmup):
    """nkl_stream_copy at 32, 48, 64, 128 and 256 MiB of traffic (half read,
    half written), and a 16-byte copy (one workgroup: the launch alone), in
    the same graph harness and buffer rotation as the row kernels.  A least
    squares line through the five sizes splits a launch into a fixed cost and
    a steady bandwidth."""
    import torch

    from nkilab import _lib
    from nkilab._tensors import stream_handle

    def one(nb):
        sets = min(n_sets(2 * nb), 32)
        bufs = [(torch.empty(nb // 2, dtype=torch.bfloat16, device="cuda").normal_(),
                 torch.empty(nb // 2, dtype=torch.bfloat16, device="cuda")) for _ in range(sets)]
        sec = time_launches([lambda b=b: _lib.call("nkl_stream_copy", b[0].data_ptr(), b[1].data_ptr(), nb,
                                                    stream_handle()) for b in bufs], reps, warmup)
        del bufs
        return sec * 1e6

    points = []
    for mib in (32, 48, 64, 128, 256):
        traffic = mib << 20
        us = one(traffic // 2)
        points.append({"traffic_MiB": mib, "us": round(us, 3), "GB/s": round(traffic / us / 1e3, 1),
                       "frac": round(traffic / us / 1e3 / PEAK_HBM_GBS, 4)})
    empty_us = one(16)
    xs = [p["traffic_MiB"] * (1 << 20) for p in points]
    ys = [p["us"] for p in points]
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    return {"points": points, "empty_launch_us": round(empty_us, 3),
            "fit": {"fixed_us": round(my - slope * mx, 3), "steady_GB/s": round(1e-3 / slope, 1)},
            "kernel": "nkl_stream_copy (2 x 16-byte loads per lane, non-temporal stores)"}


def bench_row_curve(reps, warmup):
    """The row kernels (bf16, 2048 columns) and the streaming copy from 1 to
    256 MiB of traffic, each size its own graph in the usual harness: time per
    launch against bytes moved, and a least-squares line per kernel that
    splits a launch into a fixed cost and a steady bandwidth."""
    import torch

    from nkilab import _lib, ops
    from nkilab._tensors import stream_handle

    D = 2048
    out = {}

    def fit(points):
        xs = [p["bytes"] for p in points]
        ys = [p["us"] for p in points]
        n = len(xs)
        mx, my = sum(xs) / n, sum(ys) / n
        slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        return {"fixed_us": round(my - slope * mx, 3), "steady_GB/s": round(1e-3 / slope, 1)}

    for name in ("copy", "softmax", "rmsnorm", "swiglu"):
        points = []
        for R in (128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768):
            w = torch.ones(D, dtype=torch.bfloat16, device="cuda")
            if name == "swiglu":
                nbytes = 3 * R * D * 2
                sets = [(torch.randn(R, D, device="cuda").to(torch.bfloat16),
                         torch.randn(R, D, device="cuda").to(torch.bfloat16),
                         torch.empty(R, D, dtype=torch.bfloat16, device="cuda")) for _ in range(n_sets(nbytes))]
                calls = [lambda t=t: ops.swiglu_into(*t) for t in sets]
            else:
                nbytes = 2 * R * D * 2 + (D * 2 if name == "rmsnorm" else 0)
                sets = [(torch.randn(R, D, device="cuda").to(torch.bfloat16),
                         torch.empty(R, D, dtype=torch.bfloat16, device="cuda")) for _ in range(n_sets(nbytes))]
                if name == "copy":
                    calls = [lambda t=t: _lib.call("nkl_stream_copy", t[0].data_ptr(), t[1].data_ptr(), R * D * 2,
                                                   stream_handle()) for t in sets]
                elif name == "softmax":
                    calls = [lambda t=t: ops.softmax_into(*t) for t in sets]
                else:
                    calls = [lambda t=t: ops.rmsnorm_into(t[0], w, t[1], 1e-6) for t in sets]
            us = time_launches(calls, reps, warmup) * 1e6
            points.append({"rows": R, "bytes": nbytes, "us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                           "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "buffer_sets": len(sets)})
            log(f"  {name} {R}x{D}: {us:.2f} us {nbytes / us / 1e3:.0f} GB/s")
            del sets, calls
        out[name] = {"points": points, "fit": fit(points)}
    return out


def summarize_trace(csv_path: str) -> str:
    """A markdown table of a rocprofv3 kernel-trace CSV: dispatches grouped by
    kernel and grid size, with their count and median / average / minimum
    duration in microseconds."""
    import csv
    import statistics

    groups = {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name") or row.get("Kernel-Name") or ""
            grid = int(row.get("Grid_Size") or row.get("Grid_Size_X") or 0)
            wg = int(row.get("Workgroup_Size") or row.get("Workgroup_Size_X") or 0)
            dur = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1000.0
            groups.setdefault((name, grid, wg), []).append(dur)
    lines = ["| kernel | workgroups x threads | dispatches | median us | avg us | min us |", "|---|---|---|---|---|---|"]
    for (name, grid, wg), ds in sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][1])):
        short = name.split("(")[0]
        lines.append(f"| `{short}` | {grid // max(wg, 1)} x {wg} | {len(ds)} | {statistics.median(ds):.3f} | "
                     f"{sum(ds) / len(ds):.3f} | {min(ds):.3f} |")
    return "\n".join(lines)


def bench_matmul(reps, warmup):
    import torch

    from nkilab import ops, workloads

    a, b = (t.cuda() for t in workloads.matmul_inputs())
    sets = n_sets(3 * 1024 * 1024 * 2)
    bufs = [(a.clone(), b.clone(), torch.empty_like(a)) for _ in range(sets)]
    sec = time_launches([lambda t=t: ops.gemm_into(*t) for t in bufs], reps, warmup)
    flops = 2 * 1024 ** 3
    return {"M": 1024, "N": 1024, "K": 1024, "us": sec * 1e6, "tflops": flops / sec / 1e12,
            "frac": flops / sec / 1e12 / PEAK_BF16_TFLOPS}


# The decoder block's GEMMs (hidden 2048, 16 heads, FFN 5632, 2048 tokens) and
# two square ones, as (M, N, K, B layout): "nt" is B given [N, K] (a Linear
# weight), "nn" B given [K, N].
GEMM_SHAPES = [(1024, 1024, 1024, "nn"), (2048, 6144, 2048, "nt"), (2048, 2048, 2048, "nt"),
               (2048, 11264, 2048, "nt"), (2048, 2048, 5632, "nt"), (4096, 4096, 4096, "nt")]


def bench_gemm_shapes(reps, warmup):
    """nkl_gemm (its own tile choice) beside torch.mm (hipBLASLt) on the same
    rotating bf16 operands: library context for the hand-written kernel."""
    import torch

    from nkilab import ops

    out = {}
    gen = torch.Generator(device="cuda").manual_seed(0)
    for M, N, K, kind in GEMM_SHAPES:
        per_set = 2 * (M * K + N * K + 2 * M * N)
        sets = []
        for _ in range(n_sets(per_set)):
            a = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16)
            b = torch.randn(*((K, N) if kind == "nn" else (N, K)), device="cuda", generator=gen).to(torch.bfloat16)
            sets.append((a, b, torch.empty(M, N, device="cuda", dtype=torch.bfloat16),
                         torch.empty(M, N, device="cuda", dtype=torch.bfloat16)))
        if kind == "nn":
            ours = [lambda t=t: ops.gemm_into(t[0], t[1], t[2]) for t in sets]
            lib = [lambda t=t: torch.mm(t[0], t[1], out=t[3]) for t in sets]
        else:
            ours = [lambda t=t: ops.linear_into(t[0], t[1], t[2]) for t in sets]
            lib = [lambda t=t: torch.mm(t[0], t[1].t(), out=t[3]) for t in sets]
        s_ours, s_lib = time_launches(ours, reps, warmup), time_launches(lib, reps, warmup)
        flops = 2 * M * N * K
        out[f"{M}x{N}x{K}_{kind}"] = {
            "us": round(s_ours * 1e6, 3), "tflops": round(flops / s_ours / 1e12, 1),
            "frac": round(flops / s_ours / 1e12 / PEAK_BF16_TFLOPS, 4),
            "torch_mm_us": round(s_lib * 1e6, 3), "torch_mm_tflops": round(flops / s_lib / 1e12, 1),
            "max_abs_diff_vs_torch": float((sets[0][2].float() - sets[0][3].float()).abs().max())}
        del sets
    return out


def bench_decoder(reps, warmup, counters=None):
    """The decoder block (config 5): the fp16 configuration, which meets 1e-3
    against the fp32 block at the bf16 path's cost and is the one reported;
    the all-bf16 configuration (over 1e-3) and the split-operand one (fp32
    accurate, 2.7x the time) beside it; each with its measured error."""
    import torch

    from nkilab import workloads
    from nkilab.model import nki_forward

    block, x = workloads.decoder_inputs()
    block = block.cuda()
    xg = x.cuda()
    with torch.no_grad():
        ref = block(xg)
    flops = workloads.decoder_flops()
    seven = "7 launches: 2 RMSNorm, QKV, attention, out-proj, fused gate/up/SwiGLU, down-proj"
    out = {}
    for name, cd, launches in (("fp16", "float16", seven), ("bf16", "bfloat16", seven),
                               ("split", "split", "13 launches: 2 RMSNorm, 4 hi/lo splits, 5 bf16 GEMMs over K-doubled "
                                                  "operands, fp32 attention, SwiGLU")):
        y = nki_forward(block, xg, compute_dtype=cd)  # fills the weight cache and the attention scratch
        torch.cuda.synchronize()
        err = float((y.float() - ref).abs().max() / ref.abs().max())
        sec = time_launches([lambda cd=cd: nki_forward(block, xg, compute_dtype=cd)], reps, warmup)
        out[name] = {"us": round(sec * 1e6, 3), "tflops": round(flops / sec / 1e12, 3),
                     "rel_err_vs_fp32_block": err, "launches": launches}
    rep = out["fp16"]
    return {"us": rep["us"], "tflops": rep["tflops"], "rel_err_vs_fp32_block": rep["rel_err_vs_fp32_block"],
            "llc": "warm: one input and the block's weights (~100 MB) serve every launch",
            "compute": "fp16 activations and weights (fp32 accumulation, fp32 residual stream), P rounded to fp16",
            "roofline": roofline("mfma", rep["tflops"], "TFLOP/s", (counters or {}).get("decoder")),
            "flops_per_step": flops, "fp16_activations": out["fp16"], "bf16_activations": out["bf16"],
            "split_detail": out["split"]}


# ---------------------------------------------------------- CPU baseline --

def cpu_baseline(q, k, v, gpu_out):
    """The oracle's flash attention (NumPy) and PyTorch CPU SDPA on this host."""
    import numpy as np
    import torch

    import oracle as O

    from nkilab import workloads

    H, S, d = q.shape
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    flops = workloads.causal_flops(H, S, d)
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover
        blas_threads = os.cpu_count() or 1
    reps, t0 = 0, time.perf_counter()
    while True:
        ref = O.ops_attention(qn, kn, vn, "flash_pipelined", O.BF16)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 64:  # about 10 s of CPU work
            break
    sec = (time.perf_counter() - t0) / reps
    parity = O.rel_err(gpu_out.float().cpu().numpy(), ref)
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    tq, tk, tv = (t.float().cpu() for t in (q, k, v))
    torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    t0 = time.perf_counter()
    torch_reps = 3
    for _ in range(torch_reps):
        sdpa = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    tsec = (time.perf_counter() - t0) / torch_reps
    sdpa_err = O.rel_err(gpu_out.float().cpu().numpy(), sdpa.numpy())
    try:
        model = next(ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name"))
    except Exception:  # pragma: no cover
        model = "unknown"
    rows = cpu_rows_baseline(ncores)
    other = cpu_gemm_decoder_baseline(ncores)
    base = {"value": round(flops / sec / 1e12, 5), "unit": "TFLOP/s", "cores": blas_threads, "kind": "port",
            "sample": f"full workload {H}x{S}x{d} bf16 values, oracle flash_pipelined (NumPy fp32, 128x128 tiles), "
                      f"mean of {reps} runs, {sec:.2f} s each",
            "cpu": model,
            "torch_cpu_sdpa_fp32": {"value": round(flops / tsec / 1e12, 5), "unit": "TFLOP/s", "cores": ncores,
                                    "sec": round(tsec, 4)},
            "row_kernels": rows, **other}
    return base, {"attention_rel_err_vs_oracle": parity, "attention_rel_err_vs_fp32_sdpa": sdpa_err}


def cpu_gemm_decoder_baseline(ncores: int) -> dict:
    """The 1024^3 matmul (the oracle's K-chunked NumPy restatement on one
    BLAS pool, and torch.matmul in fp32 and bf16) and one forward of the fp32
    DecoderBlock at the decoder config, on this host's cores."""
    import torch

    import oracle as O
    from nkilab import workloads

    a, b = workloads.matmul_inputs()
    an, bn = a.float().numpy(), b.float().numpy()

    def timed(fn, reps):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    mm_flops = 2 * 1024 ** 3
    out = {"matmul_1024": {
        "oracle_numpy": {"TFLOP/s": round(mm_flops / timed(lambda: O.ops_matmul(an, bn, "blocked", O.BF16), 2) / 1e12, 5)},
        "torch_cpu_float32": {"TFLOP/s": round(mm_flops / timed(lambda: a.float() @ b.float(), 3) / 1e12, 5)},
        "torch_cpu_bfloat16": {"TFLOP/s": round(mm_flops / timed(lambda: a @ b, 3) / 1e12, 5)},
        "cores": ncores}}
    block, x = workloads.decoder_inputs()
    with torch.no_grad():
        sec = timed(lambda: block(x), 1)
    out["decoder_block"] = {"torch_cpu_float32": {"TFLOP/s": round(227_641_655_296 / sec / 1e12, 5), "sec": round(sec, 3)},
                            "cores": ncores, "sample": "one forward of the fp32 DecoderBlock, S=2048, after one warm-up"}
    return out


def cpu_rows_baseline(ncores: int) -> dict:
    """Softmax / RMSNorm / SwiGLU at 4096 x 2048 on the host: the oracle's NumPy
    restatement (one thread) and PyTorch CPU in fp32 and bf16 (all cores), in
    GB/s of the same algorithmic bytes as the GPU kernels."""
    import numpy as np
    import torch

    import oracle as O
    from nkilab import workloads

    x, w, gate, up = workloads.rows_inputs(4096, 2048)
    R, D = x.shape
    nbytes = {"softmax": 2 * R * D * 2, "rmsnorm": 2 * R * D * 2 + D * 2, "swiglu": 3 * R * D * 2}
    xn, wn, gn, un = (t.float().numpy() for t in (x, w, gate, up))

    def timed(fn, reps=3):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    out = {}
    oracle_fns = {"softmax": lambda: O.softmax_fused(xn, O.BF16),
                  "rmsnorm": lambda: O.rmsnorm_fused(xn, wn, 1e-6, O.BF16),
                  "swiglu": lambda: O.swiglu_fused(gn, un, O.BF16)}
    for dt in (torch.float32, torch.bfloat16):
        tx, tw, tg, tu = (t.to(dt) for t in (x, w, gate, up))
        fns = {"softmax": lambda: torch.softmax(tx, dim=-1),
               "rmsnorm": lambda: tx * torch.rsqrt(tx.float().pow(2).mean(-1, keepdim=True) + 1e-6).to(dt) * tw,
               "swiglu": lambda: torch.nn.functional.silu(tg) * tu}
        for name, fn in fns.items():
            sec = timed(fn)
            out.setdefault(name, {})[f"torch_cpu_{str(dt).split('.')[1]}"] = {
                "GB/s": round(nbytes[name] / sec / 1e9, 3), "sec": round(sec, 5), "cores": ncores}
    for name, fn in oracle_fns.items():
        sec = timed(fn, reps=2)
        out[name]["oracle_numpy"] = {"GB/s": round(nbytes[name] / sec / 1e9, 3), "sec": round(sec, 5), "cores": 1}
    return out


# -------------------------------------------------------- counters --
#
# profiles/counters.json holds, per workload, what rocprofv3 counters read for
# its kernels: HBM bytes per launch (FETCH_SIZE, then WRITE_SIZE, in KiB per
# dispatch, each scaled by what the same counter reads per byte for a plain
# streaming kernel -- torch.neg over 256 MiB of fp32 -- in the same run) and
# the MFMA busy fraction
#     mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 * CUs * GRBM_GUI_ACTIVE / XCDs)
# (MFMA-busy SIMD-cycles over the SIMD-cycles of the dispatch; GRBM_GUI_ACTIVE
# sums the busy cycles of the XCDs' command front ends), next to the FLOPs the
# MFMAs issued, SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512.  Written by
#     python bench.py --collect-counters OUT
# which runs one rocprofv3 pass per workload and counter set over
# `bench.py --pmc-pass WORKLOAD` (graph-replayed launches, as in the timing).

COUNTERS_FILE = os.path.join(ROOT, "profiles", "counters.json")
COPY_BYTES = 256 << 20
COUNTER_SETS = {"fetch": ["FETCH_SIZE"], "write": ["WRITE_SIZE"],
                "mfma": ["SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_VALU_MFMA_BUSY_CYCLES",
                         "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE"]}
# workload -> kernel-name substring of its dominant kernel ("" = every kernel
# of the workload but the calibration copy)
PMC_WORKLOADS = {"attention": "flash", "attention_1x4096": "flash", "attention_32x16384": "flash",
                 "matmul": "gemm", "softmax": "softmax_vec", "rmsnorm": "rmsnorm_vec", "swiglu": "swiglu_vec",
                 "decoder": "", "gemm_qkv": "gemm", "gemm_wo": "gemm", "gemm_gate_up": "gemm", "gemm_down": "gemm",
                 "gemm_4096": "gemm", "hipblaslt_4096": "Cijk"}
# The decoder block's four projections at hidden 2048, FFN 5632, 2048 tokens:
# (M, N, K); gate/up is the fused GEMM with the SwiGLU epilogue (N = 2 x 5632).
DECODER_GEMMS = {"gemm_qkv": (2048, 6144, 2048), "gemm_wo": (2048, 2048, 2048), "gemm_gate_up": (2048, 11264, 2048),
                 "gemm_down": (2048, 2048, 5632)}
PMC_REPS = 8
# Calls of the workload in one counter pass where not PMC_REPS.  Counters are
# reported per call: a call can be several dispatches (the decoder forward;
# the gate/up GEMM split over two column ranges).
PMC_CALLS = {"attention_32x16384": 2, "attention_1x4096": 16, "decoder": 2}


def pmc_pass(workload: str) -> None:
    """Launches for one counter pass, as the timing runs them: the workload's
    calls (PMC_REPS of them, or PMC_CALLS, on rotating buffer sets) captured
    in a HIP graph after one eager pass, then the calibration copy, then one
    replay of the graph.  parse_counters() counts only the dispatches after
    the last calibration copy: the replayed ones."""
    import torch

    from nkilab import ops, workloads

    calls = []
    keep = []  # the buffers the graph's calls use
    if workload.startswith("attention"):
        H, S = {"attention": (8, 2048), "attention_1x4096": (1, 4096), "attention_32x16384": (32, 16384)}[workload]
        q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, 128))
        n = PMC_CALLS.get(workload, PMC_REPS)
        sets = [(q.clone(), k.clone(), v.clone(), torch.empty_like(q)) for _ in range(n)]
        keep.append(sets)
        calls = [lambda b=b: ops.attention_into(*b) for b in sets]
    elif workload == "matmul":
        a, b = (t.cuda() for t in workloads.matmul_inputs())
        sets = [(a.clone(), b.clone(), torch.empty_like(a)) for _ in range(PMC_REPS)]
        keep.append(sets)
        calls = [lambda t=t: ops.gemm_into(*t) for t in sets]
    elif workload in ("softmax", "rmsnorm", "swiglu"):
        x, w, gate, up = (t.cuda() for t in workloads.rows_inputs(4096, 2048))
        if workload == "softmax":
            sets = [(x.clone(), torch.empty_like(x)) for _ in range(PMC_REPS)]
            calls = [lambda t=t: ops.softmax_into(*t) for t in sets]
        elif workload == "rmsnorm":
            sets = [(x.clone(), torch.empty_like(x)) for _ in range(PMC_REPS)]
            calls = [lambda t=t: ops.rmsnorm_into(t[0], w, t[1], 1e-6) for t in sets]
        else:
            sets = [(gate.clone(), up.clone(), torch.empty_like(gate)) for _ in range(PMC_REPS)]
            calls = [lambda t=t: ops.swiglu_into(*t) for t in sets]
        keep.append(sets)
    elif workload in DECODER_GEMMS or workload in ("gemm_4096", "hipblaslt_4096"):
        M, N, K = DECODER_GEMMS.get(workload, (4096, 4096, 4096))
        g = torch.Generator().manual_seed(0)
        a = (torch.randn(M, K, generator=g) * 1.0).to(torch.bfloat16).cuda()
        sets = []
        for _ in range(4):
            w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
            if workload == "gemm_gate_up":
                w = ops.pack_gate_up(w[: N // 2], w[N // 2:])
                sets.append((a, w, torch.empty(M, N // 2, dtype=torch.bfloat16, device="cuda")))
            else:
                sets.append((a, w, torch.empty(M, N, dtype=torch.bfloat16, device="cuda")))
        keep.append(sets)
        for i in range(PMC_REPS):
            t = sets[i % 4]
            if workload == "gemm_gate_up":
                calls.append(lambda t=t: ops.gemm_swiglu_into(*t))
            elif workload == "hipblaslt_4096":  # torch.mm: the hipBLASLt kernel on the same operands
                calls.append(lambda t=t: torch.mm(t[0], t[1].t(), out=t[2]))
            else:
                calls.append(lambda t=t: ops.linear_into(*t))
    elif workload == "decoder":
        from nkilab.model import nki_forward

        block, x = workloads.decoder_inputs()
        block, xg = block.cuda(), x.cuda()
        keep.append((block, xg))
        calls = [lambda: nki_forward(block, xg, compute_dtype="float16")] * PMC_CALLS["decoder"]
    else:
        raise SystemExit(f"unknown counter workload {workload!r}; one of {sorted(PMC_WORKLOADS)}")
    graph = capture(calls)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)  # one streaming read and write of COPY_BYTES each
    torch.cuda.synchronize()
    del src, dst
    graph.replay()
    torch.cuda.synchronize()
    log(f"pmc pass {workload} done ({len(calls)} graph-replayed calls)")


def collect_counters(out_dir: str, only: list[str] | None = None) -> dict:
    """Every counter pass of every workload (or of the workloads in `only`,
    whose entries then replace those of the existing file) under rocprofv3
    (one child process each, under `timeout -s KILL`), then
    profiles/counters.json from them."""
    import glob
    import subprocess

    out_dir = os.path.abspath(out_dir)
    env = dict(os.environ, TMPDIR="/tmp")
    for wl in (only or PMC_WORKLOADS):
        for tag, ctrs in COUNTER_SETS.items():
            d = os.path.join(out_dir, f"{wl}_{tag}")
            cmd = ["timeout", "-s", "KILL", "180", "rocprofv3", "--pmc", *ctrs, "-d", d, "-o", "c", "-f", "csv", "--",
                   sys.executable, os.path.abspath(__file__), "--pmc-pass", wl]
            log(f"counters: {wl} {tag}")
            r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
            if r.returncode != 0 or not glob.glob(os.path.join(d, "**", "c_counter_collection.csv"), recursive=True):
                raise SystemExit(f"rocprofv3 pass {wl}/{tag} failed ({r.returncode}):\n{r.stdout[-3000:]}")
    out = parse_counters(out_dir, only)
    for path in (COUNTERS_FILE, os.path.join(out_dir, "counters.json")):
        with open(path, "w") as f:
            json.dump(out, f, indent=1)
    return out


def _rows(path: str):
    import csv

    with open(path) as f:
        for row in csv.DictReader(f):
            yield (row.get("Kernel_Name") or row.get("Kernel-Name") or "", row.get("Counter_Name", ""),
                   float(row.get("Counter_Value") or 0.0), int(row.get("Dispatch_Id") or 0))


def parse_counters(out_dir: str, only: list[str] | None = None) -> dict:
    """profiles/counters.json from the CSVs of collect_counters() (with `only`,
    the other workloads keep their entries of the existing file)."""
    import glob

    def csv_of(wl, tag):
        return glob.glob(os.path.join(out_dir, f"{wl}_{tag}", "**", "c_counter_collection.csv"), recursive=True)[0]

    res = {"formula": {"traffic": "FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the same counter's KiB per "
                                  "byte for torch.neg over 256 MiB of fp32 in the same run",
                       "mfma_busy": "SQ_VALU_MFMA_BUSY_CYCLES / (4 * CUs * GRBM_GUI_ACTIVE / XCDs)",
                       "mfma_flops_issued": "(SQ_INSTS_VALU_MFMA_MOPS_BF16 + SQ_INSTS_VALU_MFMA_MOPS_F16) * 512"},
           "cus": 256, "xcds": 8, "command": "python bench.py --collect-counters OUT"}
    if only:
        old = load_counters()
        for wl in PMC_WORKLOADS:
            if wl not in only and wl in old:
                res[wl] = old[wl]
    for wl, pat in PMC_WORKLOADS.items():
        if only and wl not in only:
            continue
        ent = {"kernel": pat or "all kernels of one forward"}
        for tag in ("fetch", "write", "mfma"):
            per = {}  # counter -> (sum over the workload's dispatches, dispatches)
            calib = {}
            rows = list(_rows(csv_of(wl, tag)))
            last_calib = max(did for name, _, _, did in rows if "neg_kernel" in name)
            for name, ctr, val, did in rows:
                if "neg_kernel" in name:
                    calib[ctr] = calib.get(ctr, 0.0) + val / 3.0
                    continue
                if did < last_calib:
                    continue  # the eager pass before the graph's capture
                if pat and pat not in name:
                    continue
                if not pat and ("elementwise" in name or "Fill" in name or "copy" in name.lower()):
                    continue  # torch's own fills and copies around the block
                t, n = per.get(ctr, (0.0, 0))
                per[ctr] = (t + val, n)
            launches = PMC_CALLS.get(wl, PMC_REPS)
            if tag == "fetch":
                f = calib["FETCH_SIZE"] * 1024 / COPY_BYTES
                ent["read_bytes"] = round(per["FETCH_SIZE"][0] / launches * 1024 / f)
                ent["fetch_factor"] = round(f, 4)
            elif tag == "write":
                f = calib["WRITE_SIZE"] * 1024 / COPY_BYTES
                ent["write_bytes"] = round(per["WRITE_SIZE"][0] / launches * 1024 / f)
                ent["write_factor"] = round(f, 4)
            else:
                busy = per["SQ_VALU_MFMA_BUSY_CYCLES"][0] / launches
                gui = per["GRBM_GUI_ACTIVE"][0] / launches
                ent["mfma_busy_simd_cycles"] = busy
                ent["grbm_gui_active"] = gui
                ent["sq_busy_cu_cycles"] = per["SQ_BUSY_CU_CYCLES"][0] / launches
                mops = per.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", (0.0, 0))[0] + per.get("SQ_INSTS_VALU_MFMA_MOPS_F16", (0.0, 0))[0]
                ent["mfma_flops_issued"] = mops / launches * 512
                ent["mfma_busy"] = round(busy / (4 * res["cus"] * gui / res["xcds"]), 4) if gui else None
        ent["bytes"] = ent["read_bytes"] + ent["write_bytes"]
        res[wl] = ent
    return res


def load_counters() -> dict:
    try:
        with open(COUNTERS_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


# ------------------------------------------------------------------ main --

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--gemm-shapes", action="store_true", help="only the GEMM shapes beside torch.mm, one JSON line")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--sdpa", action="store_true", help="only attention beside torch SDPA, one JSON line")
    ap.add_argument("--attention-sweep", action="store_true",
                    help="only attention time per launch over sizes up to the headline, one JSON line")
    ap.add_argument("--row-curve", action="store_true",
                    help="only the row kernels and the copy over sizes from 1 to 256 MiB, one JSON line")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print a rocprofv3 kernel-trace CSV as a table of durations per kernel and grid")
    ap.add_argument("--report", default=None, help="write the full result dict as JSON here")
    ap.add_argument("--pmc-pass", metavar="WORKLOAD", help="eager launches of one workload for a rocprofv3 --pmc run")
    ap.add_argument("--collect-counters", metavar="OUT",
                    help=f"run every counter pass under rocprofv3 into OUT and write "
                         f"{os.path.relpath(COUNTERS_FILE, ROOT)}")
    ap.add_argument("--parse-counters", metavar="OUT", help="rewrite the counters file from an earlier OUT")
    ap.add_argument("--workloads", default=None,
                    help="with --collect-counters: only these comma-separated workloads (the others keep their entries)")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return 0
    if args.parse_counters:
        out = parse_counters(os.path.abspath(args.parse_counters))
        with open(COUNTERS_FILE, "w") as f:
            json.dump(out, f, indent=1)
        print(json.dumps(out))
        return 0
    if args.collect_counters:  # spawns the profiled runs; this process never touches the GPU
        only = args.workloads.split(",") if args.workloads else None
        if only and any(w not in PMC_WORKLOADS for w in only):
            raise SystemExit(f"unknown workload in {only}; known: {sorted(PMC_WORKLOADS)}")
        print(json.dumps(collect_counters(args.collect_counters, only)))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: the kernel set has no multi-GPU path (asked for {args.gpus} GPUs).",
              file=sys.stderr)
        return 2

    import torch

    from nkilab import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    _lib.lib()
    if args.pmc_pass:
        pmc_pass(args.pmc_pass)
        return 0
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name} CUs={props.multi_processor_count} lib={_lib.LIB_PATH}")
    if args.gemm_shapes:
        print(json.dumps({"gemm_shapes": bench_gemm_shapes(args.steps, args.warmup)}), flush=True)
        return 0
    if args.sdpa:
        print(json.dumps({"attention_beside_torch_sdpa": bench_attention_beside_sdpa(args.steps, args.warmup)}),
              flush=True)
        return 0
    if args.attention_sweep:
        print(json.dumps({"attention_sweep": bench_attention_sweep(args.steps, args.warmup)}), flush=True)
        return 0
    if args.row_curve:
        print(json.dumps({"row_curve": bench_row_curve(args.steps, args.warmup)}), flush=True)
        return 0

    ctr = load_counters()
    A = dict(H=8, S=2048, d=128)
    log(f"attention {A} ...")
    att, bufs = bench_attention(A["H"], A["S"], A["d"], args.steps, args.warmup)
    log(f"  {att['us']:.2f} us  {att['tflops']:.1f} TFLOP/s")
    log("row kernels 4096x2048 bf16 ...")
    rows = bench_rows(4096, 2048, args.steps, args.warmup)
    for k, r in rows.items():
        log(f"  {k:8s} {r['us']:.2f} us  {r['GB/s']:.0f} GB/s  {100 * r['frac']:.1f}% of HBM peak")
    copy = bench_copy_ceiling(4096, 2048, args.steps, args.warmup)
    log(f"  copy     {copy['us']:.2f} us  {copy['GB/s']:.0f} GB/s  {100 * copy['frac']:.1f}% of HBM peak "
        f"(the same 32 MiB of traffic, no arithmetic)")
    curve = bench_copy_curve(args.steps, args.warmup)
    pts = ", ".join(f"{c['traffic_MiB']} MiB {c['us']:.2f} us ({100 * c['frac']:.1f}%)" for c in curve["points"])
    log(f"  copy curve: {pts}; empty launch {curve['empty_launch_us']:.2f} us; "
        f"fit {curve['fit']['fixed_us']:.2f} us + bytes / {curve['fit']['steady_GB/s']:.0f} GB/s")
    log("matmul 1024^3 bf16 ...")
    mm = bench_matmul(args.steps, args.warmup)
    log(f"  {mm['us']:.2f} us  {mm['tflops']:.1f} TFLOP/s")
    long_ctx = {}
    for H, S in ((1, 4096), (32, 16384)):
        log(f"attention {H}x{S}x128 ...")
        big = S > 4096
        r, _ = bench_attention(H, S, 128, max(3, args.steps // 10) if big else args.steps, min(args.warmup, 2),
                               sets=2 if big else None)
        log(f"  {r['us']:.2f} us  {r['tflops']:.1f} TFLOP/s")
        long_ctx[f"attention_{H}x{S}"] = {
            "us": round(r["us"], 3), "tflops": round(r["tflops"], 3), "flops_per_launch": r["flops"],
            "roofline": roofline("mfma", r["tflops"], "TFLOP/s", ctr.get(f"attention_{H}x{S}"))}
    log("decoder block ...")
    dec = bench_decoder(max(3, args.steps // 10), 2, ctr)
    log(f"  fp16 {dec['us']:.1f} us ({dec['rel_err_vs_fp32_block']:.2e} vs fp32 block); "
        f"bf16 {dec['bf16_activations']['us']:.1f} us ({dec['bf16_activations']['rel_err_vs_fp32_block']:.2e}); "
        f"split {dec['split_detail']['us']:.1f} us ({dec['split_detail']['rel_err_vs_fp32_block']:.2e})")

    result = {
        "metric": METRIC, "value": round(att["tflops"], 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(att["us"] / 1e3, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) bf16 from numpy default_rng(0), no published GPU baseline",
        "config": {"workload": "causal attention 8 heads x S=2048 x d=128 bf16 (flash, one launch per step)",
                   "H": 8, "S": 2048, "d": 128,
                   "flops_per_step": att["flops"], "flop_count": "exact causal pairs 4*H*d*S(S+1)/2",
                   "device": props.name, "cus": props.multi_processor_count},
        "roofline": roofline("mfma", att["tflops"], "TFLOP/s", ctr.get("attention")),
        "row_kernels": {k: {"us": round(r["us"], 3), "GB/s": round(r["GB/s"], 1), "frac": round(r["frac"], 4),
                            "bytes": r["bytes"], "frac_of_copy_ceiling": round(r["GB/s"] / copy["GB/s"], 4),
                            "roofline": roofline("hbm", r["GB/s"], "GB/s", ctr.get(k))}
                        for k, r in rows.items()},
        "hbm_copy_ceiling": {"us": round(copy["us"], 3), "GB/s": round(copy["GB/s"], 1),
                             "frac": round(copy["frac"], 4), "bytes": copy["bytes"], "copy_exact": copy["copy_exact"],
                             "kernel": "nkl_stream_copy: the row kernels' loads and non-temporal stores, no arithmetic"},
        "hbm_copy_curve": curve,
        "matmul": {"M": 1024, "N": 1024, "K": 1024, "us": round(mm["us"], 3), "tflops": round(mm["tflops"], 3),
                   "flops_per_launch": 2 * 1024 ** 3,
                   "roofline": roofline("mfma", mm["tflops"], "TFLOP/s", ctr.get("matmul"))},
        **long_ctx,
        "decoder_block": dec,
    }
    if ctr:
        result["counters_source"] = os.path.relpath(COUNTERS_FILE, ROOT)
    if not args.no_cpu:
        log("CPU baseline ...")
        q, k, v, o = bufs
        result["cpu_baseline"], result["parity"] = cpu_baseline(q, k, v, o)
    if args.report:
        with open(args.report, "w") as f:
            json.dump(result, f, indent=1)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
