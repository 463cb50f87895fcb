"""Benchmark results in the reference's dashboard format, measured on the GPU.

The reference's bench/run_bench.py:200-266 writes site/data/results.json: per
kernel summaries (profiler.py:210-235), an attention ladder and scaling sweep,
a decoder-block breakdown, a correctness matrix, and per-instruction trace
events ``{op, lane, t0, t1, bytes, flops}`` (profiler.py:237-244), all from an
analytic Trainium model.  This module writes the same schema from measurements
on this GPU, so the reference's site/index.html renders measured data:

  * latencies are HIP-event timings of graph-replayed launches (32 calls per
    graph, warm inputs); they keep the reference's field names
    (``modeled_latency_us``, ``modeled_tflops``) and each summary says
    ``"latency_source": "measured"``;
  * ``hbm_bytes`` is the HBM traffic rocprofv3 measured for the same kernel
    and shape (FETCH_SIZE + WRITE_SIZE, profiles/counters.json, written by
    ``bench.py --collect-counters``) where there is such a measurement, else
    the compulsory traffic of the call (inputs read once, outputs written
    once); ``hbm_bytes_source`` says which, and ``compulsory_hbm_bytes`` is
    always the latter;
  * ``engine_busy_pct`` holds the measured MFMA busy share of the SIMDs
    (``{"mfma": ...}``, SQ_VALU_MFMA_BUSY_CYCLES over the dispatch's SIMD
    cycles, same file) where measured;
  * trace events are one per kernel call, from HIP events around calls
    queued back to back behind a short spin kernel (lane ``"HIP stream"``),
    or one per dispatch from a rocprofv3 kernel-trace CSV (lane ``"queue N"``);
  * fields with no measured counterpart on a GPU (instruction counts, other
    engines' busy shares, on-chip footprints) are null or empty.

    python -m nkilab.results --out results.json [--quick] [--rocprof-csv kernel_trace.csv]
"""
from __future__ import annotations

import argparse
import csv
import datetime as dt
import json
import math
import os
import platform
import re
import subprocess
import sys

# MI355X (gfx950) in the shape of the reference's hardware_model (hwmodel.py's
# CoreSpec): the dashboard reads peak_flops.bfloat16 and hbm_bytes_per_s.
HARDWARE = {
    "name": "AMD Instinct MI355X (gfx950)",
    "cus": 256,
    "xcds": 8,
    "clock_hz": 2.4e9,
    "peak_flops": {"bfloat16": 2.5166e15, "float16": 2.5166e15, "float32": 157.3e12, "float8": 5.0e15},
    "hbm_bytes_per_s": 8.0e12,
    "hbm_bytes": 288 * 2**30,
    "lds_bytes_per_cu": 160 * 1024,
    "wavefront": 64,
}

# The reference's ladder labels (run_bench.py:128-134) for our variant names.
LADDER = [
    ("naive (scores in HBM)", "naive"),
    ("flash (online softmax, causal skip)", "flash"),
    ("+ K/V resident in SBUF", "flash_kv_resident"),
    ("+ fused, engine-balanced updates", "flash_balanced"),
    ("+ 2 query tiles interleaved (ILP)", "flash_pipelined"),
]


# ------------------------------------------------------------- summaries --

COUNTERS_FILE = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                             "profiles", "counters.json")


def load_counters(path: str = COUNTERS_FILE) -> dict:
    """rocprofv3 counter results per workload (profiles/counters.json), or {}."""
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def summary(kernel: str, latency_us: float, hbm_bytes: int, flops: int, dtype: str = "bfloat16",
            compulsory: int | None = None, extra: dict | None = None, counters: dict | None = None) -> dict:
    """One kernel's entry, field for field the reference's Profile.summary
    (profiler.py:210-235) plus run() additions (run_bench.py:44-58).
    `counters` is the kernel's entry of profiles/counters.json when this call
    is the measured workload (same kernel and shape): its HBM bytes replace
    the computed ones and its MFMA busy share fills engine_busy_pct."""
    source = "computed (compulsory traffic)"
    busy = {}
    if counters and counters.get("bytes"):
        hbm_bytes = counters["bytes"]
        source = "measured: rocprofv3 FETCH_SIZE + WRITE_SIZE per launch (profiles/counters.json)"
    if counters and counters.get("mfma_busy") is not None:
        busy = {"mfma": round(100.0 * counters["mfma_busy"], 2)}
    peak = HARDWARE["peak_flops"].get(dtype, HARDWARE["peak_flops"]["float32"])
    bw = HARDWARE["hbm_bytes_per_s"]
    t_compute, t_memory = flops / peak, hbm_bytes / bw
    bound_s = max(t_compute, t_memory)
    lat_s = latency_us * 1e-6
    s = {
        "kernel": kernel,
        "instructions": None,
        "per_engine": {},
        "dma_bytes": {"hbm_to_sbuf": None, "sbuf_to_hbm": None, "other": None},
        "hbm_bytes": int(hbm_bytes),
        "hbm_bytes_source": source,
        "flops": int(flops),
        "modeled_latency_us": latency_us,
        "latency_source": "measured",
        "serial_latency_us": None,
        "roofline_bound_us": bound_s * 1e6,
        "roofline_regime": "compute" if t_compute >= t_memory else "memory",
        "arithmetic_intensity": flops / hbm_bytes if hbm_bytes else None,
        "modeled_tflops": flops / lat_s / 1e12 if lat_s > 0 else 0.0,
        "pct_of_roofline": bound_s / lat_s * 100 if lat_s > 0 else 0.0,
        "engine_busy_pct": busy,
        "peak_sbuf_bytes_per_partition": None,
        "peak_psum_bytes_per_partition": None,
        "sbuf_capacity_ok": None,
        "psum_capacity_ok": None,
        "dtype": dtype,
        "simulator_wall_s": None,  # the reference's NKI simulator time; no simulator here
    }
    if compulsory is not None:
        s["compulsory_hbm_bytes"] = int(compulsory)
        s["ideal_bound_us"] = max(flops / peak, compulsory / bw) * 1e6
    if extra:
        s.update(extra)
    return s


# ---------------------------------------------------------------- traces --

_TEMPLATE_ARG = re.compile(r"Li(-?\d+)E|Lb([01])E|(DF16b)|(f)(?=[LDfE])")


def short_kernel_name(name: str) -> str:
    """A readable name for a (possibly mangled) kernel symbol:
    ``_ZN3nkl17flash_bf16_kernelILi128ELi4ELi2EEEv...`` -> ``flash_bf16_kernel<128,4,2>``,
    ``_ZN3nkl18softmax_vec_kernelIDF16bLi4EEEv...`` -> ``softmax_vec_kernel<bf16,4>``.
    Names that are not this library's mangled templates come back unchanged."""
    m = re.match(r"^_ZN3nkl(\d+)", name)
    if not m:
        return name
    n = int(m.group(1))
    base = name[m.end():m.end() + n]
    rest = name[m.end() + n:]
    if not rest.startswith("I"):
        return base
    args = []
    for lit, flag, bf, fl in _TEMPLATE_ARG.findall(rest[1:rest.find("EE") + 1] if "EE" in rest else rest[1:]):
        args.append(lit or flag or ("bf16" if bf else "float" if fl else "?"))
    return f"{base}<{','.join(args)}>" if args else base


def trace_events_from_rocprof(csv_path: str, work: dict | None = None) -> list[dict]:
    """One event per kernel dispatch of a rocprofv3 ``--kernel-trace`` CSV, with
    times in microseconds from the first dispatch; bytes and flops from
    ``work[short_name]`` = (bytes, flops) when given, else 0."""
    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Kind", "KERNEL_DISPATCH") != "KERNEL_DISPATCH":
                continue
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], r.get("Queue_Id", "0")))
    if not rows:
        return []
    rows.sort()
    t0 = rows[0][0]
    work = work or {}
    ev = []
    for s, e, name, q in rows:
        op = short_kernel_name(name)
        b, fl = work.get(op, (0, 0))
        ev.append({"op": op, "lane": f"queue {q}", "t0": round((s - t0) / 1e3, 4), "t1": round((e - t0) / 1e3, 4),
                   "bytes": int(b), "flops": int(fl)})
    return ev


class Recorder:
    """HIP events around each launch on the current stream: ``with
    rec.kernel(op, bytes, flops): launch()``; ``events()`` after a sync."""

    def __init__(self):
        self._marks = []

    def kernel(self, op: str, nbytes: int = 0, flops: int = 0):
        import torch

        rec = self

        class _Ctx:
            def __enter__(self):
                self.a = torch.cuda.Event(enable_timing=True)
                self.b = torch.cuda.Event(enable_timing=True)
                self.a.record()
                return self

            def __exit__(self, *exc):
                self.b.record()
                rec._marks.append((op, self.a, self.b, nbytes, flops))
                return False

        return _Ctx()

    def events(self) -> list[dict]:
        import torch

        torch.cuda.synchronize()
        if not self._marks:
            return []
        origin = self._marks[0][1]
        return [{"op": op, "lane": "HIP stream", "t0": round(origin.elapsed_time(a) * 1e3, 4),
                 "t1": round(origin.elapsed_time(b) * 1e3, 4), "bytes": int(nb), "flops": int(fl)}
                for op, a, b, nb, fl in self._marks]


# ---------------------------------------------------------------- timing --

def time_us(fn, reps: int = 10, per_graph: int = 32, warmup: int = 2) -> float:
    """Microseconds per call of fn (GPU launches only): `per_graph` calls
    captured in one HIP graph (so the graph's own launch cost is shared),
    replayed `reps` times between two events.  The inputs are the same every
    call, so they are warm in the caches."""
    import torch

    # Warm up (and let the ops allocate their scratch) on the stream the graph
    # is captured on, so nothing is allocated or cleared inside the capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for _ in range(per_graph):
            fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * per_graph)


def queue_behind_sleep(ms: float = 20.0):
    """Occupies the current stream for about `ms` milliseconds with a bounded
    spin kernel, so that launches enqueued next run back to back on the GPU
    and events between them time the kernels, not the host's launch gaps."""
    import torch

    torch.cuda._sleep(int(ms * 1e-3 * 2.4e9))


# ------------------------------------------------------------ collection --

def _rng(seed=7):
    import numpy as np

    return np.random.default_rng(seed)


def _gpu(x, dtype=None):
    import numpy as np
    import torch

    t = torch.from_numpy(np.asarray(x, np.float32)).cuda()
    return t.to(dtype) if dtype is not None else t


def bench_matmul(quick: bool) -> dict:
    import torch

    from . import ops

    n = 512 if quick else 1024
    ctr = load_counters()
    rng = _rng()
    a, b = (_gpu(rng.standard_normal((n, n)), torch.bfloat16) for _ in range(2))
    ref = a.double() @ b.double()
    comp = 3 * n * n * 2
    variants = []
    for nm in ("naive", "blocked"):
        c = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
        us = time_us(lambda: ops.gemm_into(a, b, c, variant=nm))
        err = float((c.double() - ref).abs().max() / ref.abs().max())
        label = "matmul naive" if nm == "naive" else "matmul blocked (MFMA, LDS-DMA)"
        variants.append(summary(label, us, comp, 2 * n**3, compulsory=comp, extra={"rel_err_vs_numpy": err},
                                counters=ctr.get("matmul") if nm == "blocked" and n == 1024 else None))
    sweep = []
    for m in ([512, 1024] if quick else [512, 1024, 2048]):
        x = torch.zeros((m, m), dtype=torch.bfloat16, device="cuda")
        c = torch.empty_like(x)
        for nm in ("naive", "blocked"):
            us = time_us(lambda: ops.gemm_into(x, x, c, variant=nm))
            s = summary(f"matmul {nm} {m}^3", us, 3 * m * m * 2, 2 * m**3, compulsory=3 * m * m * 2)
            sweep.append({"n": m, "variant": nm, **{k: s[k] for k in (
                "modeled_latency_us", "hbm_bytes", "flops", "arithmetic_intensity", "modeled_tflops",
                "ideal_bound_us")}})
    return {"shape": [n, n, n], "variants": variants, "sweep": sweep}


def bench_norm(quick: bool) -> dict:
    import torch

    from . import ops

    R, D = (1024, 1024) if quick else (4096, 2048)
    full = not quick  # the profiled shape
    ctr = load_counters()
    rng = _rng()
    x = _gpu(rng.standard_normal((R, D)) * 3, torch.bfloat16)
    y = torch.empty_like(x)
    ref = torch.softmax(x.float(), -1)
    variants = []
    for nm, fused in (("softmax unfused (3 HBM passes)", False), ("softmax fused", True)):
        us = time_us(lambda: ops.softmax_into(x, y, fused=fused))
        # three passes: read x twice (max, exp), write and re-read fp32 e
        nbytes = 2 * R * D * 2 if fused else R * D * (2 + 2 + 4 + 4 + 2)
        variants.append(summary(nm, us, nbytes, 0, compulsory=2 * R * D * 2,
                                counters=ctr.get("softmax") if fused and full else None,
                                extra={"max_abs_err_vs_torch": float((y.float() - ref).abs().max())}))
    w = _gpu(rng.uniform(0.5, 1.5, D), torch.bfloat16)
    us = time_us(lambda: ops.rmsnorm_into(x, w, y, 1e-6))
    variants.append(summary("rmsnorm fused", us, 2 * R * D * 2 + D * 2, 0, compulsory=2 * R * D * 2 + D * 2,
                            counters=ctr.get("rmsnorm") if full else None))
    u = _gpu(rng.standard_normal((R, D)), torch.bfloat16)
    us = time_us(lambda: ops.swiglu_into(x, u, y))
    variants.append(summary("swiglu fused", us, 3 * R * D * 2, 0, compulsory=3 * R * D * 2,
                            counters=ctr.get("swiglu") if full else None))
    return {"shape": [R, D], "variants": variants}


def bench_attention(quick: bool) -> dict:
    import torch
    import torch.nn.functional as F

    from . import ops

    H, S, d = (2, 512, 64) if quick else (8, 2048, 128)
    ctr = load_counters()
    rng = _rng()
    q, k, v = (_gpu(rng.standard_normal((H, S, d)), torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
    comp = 4 * H * S * d * 2
    exact = 4 * H * d * S * (S + 1) // 2
    tiles = (S + 127) // 128
    useful = 4 * H * d * tiles * (tiles + 1) // 2 * 128 * 128  # the reference's tile-level count
    ladder = []
    for label, var in LADDER:
        us = time_us(lambda: ops.attention_into(q, k, v, o, variant=var))
        err = float((o.float() - ref).abs().max() / ref.abs().max())
        ladder.append(summary(label, us, comp, exact, compulsory=comp,
                              extra={"useful_causal_flops": useful, "rel_err_vs_torch": err,
                                     "variant": var},
                              counters=ctr.get("attention") if var != "naive" and not quick else None))
    scaling = []
    for s_len in ([256, 512] if quick else [512, 1024, 2048, 4096]):
        qz = torch.zeros((1, s_len, d), dtype=torch.bfloat16, device="cuda")
        oz = torch.empty_like(qz)
        for nm, var in (("naive", "naive"), ("flash", "flash_pipelined")):
            us = time_us(lambda: ops.attention_into(qz, qz, qz, oz, variant=var))
            hbm = 4 * s_len * d * 2 + (s_len * s_len * (4 + 4 + 2 + 2) if nm == "naive" else 0)
            scaling.append({"S": s_len, "variant": nm, "hbm_bytes": hbm, "modeled_latency_us": us})
    return {"shape": [H, S, d], "ladder": ladder, "scaling": scaling}


def bench_block(quick: bool) -> dict:
    import dataclasses

    import torch

    from . import ops
    from .model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(0)
    cfg = BlockConfig()
    block = DecoderBlock(cfg).eval()
    S = 256 if quick else 512
    x = torch.randn(S, cfg.d_model)
    with torch.no_grad():
        ref = block(x)
    out = nki_forward(block, x)
    err = float((out - ref).abs().max())
    # per-op breakdown, each op timed alone on the GPU (the reference's parts)
    dev = torch.device("cuda")
    xs = x.to(dev)
    W = {n: getattr(block, n).weight.detach().to(dev) for n in ("wqkv", "wo", "wg", "wu", "wd")}
    g1 = block.norm1.weight.detach().to(dev)
    g2 = block.norm2.weight.detach().to(dev)
    d, H, hd, F_ = cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.d_ff
    h = torch.empty_like(xs)
    qkv = torch.empty((S, 3 * d), device=dev)
    a = torch.empty((S, d), device=dev)
    gate, up, act = (torch.empty((S, F_), device=dev) for _ in range(3))
    o = torch.empty((S, d), device=dev)
    q, k, v = (qkv[:, i * d:(i + 1) * d].view(S, H, hd).transpose(0, 1) for i in range(3))
    ops.linear_into(ops.rmsnorm_into(xs, g1, h, cfg.eps), W["wqkv"], qkv)
    fl_attn = 4 * H * hd * S * (S + 1) // 2
    parts_spec = [
        ("rmsnorm", lambda: ops.rmsnorm_into(xs, g1, h, cfg.eps), 2 * S * d * 4 + d * 4, 0),
        ("qkv matmul", lambda: ops.linear_into(h, W["wqkv"], qkv), (S * d + 3 * d * d + 3 * S * d) * 4,
         2 * S * d * 3 * d),
        ("flash attention", lambda: ops.attention_into(q, k, v, a.view(S, H, hd).transpose(0, 1)), 4 * S * d * 4,
         fl_attn),
        ("out-proj matmul", lambda: ops.linear_into(a, W["wo"], o, residual=xs), (3 * S * d + d * d) * 4,
         2 * S * d * d),
        ("rmsnorm", lambda: ops.rmsnorm_into(o, g2, h, cfg.eps), 2 * S * d * 4 + d * 4, 0),
        ("gate + up matmuls", lambda: (ops.linear_into(h, W["wg"], gate), ops.linear_into(h, W["wu"], up)),
         (S * d + 2 * F_ * d + 2 * S * F_) * 4, 4 * S * d * F_),
        ("swiglu", lambda: ops.swiglu_into(gate, up, act), 3 * S * F_ * 4, 0),
        ("down-proj matmul", lambda: ops.linear_into(act, W["wd"], o, residual=o), (S * F_ + F_ * d + 2 * S * d) * 4,
         2 * S * F_ * d),
    ]
    parts = []
    for nm, fn, nbytes, fl in parts_spec:
        us = time_us(fn)
        parts.append({"op": nm, "modeled_latency_us": us, "hbm_bytes": nbytes, "instructions": None, "flops": fl,
                      "latency_source": "measured"})
    return {"config": dataclasses.asdict(cfg), "seq_len": S, "dtype": "float32",
            "max_abs_err_vs_pytorch": err, "max_abs_ref": float(ref.abs().max()),
            "total_instructions": None, "kernel_launches": 9, "parts": parts}


def small_traces() -> dict:
    """Measured per-launch timelines at the reference's small trace shapes
    (run_bench.py:170-196): one event per kernel dispatch."""
    import torch

    from . import ops

    out = {}
    H, S, d = 1, 512, 128
    rng = _rng()
    q = _gpu(rng.standard_normal((H, S, d)), torch.bfloat16)
    o = torch.empty_like(q)
    fl = 4 * H * d * S * (S + 1) // 2
    for label, var in (("attention naive", "naive"), ("attention flash", "flash"),
                       ("attention flash, K/V resident", "flash_kv_resident"),
                       ("attention flash, balanced", "flash_balanced"),
                       ("attention flash, 2-tile ILP", "flash_pipelined")):
        ops.attention_into(q, q, q, o, variant=var)  # scratch allocated outside the timed launches
        rec = Recorder()
        queue_behind_sleep()
        for _ in range(4):
            with rec.kernel(f"attention {var}", 4 * H * S * d * 2, fl):
                ops.attention_into(q, q, q, o, variant=var)
        ev = rec.events()
        out[label] = {"shape": f"H={H} S={S} d={d} bf16", "latency_us": min(e["t1"] - e["t0"] for e in ev),
                      "events": ev}
    a = torch.zeros((512, 512), dtype=torch.bfloat16, device="cuda")
    c = torch.empty_like(a)
    for label, var in (("matmul naive", "naive"), ("matmul blocked", "blocked")):
        ops.gemm_into(a, a, c, variant=var)
        rec = Recorder()
        queue_behind_sleep()
        for _ in range(4):
            with rec.kernel(f"gemm {var}", 3 * 512 * 512 * 2, 2 * 512**3):
                ops.gemm_into(a, a, c, variant=var)
        ev = rec.events()
        out[label] = {"shape": "512x512x512 bf16", "latency_us": min(e["t1"] - e["t0"] for e in ev), "events": ev}
    x = torch.zeros((512, 2048), dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    for label, fused in (("softmax unfused", False), ("softmax fused", True)):
        ops.softmax_into(x, y, fused=fused)
        rec = Recorder()
        queue_behind_sleep()
        for _ in range(4):
            with rec.kernel("softmax fused" if fused else "softmax 3-pass", 2 * 512 * 2048 * 2, 0):
                ops.softmax_into(x, y, fused=fused)
        ev = rec.events()
        out[label] = {"shape": "512x2048 bf16", "latency_us": min(e["t1"] - e["t0"] for e in ev), "events": ev}
    return out


def correctness_matrix() -> list:
    """run_bench.py:199-219 against PyTorch (JAX is not installed here: vs_jax null)."""
    import numpy as np
    import torch

    from . import ops

    rng = _rng()
    rows = []
    x = (rng.standard_normal((300, 777)) * 4).astype(np.float32)
    o = ops.softmax(x)
    rows.append({"op": "softmax fused", "shape": "300x777",
                 "vs_torch": float(np.abs(o - torch.softmax(torch.from_numpy(x), -1).numpy()).max()), "vs_jax": None})
    q, k, v = (rng.standard_normal((2, 200, 64)).astype(np.float32) for _ in range(3))
    rt = torch.nn.functional.scaled_dot_product_attention(*map(torch.from_numpy, (q, k, v)), is_causal=True).numpy()
    for nm in ops.ATTENTION_VARIANTS:
        o = ops.attention(q, k, v, variant=nm)
        rows.append({"op": f"attention {nm}", "shape": "2x200x64", "vs_torch": float(np.abs(o - rt).max()),
                     "vs_jax": None})
    a, b = rng.standard_normal((200, 300)).astype(np.float32), rng.standard_normal((300, 130)).astype(np.float32)
    o = ops.matmul(a, b)
    rows.append({"op": "matmul blocked", "shape": "200x300 @ 300x130",
                 "vs_torch": float(np.abs(o - (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()).max()),
                 "vs_jax": None})
    return rows


def schema_gaps(result: dict, schema: dict) -> list[str]:
    """Keys the reference's results.json has that `result` lacks, as paths
    (``"attention.ladder[].rel_err_vs_torch"``); `schema` maps such a path to
    the reference's key list (``"top"`` for the top level, ``"x[]"`` for the
    items of list x, ``"x{}"`` for the values of dict x)."""
    gaps = []

    def node(path):
        if path == "top":
            return [result]
        cur = [result]
        for part in path.split("."):
            nxt = []
            for c in cur:
                c = c if isinstance(c, dict) else {}
                v = c.get(part.rstrip("[]{}"))
                if part.endswith("[]"):
                    nxt += list(v) if isinstance(v, list) else []
                elif part.endswith("{}"):
                    nxt += list(v.values()) if isinstance(v, dict) else []
                else:
                    nxt.append(v if isinstance(v, dict) else {})
            cur = nxt
        return cur

    for path, want in schema.items():
        if not isinstance(want, list) or path in ("trace_names", "hardware_model.read_by_dashboard"):
            continue
        items = node(path)
        if not items:
            gaps.append(f"{path} (empty)")
        for it in items:
            for k in want:
                if not isinstance(it, dict) or k not in it:
                    gaps.append(f"{path}.{k}")
    for name in schema.get("trace_names", []):
        if name not in (result.get("traces") or {}):
            gaps.append(f"traces.{name}")
    hw = result.get("hardware_model") or {}
    if "bfloat16" not in (hw.get("peak_flops") or {}) or "hbm_bytes_per_s" not in hw:
        gaps.append("hardware_model")
    return sorted(set(gaps))


def _git_sha() -> str:
    try:
        here = os.path.dirname(os.path.abspath(__file__))
        return subprocess.run(["git", "rev-parse", "--short", "HEAD"], capture_output=True, text=True,
                              cwd=here, timeout=10).stdout.strip()
    except Exception:
        return ""


def collect(quick: bool = False, rocprof_csv: str | None = None) -> dict:
    """Every section of the reference's results.json, measured on cuda:0."""
    import numpy as np
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("nkilab.results: a GPU is needed to measure the kernels")
    result = {
        "generated_at": dt.datetime.now(dt.timezone.utc).isoformat(timespec="seconds"),
        "git_sha": _git_sha(),
        "quick": quick,
        "versions": {"python": platform.python_version(), "nki": "", "torch": torch.__version__, "jax": "",
                     "numpy": np.__version__, "hip": getattr(torch.version, "hip", "") or "",
                     "device": torch.cuda.get_device_name(0)},
        "hardware_model": dict(HARDWARE),
        "matmul": bench_matmul(quick),
        "norm": bench_norm(quick),
        "attention": bench_attention(quick),
        "decoder_block": bench_block(quick),
        "correctness": correctness_matrix(),
        "traces": small_traces(),
    }
    if rocprof_csv:
        result["traces"]["rocprofv3 kernel trace"] = {
            "shape": os.path.basename(rocprof_csv), "latency_us": None,
            "events": trace_events_from_rocprof(rocprof_csv)}
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--out", default="results.json")
    ap.add_argument("--rocprof-csv", default=None, help="a rocprofv3 --kernel-trace CSV to add as a trace")
    a = ap.parse_args(argv)
    res = collect(a.quick, a.rocprof_csv)
    os.makedirs(os.path.dirname(os.path.abspath(a.out)) or ".", exist_ok=True)
    with open(a.out, "w") as f:
        json.dump(res, f, indent=1, default=float, allow_nan=False)
    print("wrote", os.path.abspath(a.out), f"{os.path.getsize(a.out) / 1e6:.2f} MB", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
