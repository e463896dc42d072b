#!/usr/bin/env python3
"""Forward-latency benchmark of the MI355X transformer-block path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]``

One step = one ``UserOptimizedTransformer.forward(x)`` call on the workload
(input copy into the captured graph's static buffer, hipGraph replay of the
whole forward, output clone), the unit the reference times in
``benchmark_once`` (TTB:4824-4855).  The headline workload is BASELINE.json's
``configs[1]`` (c2, fp16, "p50 latency over 1000 graph replays"), so the
default is K=1000 timed steps; ``value`` is their p50 in ms.

The same JSON line carries
* ``per_config``: latency / TFLOP/s / fraction of the MI355X dense MFMA peak
  for every GPU config (c2-c5), FLOPs by the reference formula
  (run_bench.py:102-113);
* ``roofline``: the dominant kernel of the headline workload, its algorithmic
  FLOPs (or bytes) per launch over its average duration, timed with HIP
  events on the stream it is launched on;
* ``cpu_baseline``: the eager oracle on the host cores (bounded sample).

Synthetic data: weights N(0, 0.02) from seed 0, x ~ N(0, 1) from seed 1
(transformer_optimization_amd/workloads.py).  One GPU only.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from transformer_optimization_amd import UserOptimizedTransformer, _C, workloads  # noqa: E402
from transformer_optimization_amd.flops import (  # noqa: E402
    MI355X_HBM_BYTES_PER_S, MI355X_PEAK_FLOPS, EXECUTED_PRECISION,
    attention_flops, count_dense_flops, gemm_flops,
)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_model(wl, dev):
    model = UserOptimizedTransformer(wl.config)
    workloads.init_parameters(model)
    model = workloads.apply_policy(model.to(dev, wl.dtype).eval(), wl)
    x = workloads.make_input(wl.config, wl.dtype).to(dev)
    return model, x


def time_forward(model, x, steps: int, warmup: int):
    """Per-step event timings (ms) and the wall time of the K-step region."""
    with torch.inference_mode():
        for _ in range(warmup):
            model(x)
        torch.cuda.synchronize()
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            starts[i].record()
            model(x)
            ends[i].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, wall


def config_record(wl):
    c = wl.config
    return {"workload": wl.name, "batch": c.batch_size, "seq_len": c.seq_len,
            "d_model": c.d_model, "heads": c.num_heads, "head_dim": c.d_model // c.num_heads,
            "layers": c.num_layers, "ffn_dim": c.ffn_dim, "causal": c.causal,
            "dtype": wl.dtype_name}


def mfu_fields(wl, ms):
    c = wl.config
    flops = count_dense_flops(c.batch_size, c.seq_len, c.d_model, c.ffn_dim, c.num_layers)
    peak = MI355X_PEAK_FLOPS[EXECUTED_PRECISION[wl.dtype_name]]
    tflops = flops / (ms / 1e3) / 1e12
    return {"gflop": round(flops / 1e9, 3), "tflop_s": round(tflops, 2),
            "mfu": round(tflops * 1e12 / peak, 4)}


# --------------------------------------------------------------- per-kernel
def kernel_ops(model, x):
    """The launches of one layer of ``_forward_core`` as (name, fn, work, unit).

    Buffers are allocated once; each fn enqueues exactly one kernel on the
    current stream.  ``work`` is the algorithmic FLOPs (mfma) or bytes (hbm)
    of one launch.
    """
    cfg = model.config
    b, s, d = x.shape
    h, hd, f = cfg.num_heads, d // cfg.num_heads, cfg.ffn_dim
    m = b * s
    es = x.element_size()
    dev, dt = x.device, x.dtype
    layer = model.layers[0]
    att = layer.attention
    w_qkv, b_qkv = model.packed_qkv(0)
    xs = x.reshape(m, d).clone()
    y = torch.empty((m, d), dtype=dt, device=dev)
    qk = torch.empty((m, 2 * d), dtype=dt, device=dev)
    vt = torch.zeros((b, h, hd, _C.vt_ld(s)), dtype=dt, device=dev)
    o = torch.empty((m, d), dtype=dt, device=dev)
    hid = torch.empty((m, f), dtype=dt, device=dev)
    ops = [
        ("layernorm", lambda: _C.layernorm_residual(xs, layer.norm1.weight, layer.norm1.bias, y=y),
         (2 * m * d + 2 * d) * es, "hbm", 2 * cfg.num_layers + 1),
        ("qkv_proj", lambda: _C.qkv_proj(y, w_qkv, b_qkv, b, s, h, qk=qk, vt=vt),
         gemm_flops(m, 3 * d, d), "mfma", cfg.num_layers),
        ("flash_attn", lambda: _C.flash_attn(qk, vt, b, s, h, hd, att.scale, cfg.causal, out=o,
                                             softmax=model.softmax),
         attention_flops(b, h, s, hd), "mfma", cfg.num_layers),
        ("gemm_out_proj", lambda: _C.gemm(o, att.out_proj.weight, att.out_proj.bias, residual=xs, out=xs),
         gemm_flops(m, d, d), "mfma", cfg.num_layers),
        ("gemm_ffn_in_gelu", lambda: _C.gemm(y, layer.ffn_in.weight, layer.ffn_in.bias, out=hid, gelu=True),
         gemm_flops(m, f, d), "mfma", cfg.num_layers),
        ("gemm_ffn_out", lambda: _C.gemm(hid, layer.ffn_out.weight, layer.ffn_out.bias, residual=xs, out=xs),
         gemm_flops(m, d, f), "mfma", cfg.num_layers),
    ]
    return ops


def time_kernel(fn, reps: int) -> float:
    """Average duration (ms) of one launch.  The reps launches are captured
    into one hipGraph (so host launch cost is excluded, as in the forward's
    own graph) and the replay is bracketed by two HIP events recorded on the
    stream the kernels run on."""
    with torch.inference_mode():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def kernel_breakdown(model, x, reps):
    rows = []
    for name, fn, work, bound, per_fwd in kernel_ops(model, x):
        ms = time_kernel(fn, reps)
        rows.append({"kernel": name, "avg_ms": ms, "work": work, "bound": bound,
                     "launches_per_forward": per_fwd, "ms_per_forward": ms * per_fwd})
    return rows


def roofline_of(row, dtype_name, traffic=None):
    if row["bound"] == "mfma":
        achieved = row["work"] / (row["avg_ms"] / 1e3) / 1e12
        peak = MI355X_PEAK_FLOPS[EXECUTED_PRECISION[dtype_name]] / 1e12
        unit = "TFLOP/s"
    else:
        achieved = row["work"] / (row["avg_ms"] / 1e3) / 1e9
        peak = MI355X_HBM_BYTES_PER_S / 1e9
        unit = "GB/s"
    return {"kernel": row["kernel"], "bound": row["bound"], "achieved": round(achieved, 2),
            "peak": round(peak, 1), "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": traffic, "avg_us": round(row["avg_ms"] * 1e3, 3),
            "work_per_launch": row["work"]}


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summaries, if any."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        data = json.loads(p.read_text())
        return data.get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None


# -------------------------------------------------------------- CPU baseline
def cpu_baseline(wl, budget_s: float):
    """Eager oracle on the host cores: median forward latency (ms) of the
    workload in its dtype, repeated until ~budget_s of CPU work."""
    import oracle  # the checker's restatement; timed here as the CPU baseline only

    threads = len(os.sched_getaffinity(0))
    threads = max(1, min(threads, 16))
    torch.set_num_threads(threads)
    model = oracle.BaselineTransformer(wl.config)
    workloads.init_parameters(model)
    model = model.to(wl.dtype).eval()
    x = workloads.make_input(wl.config, wl.dtype)
    times = []
    with torch.inference_mode():
        t0 = time.perf_counter_ns()
        model(x)  # warmup
        first = (time.perf_counter_ns() - t0) / 1e6
        reps = max(3, min(50, int(budget_s * 1e3 / max(first, 1e-3))))
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            model(x)
            times.append((time.perf_counter_ns() - t0) / 1e6)
    return {"value": round(statistics.median(times), 4), "unit": "ms", "cores": threads,
            "kind": "port",
            "sample": f"{wl.name}: eager oracle BaselineTransformer, {wl.dtype_name} on CPU, "
                      f"median of {len(times)} forwards after 1 warmup (perf_counter_ns)"}


# ---------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(workloads.WORKLOADS))
    ap.add_argument("--per-config", default="c2,c3,c4,c5",
                    help="comma list of configs to report in per_config ('' = none)")
    ap.add_argument("--per-config-steps", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB "
                         "(a known-size kernel for scaling HBM counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    _C.load_library()

    wl = workloads.WORKLOADS[args.workload]
    log(f"[bench] headline workload {wl.name}: {args.warmup} warmup + {args.steps} timed steps")
    model, x = build_model(wl, dev)
    per, wall = time_forward(model, x, args.steps, args.warmup)
    p50 = statistics.median(per)
    ms_per_step = wall * 1e3 / args.steps
    log(f"[bench] p50 {p50:.4f} ms, mean {ms_per_step:.4f} ms/step")

    log("[bench] per-kernel breakdown (HIP events)")
    rows = kernel_breakdown(model, x, args.kernel_reps)
    for r in rows:
        log(f"  {r['kernel']:18s} {r['avg_ms'] * 1e3:9.2f} us x{r['launches_per_forward']}")
    dom = max(rows, key=lambda r: r["ms_per_forward"])
    roof = roofline_of(dom, wl.dtype_name, load_traffic(dom["kernel"], wl.name))
    del model, x
    torch.cuda.empty_cache()

    per_config = []
    for key in [k for k in args.per_config.split(",") if k]:
        cw = workloads.WORKLOADS[key]
        if cw.dtype == torch.float32:
            continue
        log(f"[bench] per-config {cw.name}")
        m2, x2 = build_model(cw, dev)
        steps = args.per_config_steps if key != "c2" else max(args.per_config_steps, 200)
        times, _ = time_forward(m2, x2, steps, warmup=3)
        ms = statistics.median(times)
        krows = kernel_breakdown(m2, x2, 10 if key in ("c4", "c5") else 50)
        kd = max(krows, key=lambda r: r["ms_per_forward"])
        rec = {"config": key, **config_record(cw), "precision": cw.precision,
               "softmax": cw.softmax, "latency_ms_p50": round(ms, 4),
               **mfu_fields(cw, ms),
               "kernels_us": {r["kernel"]: round(r["avg_ms"] * 1e3, 2) for r in krows},
               "dominant_kernel": roofline_of(kd, cw.dtype_name, load_traffic(kd["kernel"], cw.name))}
        log(f"  {ms:.4f} ms  {rec['tflop_s']} TFLOP/s  MFU {rec['mfu']:.2%}")
        per_config.append(rec)
        del m2, x2
        torch.cuda.empty_cache()

    if args.calibration_copy_mib > 0:
        n = args.calibration_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {args.calibration_copy_mib} MiB read + written")
        del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline ({wl.name})")
        cpu = cpu_baseline(wl, args.cpu_budget_s)
        log(f"  {cpu['value']} ms on {cpu['cores']} threads")

    out = {
        "metric": "forward latency (ms), p50 over graph replays; MFU vs MI355X dense MFMA peak per config",
        "value": round(p50, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float16": "fp16", "bfloat16": "bf16"}.get(wl.dtype_name, wl.dtype_name),
        "data": "synthetic (weights N(0,0.02) seed 0, x ~ N(0,1) seed 1)",
        "config": config_record(wl),
        **mfu_fields(wl, p50),
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_config": per_config,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
