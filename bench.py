#!/usr/bin/env python3
"""Forward-latency benchmark of the MI355X transformer-block path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]``

One step = one ``UserOptimizedTransformer.forward(x)`` call on the workload
(input copy into the captured graph's static buffer, hipGraph replay of the
layers, the final LayerNorm into a new output tensor), the unit the reference times in
``benchmark_once`` (TTB:4824-4855).  The headline workload is BASELINE.json's
``configs[1]`` (c2, fp16, "p50 latency over 1000 graph replays"), so the
default is K=1000 timed steps; ``value`` is their p50 in ms.

The same JSON line carries
* ``per_config``: latency / TFLOP/s / fraction of the MI355X dense MFMA peak
  for every config (c1-c5), FLOPs by the reference formula
  (run_bench.py:102-113), next to the eager oracle on the same GPU
  (``eager_gpu_ms``; c5 has none, its dense scores would not fit) and on the
  host cores (``cpu_baseline``, bounded sample, method stated);
* ``geomean_speedup_vs_eager_gpu_c2_c4``: the reference's headline statistic
  (geomean latency gain over its eager baseline) for c2-c4;
* ``roofline``: the dominant kernel of the headline workload, its algorithmic
  FLOPs (or bytes) per launch over its average duration, timed with HIP
  events on the stream it is launched on;
* ``cpu_baseline``: the eager oracle on the host cores for the headline
  workload (bounded sample).

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
    dev, dt = x.device, x.dtype
    # fp32 model: fp16 GEMM / attention operands, fp32 residual (see model.py).
    ot = torch.float16 if dt == torch.float32 else dt
    softmax = "online" if dt == torch.float32 else model.softmax
    layer = model.layers[0]
    att = layer.attention
    w_qkv, b_qkv = model.packed_qkv(0)
    if dt == torch.float32:
        w_out, w_in, w_o2 = (model._half[0][k] for k in ("out_proj", "ffn_in", "ffn_out"))
    else:
        w_out = (att.out_proj.weight, att.out_proj.bias)
        w_in = (layer.ffn_in.weight, layer.ffn_in.bias)
        w_o2 = (layer.ffn_out.weight, layer.ffn_out.bias)
    xs = x.reshape(m, d).clone()
    y = torch.empty((m, d), dtype=ot, device=dev)
    qk = torch.empty((m, 2 * d), dtype=ot, device=dev)
    vt = torch.zeros((b, h, hd, _C.vt_ld(s)), dtype=ot, device=dev)
    o = torch.empty((m, d), dtype=ot, device=dev)
    hid = torch.empty((m, f), dtype=ot, device=dev)
    ln_bytes = m * d * (x.element_size() + y.element_size()) + 2 * d * layer.norm1.weight.element_size()
    ops = [
        ("layernorm", lambda: _C.layernorm_residual(xs, layer.norm1.weight, layer.norm1.bias, y=y),
         ln_bytes, "hbm", 2 * cfg.num_layers + 1),
        ("qkv_proj", lambda: _C.qkv_proj(y, w_qkv, b_qkv, b, s, h, qk=qk, vt=vt),
         gemm_flops(m, 3 * d, d), "mfma", cfg.num_layers),
        ("flash_attn", lambda: _C.flash_attn(qk, vt, b, s, h, hd, att.scale, cfg.causal, out=o,
                                             softmax=softmax),
         attention_flops(b, h, s, hd), "mfma", cfg.num_layers),
        ("gemm_out_proj", lambda: _C.gemm(o, *w_out, residual=xs, out=xs),
         gemm_flops(m, d, d), "mfma", cfg.num_layers),
        ("gemm_ffn_in_gelu", lambda: _C.gemm(y, *w_in, out=hid, gelu=True),
         gemm_flops(m, f, d), "mfma", cfg.num_layers),
        ("gemm_ffn_out", lambda: _C.gemm(hid, *w_o2, residual=xs, out=xs),
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
def _cpu_threads() -> int:
    return max(1, min(len(os.sched_getaffinity(0)), 16))


def cpu_baseline(wl, budget_s: float):
    """The eager oracle (the reference's BaselineTransformer, restated) on the
    host cores, in the workload's dtype, timed with perf_counter_ns per call
    (TTB:4848-4853).  Bounded sample: one block of the stack is timed
    (repeated until ~budget_s, median) and the forward is that times the
    layer count plus the final LayerNorm, since every block has the same
    cost.  For sequences with no dense baseline (S = 100000) the block is
    timed on a subset of query rows -- LN1 and the K/V projections of all
    rows, attention and the block tail of the subset -- and the row-dependent
    part is extrapolated linearly to all rows."""
    import oracle  # the checker's restatement; timed here as the CPU baseline only
    from oracle.chunked import _attention_rows, head_split_kv

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    c = wl.config
    model = oracle.BaselineTransformer(c)
    workloads.init_parameters(model)
    model = model.to(wl.dtype).eval()
    x = workloads.make_input(c, wl.dtype)
    block = model.layers[0]

    def timed(fn, reps_max=50):
        t0 = time.perf_counter_ns()
        fn()
        first = (time.perf_counter_ns() - t0) / 1e6
        times = [first]
        reps = max(0, min(reps_max, int(budget_s * 1e3 / max(first, 1e-3)) - 1))
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            fn()
            times.append((time.perf_counter_ns() - t0) / 1e6)
        return statistics.median(times), len(times)

    with torch.inference_mode():
        t_ln, _ = timed(lambda: model.final_norm(x), 5)
        if c.seq_len <= 16384:
            t_blk, n = timed(lambda: block(x, None, c.causal))
            value = t_blk * c.num_layers + t_ln
            sample = (f"{wl.name}: eager oracle block 0 of {c.num_layers}, {wl.dtype_name} on CPU, "
                      f"median of {n} calls, x{c.num_layers} layers + final LayerNorm")
            kind_note = "measured per block"
        else:
            rows_n = 256
            rows = torch.arange(0, c.seq_len, c.seq_len // rows_n)[:rows_n]

            def all_rows_part():
                xn = block.norm1(x)
                return xn, head_split_kv(block.attention, xn)

            t_all, _ = timed(all_rows_part, 3)
            xn, kv = all_rows_part()

            def subset_part():
                xr = x[:, rows, :] + _attention_rows(block.attention, xn, rows, None, c.causal, 64, kv)
                xr = xr + block.ffn_out(torch.nn.functional.gelu(block.ffn_in(block.norm2(xr))))
                return model.final_norm(xr)

            t_sub, n = timed(subset_part, 3)
            value = (t_all + t_sub * c.seq_len / rows_n) * c.num_layers
            sample = (f"{wl.name}: eager oracle, {wl.dtype_name} on CPU; LN1 + K/V projections of all "
                      f"{c.seq_len} rows ({t_all:.0f} ms) + attention and block tail of {rows_n} "
                      f"query rows ({t_sub:.0f} ms, median of {n}) extrapolated linearly to all rows")
            kind_note = "extrapolated"
    return {"value": round(value, 4), "unit": "ms", "cores": threads, "kind": "port",
            "sample": sample, "method": kind_note}


def eager_gpu_baseline(wl, dev, steps: int):
    """The eager oracle on the same GPU and dtype (the reference's baseline
    model), median of CUDA-event-timed forwards."""
    import oracle

    c = wl.config
    if c.seq_len > 16384:
        return None  # dense scores do not fit (S = 100000: 320 GB in bf16)
    model = oracle.BaselineTransformer(c)
    workloads.init_parameters(model)
    model = model.to(dev, wl.dtype).eval()
    x = workloads.make_input(c, wl.dtype).to(dev)
    times, _ = time_forward(model, x, steps, warmup=2)
    del model, x
    torch.cuda.empty_cache()
    return round(statistics.median(times), 4)


# ---------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(workloads.WORKLOADS))
    ap.add_argument("--per-config", default="c1,c2,c3,c4,c5",
                    help="comma list of configs to report in per_config ('' = none)")
    ap.add_argument("--per-config-steps", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--cpu-budget-s", type=float, default=15.0,
                    help="CPU-baseline time budget of the headline workload")
    ap.add_argument("--cpu-config-budget-s", type=float, default=4.0,
                    help="CPU-baseline time budget per other config")
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
        log(f"[bench] per-config {cw.name}")
        m2, x2 = build_model(cw, dev)
        steps = args.per_config_steps if key != "c2" else max(args.per_config_steps, 200)
        times, _ = time_forward(m2, x2, steps, warmup=3)
        ms = statistics.median(times)
        krows = kernel_breakdown(m2, x2, 10 if key in ("c4", "c5") else 50)
        kd = max(krows, key=lambda r: r["ms_per_forward"])
        rec = {"config": key, **config_record(cw), "precision": cw.precision,
               "softmax": "online" if cw.dtype == torch.float32 else cw.softmax,
               "latency_ms_p50": round(ms, 4), **mfu_fields(cw, ms),
               "kernels_us": {r["kernel"]: round(r["avg_ms"] * 1e3, 2) for r in krows},
               "dominant_kernel": roofline_of(kd, cw.dtype_name, load_traffic(kd["kernel"], cw.name))}
        del m2, x2
        torch.cuda.empty_cache()
        eager = eager_gpu_baseline(cw, dev, 10 if key in ("c3", "c4") else 50)
        rec["eager_gpu_ms"] = eager
        rec["speedup_vs_eager_gpu"] = round(eager / ms, 3) if eager else None
        if not args.no_cpu_baseline:
            cb = cpu_baseline(cw, args.cpu_budget_s if key == args.workload else args.cpu_config_budget_s)
            rec["cpu_baseline"] = cb
            rec["speedup_vs_cpu"] = round(cb["value"] / ms, 2)
        log(f"  {ms:.4f} ms  {rec['tflop_s']} TFLOP/s  MFU {rec['mfu']:.2%}  eager-GPU {eager} ms"
            + (f"  CPU {rec['cpu_baseline']['value']} ms ({rec['cpu_baseline']['method']})"
               if "cpu_baseline" in rec else ""))
        per_config.append(rec)

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
        cpu = next((r["cpu_baseline"] for r in per_config if r["config"] == args.workload), None)
        if cpu is None:
            log(f"[bench] CPU baseline ({wl.name})")
            cpu = cpu_baseline(wl, args.cpu_budget_s)
        log(f"[bench] CPU baseline {wl.name}: {cpu['value']} ms on {cpu['cores']} threads")
    sp = [r["speedup_vs_eager_gpu"] for r in per_config
          if r["config"] in ("c2", "c3", "c4") and r.get("speedup_vs_eager_gpu")]
    geomean = round(math.exp(sum(math.log(v) for v in sp) / len(sp)), 3) if sp else None

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
        "geomean_speedup_vs_eager_gpu_c2_c4": geomean,
        "per_config": per_config,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
