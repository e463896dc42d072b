"""A/B timing of kernel variants on one GPU, in one process.

The GEMM dispatcher reads ``TX_GEMM_VARIANT`` on every call ("default" = the
dispatcher's own choice; 20 / 19 = the 128x128 / 256x256 ``gemm_big_kernel``;
256 / 192 / 128 = ``gemm_hp_kernel`` at that tile width; 0 = the
register-staged ``gemm_kernel``), so variants of one shape
can be timed side by side, alternating, against the same operands.  Each
launch is timed as ``bench.py`` times its per-op figures: ``reps`` launches
captured into one hipGraph, the replay bracketed by HIP events on the
launching stream.  Every variant's output is compared bitwise with the
library op eager calls (``F.linear``, then ``F.gelu`` or the residual add).

    python -m transformer_optimization_amd.variants gemm 8192 3072 1024 --variants default,20
    python -m transformer_optimization_amd.variants gemm 8192 4096 1024 --epi gelu
    python -m transformer_optimization_amd.variants layernorm 8192 1024

``layernorm`` times ``tx_layernorm_residual`` (x read, y written) and checks
its output bitwise against ``torch.native_layer_norm``.
"""
from __future__ import annotations

import argparse
import os
import statistics
import sys

import torch
import torch.nn.functional as F

from . import _C

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}


def graph_time_us(fn, reps: int) -> float:
    """Average duration of one ``fn()`` launch in microseconds."""
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
    return e0.elapsed_time(e1) * 1e3 / reps


def ab_gemm(m: int, n: int, k: int, epi: str, dtype: torch.dtype, variants, rounds: int, reps: int):
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn((m, k), generator=g, device=dev).to(dtype)
    w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(dtype)
    b = (0.02 * torch.randn((n,), generator=g, device=dev)).to(dtype)
    res = torch.randn((m, n), generator=g, device=dev).to(dtype) if epi == "residual" else None
    with torch.inference_mode():
        ref = F.linear(a, w, b)
        if epi == "gelu":
            ref = F.gelu(ref)
        elif epi == "residual":
            ref = res + ref
    outs = {v: torch.empty((m, n), dtype=dtype, device=dev) for v in variants}
    fns = {}
    for v in variants:
        def launch(v=v):
            _C.gemm(a, w, b, residual=res, out=outs[v], gelu=(epi == "gelu"))
        fns[v] = launch
    times = {v: [] for v in variants}
    for _ in range(rounds):
        for v in variants:
            # Set while the graph is captured: it records the kernel the
            # dispatcher picked for this variant.
            os.environ["TX_GEMM_VARIANT"] = str(v)
            try:
                times[v].append(graph_time_us(fns[v], reps))
            finally:
                os.environ.pop("TX_GEMM_VARIANT", None)
    flops = 2.0 * m * n * k
    for v in variants:
        same = torch.equal(outs[v], ref)
        t = statistics.median(times[v])
        name = "default" if v < 0 else str(v)
        print(f"gemm {m}x{n}x{k} {epi:8s} variant {name:>7s}: {t:9.2f} us "
              f"({flops / t / 1e6:7.1f} TFLOP/s; rounds {min(times[v]):.2f}-{max(times[v]):.2f}) "
              f"equal to eager: {same}", flush=True)


def ab_layernorm(m: int, d: int, dtype: torch.dtype, rounds: int, reps: int):
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((m, d), generator=g, device=dev).to(dtype)
    w = (1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(dtype)
    b = (0.1 * torch.randn((d,), generator=g, device=dev)).to(dtype)
    y = torch.empty_like(x)
    with torch.inference_mode():
        ref = torch.native_layer_norm(x, (d,), w, b, 1e-5)[0]
    fn = lambda: _C.layernorm_residual(x, w, b, y=y, eps=1e-5)  # noqa: E731
    times = [graph_time_us(fn, reps) for _ in range(rounds)]
    t = statistics.median(times)
    nbytes = m * d * 2 * x.element_size() + 2 * d * w.element_size()
    print(f"layernorm {m}x{d}: {t:.2f} us ({nbytes / t / 1e3:.0f} GB/s; rounds "
          f"{min(times):.2f}-{max(times):.2f}) equal to native_layer_norm: {torch.equal(y, ref)}",
          flush=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="op", required=True)
    pg = sub.add_parser("gemm")
    pg.add_argument("m", type=int)
    pg.add_argument("n", type=int)
    pg.add_argument("k", type=int)
    pg.add_argument("--epi", choices=("bias", "gelu", "residual"), default="bias")
    pg.add_argument("--variants", default="default,20",
                    help="comma list of TX_GEMM_VARIANT values; 'default' = the dispatcher's choice")
    pl = sub.add_parser("layernorm")
    pl.add_argument("m", type=int)
    pl.add_argument("d", type=int)
    for p in (pg, pl):
        p.add_argument("--dtype", choices=sorted(DTYPES), default="bf16")
        p.add_argument("--rounds", type=int, default=5)
        p.add_argument("--reps", type=int, default=20)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("variants: needs a GPU", file=sys.stderr)
        return 2
    _C.load_library()
    if args.op == "gemm":
        ab_gemm(args.m, args.n, args.k, args.epi, DTYPES[args.dtype],
                [-1 if v == "default" else int(v) for v in args.variants.split(",") if v],
                args.rounds, args.reps)
    else:
        ab_layernorm(args.m, args.d, DTYPES[args.dtype], args.rounds, args.reps)
    return 0


if __name__ == "__main__":
    sys.exit(main())
