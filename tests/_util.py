"""Shared helpers for the GPU parity tests (not collected by pytest)."""

import sys

import torch

MANT_BITS = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}


def ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of ``dtype`` values at |x| (fp32 tensor in, fp32 out)."""
    x = x.abs().float().clamp_min(torch.finfo(dtype).tiny)
    _, e = torch.frexp(x)
    return torch.ldexp(torch.ones_like(x), (e - MANT_BITS[dtype]).to(torch.int32))


def ulp_diff_stats(got: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype):
    """(max difference in ulps of dtype, fraction of elements that differ)."""
    g, r = got.float(), ref.float()
    d = (g - r).abs()
    u = ulp(torch.maximum(g.abs(), r.abs()), dtype)
    return float((d / u).max()), float((d > 0).float().mean())


def log(*args):
    print(*args, flush=True, file=sys.stderr)
