"""The reference's accuracy gate (test infrastructure only).

Restates ``AccuracyResult`` / ``compare_outputs`` from TTB:4534-4615.  An
element passes when it is finite in both tensors and
``|opt - ref| <= atol  OR  |opt - ref| <= rtol * |ref|`` -- the exact OR of the
two branches, deliberately not ``torch.isclose`` (which uses the sum
``atol + rtol*|ref|``).  The run passes only with zero failing elements.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import torch

# The repository's own gate (BASELINE.json / TTB:5048-5049 defaults used by the suites).
GATE_ATOL = 0.002
GATE_RTOL = 0.02


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float

    def summary(self) -> str:
        return (
            f"{'PASS' if self.passed else 'FAIL'} | max_abs={self.max_abs_error:.6g} | "
            f"max_rel={self.max_relative_error:.6g} | "
            f"failed={self.failed_elements}/{self.total_elements} | "
            f"worst={self.worst_index} ref={self.reference_at_worst:.8g} "
            f"opt={self.optimized_at_worst:.8g}"
        )


def compare_outputs(
    reference: torch.Tensor,
    optimized: torch.Tensor,
    rtol: float = GATE_RTOL,
    atol: float = GATE_ATOL,
) -> AccuracyResult:
    """Elementwise OR gate with a finiteness requirement (TTB:4548-4615)."""
    if tuple(reference.shape) != tuple(optimized.shape):
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, "
            f"optimized={tuple(optimized.shape)}"
        )
    ref = reference.detach().to("cpu", torch.float32)
    opt = optimized.detach().to("cpu", torch.float32)

    err = (opt - ref).abs()
    ok = torch.isfinite(ref) & torch.isfinite(opt) & ((err <= atol) | (err <= rtol * ref.abs()))
    bad = ~ok
    n_bad = int(bad.sum())

    # Worst element by absolute error (NaN compares as the largest, like argmax).
    err_for_argmax = torch.where(torch.isnan(err), torch.full_like(err, float("inf")), err)
    flat = int(err_for_argmax.reshape(-1).argmax()) if err.numel() else 0
    worst = tuple(int(i) for i in torch.unravel_index(torch.tensor(flat), ref.shape)) if ref.ndim else ()

    rel = err / ref.abs().clamp_min(1e-12)
    if ref.ndim == 0:
        dims = [0] if n_bad else []
    elif ref.ndim == 1:
        dims = torch.nonzero(bad).flatten().tolist()
    else:
        dims = torch.nonzero(bad.reshape(-1, ref.shape[-1]).any(dim=0)).flatten().tolist()

    return AccuracyResult(
        passed=n_bad == 0,
        total_elements=ref.numel(),
        failed_elements=n_bad,
        max_abs_error=float(err.max()) if err.numel() else 0.0,
        max_relative_error=float(rel.max()) if rel.numel() else 0.0,
        mean_abs_error=float(err.mean()) if err.numel() else 0.0,
        failed_feature_dims=dims,
        worst_index=worst,
        reference_at_worst=float(ref[worst]) if ref.numel() else 0.0,
        optimized_at_worst=float(opt[worst]) if opt.numel() else 0.0,
    )
