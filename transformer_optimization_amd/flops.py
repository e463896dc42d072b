"""FLOP count and MFU, re-based on MI355X (run_bench.py:67-124 of the reference).

``count_dense_flops`` is the reference's formula: per layer
``8*B*S*D^2 + 4*B*S^2*D + 4*B*S*D*F`` (QKV + out_proj, QK^T + PV, FFN in/out),
LayerNorm / softmax / GELU excluded, no causal discount.  MFU divides the
achieved FLOP/s by the dense MFMA peak of the precision actually executed
(bf16 and fp16 models run bf16 / fp16 MFMA; an fp32 model runs fp16 MFMA).
"""

from __future__ import annotations

# MI355X published dense peaks (no sparsity), per second.
MI355X_PEAK_FLOPS = {
    "bfloat16": 2.5e15,
    "float16": 2.5e15,
    "float8": 5.0e15,
    "float32": 157.3e12,   # vector / matrix fp32
    "float64": 78.6e12,
}
MI355X_HBM_BYTES_PER_S = 8.0e12

# Precision of the MFMA instructions each model dtype executes on.
EXECUTED_PRECISION = {"bfloat16": "bfloat16", "float16": "float16", "float32": "float16"}


def count_dense_flops(batch: int, seq: int, d_model: int, ffn_dim: int, layers: int) -> int:
    """Dense forward matmul FLOPs (reference formula, run_bench.py:102-113)."""
    b, s, d, f = batch, seq, d_model, ffn_dim
    per_layer = 8 * b * s * d * d + 4 * b * s * s * d + 4 * b * s * d * f
    return layers * per_layer


def gemm_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def attention_flops(batch: int, heads: int, seq: int, head_dim: int) -> int:
    """QK^T + PV, non-causal: 4*B*H*S^2*hd."""
    return 4 * batch * heads * seq * seq * head_dim


def compute_mfu(flops: float, latency_ms: float, dtype: str) -> float:
    """Fraction of the MI355X dense MFMA peak of the executed precision."""
    if not latency_ms or latency_ms <= 0:
        raise ValueError("latency must be positive")
    peak = MI355X_PEAK_FLOPS[EXECUTED_PRECISION.get(dtype, dtype)]
    return flops / (latency_ms / 1e3) / peak
