"""The five measured workloads and their seeded synthetic weights and inputs.

Seeding rule (one rule for every workload, device-independent):

* weights: ``torch.Generator('cpu').manual_seed(0)``; walk ``named_modules()``
  in registration order; every ``nn.Linear`` weight draws ``N(0, 0.02)`` in
  fp32, every Linear bias is 0, every ``nn.LayerNorm`` gets weight 1 and
  bias 0.  Then the model is moved with ``.to(device, dtype)``.
* input: ``torch.randn(B, S, D)`` in fp32 from
  ``torch.Generator('cpu').manual_seed(1)``, cast to the workload dtype.

The reference itself initialises with the default ``nn`` init after
``torch.manual_seed(1234)`` (TTB:5152, 5182); the rule above is the one the
measured configurations specify.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict

import torch
import torch.nn as nn

from .config import TransformerConfig


@dataclass(frozen=True)
class Workload:
    name: str
    config: TransformerConfig
    dtype: torch.dtype
    note: str
    # Numeric policy UserOptimizedTransformer's default ("auto") rule picks
    # for this workload: the eager rounding chain where the gate compares
    # against eager, the fp32-residual policy with the online softmax where no
    # eager result can exist and the gate compares against an fp32
    # evaluation.  Recorded for the reports; the model resolves it itself.
    precision: str = "eager"
    softmax: str = "eager"

    @property
    def dtype_name(self) -> str:
        return str(self.dtype).replace("torch.", "")


WORKLOADS: Dict[str, Workload] = {
    "c1": Workload(
        "c1_plumbing_fp32",
        TransformerConfig(2, 128, 256, 4, 1024, 2, False),
        torch.float32,
        "tiny plumbing case, eager fp32",
    ),
    "c2": Workload(
        "c2_launch_bound_fp16",
        TransformerConfig(1, 64, 512, 8, 2048, 6, False),
        torch.float16,
        "launch-bound; p50 over 1000 graph replays",
    ),
    "c3": Workload(
        "c3_gemm_bound_bf16",
        TransformerConfig(8, 1024, 1024, 16, 4096, 4, False),
        torch.bfloat16,
        "GEMM-bound medium shape",
    ),
    "c4": Workload(
        "c4_attention_bound_bf16",
        TransformerConfig(1, 8192, 2048, 16, 8192, 2, False),
        torch.bfloat16,
        "attention-bound, head_dim 128",
    ),
    "c5": Workload(
        "c5_extreme_seq_bf16",
        TransformerConfig(1, 100000, 1024, 16, 4096, 1, False),
        torch.bfloat16,
        "S=100000, HBM-resident attention; gate on 512 seeded query rows vs fp32",
        precision="fp32_residual",
        softmax="online",
    ),
}

def workload(key: str) -> Workload:
    """``cN`` or ``cN:causal``: the same shape with causal masking (the
    reference's canonical matrix is all causal, run_bench.py:227-242)."""
    name, _, variant = key.partition(":")
    wl = WORKLOADS[name]
    if variant == "causal":
        c = wl.config
        cfg = TransformerConfig(c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim,
                                c.num_layers, True)
        return Workload(wl.name + "_causal", cfg, wl.dtype, wl.note + "; causal", wl.precision, wl.softmax)
    if variant:
        raise ValueError(f"unknown workload variant {key!r}")
    return wl


# The reference's "full" suite rows (run_bench.py:202-218) over its CLI
# default shape B8 S128 D512 H8 F2048 L6 (TTB:5028-5034):
# (batch, seq, d_model, heads, ffn, layers, causal, dtype, padding ratio).
SUITE_FULL = {
    "default_fp16": (8, 128, 512, 8, 2048, 6, False, torch.float16, 0.0),
    "default_bf16": (8, 128, 512, 8, 2048, 6, False, torch.bfloat16, 0.0),
    "causal_fp16": (8, 128, 512, 8, 2048, 6, True, torch.float16, 0.0),
    "padded_fp16": (8, 128, 512, 8, 2048, 6, False, torch.float16, 0.4),
    "big_fp16": (32, 512, 512, 8, 2048, 6, False, torch.float16, 0.0),
    "big_causal_fp16": (32, 512, 512, 8, 2048, 6, True, torch.float16, 0.0),
    "long_fp16": (4, 2048, 512, 8, 2048, 6, False, torch.float16, 0.0),
    "small_fp16": (1, 64, 512, 8, 2048, 6, False, torch.float16, 0.0),
    "wide_fp16": (16, 256, 1024, 16, 4096, 12, False, torch.float16, 0.0),
}

WEIGHT_SEED = 0
INPUT_SEED = 1
ROW_SAMPLE_SEED = 2
ROW_SAMPLE_COUNT = 512


@torch.no_grad()
def init_parameters(model: nn.Module, seed: int = WEIGHT_SEED, std: float = 0.02) -> nn.Module:
    """Seeded init (see module docstring); call before ``.to(device, dtype)``."""
    g = torch.Generator("cpu").manual_seed(seed)
    for _, mod in model.named_modules():
        if isinstance(mod, nn.Linear):
            w = torch.empty(mod.weight.shape, dtype=torch.float32)
            w.normal_(0.0, std, generator=g)
            mod.weight.copy_(w)
            if mod.bias is not None:
                mod.bias.zero_()
        elif isinstance(mod, nn.LayerNorm):
            if mod.weight is not None:
                mod.weight.fill_(1.0)
            if mod.bias is not None:
                mod.bias.zero_()
    return model


def make_input(config: TransformerConfig, dtype: torch.dtype, seed: int = INPUT_SEED) -> torch.Tensor:
    """``x ~ N(0,1)`` of shape [B, S, D], generated in fp32 on the CPU."""
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, dtype=torch.float32)
    return x.to(dtype)


def sample_rows(seq_len: int, count: int = ROW_SAMPLE_COUNT, seed: int = ROW_SAMPLE_SEED) -> torch.Tensor:
    """Seeded query-row sample (sorted) used to check sequences too long for dense scores."""
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randperm(seq_len, generator=g)[: min(count, seq_len)].sort().values


def padding_mask(batch: int, seq: int, min_fraction: float, seed: int) -> torch.Tensor:
    """Prefix-valid ``[B, S]`` bool mask with random lengths in
    ``[round(S*min_fraction), S]`` (the reference's padding generator,
    TTB:4380-4396, seeded on the CPU)."""
    g = torch.Generator("cpu").manual_seed(seed)
    lo = max(1, int(round(seq * min_fraction)))
    lengths = torch.randint(lo, seq + 1, (batch,), generator=g)
    return torch.arange(seq)[None, :] < lengths[:, None]
