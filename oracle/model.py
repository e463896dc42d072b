"""Eager restatement of the reference's oracle models (test infrastructure only).

Restates TTB:43-70 (``TransformerConfig``), TTB:135-248 (``BaselineSelfAttention``,
``BaselineTransformerBlock``, ``BaselineTransformer``) and TTB:4328-4338
(``copy_model_weights``).  Module attribute names are the reference's, so the
``state_dict`` key set is identical:
``layers.{i}.norm1``, ``layers.{i}.attention.{q,k,v,out}_proj``,
``layers.{i}.norm2``, ``layers.{i}.ffn_in``, ``layers.{i}.ffn_out``,
``final_norm``.

Every materialisation point of the reference is kept, because on a bf16 or
fp16 model each one is a rounding to the model dtype that the GPU kernels must
mirror:

1. ``q/k/v = Linear(x)``                       (rounded)
2. ``s = matmul(q, k^T)``                      (rounded)   TTB:173
3. ``s = s * head_dim**-0.5``                  (rounded)   TTB:173
4. causal ``triu(1)`` and invalid keys -> -inf             TTB:175-184
5. ``p = softmax(s.float()).to(dtype)``        (rounded)   TTB:187
6. ``ctx = matmul(p, v)``                      (rounded)   TTB:188
7. ``out_proj``; invalid query rows -> 0                   TTB:193-197
8. ``x + attn``; ``ffn_out(gelu_erf(ffn_in(norm2(x))))``   TTB:219-220
9. invalid rows of x -> 0 after each block and after the final LayerNorm.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class TransformerConfig:
    """Shape record, TTB:43-70 (same fields, same validation rules)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )
        for name in ("ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")


class BaselineSelfAttention(nn.Module):
    """Multi-head self-attention, eager ATen ops (TTB:135-198)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        # TTB:146: a Python float, applied after the matmul.
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        b, s, _ = t.shape
        # [B,S,D] -> [B,H,S,hd], materialised as the reference does (TTB:151-159).
        return t.reshape(b, s, self.num_heads, self.head_dim).permute(0, 2, 1, 3).contiguous()

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
        causal: bool = False,
    ) -> torch.Tensor:
        b, s, _ = x.shape
        q = self._heads(self.q_proj(x))
        k = self._heads(self.k_proj(x))
        v = self._heads(self.v_proj(x))
        # Rounding points 2 and 3: matmul result, then the scaled product.
        # TTB:173 verbatim: the transposed view goes to the batched GEMM as is
        # (the library's NT layout).  One exception: bf16 batched products
        # with a transposed right operand have faulted MI355X GPUs on the
        # test pool, so on a GPU in bf16 the transpose is materialised (NN
        # layout).  Whether the two layouts give the same bits is measured in
        # fp16, where both are safe (tests/test_kernels_gpu.py).
        kt = k.transpose(-2, -1)
        if kt.is_cuda and kt.dtype == torch.bfloat16:
            kt = kt.contiguous()
        scores = torch.matmul(q, kt) * self.scale
        neg_inf = float("-inf")
        if causal:
            upper = torch.ones((s, s), dtype=torch.bool, device=x.device).triu(1)
            scores = scores.masked_fill(upper, neg_inf)
        if valid_token_mask is not None:
            scores = scores.masked_fill(~valid_token_mask.view(b, 1, 1, s), neg_inf)
        # Rounding point 5: fp32 softmax, cast back to the model dtype (TTB:187).
        probs = torch.softmax(scores.float(), dim=-1).to(x.dtype)
        ctx = torch.matmul(probs, v)
        ctx = ctx.permute(0, 2, 1, 3).contiguous().reshape(b, s, self.d_model)
        out = self.out_proj(ctx)
        if valid_token_mask is not None:
            out = out.masked_fill(~valid_token_mask.unsqueeze(-1), 0)
        return out


class BaselineTransformerBlock(nn.Module):
    """Pre-LayerNorm block (TTB:201-221)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor],
        causal: bool,
    ) -> torch.Tensor:
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        hidden = F.gelu(self.ffn_in(self.norm2(x)), approximate="none")
        x = x + self.ffn_out(hidden)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask.unsqueeze(-1), 0)
        return x


class BaselineTransformer(nn.Module):
    """Stack of blocks plus a final LayerNorm (TTB:224-248)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
            for _ in range(config.num_layers)
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
    ) -> torch.Tensor:
        for block in self.layers:
            x = block(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask.unsqueeze(-1), 0)
        return x


def copy_model_weights(baseline: nn.Module, optimized: nn.Module, strict: bool = True) -> None:
    """Strict state-dict copy from one model into the other (TTB:4328-4338)."""
    result = optimized.load_state_dict(copy.deepcopy(baseline.state_dict()), strict=strict)
    if not strict:
        if result.missing_keys:
            print(f"[warning] missing optimized keys: {result.missing_keys}")
        if result.unexpected_keys:
            print(f"[warning] unexpected optimized keys: {result.unexpected_keys}")
