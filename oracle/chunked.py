"""Query-row-subset reference of the whole stack (test infrastructure only).

For sequences whose dense ``[B,H,S,S]`` scores cannot be materialised
(S = 100000: 640 GB of fp32 scores), this computes the oracle's output for a
chosen subset of query rows.  It follows the reference's query-tiled form
(TTB:341-421): every key and value row is computed, while scores are formed
for a bounded chunk of query rows at a time against all keys.

Arithmetic is the oracle's (same modules, same order of operations) run in
the dtype of the weights it is given -- float32 for the config-5 check.
Layers before the last are evaluated for all rows (query-chunked); the last
layer and the final LayerNorm only for the requested rows.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .model import BaselineTransformer


def head_split_kv(attn, x_norm: torch.Tensor):
    """K and V of every row, split into heads: two [B,H,S,hd] tensors."""
    b, s, _ = x_norm.shape
    h, hd = attn.num_heads, attn.head_dim
    k = attn.k_proj(x_norm).reshape(b, s, h, hd).permute(0, 2, 1, 3).contiguous()
    v = attn.v_proj(x_norm).reshape(b, s, h, hd).permute(0, 2, 1, 3).contiguous()
    return k, v


def _attention_rows(
    attn,
    x_norm: torch.Tensor,
    rows: torch.Tensor,
    valid: Optional[torch.Tensor],
    causal: bool,
    q_chunk: int,
    kv: Optional[tuple] = None,
) -> torch.Tensor:
    """Attention output (after out_proj and the query-row mask) for ``rows`` of
    every batch element.  ``x_norm`` is LN1(x) for all rows, shape [B,S,D];
    ``kv`` optionally holds the head-split K and V already computed by
    ``head_split_kv``."""
    b, s, d = x_norm.shape
    h, hd = attn.num_heads, attn.head_dim
    k, v = kv if kv is not None else head_split_kv(attn, x_norm)
    out = []
    for start in range(0, rows.numel(), q_chunk):
        r = rows[start:start + q_chunk]
        q = attn.q_proj(x_norm[:, r, :]).reshape(b, r.numel(), h, hd).permute(0, 2, 1, 3)
        scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * attn.scale
        if causal:
            keys = torch.arange(s, device=x_norm.device)
            scores = scores.masked_fill(keys.view(1, 1, 1, s) > r.view(1, 1, -1, 1), float("-inf"))
        if valid is not None:
            scores = scores.masked_fill(~valid.view(b, 1, 1, s), float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(x_norm.dtype)
        ctx = torch.matmul(probs, v).permute(0, 2, 1, 3).reshape(b, r.numel(), d)
        o = attn.out_proj(ctx)
        if valid is not None:
            o = o.masked_fill(~valid[:, r].unsqueeze(-1), 0)
        out.append(o)
    return torch.cat(out, dim=1)


def _block_rows(block, x, rows, valid, causal, q_chunk):
    """One block's output for ``rows`` given the block input ``x`` for all rows."""
    x_norm = block.norm1(x)
    xr = x[:, rows, :] + _attention_rows(block.attention, x_norm, rows, valid, causal, q_chunk)
    xr = xr + block.ffn_out(F.gelu(block.ffn_in(block.norm2(xr)), approximate="none"))
    if valid is not None:
        xr = xr.masked_fill(~valid[:, rows].unsqueeze(-1), 0)
    return xr


@torch.inference_mode()
def chunked_reference_rows(
    model: BaselineTransformer,
    x: torch.Tensor,
    rows: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    q_chunk: int = 64,
) -> torch.Tensor:
    """Oracle output ``model(x, mask)[:, rows, :]`` without dense scores.

    ``rows`` is a 1-D index tensor into the sequence axis, applied to every
    batch element.  Returns ``[B, len(rows), D]``.
    """
    causal = model.config.causal
    rows = rows.to(device=x.device, dtype=torch.long)
    all_rows = torch.arange(x.shape[1], device=x.device)
    for block in list(model.layers)[:-1]:
        x = _block_rows(block, x, all_rows, valid_token_mask, causal, q_chunk)
    xr = _block_rows(model.layers[-1], x, rows, valid_token_mask, causal, q_chunk)
    y = model.final_norm(xr)
    if valid_token_mask is not None:
        y = y.masked_fill(~valid_token_mask[:, rows].unsqueeze(-1), 0)
    return y
