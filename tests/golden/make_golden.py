"""Write the golden fixtures of the oracle (``tests/golden/oracle_golden.npz``).

The reference commits no golden vectors (its correctness checks recompute the
eager model at run time), so these fixtures come from this repository's own
CPU oracle and serve as regression anchors.  The oracle itself is pinned
independently (``tests/test_oracle.py``: equality with
``torch.nn.TransformerEncoderLayer``, closed forms, invariants).

Contents (all float32 unless noted):

* ``c1_out``  -- the whole stack at the reference's tiny CPU configuration
  (B2 S128 D256 H4 L2 F1024, fp32, non-causal), weights N(0, 0.02) from seed
  0 and x ~ N(0, 1) from seed 1, as ``BaselineTransformer`` computes it
  (TTB:135-248);
* ``ln_*``    -- LayerNorm known answers computed in float64 (TTB:204-217);
* ``gemm_*``  -- ``X W^T + b`` / GELU-erf / residual known answers, float64;
* ``attn_*``  -- attention (TTB:161-194) known answers in float64 for
  (B1, H2, S128, hd64), non-causal and causal, with and without a key mask.

Usage: ``python tests/golden/make_golden.py`` (CPU only, a few seconds).
"""

from __future__ import annotations

import hashlib
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from transformer_optimization_amd import workloads  # noqa: E402

OUT = HERE / "oracle_golden.npz"


def _g(seed):
    return torch.Generator("cpu").manual_seed(seed)


def c1_output() -> torch.Tensor:
    wl = workloads.WORKLOADS["c1"]
    model = oracle.BaselineTransformer(wl.config)
    workloads.init_parameters(model)
    model = model.to(torch.float32).eval()
    x = workloads.make_input(wl.config, torch.float32)
    torch.set_num_threads(1)  # one reduction order for the fp32 GEMMs
    with torch.inference_mode():
        return model(x)


def layernorm_known_answers():
    x = torch.randn(4, 256, generator=_g(101), dtype=torch.float64) * 1.5 + 0.3
    x[1] = 2.5  # a constant row: the output is beta
    gamma = 1 + 0.1 * torch.randn(256, generator=_g(102), dtype=torch.float64)
    beta = 0.1 * torch.randn(256, generator=_g(103), dtype=torch.float64)
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    y = (x - mu) / torch.sqrt(var + 1e-5) * gamma + beta
    return {"ln_x": x, "ln_gamma": gamma, "ln_beta": beta, "ln_y": y}


def gemm_known_answers():
    a = torch.randn(64, 64, generator=_g(201), dtype=torch.float64)
    w = torch.randn(64, 64, generator=_g(202), dtype=torch.float64) * 0.1
    b = torch.randn(64, generator=_g(203), dtype=torch.float64) * 0.1
    r = torch.randn(64, 64, generator=_g(204), dtype=torch.float64)
    lin = a @ w.t() + b
    gelu = lin * 0.5 * (1 + torch.erf(lin / math.sqrt(2.0)))
    return {"gemm_a": a, "gemm_w": w, "gemm_b": b, "gemm_res": r,
            "gemm_lin": lin, "gemm_gelu": gelu, "gemm_resout": r + lin}


def attention_known_answers():
    b, h, s, hd = 1, 2, 128, 64
    q = torch.randn(b, h, s, hd, generator=_g(301), dtype=torch.float64)
    k = torch.randn(b, h, s, hd, generator=_g(302), dtype=torch.float64)
    v = torch.randn(b, h, s, hd, generator=_g(303), dtype=torch.float64)
    valid = torch.ones(b, s, dtype=torch.bool)
    valid[0, 100:] = False
    out = {"attn_q": q, "attn_k": k, "attn_v": v, "attn_valid": valid.numpy().astype(np.uint8)}
    scale = hd ** -0.5
    for causal in (False, True):
        for masked in (False, True):
            sc = (q @ k.transpose(-2, -1)) * scale
            if causal:
                sc = sc.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
            if masked:
                sc = sc.masked_fill(~valid[:, None, None, :], float("-inf"))
            p = torch.softmax(sc, -1)
            out[f"attn_out_c{int(causal)}_m{int(masked)}"] = p @ v
    return out


def main() -> None:
    arrays = {}
    c1 = c1_output()
    arrays["c1_out"] = c1.numpy().astype(np.float32)
    for part in (layernorm_known_answers(), gemm_known_answers(), attention_known_answers()):
        for key, val in part.items():
            arrays[key] = val.numpy().astype(np.float32) if isinstance(val, torch.Tensor) else val
    np.savez_compressed(OUT, **arrays)
    digest = hashlib.sha256(arrays["c1_out"].tobytes()).hexdigest()
    (HERE / "c1_out.sha256").write_text(digest + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes); c1_out sha256 {digest}")


if __name__ == "__main__":
    main()
