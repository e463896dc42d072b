"""Kernel-level parity on the GPU, through the C ABI (via the ctypes wrappers).

Comparators are the eager ATen ops of the oracle on the same device and
dtype (the rounding chain each kernel mirrors) and an fp32 evaluation of the
same inputs.  Tolerances are stated per test:

* GEMM / LayerNorm: same rounding points as the eager op, so results agree to
  1 ulp of the output dtype and differ (by that 1 ulp, from fp32 accumulation
  order) in a small fraction of elements;
* attention: the flash kernel rounds exp(s - m_running) instead of the
  normalised probability, so it is compared to fp32 attention with a bound
  no worse than eager's own error, and to eager within the repository gate.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from transformer_optimization_amd import _C
from _util import log, ulp_diff_stats

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _randn(shape, dtype, dev, seed, scale=1.0):
    return (torch.randn(shape, generator=_gen(seed)) * scale).to(dev, dtype)


# ------------------------------------------------------------------ LayerNorm
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,d", [(256, 256), (64, 512), (8192, 1024), (8192, 2048), (100000, 1024), (7, 1032)])
def test_layernorm_matches_eager(cuda, dtype, rows, d):
    log(f"layernorm {rows}x{d} {dtype}")
    x = _randn((rows, d), dtype, cuda, 1, 2.0) + 0.5
    g = _randn((d,), dtype, cuda, 2, 0.2) + 1.0
    b = _randn((d,), dtype, cuda, 3, 0.2)
    y = _C.layernorm_residual(x, g, b)
    ref = F.layer_norm(x, (d,), g, b, 1e-5)
    mx, frac = ulp_diff_stats(y, ref, dtype)
    log(f"  max_ulp={mx:.2f} frac_diff={frac:.2e}")
    assert mx <= 1.0 and frac < 0.01


@pytest.mark.parametrize("dtype", DTYPES)
def test_layernorm_residual_flags(cuda, dtype):
    rows, d = 1000, 1024
    x = _randn((rows, d), dtype, cuda, 4)
    delta = _randn((rows, d), dtype, cuda, 5, 0.3)
    g = _randn((d,), dtype, cuda, 6, 0.2) + 1.0
    b = _randn((d,), dtype, cuda, 7, 0.2)
    valid = torch.rand(rows, generator=_gen(8)) > 0.3
    valid = valid.to(cuda)
    x_out = torch.empty_like(x)
    flags = _C.LN_MASK_DELTA | _C.LN_MASK_X | _C.LN_MASK_OUT
    y = _C.layernorm_residual(x, g, b, delta=delta, x_out=x_out, row_valid=valid, flags=flags)
    # eager chain: x' = mask_x(x + mask_d(delta)); y = mask_o(LN(x'))
    dm = delta.masked_fill(~valid[:, None], 0)
    xr = (x + dm).masked_fill(~valid[:, None], 0)
    assert torch.equal(x_out, xr)
    ref = F.layer_norm(xr, (d,), g, b, 1e-5).masked_fill(~valid[:, None], 0)
    mx, frac = ulp_diff_stats(y, ref, dtype)
    assert mx <= 1.0 and frac < 0.01
    assert torch.count_nonzero(y[~valid]) == 0


# ----------------------------------------------------------------------- GEMM
GEMM_SHAPES = [
    (64, 64, 64),
    (100, 192, 136),       # ragged M, N; K not a multiple of 64
    (64, 1536, 512),       # c2 QKV
    (64, 512, 2048),       # c2 FFN out
    (256, 768, 256),       # c1 QKV
    (8192, 3072, 1024),    # c3 QKV
    (8192, 1024, 1024),    # c3 out_proj
    (8192, 4096, 1024),    # c3 FFN in
    (8192, 1024, 4096),    # c3 FFN out
    (8192, 2048, 8192),    # c4 FFN out
    (100000, 1024, 1024),  # c5 out_proj
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_bias_matches_eager_linear(cuda, dtype, m, n, k):
    log(f"gemm {m}x{n}x{k} {dtype}")
    a = _randn((m, k), dtype, cuda, 11)
    w = _randn((n, k), dtype, cuda, 12, 0.02)
    bias = _randn((n,), dtype, cuda, 13, 0.1)
    c = _C.gemm(a, w, bias)
    ref = F.linear(a, w, bias)
    mx, frac = ulp_diff_stats(c, ref, dtype)
    # fp32 reference rounded once: our result must be within 1 ulp of it as well.
    ref32 = (a.float() @ w.float().t() + bias.float()).to(dtype)
    mx32, _ = ulp_diff_stats(c, ref32, dtype)
    log(f"  vs eager max_ulp={mx:.2f} frac={frac:.2e}; vs fp32 max_ulp={mx32:.2f}")
    assert mx32 <= 1.0
    assert mx <= 1.0 and frac < 0.02


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(300, 1024, 512), (8192, 4096, 1024)])
def test_gemm_gelu_epilogue(cuda, dtype, m, n, k):
    a = _randn((m, k), dtype, cuda, 21)
    w = _randn((n, k), dtype, cuda, 22, 0.05)
    bias = _randn((n,), dtype, cuda, 23, 0.1)
    c = _C.gemm(a, w, bias, gelu=True)
    ref = F.gelu(F.linear(a, w, bias), approximate="none")
    mx, frac = ulp_diff_stats(c, ref, dtype)
    log(f"gelu {m}x{n}x{k} max_ulp={mx:.2f} frac={frac:.2e}")
    # GELU reads the rounded GEMM value; a 1-ulp difference there can move
    # the GELU output by ~1 ulp, so allow 2.
    assert mx <= 2.0 and frac < 0.02


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("masked", [False, True])
def test_gemm_residual_epilogue_inplace(cuda, dtype, masked):
    m, n, k = 1000, 1024, 4096
    a = _randn((m, k), dtype, cuda, 31)
    w = _randn((n, k), dtype, cuda, 32, 0.02)
    bias = _randn((n,), dtype, cuda, 33, 0.1)
    x = _randn((m, n), dtype, cuda, 34)
    valid = (torch.rand(m, generator=_gen(35)) > 0.25).to(cuda) if masked else None
    delta = F.linear(a, w, bias)
    # mask_delta: invalid rows keep x; eager x + masked_fill(delta, 0)
    want_d = x + (delta.masked_fill(~valid[:, None], 0) if masked else delta)
    xs = x.clone()
    _C.gemm(a, w, bias, residual=xs, out=xs, row_valid=valid, mask_delta=masked)
    mx, frac = ulp_diff_stats(xs, want_d, dtype)
    log(f"residual mask={masked} max_ulp={mx:.2f} frac={frac:.2e}")
    assert mx <= 1.0 and frac < 0.02
    if masked:
        assert torch.equal(xs[~valid], x[~valid])
        # mask_out: invalid rows become 0 (end of block, TTB:219-220)
        xo = x.clone()
        _C.gemm(a, w, bias, residual=xo, out=xo, row_valid=valid, mask_out=True)
        assert torch.count_nonzero(xo[~valid]) == 0
        assert torch.equal(xo[valid], (x + delta)[valid]) or ulp_diff_stats(xo[valid], (x + delta)[valid], dtype)[0] <= 1


# ------------------------------------------------------------ packed QKV
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("b,s,d,h", [(1, 64, 512, 8), (2, 100, 256, 4), (8, 1024, 1024, 16), (1, 8192, 2048, 16)])
def test_qkv_proj_layouts(cuda, dtype, b, s, d, h):
    log(f"qkv b{b} s{s} d{d} h{h} {dtype}")
    hd = d // h
    x = _randn((b * s, d), dtype, cuda, 41)
    w = _randn((3 * d, d), dtype, cuda, 42, 0.02)
    bias = _randn((3 * d,), dtype, cuda, 43, 0.1)
    qk, vt = _C.qkv_proj(x, w, bias, b, s, h)
    ref = F.linear(x, w, bias)
    mx, frac = ulp_diff_stats(qk, ref[:, : 2 * d], dtype)
    assert mx <= 1.0 and frac < 0.02
    v_ref = ref[:, 2 * d:].reshape(b, s, h, hd).permute(0, 2, 3, 1)  # [B,H,hd,S]
    mx, frac = ulp_diff_stats(vt[..., :s], v_ref, dtype)
    assert mx <= 1.0 and frac < 0.02


# ------------------------------------------------------------------ attention
def _split(qk, vt, b, s, h, hd):
    d = h * hd
    q = qk[:, :d].reshape(b, s, h, hd).permute(0, 2, 1, 3).contiguous()
    k = qk[:, d:].reshape(b, s, h, hd).permute(0, 2, 1, 3).contiguous()
    v = vt[..., :s].permute(0, 1, 3, 2).contiguous()
    return q, k, v


def _eager_attention(q, k, v, scale, causal, valid):
    """The oracle's chain (TTB:173-188) in the model dtype."""
    s = q.shape[2]
    scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    if causal:
        scores = scores.masked_fill(torch.ones(s, s, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    if valid is not None:
        scores = scores.masked_fill(~valid[:, None, None, :], float("-inf"))
    p = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(p, v)


def _fp32_attention(q, k, v, scale, causal, valid, q_rows=None):
    qf = q.float() if q_rows is None else q[:, :, q_rows].float()
    scores = torch.matmul(qf, k.float().transpose(-2, -1).contiguous()) * scale
    s = k.shape[2]
    if causal:
        rows = torch.arange(q.shape[2], device=q.device) if q_rows is None else q_rows
        scores = scores.masked_fill(torch.arange(s, device=q.device)[None, :] > rows[:, None], float("-inf"))
    if valid is not None:
        scores = scores.masked_fill(~valid[:, None, None, :], float("-inf"))
    return torch.matmul(torch.softmax(scores, -1), v.float())


ATTN_CASES = [
    # b, h, s, hd, causal, masked
    (1, 8, 64, 64, False, False),      # c2
    (2, 4, 128, 64, True, False),      # c1 shape, causal
    (2, 4, 200, 64, False, True),      # ragged S, key padding
    (8, 16, 1024, 64, False, False),   # c3
    (2, 16, 1024, 64, True, True),
    (1, 16, 8192, 128, False, False),  # c4
    (1, 4, 1000, 128, True, True),
    (3, 2, 77, 128, False, True),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("b,h,s,hd,causal,masked", ATTN_CASES)
def test_flash_attention(cuda, dtype, b, h, s, hd, causal, masked):
    log(f"attn b{b} h{h} s{s} hd{hd} causal={causal} masked={masked} {dtype}")
    d = h * hd
    qk = _randn((b * s, 2 * d), dtype, cuda, 51, 0.8)
    vt = torch.zeros((b, h, hd, _C.vt_ld(s)), dtype=dtype, device=cuda)
    vt[..., :s] = _randn((b, h, hd, s), dtype, cuda, 52)
    valid = None
    if masked:
        from transformer_optimization_amd.workloads import padding_mask
        valid = padding_mask(b, s, 0.5, seed=53).to(cuda)
    scale = hd ** -0.5
    o = _C.flash_attn(qk, vt, b, s, h, hd, scale, causal, key_valid=valid)
    q, k, v = _split(qk, vt, b, s, h, hd)
    ours = o.reshape(b, s, h, hd).permute(0, 2, 1, 3).float()
    eager = _eager_attention(q, k, v, scale, causal, valid).float()
    exact = _fp32_attention(q, k, v, scale, causal, valid)
    err_ours = (ours - exact).abs().max().item()
    err_eager = (eager - exact).abs().max().item()
    diff = (ours - eager).abs().max().item()
    log(f"  |ours-fp32|={err_ours:.3e} |eager-fp32|={err_eager:.3e} |ours-eager|={diff:.3e}")
    assert torch.isfinite(ours).all()
    # No worse than twice eager's own deviation from fp32, plus one output ulp.
    tol = 2 * err_eager + (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11) * exact.abs().max().item()
    assert err_ours <= tol
    assert diff <= 2 * tol


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_flash_attention_c5_rows(cuda, dtype):
    # S = 100000, hd 64: dense scores are impossible; check 512 seeded query
    # rows against fp32 attention over all keys.
    from transformer_optimization_amd.workloads import sample_rows
    b, h, s, hd = 1, 16, 100000, 64
    d = h * hd
    log("attn c5 S=100000")
    qk = _randn((b * s, 2 * d), dtype, cuda, 61, 0.8)
    vt = torch.zeros((b, h, hd, _C.vt_ld(s)), dtype=dtype, device=cuda)
    vt[..., :s] = _randn((b, h, hd, s), dtype, cuda, 62)
    scale = hd ** -0.5
    o = _C.flash_attn(qk, vt, b, s, h, hd, scale, False)
    torch.cuda.synchronize()
    rows = sample_rows(s).to(cuda)
    q, k, v = _split(qk, vt, b, s, h, hd)
    exact = torch.cat([_fp32_attention(q, k, v, scale, False, None, rows[i:i + 64])
                       for i in range(0, rows.numel(), 64)], dim=2)
    ours = o.reshape(b, s, h, hd)[:, rows].permute(0, 2, 1, 3).float()
    err = (ours - exact).abs().max().item()
    log(f"  c5 rows |ours-fp32| = {err:.3e}")
    assert err <= 4 * 2.0 ** -8 * max(exact.abs().max().item(), 1e-3)


def test_fully_masked_rows_are_zero_not_nan(cuda):
    b, h, s, hd = 2, 2, 96, 64
    d = h * hd
    qk = _randn((b * s, 2 * d), torch.bfloat16, cuda, 71)
    vt = _randn((b, h, hd, _C.vt_ld(s)), torch.bfloat16, cuda, 72)
    valid = torch.ones(b, s, dtype=torch.bool, device=cuda)
    valid[1] = False  # batch 1 has no valid key at all
    o = _C.flash_attn(qk, vt, b, s, h, hd, hd ** -0.5, False, key_valid=valid)
    assert torch.isfinite(o).all()
    assert torch.count_nonzero(o[s:]) == 0
