"""tx_flash_attn_fwd_noalloc against tx_flash_attn_fwd, through the C ABI.

The no-allocation entry point keeps the eager softmax's row statistics in
the library's fixed device scratch instead of a caller workspace.  Two calls
in a row (the second smaller, so stale statistics of the first call sit in
the scratch beyond the rows the second covers) must each equal the
workspace entry point bit for bit, and oversize problems must be refused
on the host (TX_ESCRATCH) before anything is launched.
"""

import pytest
import torch

from transformer_optimization_amd import _C
from transformer_optimization_amd.workloads import padding_mask
from _util import log

pytestmark = pytest.mark.gpu


def _case(b, h, s, hd, dtype, dev, seed, masked):
    g = torch.Generator("cpu").manual_seed(seed)
    d = h * hd
    qk = (torch.randn(b * s, 2 * d, generator=g) * 0.8).to(dev, dtype)
    vt = torch.zeros((b, h, hd, _C.vt_ld(s)), dtype=dtype, device=dev)
    vt[..., :s] = torch.randn(b, h, hd, s, generator=g).to(dev, dtype)
    valid = padding_mask(b, s, 0.5, seed=seed + 1).to(dev) if masked else None
    return qk, vt, valid


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_two_calls(cuda, dtype):
    cases = [  # b, h, s, hd, causal, masked -- the second call is smaller
        (8, 16, 1024, 64, False, False),
        (2, 4, 200, 128, True, True),
    ]
    for i, (b, h, s, hd, causal, masked) in enumerate(cases):
        log(f"noalloc call {i + 1}: b{b} h{h} s{s} hd{hd} causal={causal} masked={masked} {dtype}")
        qk, vt, valid = _case(b, h, s, hd, dtype, cuda, 300 + i, masked)
        scale = hd ** -0.5
        want = _C.flash_attn(qk, vt, b, s, h, hd, scale, causal, key_valid=valid, softmax="eager")
        out = torch.empty_like(want)
        got = _C.flash_attn_noalloc(qk, vt, b, s, h, hd, scale, causal, key_valid=valid, out=out)
        torch.cuda.synchronize()
        n_diff = int((got != want).sum())
        log(f"  differing elements {n_diff} of {got.numel()}")
        assert got.data_ptr() == out.data_ptr()
        assert n_diff == 0


def test_noalloc_refuses_oversize_on_host(cuda):
    # batch * heads * seq = 2^21 rows > the 2^20-row scratch: refused before
    # any launch (the sizes are never used to address memory).
    lib = _C.load_library()
    dummy = torch.empty(16, dtype=torch.bfloat16, device=cuda)
    code = lib.tx_flash_attn_fwd_noalloc(dummy.data_ptr(), dummy.data_ptr(), 4096, dummy.data_ptr(), None,
                                         1, 4096, 512, 64, 0.125, 0, _C.SOFTMAX_EAGER, _C.TX_BF16,
                                         torch.cuda.current_stream().cuda_stream)
    assert code == _C.TX_ESCRATCH
    assert "scratch" in _C.status_string(code)
