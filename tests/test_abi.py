"""C-ABI and host-glue checks that need no GPU.

* libtx_hip.so loads after ``import torch`` and exports every function that
  include/tx_api.h declares;
* host-side validation returns TX_EINVAL / TX_EUNSUPPORTED before anything
  touches a device (fake non-null pointers are never dereferenced);
* the Python wrappers turn statuses into exceptions and refuse CPU tensors;
* ``UserOptimizedTransformer`` keeps the oracle's state_dict key set and has
  no CPU fallback.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import oracle
from transformer_optimization_amd import TransformerConfig, UserOptimizedTransformer, _C, workloads

ROOT = Path(__file__).resolve().parent.parent
FAKE = 4096  # a non-null, 16-byte aligned address that validation must reject first


def _header_functions():
    text = (ROOT / "include" / "tx_api.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(tx_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _C.load_library()
    declared = _header_functions()
    assert declared == sorted(_C.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.tx_abi_version() == _C.ABI_VERSION


def test_single_hip_runtime_mapped():
    _C.load_library()
    assert len(_C._hip_runtime_mappings()) <= 1


def test_status_strings():
    for code in (0, 1, 2, 3):
        assert _C.status_string(code)
    assert "unknown" in _C.status_string(99)


def test_gemm_validation_without_gpu():
    lib = _C.load_library()
    g = lib.tx_gemm
    # null operand
    assert g(None, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, 0, None, None) == _C.TX_EINVAL
    # non-positive sizes
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 0, 64, 64, 2, 2, 2, 2, 0, None, None) == _C.TX_EINVAL
    # lda < k
    assert g(FAKE, 32, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, 0, None, None) == _C.TX_EINVAL
    # bias flag without bias
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, _C.EPI_BIAS, None, None) == _C.TX_EINVAL
    # K not a multiple of 8
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 12, 2, 2, 2, 2, 0, None, None) == _C.TX_EUNSUPPORTED
    # fp32 operands are not an MFMA input type here
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 0, 0, 0, 0, 0, None, None) == _C.TX_EINVAL
    # misaligned A
    assert g(FAKE + 2, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, 0, None, None) == _C.TX_EUNSUPPORTED
    # unknown epilogue bits
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, 64, None, None) == _C.TX_EINVAL
    # split output needs ldc >= 2N and excludes the residual epilogue
    assert g(FAKE, 64, FAKE, 64, None, None, 0, FAKE, 64, 64, 64, 64, 2, 2, 2, 2, _C.EPI_SPLIT_OUT, None, None) == _C.TX_EINVAL
    assert g(FAKE, 64, FAKE, 64, None, FAKE, 64, FAKE, 128, 64, 64, 64, 2, 2, 2, 2,
             _C.EPI_SPLIT_OUT | _C.EPI_RESIDUAL, None, None) == _C.TX_EINVAL


def test_attention_and_qkv_validation_without_gpu():
    lib = _C.load_library()
    fa = lib.tx_flash_attn_fwd
    E, O = _C.SOFTMAX_EAGER, _C.SOFTMAX_ONLINE
    assert fa(FAKE, FAKE, 64, FAKE, None, 1, 64, 8, 96, 0.1, 0, O, None, 2, None) == _C.TX_EUNSUPPORTED  # head_dim
    assert fa(FAKE, FAKE, 60, FAKE, None, 1, 64, 8, 64, 0.1, 0, O, None, 2, None) == _C.TX_EINVAL  # ldvt < seq
    assert fa(FAKE, FAKE, 68, FAKE, None, 1, 64, 8, 64, 0.1, 0, O, None, 2, None) == _C.TX_EUNSUPPORTED  # ldvt % 8
    assert fa(FAKE, FAKE, 64, FAKE, None, 1, 64, 8, 64, -1.0, 0, O, None, 2, None) == _C.TX_EINVAL  # scale
    assert fa(FAKE, FAKE, 64, FAKE, None, 1, 64, 8, 64, 0.1, 0, O, None, 0, None) == _C.TX_EUNSUPPORTED  # fp32
    assert fa(None, FAKE, 64, FAKE, None, 1, 64, 8, 64, 0.1, 0, O, None, 2, None) == _C.TX_EINVAL
    # eager softmax needs its row-stats workspace; unknown modes are rejected
    assert fa(FAKE, FAKE, 64, FAKE, None, 1, 64, 8, 64, 0.1, 0, E, None, 2, None) == _C.TX_EINVAL
    assert fa(FAKE, FAKE, 64, FAKE, None, 1, 64, 8, 64, 0.1, 0, 7, FAKE, 2, None) == _C.TX_EINVAL
    # o overlapping qk or vt: refused (other workgroups still read them)
    QK, VT, OUT = 1 << 30, 1 << 31, 1 << 32
    assert fa(QK, VT, 64, QK + 512, None, 1, 64, 8, 64, 0.1, 0, O, None, 2, None) == _C.TX_EINVAL
    assert fa(QK, VT, 64, VT, None, 1, 64, 8, 64, 0.1, 0, O, None, 2, None) == _C.TX_EINVAL
    # 32-bit tile offsets: heads * head_dim < 2^24, head_dim * ldvt * 2 + 256 < 2^32
    assert fa(QK, VT, 64, OUT, None, 1, 64, 1 << 18, 64, 0.1, 0, O, None, 2, None) == _C.TX_EUNSUPPORTED
    assert fa(QK, VT, 1 << 25, OUT, None, 1, 64, 8, 128, 0.1, 0, O, None, 2, None) == _C.TX_EUNSUPPORTED
    qkv = lib.tx_qkv_proj
    assert qkv(FAKE, FAKE, FAKE, FAKE, FAKE, 64, 1, 64, 96, 2, 2, None) == _C.TX_EUNSUPPORTED  # D % 64
    assert qkv(FAKE, FAKE, FAKE, FAKE, FAKE, 64, 1, 64, 128, 3, 2, None) == _C.TX_EINVAL  # D % H
    assert qkv(FAKE, FAKE, None, FAKE, FAKE, 64, 1, 64, 128, 2, 2, None) == _C.TX_EINVAL


def test_layernorm_validation_without_gpu():
    lib = _C.load_library()
    ln = lib.tx_layernorm_residual
    assert ln(FAKE, None, None, FAKE, FAKE, FAKE, None, None, None, 4, 12, 1e-5, 2, 2, 2, 2, 0, None) == _C.TX_EUNSUPPORTED
    assert ln(FAKE, None, None, FAKE, FAKE, FAKE, None, None, None, 4, 64, 1e-5, 2, 2, 2, 2, _C.LN_HAS_DELTA, None) == _C.TX_EINVAL
    assert ln(FAKE, None, None, FAKE, FAKE, FAKE, None, None, None, 0, 64, 1e-5, 2, 2, 2, 2, 0, None) == _C.TX_EINVAL
    assert ln(FAKE, None, None, FAKE, FAKE, FAKE, None, None, None, 4, 64, 1e-5, 2, 2, 7, 2, 0, None) == _C.TX_EINVAL
    assert ln(FAKE, None, None, FAKE, FAKE, FAKE, None, None, None, 4, 64, 1e-5, 2, 2, 1, 2, 0, None) == _C.TX_EUNSUPPORTED


def test_status_maps_to_exception():
    with pytest.raises(_C.TxError) as info:
        _C._check("tx_gemm", _C.TX_EUNSUPPORTED)
    assert info.value.code == _C.TX_EUNSUPPORTED and "tx_gemm" in str(info.value)


def test_wrappers_refuse_cpu_tensors():
    a = torch.zeros(64, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _C.gemm(a, a)
    with pytest.raises(ValueError):
        _C.layernorm_residual(a, a[0], a[0])


def _pair(cfg):
    base = oracle.BaselineTransformer(cfg)
    workloads.init_parameters(base)
    opt = UserOptimizedTransformer(cfg)
    return base, opt


def test_state_dict_compatibility_both_directions():
    cfg = TransformerConfig(2, 16, 128, 2, 256, 3, False)
    base, opt = _pair(cfg)
    assert list(base.state_dict().keys()) == list(opt.state_dict().keys())
    oracle.copy_model_weights(base, opt, strict=True)
    for k, v in base.state_dict().items():
        assert torch.equal(v, opt.state_dict()[k])
    base2 = oracle.BaselineTransformer(cfg)
    base2.load_state_dict(opt.state_dict(), strict=True)


def test_derived_caches_are_not_state():
    cfg = TransformerConfig(1, 8, 128, 2, 256, 2, False)
    _, opt = _pair(cfg)
    keys_before = set(opt.state_dict())
    w, b = opt.packed_qkv(1)
    assert set(opt.state_dict()) == keys_before
    att = opt.layers[1].attention
    # fp32 model: the GEMMs read fp16 copies (the reference's *_fp16 caches)
    assert w.dtype == torch.float16
    assert torch.equal(w, torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).half())
    assert torch.equal(b, torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]).half())
    assert set(opt._half[1]) == {"out_proj", "ffn_in", "ffn_out"}
    # in-place update invalidates the packed copy
    with torch.no_grad():
        att.k_proj.weight.add_(1.0)
    w2, _ = opt.packed_qkv(1)
    assert torch.equal(w2[128:256], att.k_proj.weight.half())
    # a bf16 model keeps its own dtype
    opt16 = opt.to(torch.bfloat16)
    w3, _ = opt16.packed_qkv(0)
    att0 = opt16.layers[0].attention
    assert w3.dtype == torch.bfloat16
    assert torch.equal(w3, torch.cat([att0.q_proj.weight, att0.k_proj.weight, att0.v_proj.weight]))
    assert opt16._half == {}


def test_no_cpu_fallback():
    cfg = TransformerConfig(1, 8, 128, 2, 256, 1, False)
    _, opt = _pair(cfg)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        opt(torch.zeros(1, 8, 128))


def test_mask_kind_memo():
    cfg = TransformerConfig(2, 8, 128, 2, 256, 1, False)
    _, opt = _pair(cfg)
    assert opt._mask_kind(None) == "none"
    m = torch.ones(2, 8, dtype=torch.bool)
    assert opt._mask_kind(m) == "all_true"
    m2 = m.clone()
    m2[1, 5:] = False
    assert opt._mask_kind(m2) == "partial"
    assert len(opt._mask_all_true) == 2
    opt._mask_kind(m2)
    assert len(opt._mask_all_true) == 2


def test_default_policy_rule():
    """The default ("auto") numeric policy: the eager mirror wherever the
    eager attention serves the length, the long-sequence policy beyond it
    (so config 5 runs through the plain drop-in API), the fp32 policy for
    fp32 models; explicit attributes pin a policy."""
    cfg = TransformerConfig(1, 8, 128, 2, 256, 1, False)
    _, opt = _pair(cfg)
    assert (opt.softmax, opt.precision) == ("auto", "auto")
    assert opt.resolve_policy(_C.EAGER_MAX_SEQ, torch.bfloat16) == ("eager", "eager")
    assert opt.resolve_policy(_C.EAGER_MAX_SEQ + 1, torch.bfloat16) == ("online", "fp32_residual")
    assert opt.resolve_policy(100000, torch.float32) == ("online", "fp32_model")
    for key, wl in workloads.WORKLOADS.items():
        if wl.dtype != torch.float32:
            assert opt.resolve_policy(wl.config.seq_len, wl.dtype) == (wl.softmax, wl.precision), key
    # Lengths whose ATen block-softmax order is not reproduced take the
    # long-sequence policy (tx_eager_softmax_supported; 64 KiB assumed here).
    assert opt.resolve_policy(1501, torch.bfloat16) == ("eager", "eager")
    assert opt.resolve_policy(2052, torch.bfloat16) == ("eager", "eager")
    assert opt.resolve_policy(2050, torch.bfloat16) == ("online", "fp32_residual")
    assert opt.resolve_policy(20000, torch.bfloat16) == ("online", "fp32_residual")
    assert _C.eager_softmax_supported(2047) and not _C.eager_softmax_supported(2049)
    opt.softmax = "online"
    assert opt.resolve_policy(128, torch.float16) == ("online", "eager")
    opt.precision = "bogus"
    with pytest.raises(ValueError):
        opt.resolve_policy(128, torch.float16)


def test_weights_key_tracks_in_place_updates_and_moves():
    cfg = TransformerConfig(1, 8, 128, 2, 256, 2, False)
    _, opt = _pair(cfg)
    k0 = opt._current_weights_key()
    assert opt._current_weights_key() == k0
    with torch.no_grad():
        opt.layers[1].ffn_out.bias.add_(1.0)
    k1 = opt._current_weights_key()
    assert k1 != k0
    opt = opt.to(torch.float16)  # new storages
    assert opt._current_weights_key()[1] != k1[1]
    opt.invalidate_caches()
    assert opt._params_cache is None and opt._weights_key is None


def test_strided_attention_validation_without_gpu():
    """tx_flash_attn_fwd_strided refuses bad views on the host (nothing launches)."""
    lib = _C.load_library()
    f = lib.tx_flash_attn_fwd_strided

    keep = []  # the stride arrays must outlive the calls that read them

    def st(*v):
        arr = (ctypes.c_int64 * 4)(*v)
        keep.append(arr)
        return ctypes.addressof(arr)

    good = (1 << 20, 64, 3 * 1024, 1)       # [B,H,S,hd] view of a [B,S,3D] projection, D = 1024
    o_good = (1 << 19, 64, 1024, 1)

    def call(q=good, k=good, v=good, o=o_good, kv=None, kv_sb=0, hd=64, mode=_C.SOFTMAX_ONLINE, stats=None):
        return f(FAKE, FAKE, FAKE, FAKE, st(*q), st(*k), st(*v), st(*o), kv, kv_sb,
                 2, 16, 512, hd, 0.125, 0, mode, stats, _C.TX_BF16, None)

    assert call(q=(1 << 20, 64, 3 * 1024, 2)) == _C.TX_EUNSUPPORTED   # head_dim not contiguous
    assert call(k=(-8, 64, 3 * 1024, 1)) == _C.TX_EINVAL              # negative stride
    assert call(v=(1 << 20, 64, 3 * 1024 + 4, 1)) == _C.TX_EUNSUPPORTED  # rows not 16-byte aligned
    assert call(o=(1 << 19, 64, 32, 1)) == _C.TX_EINVAL               # rows overlap (stride < head_dim)
    assert call(o=(1 << 19, 0, 1024, 1)) == _C.TX_EINVAL              # every head on one row
    assert call(o=(32, 1 << 19, 1024, 1)) == _C.TX_EINVAL             # batch 1 overlaps batch 0's rows
    assert call(kv=FAKE, kv_sb=100) == _C.TX_EINVAL                   # mask row shorter than seq
    assert call(hd=96) == _C.TX_EUNSUPPORTED                          # head_dim 64 / 128 only
    assert call(mode=_C.SOFTMAX_EAGER) == _C.TX_EINVAL                # eager softmax needs row_stats
    assert f(None, FAKE, FAKE, FAKE, st(*good), st(*good), st(*good), st(*o_good), None, 0,
             2, 16, 512, 64, 0.125, 0, _C.SOFTMAX_ONLINE, None, _C.TX_BF16, None) == _C.TX_EINVAL
    # o inside the q / k / v projection: refused (q, k, v are at FAKE and span
    # 2 * 512 * 3072 elements; o starting 1 KB in overlaps them all)
    assert f(FAKE, FAKE, FAKE, FAKE + 1024, st(*good), st(*good), st(*good), st(*o_good), None, 0,
             2, 16, 512, 64, 0.125, 0, _C.SOFTMAX_ONLINE, None, _C.TX_BF16, None) == _C.TX_EINVAL


def test_bench_provenance_from_the_build_record(tmp_path, monkeypatch):
    """On a copy of the tree without .git (the GPU box), the bench names the
    commit from the record the build writes next to the library, and says
    whether the kernel sources still match it."""
    import json
    import shutil
    import bench
    from transformer_optimization_amd import build as txbuild

    root = tmp_path / "tree"
    (root / "transformer_optimization_amd" / "_lib").mkdir(parents=True)
    shutil.copytree(txbuild.CSRC, root / "transformer_optimization_amd" / "csrc")
    shutil.copytree(txbuild.INCLUDE, root / "include")
    monkeypatch.setattr(bench, "ROOT", root)
    assert bench.git_state()["head"] is None  # no record yet
    record = {"git_head": "0" * 40, "git_dirty": False, "built_utc": "2026-01-01T00:00:00+00:00",
              "kernel_sources_sha256": bench.kernel_sources_hash()}
    (root / "transformer_optimization_amd" / "_lib" / "build_info.json").write_text(json.dumps(record))
    st = bench.git_state()
    assert st["head"] == "0" * 40 and st["dirty"] is False and st["kernel_sources_match_build"] is True
    (root / "include" / "tx_api.h").write_text("changed\n")
    assert bench.git_state()["kernel_sources_match_build"] is False
