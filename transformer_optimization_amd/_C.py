"""ctypes binding of ``libtx_hip.so`` (declared in ``include/tx_api.h``).

The library is loaded lazily, after ``import torch``, so that it binds to the
HIP runtime torch already mapped (both resolve ``libamdhip64.so.7`` by
SONAME).  If the library is missing, every wrapper raises -- there is no
fallback path.  Wrappers take torch tensors, check devices / dtypes /
contiguity, pass raw pointers and ``torch.cuda.current_stream()`` and turn a
non-zero status into :class:`TxError`.  They never synchronise, so they are
capturable into a graph.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path
from typing import Optional, Tuple

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtx_hip.so"
ABI_VERSION = 4

TX_OK, TX_EINVAL, TX_EUNSUPPORTED, TX_EHIP, TX_ESCRATCH = 0, 1, 2, 3, 4
TX_F32, TX_F16, TX_BF16 = 0, 1, 2

LN_HAS_DELTA, LN_MASK_DELTA, LN_MASK_X, LN_MASK_OUT, LN_WRITE_X, LN_SPLIT_Y = 1, 2, 4, 8, 16, 32
EPI_BIAS, EPI_GELU_ERF, EPI_RESIDUAL, EPI_MASK_DELTA, EPI_MASK_OUT, EPI_SPLIT_OUT = 1, 2, 4, 8, 16, 32
SOFTMAX_EAGER, SOFTMAX_ONLINE = 0, 1
SOFTMAX_MODES = {"eager": SOFTMAX_EAGER, "online": SOFTMAX_ONLINE}
# Longest sequence the eager-exact softmax serves (tx_flash_attn_fwd returns
# TX_EUNSUPPORTED above it: 1024 key tiles of 64); below it, the lengths
# eager_softmax_supported accepts.
EAGER_MAX_SEQ = 65536
# Shared memory per block assumed where no device can be asked (the usual
# value; it only decides lengths from ~16K keys up).
DEFAULT_SHARED_MEM_PER_BLOCK = 65536

# Every symbol include/tx_api.h declares.
EXPORTED_SYMBOLS = (
    "tx_abi_version",
    "tx_status_string",
    "tx_device_cu_count",
    "tx_eager_softmax_supported",
    "tx_layernorm_residual",
    "tx_gemm",
    "tx_qkv_proj",
    "tx_flash_attn_fwd",
    "tx_flash_attn_fwd_strided",
    "tx_flash_attn_fwd_noalloc",
)

# Rows (batch * heads * seq) the fixed scratch of tx_flash_attn_fwd_noalloc holds.
NOALLOC_MAX_STAT_ROWS = 1 << 20

_DT = {torch.float32: TX_F32, torch.float16: TX_F16, torch.bfloat16: TX_BF16}


class TxError(RuntimeError):
    """A libtx_hip entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed: {msg} (status {code})")
        self.code = code
        self.fn = fn


_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

_i64, _i32, _u32, _f32, _vp = ctypes.c_int64, ctypes.c_int, ctypes.c_uint32, ctypes.c_float, ctypes.c_void_p


def _declare(lib: ctypes.CDLL) -> None:
    lib.tx_abi_version.restype = _i32
    lib.tx_abi_version.argtypes = []
    lib.tx_status_string.restype = ctypes.c_char_p
    lib.tx_status_string.argtypes = [_i32]
    lib.tx_device_cu_count.restype = _i32
    lib.tx_device_cu_count.argtypes = []
    lib.tx_eager_softmax_supported.restype = _i32
    lib.tx_eager_softmax_supported.argtypes = [_i64, _i64]
    lib.tx_layernorm_residual.restype = _i32
    lib.tx_layernorm_residual.argtypes = [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp,  # x delta x_out y gamma beta row_valid
        _vp, _vp,                           # mean_out rstd_out
        _i64, _i64, _f32,                   # rows d eps
        _i32, _i32, _i32, _i32,             # x_dt delta_dt y_dt param_dt
        _u32, _vp,                          # flags stream
    ]
    lib.tx_gemm.restype = _i32
    lib.tx_gemm.argtypes = [
        _vp, _i64, _vp, _i64,               # a lda w ldw
        _vp, _vp, _i64,                     # bias residual ldr
        _vp, _i64, _i64, _i64, _i64,        # c ldc m n k
        _i32, _i32, _i32, _i32, _u32,       # ab_dt c_dt bias_dt res_dt epilogue
        _vp, _vp,                           # row_valid stream
    ]
    lib.tx_qkv_proj.restype = _i32
    lib.tx_qkv_proj.argtypes = [
        _vp, _vp, _vp, _vp, _vp, _i64,      # a w_qkv b_qkv qk vt ldvt
        _i64, _i64, _i64, _i64, _i32, _vp,  # batch seq d_model heads dt stream
    ]
    lib.tx_flash_attn_fwd.restype = _i32
    lib.tx_flash_attn_fwd.argtypes = [
        _vp, _vp, _i64, _vp, _vp,           # qk vt ldvt o key_valid
        _i64, _i64, _i64, _i64,             # batch seq heads head_dim
        _f32, _i32, _i32, _vp,              # scale causal softmax_mode row_stats
        _i32, _vp,                          # dt stream
    ]
    lib.tx_flash_attn_fwd_strided.restype = _i32
    lib.tx_flash_attn_fwd_strided.argtypes = [
        _vp, _vp, _vp, _vp,                 # q k v o
        _vp, _vp, _vp, _vp,                 # q/k/v/o strides (int64[4] each)
        _vp, _i64,                          # key_valid key_valid_sb
        _i64, _i64, _i64, _i64,             # batch heads seq head_dim
        _f32, _i32, _i32, _vp,              # scale causal softmax_mode row_stats
        _i32, _vp,                          # dt stream
    ]
    lib.tx_flash_attn_fwd_noalloc.restype = _i32
    lib.tx_flash_attn_fwd_noalloc.argtypes = [
        _vp, _vp, _i64, _vp, _vp,           # qk vt ldvt o key_valid
        _i64, _i64, _i64, _i64,             # batch seq heads head_dim
        _f32, _i32, _i32, _i32, _vp,        # scale causal softmax_mode dt stream
    ]


def _hip_runtime_mappings() -> set:
    paths = set()
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                if "libamdhip64" in line:
                    paths.add(line.split()[-1])
    except OSError:
        pass
    return paths


def load_library() -> ctypes.CDLL:
    """Load and check libtx_hip.so once per process (raises if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m transformer_optimization_amd.build` "
                "(or __graft_entry__.build()). There is no fallback path."
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        _declare(lib)
        if lib.tx_abi_version() != ABI_VERSION:
            raise ImportError(f"libtx_hip ABI {lib.tx_abi_version()} != expected {ABI_VERSION}")
        maps = _hip_runtime_mappings()
        if len(maps) > 1:
            raise ImportError(
                "two HIP runtimes are mapped into this process "
                f"({sorted(maps)}); load libtx_hip after `import torch`"
            )
        _lib = lib
        return lib


def status_string(code: int) -> str:
    return load_library().tx_status_string(code).decode()


def _check(fn: str, code: int) -> None:
    if code != TX_OK:
        raise TxError(fn, code, status_string(code))


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require_cuda(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise ValueError("libtx_hip operates on GPU tensors only (got a CPU tensor)")


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def cu_count() -> int:
    return int(load_library().tx_device_cu_count())


_eager_ok: dict = {}


def eager_softmax_supported(seq: int, device: Optional[torch.device] = None) -> bool:
    """Whether the eager-exact softmax serves rows of ``seq`` keys on
    ``device`` (``tx_eager_softmax_supported``; the device's shared memory
    per block, as torch reports it, decides the longest lengths).  Without a
    device, the usual 64 KiB is assumed.  Memoised per (seq, device)."""
    key = (int(seq), device)
    got = _eager_ok.get(key)
    if got is None:
        if device is not None and device.type == "cuda":
            smem = int(torch.cuda.get_device_properties(device).shared_memory_per_block)
        else:
            smem = DEFAULT_SHARED_MEM_PER_BLOCK
        got = _eager_ok[key] = load_library().tx_eager_softmax_supported(int(seq), smem) == 1
    return got


# ------------------------------------------------------------ launch record
class Launch:
    """One entry-point call as the wrappers made it: the C function, its
    arguments (all but the trailing stream), the tensors they point into
    (kept alive) and a description of the work.  Calling it enqueues the same
    launch again on the current stream."""

    __slots__ = ("fn", "args", "keep", "info")

    def __init__(self, fn: str, args: tuple, keep: tuple, info: dict):
        self.fn, self.args, self.keep, self.info = fn, args, keep, info

    def __call__(self) -> None:
        _check(self.fn, getattr(load_library(), self.fn)(*self.args, _stream()))

    def __repr__(self) -> str:
        return f"Launch({self.fn}, {self.info})"


_recorder: Optional[list] = None


@contextlib.contextmanager
def record_launches():
    """Collect every launch the wrappers make inside the block, in order, as
    :class:`Launch` objects (used to time exactly the kernels a forward runs)."""
    global _recorder
    prev, _recorder = _recorder, []
    try:
        yield _recorder
    finally:
        _recorder = prev


def _launch(fn: str, args: tuple, keep: tuple, info: dict) -> None:
    """Call ``lib.<fn>(*args, stream)`` on the current stream; raise on a
    non-zero status; record the call when a recording is active."""
    _check(fn, getattr(load_library(), fn)(*args, _stream()))
    if _recorder is not None:
        _recorder.append(Launch(fn, args, keep, info))


# ----------------------------------------------------------------- wrappers
def layernorm_residual(
    x: torch.Tensor,
    gamma: torch.Tensor,
    beta: torch.Tensor,
    *,
    delta: Optional[torch.Tensor] = None,
    x_out: Optional[torch.Tensor] = None,
    y: Optional[torch.Tensor] = None,
    y_dtype: Optional[torch.dtype] = None,
    row_valid: Optional[torch.Tensor] = None,
    flags: int = 0,
    eps: float = 1e-5,
    mean_out: Optional[torch.Tensor] = None,
    rstd_out: Optional[torch.Tensor] = None,
    split: bool = False,
) -> torch.Tensor:
    """``y = LN(x [+ delta])`` over the last dim; see ``tx_layernorm_residual``.
    ``mean_out`` / ``rstd_out`` (fp32, one per row) receive the row statistics.
    ``split=True`` writes y as [rows, 2d]: the rounded value, then the rounded
    remainder (a two-term operand for the fp32-residual policy)."""
    load_library()
    _require_cuda(x, gamma, beta, delta, x_out, y, row_valid, mean_out, rstd_out)
    d = x.shape[-1]
    rows = x.numel() // d
    if y is None:
        shape = (*x.shape[:-1], 2 * d) if split else x.shape
        y = torch.empty(shape, dtype=y_dtype or x.dtype, device=x.device)
    if y.numel() != rows * d * (2 if split else 1):
        raise ValueError("y has the wrong number of elements")
    if split:
        flags |= LN_SPLIT_Y
    for t in (x, y, delta, x_out):
        if t is not None and not t.is_contiguous():
            raise ValueError("layernorm_residual needs contiguous rows")
    if delta is not None:
        flags |= LN_HAS_DELTA
    if x_out is not None:
        flags |= LN_WRITE_X
    for t in (mean_out, rstd_out):
        if t is not None and (t.dtype != torch.float32 or t.numel() != rows or not t.is_contiguous()):
            raise ValueError("mean_out / rstd_out must be contiguous fp32 with one entry per row")
    rv = row_valid.contiguous() if row_valid is not None else None
    args = (
        x.data_ptr(), _ptr(delta), _ptr(x_out), y.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
        _ptr(rv), _ptr(mean_out), _ptr(rstd_out), rows, d, float(eps), _dt(x),
        _dt(delta) if delta is not None else _dt(x), _dt(y), _dt(gamma), flags,
    )
    info = {"op": "layernorm", "rows": rows, "d": d, "x_bytes": x.element_size(),
            "y_bytes": y.element_size(), "param_bytes": gamma.element_size(), "flags": flags,
            "delta_bytes": delta.element_size() if delta is not None else 0}
    _launch("tx_layernorm_residual", args, (x, delta, x_out, y, gamma, beta, rv, mean_out, rstd_out), info)
    return y


def gemm(
    a: torch.Tensor,
    w: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    *,
    residual: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    gelu: bool = False,
    row_valid: Optional[torch.Tensor] = None,
    mask_delta: bool = False,
    mask_out: bool = False,
    split_out: bool = False,
) -> torch.Tensor:
    """``out = epilogue(a @ w.T)`` for a 2-D ``a`` [M,K] and nn.Linear ``w`` [N,K].
    ``split_out=True`` stores the unrounded fp32 result as a hi/lo pair in
    ``out`` [M, 2N] (``out_dtype`` = the operand dtype)."""
    load_library()
    _require_cuda(a, w, bias, residual, out, row_valid)
    if a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise ValueError(f"gemm shapes: a {tuple(a.shape)} w {tuple(w.shape)}")
    m, k = a.shape
    n = w.shape[0]
    if a.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("gemm operands must be K-contiguous")
    ncols = 2 * n if split_out else n
    if out is None:
        out = torch.empty((m, ncols), dtype=out_dtype or a.dtype, device=a.device)
    if out.shape != (m, ncols) or out.stride(1) != 1:
        raise ValueError(f"gemm output must be [M, {ncols}] with unit column stride")
    epi = 0
    if bias is not None:
        epi |= EPI_BIAS
    if gelu:
        epi |= EPI_GELU_ERF
    ldr = 0
    if residual is not None:
        if residual.shape != (m, n) or residual.stride(1) != 1:
            raise ValueError("residual must be [M, N] with unit column stride")
        epi |= EPI_RESIDUAL
        ldr = residual.stride(0)
    if split_out:
        epi |= EPI_SPLIT_OUT
    if mask_delta:
        epi |= EPI_MASK_DELTA
    if mask_out:
        epi |= EPI_MASK_OUT
    rv = row_valid.contiguous() if row_valid is not None else None
    args = (
        a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
        _ptr(bias), _ptr(residual), ldr,
        out.data_ptr(), out.stride(0), m, n, k,
        _dt(a), _dt(out), _dt(bias) if bias is not None else _dt(a),
        _dt(residual) if residual is not None else _dt(out), epi,
        _ptr(rv),
    )
    info = {"op": "gemm", "m": m, "n": n, "k": k, "epilogue": epi, "ab_bytes": a.element_size(),
            "c_bytes": out.element_size()}
    _launch("tx_gemm", args, (a, w, bias, residual, out, rv), info)
    return out


def vt_ld(seq: int) -> int:
    """Row stride of the head-transposed V buffer: seq rounded up to 8."""
    return (seq + 7) // 8 * 8


def qkv_proj(
    a: torch.Tensor,
    w_qkv: torch.Tensor,
    b_qkv: torch.Tensor,
    batch: int,
    seq: int,
    heads: int,
    *,
    qk: Optional[torch.Tensor] = None,
    vt: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Packed QKV projection -> (qk [M, 2D], vt [B, H, hd, ldvt])."""
    load_library()
    _require_cuda(a, w_qkv, b_qkv, qk, vt)
    m, d = a.shape
    if m != batch * seq or w_qkv.shape != (3 * d, d) or b_qkv.shape != (3 * d,):
        raise ValueError("qkv_proj shapes")
    for t in (a, w_qkv, b_qkv):
        if not t.is_contiguous():
            raise ValueError("qkv_proj operands must be contiguous")
    hd = d // heads
    ld = vt_ld(seq)
    if qk is None:
        qk = torch.empty((m, 2 * d), dtype=a.dtype, device=a.device)
    if vt is None:
        vt = torch.empty((batch, heads, hd, ld), dtype=a.dtype, device=a.device)
    args = (a.data_ptr(), w_qkv.data_ptr(), b_qkv.data_ptr(), qk.data_ptr(), vt.data_ptr(), ld,
            batch, seq, d, heads, _dt(a))
    info = {"op": "qkv_proj", "m": m, "n": 3 * d, "k": d, "ab_bytes": a.element_size()}
    _launch("tx_qkv_proj", args, (a, w_qkv, b_qkv, qk, vt), info)
    return qk, vt


def flash_attn(
    qk: torch.Tensor,
    vt: torch.Tensor,
    batch: int,
    seq: int,
    heads: int,
    head_dim: int,
    scale: float,
    causal: bool,
    *,
    key_valid: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    softmax: str = "eager",
    row_stats: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention over the ``qkv_proj`` layouts -> o [B*S, H*hd].

    ``softmax="eager"`` reproduces the eager fp32 softmax bit for bit and uses
    ``row_stats`` (fp32, 2*B*H*S; allocated here when omitted);
    ``softmax="online"`` is the one-pass online softmax."""
    load_library()
    _require_cuda(qk, vt, key_valid, out, row_stats)
    if softmax not in SOFTMAX_MODES:
        raise ValueError(f"softmax must be one of {sorted(SOFTMAX_MODES)}")
    mode = SOFTMAX_MODES[softmax]
    d = heads * head_dim
    if qk.shape != (batch * seq, 2 * d) or not qk.is_contiguous():
        raise ValueError("qk must be contiguous [B*S, 2D]")
    if vt.dim() != 4 or tuple(vt.shape[:3]) != (batch, heads, head_dim) or not vt.is_contiguous():
        raise ValueError("vt must be contiguous [B, H, hd, ldvt]")
    if out is None:
        out = torch.empty((batch * seq, d), dtype=qk.dtype, device=qk.device)
    kv = None
    if key_valid is not None:
        if key_valid.dtype not in (torch.bool, torch.uint8) or key_valid.numel() != batch * seq:
            raise ValueError("key_valid must be bool/uint8 with B*S elements")
        kv = key_valid.contiguous()
    if mode == SOFTMAX_EAGER:
        if row_stats is None:
            row_stats = torch.empty(2 * batch * heads * seq, dtype=torch.float32, device=qk.device)
        if row_stats.dtype != torch.float32 or row_stats.numel() < 2 * batch * heads * seq:
            raise ValueError("row_stats must be fp32 with at least 2*B*H*S elements")
    args = (qk.data_ptr(), vt.data_ptr(), vt.shape[3], out.data_ptr(), _ptr(kv),
            batch, seq, heads, head_dim, float(scale), 1 if causal else 0, mode,
            _ptr(row_stats) if mode == SOFTMAX_EAGER else None, _dt(qk))
    info = {"op": "flash_attn", "batch": batch, "seq": seq, "heads": heads, "head_dim": head_dim,
            "causal": bool(causal), "softmax": softmax}
    _launch("tx_flash_attn_fwd", args, (qk, vt, out, kv, row_stats), info)
    return out


def _strides4(t: torch.Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def flash_attn_strided(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal: bool,
    *,
    key_valid: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    softmax: str = "eager",
    row_stats: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention over strided [B, H, S, hd] views (``tx_flash_attn_fwd_strided``),
    the call shape of the reference's ``_triton_short_attention(q, k, v, scale,
    causal, mask_active, valid_token_mask)`` (TTB:1596-1668): q / k / v may be
    column slices of a packed [B, S, 3D] projection viewed as [B, H, S, hd].
    Returns ``out``, a [B, H, S, hd] view; by default the permuted view of a
    fresh [B, S, H, hd] tensor, i.e. heads merged in memory ([B, S, D])."""
    load_library()
    _require_cuda(q, k, v, key_valid, out, row_stats)
    if softmax not in SOFTMAX_MODES:
        raise ValueError(f"softmax must be one of {sorted(SOFTMAX_MODES)}")
    mode = SOFTMAX_MODES[softmax]
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must be [B, H, S, hd] views of one shape")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    b, h, s, hd = q.shape
    if out is None:
        out = torch.empty((b, s, h, hd), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    if out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must be a [B, H, S, hd] view of the operand dtype")
    kv, kv_sb = None, 0
    if key_valid is not None:
        if key_valid.dtype not in (torch.bool, torch.uint8) or tuple(key_valid.shape) != (b, s):
            raise ValueError("key_valid must be a bool/uint8 [B, S] tensor")
        kv = key_valid if key_valid.stride(1) == 1 else key_valid.contiguous()
        kv_sb = kv.stride(0)
    if mode == SOFTMAX_EAGER:
        if row_stats is None:
            row_stats = torch.empty(2 * b * h * s, dtype=torch.float32, device=q.device)
        if row_stats.dtype != torch.float32 or row_stats.numel() < 2 * b * h * s:
            raise ValueError("row_stats must be fp32 with at least 2*B*H*S elements")
    st = tuple(_strides4(t) for t in (q, k, v, out))
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            ctypes.addressof(st[0]), ctypes.addressof(st[1]), ctypes.addressof(st[2]),
            ctypes.addressof(st[3]), _ptr(kv), kv_sb, b, h, s, hd, float(scale), 1 if causal else 0,
            mode, _ptr(row_stats) if mode == SOFTMAX_EAGER else None, _dt(q))
    info = {"op": "flash_attn", "batch": b, "seq": s, "heads": h, "head_dim": hd,
            "causal": bool(causal), "softmax": softmax}
    # st stays with the recorded launch: a re-launch passes the same stride arrays.
    _launch("tx_flash_attn_fwd_strided", args, (q, k, v, out, kv, row_stats, st), info)
    return out


def flash_attn_noalloc(
    qk: torch.Tensor,
    vt: torch.Tensor,
    batch: int,
    seq: int,
    heads: int,
    head_dim: int,
    scale: float,
    causal: bool,
    *,
    key_valid: Optional[torch.Tensor] = None,
    out: torch.Tensor,
    softmax: str = "eager",
) -> torch.Tensor:
    """``flash_attn`` through ``tx_flash_attn_fwd_noalloc``: the eager softmax's
    row statistics live in the library's fixed device scratch, so nothing is
    allocated (``out`` is the caller's).  batch * heads * seq above
    ``NOALLOC_MAX_STAT_ROWS`` raises TxError (TX_ESCRATCH)."""
    load_library()
    _require_cuda(qk, vt, key_valid, out)
    if softmax not in SOFTMAX_MODES:
        raise ValueError(f"softmax must be one of {sorted(SOFTMAX_MODES)}")
    d = heads * head_dim
    if qk.shape != (batch * seq, 2 * d) or not qk.is_contiguous():
        raise ValueError("qk must be contiguous [B*S, 2D]")
    if vt.dim() != 4 or tuple(vt.shape[:3]) != (batch, heads, head_dim) or not vt.is_contiguous():
        raise ValueError("vt must be contiguous [B, H, hd, ldvt]")
    if out.shape != (batch * seq, d) or not out.is_contiguous() or out.dtype != qk.dtype:
        raise ValueError("out must be contiguous [B*S, D] of the operand dtype")
    kv = None
    if key_valid is not None:
        if key_valid.dtype not in (torch.bool, torch.uint8) or key_valid.numel() != batch * seq:
            raise ValueError("key_valid must be bool/uint8 with B*S elements")
        if not key_valid.is_contiguous():
            raise ValueError("key_valid must be contiguous (no copy is made)")
        kv = key_valid
    args = (qk.data_ptr(), vt.data_ptr(), vt.shape[3], out.data_ptr(), _ptr(kv),
            batch, seq, heads, head_dim, float(scale), 1 if causal else 0, SOFTMAX_MODES[softmax], _dt(qk))
    info = {"op": "flash_attn", "batch": batch, "seq": seq, "heads": heads, "head_dim": head_dim,
            "causal": bool(causal), "softmax": softmax, "noalloc": True}
    _launch("tx_flash_attn_fwd_noalloc", args, (qk, vt, out, kv), info)
    return out
