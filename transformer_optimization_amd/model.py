"""``UserOptimizedTransformer``: the reference's optimised-model API over the
gfx950 kernels of ``libtx_hip.so``.

Module API kept from the reference (TTB:2144, 2282, 3509-3611):

* ``UserOptimizedTransformer(config)`` holds exactly the parameters of
  ``BaselineTransformer`` under the same names (``layers.{i}.norm1``,
  ``layers.{i}.attention.{q,k,v,out}_proj``, ``layers.{i}.norm2``,
  ``layers.{i}.ffn_in``, ``layers.{i}.ffn_out``, ``final_norm``), so a strict
  ``load_state_dict`` works in both directions.  Derived state (the packed
  QKV weights, captured graphs, the mask memo) lives in plain attributes.
* ``forward(x, valid_token_mask=None) -> Tensor`` returns a fresh tensor.

Forward schedule per layer (TTB:4115-4314; seven launches):

  LN1            tx_layernorm_residual          x -> y
  QKV            tx_qkv_proj                    y -> qk [M,2D], vt [B,H,hd,S']
  attention      tx_flash_attn_fwd              qk, vt -> o [M,D] (heads merged)
  (or, with the strided layout: tx_gemm -> qkv [M,3D], then
   tx_flash_attn_fwd_strided on [B,H,S,hd] column views of qkv)
  out_proj       tx_gemm BIAS|RESIDUAL          x <- round(x + round(o Wo^T + bo))
  LN2            tx_layernorm_residual          x -> y
  FFN in         tx_gemm BIAS|GELU_ERF          y -> h [M,F]
  FFN out        tx_gemm BIAS|RESIDUAL          x <- round(x + round(h W2^T + b2))

then the final LayerNorm.  With a partial ``valid_token_mask``, invalid query
rows drop the attention term (MASK_DELTA), the residual stream is zeroed after
each block (MASK_OUT on FFN out) and the final output rows are zeroed, the
three masking points of the eager model (TTB:196-197, 219-220, 246-247).

fp32 models follow the reference's shipped fp32 policy (TTB:2226-2239,
4108, 4130-4199): the residual stream, the LayerNorms and the output stay
fp32, every GEMM and the attention run on fp16 operands (fp16 copies of the
weights, LayerNorm writing fp16 directly), and the GEMM results that feed the
residual are added in fp32.

On CUDA(HIP) tensors the whole forward is captured once per
(shape, dtype, device, causal, mask kind, numeric policy) into a hipGraph
(``torch.cuda.CUDAGraph``) and replayed (TTB:3613-3725).  CPU tensors and
unsupported configurations raise: there is no eager-ATen fallback.
"""

from __future__ import annotations

import operator
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import _C
from .config import TransformerConfig


class SelfAttentionParams(nn.Module):
    """Parameters of one attention sublayer (names of TTB:135-149)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)


class BlockParams(nn.Module):
    """Parameters of one pre-LayerNorm block (names of TTB:201-208)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = SelfAttentionParams(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)


class TransformerParams(nn.Module):
    """Parameter container with ``BaselineTransformer``'s structure (TTB:224-236)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self.layers = nn.ModuleList(
            BlockParams(config.d_model, config.num_heads, config.ffn_dim)
            for _ in range(config.num_layers)
        )
        self.final_norm = nn.LayerNorm(config.d_model)


@dataclass
class _GraphEntry:
    graph: "torch.cuda.CUDAGraph"
    static_x: torch.Tensor
    static_mask: Optional[torch.Tensor]
    static_out: torch.Tensor
    # The parameter storages the graph reads (detached aliases), held so that
    # a replay can never read freed memory even when a parameter's storage
    # was replaced since the capture (the replay is then discarded, see
    # forward).
    weights: tuple = ()
    # Layer 0's first LayerNorm when it runs outside the graph (16-bit eager
    # policy): (its norm module, the LayerNorm output buffer the graph reads).
    first_ln: Optional[tuple] = None


# Share of device memory a captured graph's private pool may retain.
_GRAPH_MEMORY_FRACTION = 0.5

_VERSION = operator.attrgetter("_version")


class UserOptimizedTransformer(TransformerParams):
    """Drop-in for the reference's ``UserOptimizedTransformer`` (TTB:2144)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__(config)
        self._packed_qkv: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._weights_key: Optional[tuple] = None
        self._graph_cache: Dict[tuple, _GraphEntry] = {}
        self._graph_pool = None
        self._mask_all_true: Dict[tuple, bool] = {}
        self.use_graphs = True
        # Numeric policy of 16-bit models.  "auto" (the default) chooses per
        # input shape, as the reference's forward chooses its route itself
        # (TTB:3509-3611): the eager mirror wherever the eager chain it
        # mirrors can exist, otherwise the long-sequence policy (see
        # resolve_policy).  Explicit values pin one policy:
        # softmax "eager": attention reproduces the eager fp32 softmax bit for
        #   bit (the gate's comparator); "online": one-pass online softmax.
        # precision "eager": every intermediate rounded to the model dtype
        #   exactly where the eager model rounds it; "fp32_residual": the
        #   residual stream stays fp32 and the FFN GEMMs take their
        #   activations as hi/lo pairs of the model dtype, for comparison
        #   against an fp32 evaluation (the check used where no eager
        #   baseline can run, e.g. S = 100000).
        self.softmax = "auto"
        self.precision = "auto"
        self._params_cache: Optional[list] = None
        self._fits_cache: Dict[tuple, bool] = {}
        # Layout between the QKV projection and attention: "packed" (q/k in
        # [M, 2D], V head-transposed; the default) or "strided" (one [M, 3D]
        # GEMM output read as column views through the reference-shaped
        # entry point).  Both give identical bits; packed measured 1-2%
        # faster at the long-sequence shapes (attention's V operand is one
        # 128-bit LDS read instead of two transpose reads).  Part of the graph key.
        self._qkv_layout = "packed"
        self._dup_ffn: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
        # fp32 model: fp16 copies of out_proj / ffn_in / ffn_out per layer.
        self._half: Dict[int, Dict[str, Tuple[torch.Tensor, torch.Tensor]]] = {}

    # ------------------------------------------------------------ derived state
    def _current_weights_key(self) -> tuple:
        """Storage address and in-place version of every parameter.  Runs on
        every forward, so it is kept to two C-level attribute reads per
        parameter over a cached parameter list (dtype and device changes move
        the storage, so the address covers them)."""
        ps = self._params_cache
        if ps is None:
            ps = self._params_cache = list(self.parameters())
        return (tuple(map(_VERSION, ps)), tuple(map(torch.Tensor.data_ptr, ps)))

    def _apply(self, fn, *args, **kwargs):
        # .to() / .half() / .cuda() may replace parameter objects.
        self._params_cache = None
        self._fits_cache.clear()
        return super()._apply(fn, *args, **kwargs)

    def _refresh_derived(self) -> None:
        """Rebuild packed weights and drop graphs when any parameter changed
        (storage or in-place version), as TTB:455-462 keys its caches on
        storage identity.  Updates in place (``load_state_dict``, ``copy_``,
        ``mul_``) and ``.to()`` are seen; a Parameter object swapped into a
        submodule by assignment is not in the cached list, so such code calls
        ``invalidate_caches()`` afterwards."""
        key = self._current_weights_key()
        if key == self._weights_key:
            return
        # A parameter object may have been replaced (new storage): re-list them.
        self._params_cache = None
        key = self._current_weights_key()
        self._graph_cache.clear()
        self._packed_qkv.clear()
        self._dup_ffn.clear()
        self._half.clear()
        with torch.no_grad():
            for i, layer in enumerate(self.layers):
                att = layer.attention
                w = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight], 0).contiguous()
                b = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias], 0).contiguous()
                if w.dtype == torch.float32:
                    # fp32 model: the GEMMs read fp16 copies (TTB:440-504, the
                    # reference's *_fp16 weight caches).
                    w, b = w.half(), b.half()
                    self._half[i] = {
                        name: (lin.weight.detach().half().contiguous(), lin.bias.detach().half().contiguous())
                        for name, lin in (("out_proj", att.out_proj), ("ffn_in", layer.ffn_in),
                                          ("ffn_out", layer.ffn_out))
                    }
                self._packed_qkv[i] = (w, b)
        self._weights_key = key

    def invalidate_caches(self) -> None:
        """Forget every derived tensor and captured graph (rebuilt on the next forward)."""
        self._params_cache = None
        self._weights_key = None
        self._graph_cache.clear()
        self._fits_cache.clear()

    def _ffn_dup(self, layer: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """``[W, W]`` along K for the FFN weights: with a hi/lo activation
        operand ``[a_hi, a_lo]`` one GEMM computes ``W a_hi + W a_lo``."""
        got = self._dup_ffn.get(layer)
        if got is None:
            blk = self.layers[layer]
            with torch.no_grad():
                w1 = torch.cat([blk.ffn_in.weight, blk.ffn_in.weight], 1).contiguous()
                w2 = torch.cat([blk.ffn_out.weight, blk.ffn_out.weight], 1).contiguous()
            got = self._dup_ffn[layer] = (w1, w2)
        return got

    def packed_qkv(self, layer: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """``(cat(Wq, Wk, Wv) [3D, D], cat(bq, bk, bv) [3D])`` of a layer (TTB:440-504)."""
        self._refresh_derived()
        return self._packed_qkv[layer]

    def _mask_kind(self, mask: Optional[torch.Tensor]) -> str:
        """none / all_true / partial; at most one device->host sync per distinct
        mask tensor (TTB:2438-2477)."""
        if mask is None:
            return "none"
        try:
            version = mask._version
        except RuntimeError:  # inference tensors carry no version counter
            version = None
        key = (mask.data_ptr(), tuple(mask.shape), mask.dtype, version)
        all_true = self._mask_all_true.get(key)
        if all_true is None:
            all_true = bool(torch.all(mask))
            self._mask_all_true[key] = all_true
        return "all_true" if all_true else "partial"

    # ----------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        cfg = self.config
        if x.dim() != 3 or x.shape[-1] != cfg.d_model:
            raise ValueError(f"expected x of shape [B, S, {cfg.d_model}], got {tuple(x.shape)}")
        if x.device.type != "cuda":
            raise RuntimeError(
                "UserOptimizedTransformer runs on the MI355X HIP kernels only; "
                f"got a tensor on {x.device} (no CPU fallback exists)"
            )
        if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise NotImplementedError(f"model dtype {x.dtype} is not implemented by libtx_hip")
        if self.final_norm.weight.dtype != x.dtype or self.final_norm.weight.device != x.device:
            raise ValueError("input dtype/device must match the model's (call .to(device, dtype))")
        if valid_token_mask is not None:
            if valid_token_mask.shape != x.shape[:2] or valid_token_mask.dtype != torch.bool:
                raise ValueError("valid_token_mask must be a bool tensor of shape [B, S]")
            if valid_token_mask.device != x.device:
                raise ValueError("valid_token_mask must be on the input's device")
        # The layers run in inference mode (no autograd bookkeeping on the
        # internal buffers); the returned tensor is allocated outside it, in
        # the caller's mode, so a caller under no_grad gets an ordinary tensor
        # it can update in place or keep (the reference returns a clone of
        # its static output, TTB:3613-3627; its harness also calls forward
        # under torch.no_grad(), TTB:3683-3706).
        with torch.inference_mode():
            _C.load_library()
            kind = self._mask_kind(valid_token_mask)
            mask = valid_token_mask.contiguous() if kind == "partial" else None
            x = x.contiguous()
            cur = self._residual_stream(x, mask, kind)
        return self._final_ln(cur, mask, x.shape, x.dtype)

    def _residual_stream(self, x: torch.Tensor, mask: Optional[torch.Tensor], kind: str) -> torch.Tensor:
        """Run the layers (graph replay where possible) and return the final
        residual stream [M, D] the final LayerNorm reads."""
        cfg = self.config
        policy = self.resolve_policy(x.shape[1], x.dtype, x.device)
        if not self.use_graphs or not self._graph_fits(x):
            self._refresh_derived()
            return self._forward_layers(x, mask, policy)
        # A weight change clears the graph cache (_refresh_derived), so the
        # weights need no place in the key.
        key = (tuple(x.shape), x.dtype, x.device, cfg.causal, kind, policy, self._qkv_layout)
        entry = self._graph_cache.get(key)
        if entry is not None:
            # Replay first and check the weights while it runs: the check
            # walks every parameter (~20 us of host time at c2's 100
            # tensors), which would otherwise delay the replay.  When a
            # parameter changed since the capture, this replay (which read
            # the storages the entry holds) is discarded and the forward
            # runs again on the rebuilt state.
            self._replay(entry, x, mask)
            if self._current_weights_key() == self._weights_key:
                return entry.static_out
        self._refresh_derived()
        entry = self._graph_cache.get(key)
        if entry is None:
            entry = self._capture(x, mask, policy)
            self._graph_cache[key] = entry
        self._replay(entry, x, mask)
        return entry.static_out

    @staticmethod
    def _replay(entry: "_GraphEntry", x: torch.Tensor, mask: Optional[torch.Tensor]) -> None:
        """Load the inputs into the entry's static buffers and replay its graph;
        static_out is the residual stream the final LayerNorm then reads."""
        if entry.first_ln is not None:
            # Layer 0's LayerNorm reads the caller's tensor and also writes it
            # into the static input the graph's first residual add reads: one
            # launch instead of a copy plus the LayerNorm inside the graph.
            ln, static_y = entry.first_ln
            d = x.shape[-1]
            _C.layernorm_residual(x.reshape(-1, d), ln.weight, ln.bias, y=static_y,
                                  x_out=entry.static_x.view(-1, d), eps=ln.eps)
        else:
            entry.static_x.copy_(x)
        if mask is not None:
            entry.static_mask.copy_(mask)
        entry.graph.replay()

    def resolve_policy(self, seq_len: int, dtype: torch.dtype,
                       device: Optional[torch.device] = None) -> Tuple[str, str]:
        """``(softmax, precision)`` of a forward over sequences of ``seq_len``.

        Rule for ``"auto"``: a 16-bit model mirrors the eager chain bit for bit
        (``("eager", "eager")``) wherever the eager-exact attention reproduces
        the eager softmax at that length (``_C.eager_softmax_supported``:
        every length up to 1024; above, ATen's block softmax for lengths that
        are multiples of 4 up to 65536 that it reads as whole vectors -- the
        eager chain itself would hold ``seq_len^2`` scores per head, 137 GB
        at 65536 and one batch of 16 heads).  Other lengths have no eager
        result the kernels can mirror; they take the one-pass online softmax
        and the fp32 residual stream (``("online", "fp32_residual")``), whose
        output is compared against an fp32 evaluation instead.  fp32 models
        always run the reference's fp32 policy (fp16 operands, fp32
        residual), whatever these say.
        """
        softmax, precision = self.softmax, self.precision
        if softmax not in ("auto", "eager", "online"):
            raise ValueError(f"unknown softmax policy {softmax!r}")
        if precision not in ("auto", "eager", "fp32_residual"):
            raise ValueError(f"unknown precision policy {precision!r}")
        if dtype == torch.float32:
            return ("online", "fp32_model")
        mirror = _C.eager_softmax_supported(seq_len, device)
        if softmax == "auto":
            softmax = "eager" if mirror else "online"
        if precision == "auto":
            precision = "eager" if mirror else "fp32_residual"
        return (softmax, precision)

    def _graph_fits(self, x: torch.Tensor) -> bool:
        key = (tuple(x.shape), x.dtype, x.device)
        fits = self._fits_cache.get(key)
        if fits is None:
            b, s, d = x.shape
            es = x.element_size()
            m = b * s
            est = es * (m * d * 6 + m * self.config.ffn_dim + b * d * _C.vt_ld(s))
            total = torch.cuda.get_device_properties(x.device).total_memory
            fits = self._fits_cache[key] = est <= _GRAPH_MEMORY_FRACTION * total
        return fits

    def _capture(self, x: torch.Tensor, mask: Optional[torch.Tensor], policy) -> _GraphEntry:
        if self._graph_pool is None:
            self._graph_pool = torch.cuda.graph_pool_handle()
        static_x = x.clone()
        static_mask = mask.clone() if mask is not None else None
        first_ln = None
        if policy[1] == "eager" and x.dtype != torch.float32:
            d = x.shape[-1]
            first_ln = (self.layers[0].norm1, torch.empty((x.numel() // d, d), dtype=x.dtype, device=x.device))
        y0 = first_ln[1] if first_ln is not None else None
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            if first_ln is not None:
                ln = first_ln[0]
                _C.layernorm_residual(static_x.view(-1, static_x.shape[-1]), ln.weight, ln.bias, y=y0, eps=ln.eps)
            self._forward_layers(static_x, static_mask, policy, y0=y0)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._graph_pool):
            static_out = self._forward_layers(static_x, static_mask, policy, y0=y0)
        return _GraphEntry(graph, static_x, static_mask, static_out,
                           tuple(t.detach() for t in self._params_cache or self.parameters()), first_ln)

    def _forward_core(self, x: torch.Tensor, mask: Optional[torch.Tensor], policy=None) -> torch.Tensor:
        """The whole launch sequence: the layers, then the final LayerNorm."""
        if policy is None:
            policy = self.resolve_policy(x.shape[1], x.dtype, x.device)
        return self._final_ln(self._forward_layers(x, mask, policy), mask, x.shape, x.dtype)

    def _final_ln(self, cur: torch.Tensor, mask: Optional[torch.Tensor], shape, dtype) -> torch.Tensor:
        """Final LayerNorm of the residual stream ``cur`` [M, D] (TTB:4319-4320) into a new
        tensor of the model dtype; rows with mask 0 become 0.  Runs after the graph
        replay, so the caller's tensor is written directly (no copy out of the graph)."""
        b, s, d = shape
        rows = mask.reshape(b * s) if mask is not None else None
        out = torch.empty((b * s, d), dtype=dtype, device=cur.device)
        _C.layernorm_residual(cur, self.final_norm.weight, self.final_norm.bias, y=out,
                              eps=self.final_norm.eps, row_valid=rows,
                              flags=_C.LN_MASK_OUT if rows is not None else 0)
        return out.view(b, s, d)

    def _qkv_buffers(self, b: int, s: int, dtype: torch.dtype, dev) -> tuple:
        """Projection buffers of one forward: [M, 3D] for the strided layout,
        (qk [M, 2D], vt [B, H, hd, S']) for the packed one."""
        cfg = self.config
        d, h = cfg.d_model, cfg.num_heads
        if self._qkv_layout == "strided":
            return (torch.empty((b * s, 3 * d), dtype=dtype, device=dev),)
        return (torch.empty((b * s, 2 * d), dtype=dtype, device=dev),
                torch.empty((b, h, d // h, _C.vt_ld(s)), dtype=dtype, device=dev))

    def _qkv_attention(self, i: int, y: torch.Tensor, bufs: tuple, b: int, s: int,
                       mask: Optional[torch.Tensor], softmax: str, stats: Optional[torch.Tensor],
                       out: torch.Tensor) -> None:
        """Layer i's packed Q/K/V projection of y [M, D] and attention into out
        [M, D] (heads merged).  Packed layout (the default): the projection
        stores q, k in [M, 2D] and V head-transposed, read by
        tx_flash_attn_fwd.  Strided layout (the reference's call shape): one
        GEMM writes [M, 3D] = y W_qkv^T + b_qkv (TTB:4220-4222) and attention
        reads q / k / v as [B, H, S, hd] column views of it, as the
        reference's attention wrapper does (TTB:1596-1668)."""
        cfg = self.config
        h, d = cfg.num_heads, cfg.d_model
        hd = d // h
        m = b * s
        att = self.layers[i].attention
        w_qkv, b_qkv = self._packed_qkv[i]
        if self._qkv_layout == "strided":
            qkv = bufs[0]
            _C.gemm(y, w_qkv, b_qkv, out=qkv)
            q, k, v = (qkv[:, j * d:(j + 1) * d].view(b, s, h, hd).transpose(1, 2) for j in range(3))
            _C.flash_attn_strided(q, k, v, att.scale, cfg.causal, key_valid=mask,
                                  out=out.view(b, s, h, hd).transpose(1, 2), softmax=softmax,
                                  row_stats=stats)
        else:
            qk, vt = bufs
            _C.qkv_proj(y, w_qkv, b_qkv, b, s, h, qk=qk, vt=vt)
            _C.flash_attn(qk, vt, b, s, h, hd, att.scale, cfg.causal,
                          key_valid=mask.reshape(m) if mask is not None else None, out=out,
                          softmax=softmax, row_stats=stats)

    def _forward_layers(self, x: torch.Tensor, mask: Optional[torch.Tensor], policy,
                        y0: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The layers' launch sequence (capturable: no syncs, no host reads of device
        data); returns the final residual stream [M, D].  ``y0`` (16-bit eager policy
        only): layer 0's first LayerNorm output, already formed from ``x`` by the caller."""
        softmax, precision = policy
        if y0 is not None and (x.dtype == torch.float32 or precision != "eager"):
            raise ValueError("y0 applies to the 16-bit eager policy only")
        if x.dtype == torch.float32:
            return self._layers_fp32_model(x, mask)
        if precision == "fp32_residual":
            return self._layers_fp32_residual(x, mask, softmax)
        if precision != "eager":
            raise ValueError(f"unknown precision policy {precision!r}")
        cfg = self.config
        b, s, d = x.shape
        h, hd = cfg.num_heads, cfg.d_model // cfg.num_heads
        m = b * s
        dev, dt = x.device, x.dtype
        rows = mask.reshape(m) if mask is not None else None
        x_in = x.reshape(m, d)

        y = y0 if y0 is not None else torch.empty((m, d), dtype=dt, device=dev)
        qkv = self._qkv_buffers(b, s, dt, dev)
        hid = torch.empty((m, cfg.ffn_dim), dtype=dt, device=dev)
        xs = torch.empty((m, d), dtype=dt, device=dev)  # residual stream, updated in place
        stats = (torch.empty(2 * b * h * s, dtype=torch.float32, device=dev)
                 if softmax == "eager" else None)

        cur = x_in
        for i, layer in enumerate(self.layers):
            att = layer.attention
            if i > 0 or y0 is None:
                _C.layernorm_residual(cur, layer.norm1.weight, layer.norm1.bias, y=y, eps=layer.norm1.eps)
            o = y  # LN1 output is consumed; reuse its buffer for the attention output
            self._qkv_attention(i, y, qkv, b, s, mask, softmax, stats, out=o)
            _C.gemm(o, att.out_proj.weight, att.out_proj.bias, residual=cur, out=xs,
                    row_valid=rows, mask_delta=rows is not None)
            cur = xs
            _C.layernorm_residual(cur, layer.norm2.weight, layer.norm2.bias, y=y, eps=layer.norm2.eps)
            _C.gemm(y, layer.ffn_in.weight, layer.ffn_in.bias, out=hid, gelu=True)
            _C.gemm(hid, layer.ffn_out.weight, layer.ffn_out.bias, residual=cur, out=xs,
                    row_valid=rows, mask_out=rows is not None)
        return cur

    def _layers_fp32_residual(self, x: torch.Tensor, mask: Optional[torch.Tensor], softmax: str) -> torch.Tensor:
        """fp32 residual stream; hi/lo operands for the FFN GEMMs.

        LN1 -> y (model dtype) -> QKV -> attention -> out_proj adds
        acc + b to the fp32 residual without rounding; LN2 writes y2 as a
        [M, 2D] hi/lo pair; FFN-in takes it against [W1, W1], applies GELU to
        the fp32 value and stores a [M, 2F] hi/lo pair; FFN-out adds
        [W2, W2] x that pair to the fp32 residual; the final LayerNorm reads
        the fp32 residual.
        """
        cfg = self.config
        b, s, d = x.shape
        h, hd, f = cfg.num_heads, cfg.d_model // cfg.num_heads, cfg.ffn_dim
        m = b * s
        dev, dt = x.device, x.dtype
        rows = mask.reshape(m) if mask is not None else None
        x_in = x.reshape(m, d)
        y = torch.empty((m, d), dtype=dt, device=dev)
        y2 = torch.empty((m, 2 * d), dtype=dt, device=dev)
        qkv = self._qkv_buffers(b, s, dt, dev)
        hid = torch.empty((m, 2 * f), dtype=dt, device=dev)
        xs = torch.empty((m, d), dtype=torch.float32, device=dev)
        stats = (torch.empty(2 * b * h * s, dtype=torch.float32, device=dev)
                 if softmax == "eager" else None)
        cur = x_in
        for i, layer in enumerate(self.layers):
            att = layer.attention
            _C.layernorm_residual(cur, layer.norm1.weight, layer.norm1.bias, y=y, eps=layer.norm1.eps)
            self._qkv_attention(i, y, qkv, b, s, mask, softmax, stats, out=y)
            _C.gemm(y, att.out_proj.weight, att.out_proj.bias, residual=cur, out=xs,
                    row_valid=rows, mask_delta=rows is not None)
            cur = xs
            _C.layernorm_residual(cur, layer.norm2.weight, layer.norm2.bias, y=y2, y_dtype=dt,
                                  eps=layer.norm2.eps, split=True)
            w1d, w2d = self._ffn_dup(i)
            _C.gemm(y2, w1d, layer.ffn_in.bias, out=hid, gelu=True, split_out=True)
            _C.gemm(hid, w2d, layer.ffn_out.bias, residual=cur, out=xs,
                    row_valid=rows, mask_out=rows is not None)
        return cur

    def _layers_fp32_model(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
        """fp32 model: fp32 residual / LayerNorm / output, fp16 GEMM operands.

        LN1 writes y in fp16 -> packed QKV (fp16 weights) -> attention on fp16
        (one-pass softmax in fp32) -> out_proj adds round16-operand GEMM +
        bias to the fp32 residual -> LN2 (fp16 y) -> FFN-in + GELU (fp16 h)
        -> FFN-out adds into the fp32 residual -> final LN in fp32.
        """
        cfg = self.config
        b, s, d = x.shape
        h, hd = cfg.num_heads, cfg.d_model // cfg.num_heads
        m = b * s
        dev = x.device
        f16 = torch.float16
        rows = mask.reshape(m) if mask is not None else None
        y = torch.empty((m, d), dtype=f16, device=dev)
        qkv = self._qkv_buffers(b, s, f16, dev)
        hid = torch.empty((m, cfg.ffn_dim), dtype=f16, device=dev)
        xs = torch.empty((m, d), dtype=torch.float32, device=dev)
        cur = x.reshape(m, d)
        for i, layer in enumerate(self.layers):
            att = layer.attention
            w16 = self._half[i]
            _C.layernorm_residual(cur, layer.norm1.weight, layer.norm1.bias, y=y, y_dtype=f16,
                                  eps=layer.norm1.eps)
            self._qkv_attention(i, y, qkv, b, s, mask, "online", None, out=y)
            _C.gemm(y, *w16["out_proj"], residual=cur, out=xs, row_valid=rows,
                    mask_delta=rows is not None)
            cur = xs
            _C.layernorm_residual(cur, layer.norm2.weight, layer.norm2.bias, y=y, y_dtype=f16,
                                  eps=layer.norm2.eps)
            _C.gemm(y, *w16["ffn_in"], out=hid, gelu=True)
            _C.gemm(hid, *w16["ffn_out"], residual=cur, out=xs, row_valid=rows,
                    mask_out=rows is not None)
        return cur
