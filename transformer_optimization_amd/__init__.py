"""MI355X (gfx950) transformer-block forward.

Drop-in for the reference's ``UserOptimizedTransformer``: same constructor,
``state_dict`` keys and ``forward(x, valid_token_mask=None)``; the hot path is
hand-written HIP (``csrc/``) behind the C ABI declared in ``include/tx_api.h``.
``import torch`` happens first so that ``libtx_hip.so`` binds to the HIP
runtime torch has mapped.
"""

import torch  # noqa: F401  (must precede loading libtx_hip.so)

from .config import TransformerConfig
from .model import UserOptimizedTransformer, TransformerParams
from .flops import count_dense_flops, compute_mfu
from . import _C, workloads

__all__ = [
    "TransformerConfig",
    "UserOptimizedTransformer",
    "TransformerParams",
    "count_dense_flops",
    "compute_mfu",
    "_C",
    "workloads",
]
