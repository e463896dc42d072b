"""CPU restatement of the reference's eager transformer-block forward.

TEST INFRASTRUCTURE ONLY.  Nothing in ``transformer_optimization_amd`` imports
this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, in ``bench.py``, as the timed CPU baseline) -- never as a product path.

Contents (each function cites the reference file:line it restates;
``TTB`` = ``torch_transformer_benchmark.py`` of namsengi11/transformer_optimization):

* ``model``   -- ``TransformerConfig``, ``BaselineSelfAttention``,
  ``BaselineTransformerBlock``, ``BaselineTransformer``, ``copy_model_weights``
  (TTB:43-70, 135-248, 4328-4338).
* ``gate``    -- ``AccuracyResult`` / ``compare_outputs`` (TTB:4534-4615).
* ``chunked`` -- query-row-subset fp32 reference of the whole stack for
  sequences too long for dense scores (TTB:341-421 pattern).

How each part is pinned (none of these re-types the formula under test):

* the block stack equals ``torch.nn.TransformerEncoderLayer(norm_first=True,
  activation="gelu")`` followed by ``nn.LayerNorm`` in float64, with and
  without causal / key-padding masks (``tests/test_oracle.py``);
* attention equals ``F.scaled_dot_product_attention`` in float64;
* closed forms: constant rows -> LayerNorm bias, identical keys -> mean of V,
  causal row 0 -> v0, padded rows exactly 0, causality under perturbation,
  batch-permutation equivariance;
* the gate by a truth table (NaN fails, boundary equality passes, the OR of
  the absolute and relative branches, not ``isclose``);
* the chunked reference equals the dense oracle on shapes where both run.

No reference golden vectors exist (the reference commits none); the fixtures
under ``tests/golden/`` are produced by ``tests/golden/make_golden.py`` from
this oracle and serve as regression anchors.
"""

from .model import (  # noqa: F401
    TransformerConfig,
    BaselineSelfAttention,
    BaselineTransformerBlock,
    BaselineTransformer,
    copy_model_weights,
)
from .gate import AccuracyResult, compare_outputs  # noqa: F401
from .chunked import chunked_reference_rows  # noqa: F401
