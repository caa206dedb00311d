"""CPU restatement of the DiT residual stream around the drafter's attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The reference runs it as eager bf16
torch ops, each rounding its result to bf16:

  * AdaLN-zero norm: ``F.layer_norm(x, (dim,), eps) * (1 + scale) + shift``
    (flashmap/modeling_flashmap.py:114-117), LayerNorm without affine weights;
  * gated residual: ``x + gate * y`` (flashmap/modeling_flashmap.py:185-192).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def adaln_residual(x, y, gate, scale, shift, eps):
    """``(x', h)`` with ``x' = x + gate * y`` (``x`` when ``y`` is None) and ``h =
    LN(x') * (1 + scale) + shift`` (None when ``scale`` is None), in ``x``'s dtype with
    the reference's per-op rounding. ``gate``, ``scale``, ``shift`` broadcast over the
    rows. Pinned by: float64 brute force within the bf16 rounding points, ``gate = 0``
    gives ``x`` exactly, ``scale = shift = 0`` gives rows of mean 0 and variance 1
    (tests/test_oracle_dit.py)."""
    xn = x if y is None else x + gate * y
    if scale is None:
        return xn, None
    return xn, F.layer_norm(xn, xn.shape[-1:], eps=eps) * (1 + scale) + shift
