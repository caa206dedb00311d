"""Load-time folds of the one-jump draft step, with the API of the reference's
flashmap/vllm/fold.py (pure torch: computed once when the drafter is prepared, off the
per-step path).

- ``fold_noise``: a one-jump draft reads its starting noise ``x0 ~ N(0, I_V)`` only as
  ``x_embed(noise_norm(x0 @ E))``. ``x0 @ E`` is Gaussian with covariance ``E^T E = Q
  Lambda Q^T``, so it is drawn as ``z @ A``, ``z ~ N(0, I_H)``, ``A = sqrt(Lambda) Q^T``;
  then ``A A^T = Lambda`` makes the norm's mean square ``(z^2 @ lambda) / H``, and the
  norm weight ``w`` and ``x_embed``'s weight fold into one matrix:
  ``x_embed(noise_norm(z @ A)) = rsqrt(z^2 @ lambda / H + eps) * (z @ M^T) + b`` with
  ``M = W_x diag(w) A^T`` (flashmap/vllm/fold.py:1-15, 45-75).
- ``fold_head``: the DiT's output head (``D -> H`` with bias) followed by the target's
  LM head (``H -> V``, no nonlinearity between) as one ``(V, D)`` weight and bias
  (flashmap/vllm/fold.py:78-100).

The per-step use of the folded noise is ``ops.noise_rows`` + one GEMM +
``ops.adaln_residual`` with a per-row gate (see ``flashmap_amd.draft_step``); the folded
head is one GEMM followed by ``split_argmax`` (the gfx950 argmax kernel).
"""

from __future__ import annotations

import math

import torch

from .vllm import split_argmax

__all__ = ["fold_head", "fold_noise", "noise_factor", "quantize_fp8_per_channel", "split_argmax",
           "timestep_embedding"]


def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0) -> torch.Tensor:
    """``[cos(t f) | sin(t f)]`` float32 with ``f_i = max_period^(-i / (dim / 2))``
    (flashmap/vllm/fold.py:31-40; the expression order of the reference, so the values
    agree bit for bit on the same device)."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    angles = t.float()[..., None] * freqs
    return torch.cat([torch.cos(angles), torch.sin(angles)], dim=-1)


def _gram(embedding: torch.Tensor, chunk: int) -> torch.Tensor:
    """``E^T E`` accumulated in float32 over ``chunk``-row slices of ``E``."""
    hidden = embedding.shape[1]
    gram = torch.zeros(hidden, hidden, device=embedding.device, dtype=torch.float32)
    for rows in embedding.split(chunk):
        rows = rows.float()
        gram += rows.T @ rows
    return gram


@torch.no_grad()
def noise_factor(embedding: torch.Tensor, chunk: int = 16384) -> tuple[torch.Tensor, torch.Tensor]:
    """``(A, lambda)`` float64 for ``embedding (V, H)``: ``E^T E = Q diag(lambda) Q^T``
    (eigenvalues clamped at 0) and ``A = diag(sqrt(lambda)) Q^T``, so that ``A^T A = E^T
    E`` and ``A A^T = diag(lambda)``."""
    eigvals, eigvecs = torch.linalg.eigh(_gram(embedding, chunk).double())
    eigvals = eigvals.clamp_min(0)
    return eigvals.sqrt()[:, None] * eigvecs.T, eigvals


@torch.no_grad()
def fold_noise(embedding: torch.Tensor, noise_norm_weight: torch.Tensor, x_embed_weight: torch.Tensor,
               chunk: int = 16384) -> tuple[torch.Tensor, torch.Tensor]:
    """``(M, lambda / H)``: ``M = W_x diag(w) A^T`` ``(D, H)`` in the embedding's dtype (the
    weight ``F.linear`` takes) and the eigenvalues over ``H`` ``(H,)`` float32."""
    factor, eigvals = noise_factor(embedding, chunk)
    scaled = factor * noise_norm_weight.double()[None, :]  # A diag(w)
    folded = x_embed_weight.double() @ scaled.T
    return folded.to(embedding.dtype), (eigvals / embedding.shape[1]).float()


@torch.no_grad()
def fold_head(lm_head: torch.Tensor, head_weight: torch.Tensor, head_bias: torch.Tensor,
              rows: torch.Tensor | None = None, chunk: int = 8192) -> tuple[torch.Tensor, torch.Tensor]:
    """``(lm_head[rows] @ W_head, lm_head[rows] @ b_head)``: one ``(len(rows), D)`` weight
    and bias in the LM head's dtype, products in float32, ``chunk`` vocabulary rows at a
    time (all rows when ``rows`` is None)."""
    count = lm_head.shape[0] if rows is None else rows.numel()
    weight = torch.empty(count, head_weight.shape[1], dtype=lm_head.dtype, device=lm_head.device)
    bias = torch.empty(count, dtype=lm_head.dtype, device=lm_head.device)
    hw, hb = head_weight.float(), head_bias.float()
    for start in range(0, count, chunk):
        stop = min(count, start + chunk)
        part = (lm_head[start:stop] if rows is None else lm_head[rows[start:stop]]).float()
        weight[start:stop] = (part @ hw).to(lm_head.dtype)
        bias[start:stop] = (part @ hb).to(lm_head.dtype)
    return weight, bias


@torch.no_grad()
def quantize_fp8_per_channel(weight: torch.Tensor, dtype: torch.dtype = torch.float8_e4m3fn):
    """``(w_q, scale)`` for an ``(N, K)`` weight: ``w_q (K, N)`` in ``dtype`` (a
    column-major view, the operand form of scaled-mm kernels) and ``scale (N, 1)``
    float32, one per output channel, with ``weight ~= w_q.T * scale``
    (flashmap/vllm/fold.py:103-114)."""
    top = torch.finfo(dtype).max
    w = weight.float()
    scale = w.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / top
    return (w / scale).clamp(-top, top).to(dtype).t(), scale.contiguous()
