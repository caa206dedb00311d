"""Weight folds the vLLM plugin's draft step applies once, when the drafter is prepared
(the public names and signatures of the reference's flashmap/vllm/fold.py, which the
plugin's ``prepare`` imports; pure torch, nothing here runs per step).

Noise. A draft of one jump starts from Gaussian noise over the vocabulary and reads it
through one path only: the embedding ``E (V, H)``, then the noise norm, then ``x_embed``.
The embedded noise is Gaussian with covariance ``E^T E``. Writing that covariance's
eigendecomposition as ``Q diag(lambda) Q^T`` and ``A = diag(sqrt(lambda)) Q^T``, the same
distribution comes from ``z @ A`` with ``z`` standard normal of width ``H`` instead of
``V``. Because the rows of ``A`` are orthogonal (``A A^T = diag(lambda)``), the norm's mean
square of ``z @ A`` is ``sum_i lambda_i z_i^2 / H``, so only a per-row scale is left to
compute at run time, and the noise norm's weights ``w`` and ``x_embed``'s weight ``W_x``
multiply with ``A`` into one ``(D, H)`` matrix ``M = W_x diag(w) A^T``
(flashmap/vllm/fold.py:45-75): ``x_embed(noise_norm(z @ A)) = (z @ M^T) / rms + b``.

Head. The DiT's output projection ``(D -> H, with bias)`` feeds the target's LM head
``(H -> V)`` directly; as both are linear, their product ``lm_head @ W_head`` and the
projected bias ``lm_head @ b_head`` replace the pair with one ``(V, D)`` GEMM
(flashmap/vllm/fold.py:78-100).

At run time the folded noise is ``ops.noise_rows`` (the row scales) + one GEMM +
``ops.adaln_residual`` with a per-row gate (``flashmap_amd.draft_step``), and the folded
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
    """The DiT head and the LM head as one linear map over the vocabulary rows ``rows``
    (every row when None): weight ``lm_head[rows] @ W_head`` ``(len(rows), D)`` and bias
    ``lm_head[rows] @ b_head``, multiplied in float32 and stored in the LM head's dtype,
    ``chunk`` rows at a time so the float32 copies stay small."""
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
