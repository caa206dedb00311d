"""Drop-in FlashMap drafter for the transformers path, on the gfx950 kernels.

Public names, parameter names and signatures are the reference's
(flashmap/modeling_flashmap.py), so a reference checkpoint (``config.json`` plus
safetensors, or a live model's ``state_dict()``) loads unchanged and a caller written
against ``FlashMapAttention.forward(x, rope, keys, values)`` / ``project_kv(x, rope)``,
``FlashMapLayer``, ``FlashMapCache``, ``draft`` or ``spec_generate`` keeps working.

How it runs on the GPU (bf16 models only; every kernel call fails loudly off the GPU):

- ``FlashMapAttention.forward``: the query's QK-RMSNorm + RoPE applied inside the
  split-KV block attention over the cache's strided views (``fm_block_attn_contig``);
- self-attention across a block's slots: one projection GEMM over the concatenated
  q/k/v weights and one fused norm + RoPE + 16 x 16 attention launch
  (``fm_block_self_attention``);
- the residual stream: each sublayer's gated residual and the next sublayer's
  time-modulated LayerNorm in one pass (``fm_adaln_residual``), so a layer makes three
  such launches instead of the eager chain of about twenty-four;
- the context's keys and values of every layer: one GEMM over all layers' concatenated
  k/v weights and one launch of the context writer (``fm_write_context_kv``, k-norm +
  RoPE + store) into the cache's ``(layers, 2, B, heads, positions, head_dim)`` tensor,
  addressed as a paged cache with one page per sequence.

Time embeddings, the state featurization, the output head and the speculative-decoding
loop are torch, as in the reference.
"""

from __future__ import annotations

import json
import math
import os
import warnings
from contextlib import contextmanager
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import ops

__all__ = [
    "FlashMapAdaLayerNorm",
    "FlashMapAttention",
    "FlashMapCache",
    "FlashMapDraftModel",
    "FlashMapGenerateOutput",
    "FlashMapLayer",
    "FlashMapMLP",
    "FlashMapRMSNorm",
    "FlashMapTimeEmbedding",
    "drafter_config",
    "jump_times",
    "rope_tables",
]

# Defaults of the reference's FlashMapConfig (flashmap/configuration_flashmap.py:88-112).
_JUMP_GRIDS = {
    "1": [0.0, 1.0],
    "2": [0.0, 0.8172569274902344, 1.0],
    "3": [0.0, 0.8010796308517456, 0.8310279846191406, 1.0],
    "4": [0.0, 0.7906050682067871, 0.8172569274902344, 0.8379518389701843, 1.0],
}
_DEFAULTS = dict(
    target_model="Qwen/Qwen3-8B", target_hidden_size=4096, vocab_size=151936, state_vocab_size=None,
    target_layer_ids=[1, 9, 17, 25, 33], block_size=16, hidden_size=2048, num_hidden_layers=6,
    num_attention_heads=16, intermediate_size=8192, mlp_type="gelu", cond_dim=256, time_embed_dim=256,
    time_scale=1000.0, rope_theta=10000.0, rms_norm_eps=1e-6, qk_norm_eps=1e-5, layer_norm_eps=1e-6,
    noise_gate="jump", time_schedule="decoding_error", num_steps=1, jump_grids=None,
)
# Target layer kinds whose state a rejected draft can be cropped from.
_CROPPABLE = frozenset({"full_attention", "sliding_attention", "chunked_attention"})


def drafter_config(config=None, **overrides) -> SimpleNamespace:
    """A drafter configuration from a reference ``FlashMapConfig``, a ``config.json``
    dict or keyword arguments (missing fields take the reference's defaults)."""
    if isinstance(config, SimpleNamespace) and not overrides:
        return config
    if config is None:
        given = {}
    elif isinstance(config, dict):
        given = dict(config)
    else:
        given = {k: getattr(config, k) for k in _DEFAULTS if hasattr(config, k)}
    cfg = dict(_DEFAULTS)
    cfg.update((k, v) for k, v in given.items() if k in _DEFAULTS)
    cfg.update(overrides)
    cfg["target_layer_ids"] = list(cfg["target_layer_ids"])
    cfg["jump_grids"] = dict(cfg["jump_grids"] or _JUMP_GRIDS)
    if cfg["mlp_type"] not in ("gelu", "swiglu"):
        raise ValueError(f"mlp_type must be gelu or swiglu, got {cfg['mlp_type']!r}")
    return SimpleNamespace(**cfg)


def jump_times(grid) -> list:
    """``(s, t, next)`` per jump over ``grid``: the network jumps from ``s`` to ``t``
    and the state then moves to ``next``; each jump lands where the next starts, so
    ``t == next`` (flashmap/configuration_flashmap.py:23-31)."""
    times = [float(v) for v in grid]
    return [(a, b, b) for a, b in zip(times, times[1:])]


# ---------------------------------------------------------------------------- rotary


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """``cos`` and ``sin`` ``(B, T, 1, head_dim / 2)`` float32 of the rotary angles at
    ``positions (B, T)``, with the torch expression of flashmap/modeling_flashmap.py:53-58
    (so the values are the reference's bit for bit on the same device)."""
    inv_freq = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=positions.device).float() / head_dim)
    angles = positions.float()[..., None, None] * inv_freq
    return angles.cos(), angles.sin()


def _token_rope(rope, batch: int, length: int) -> ops.Rope:
    """The kernels' rotary descriptor with one row per token (``b * length + t``) from
    the reference's ``(cos, sin)`` pair (any shape broadcasting to ``(B, T, 1, D/2)``),
    or an ``ops.Rope`` already in that form."""
    if isinstance(rope, ops.Rope):
        return rope
    cos, sin = rope
    half = cos.shape[-1]
    rows = [torch.broadcast_to(c, (batch, length, 1, half)).reshape(batch * length, half) for c in (cos, sin)]
    return ops.rope_from_split(*rows)


class _Joined:
    """Parameters concatenated along dim 0 (fused projection weights, stacked norm
    weights), rebuilt whenever one of them is replaced, moved or changed in place."""

    def __init__(self):
        self._key, self._value = None, None

    def __call__(self, params, dtype=None) -> torch.Tensor:
        key = tuple((p.data_ptr(), p._version, tuple(p.shape), p.dtype, p.device) for p in params) + (dtype,)
        if key != self._key:
            self._value = None  # release the old copy first
            joined = torch.cat([p.detach().reshape(-1, *p.shape[1:]) for p in params])
            self._value = joined if dtype is None else joined.to(dtype)
            self._key = key
        return self._value


# --------------------------------------------------------------------------- modules


class FlashMapRMSNorm(nn.Module):
    """RMSNorm whose scale ``weight / rms(x)`` is rounded to ``x``'s dtype before the
    multiply (flashmap/modeling_flashmap.py:69-80). As the q/k norm of an attention its
    weight feeds the kernels; as a hidden-state norm it runs in torch."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        inv_rms = torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return x * (self.weight.float() * inv_rms).to(x.dtype)


def _time_features(t: torch.Tensor, dim: int, scale: float) -> torch.Tensor:
    """``[cos(a) | sin(a)]`` with ``a = scale * t * 10000^(-i / (dim / 2))``: the
    sinusoidal features of flashmap/modeling_flashmap.py:94-98, in float32."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device).float() / half)
    angles = (t.float() * scale)[..., None] * freqs
    return torch.cat([angles.cos(), angles.sin()], dim=-1)


class FlashMapTimeEmbedding(nn.Module):
    """A time in [0, 1] -> sinusoidal features -> two-layer SiLU MLP
    (flashmap/modeling_flashmap.py:83-99)."""

    def __init__(self, config):
        super().__init__()
        self.dim, self.scale = config.time_embed_dim, config.time_scale
        self.linear_1 = nn.Linear(config.time_embed_dim, config.cond_dim)
        self.linear_2 = nn.Linear(config.cond_dim, config.cond_dim)

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        feats = _time_features(t, self.dim, self.scale).to(self.linear_1.weight.dtype)
        return self.linear_2(F.silu(self.linear_1(feats)))


class FlashMapAdaLayerNorm(nn.Module):
    """AdaLN-zero: a LayerNorm without affine weights modulated by ``(scale, shift)`` and
    a residual ``gate``, the three from one linear map of ``silu(cond)``
    (flashmap/modeling_flashmap.py:102-117). ``forward`` is one ``fm_adaln_residual``
    launch; the layers call that kernel with the preceding residual fused in."""

    def __init__(self, config):
        super().__init__()
        self.linear = nn.Linear(config.cond_dim, 3 * config.hidden_size)
        self.eps = config.layer_norm_eps

    def modulation(self, cond: torch.Tensor):
        """``(scale, shift, gate)`` of the conditioning ``cond``."""
        return self.linear(F.silu(cond)).chunk(3, dim=-1)

    def forward(self, x: torch.Tensor, modulation):
        scale, shift, gate = modulation
        return ops.adaln_residual(x, None, None, (scale, shift), self.eps)[1], gate


class FlashMapAttention(nn.Module):
    """Attention with RMS-normed queries and keys and interleaved rotary positions
    (flashmap/modeling_flashmap.py:118-147), on the kernels. ``rope`` is the reference's
    ``(cos, sin)`` pair from :func:`rope_tables` or an ``ops.Rope`` with one row per token.

    - ``project_kv(x, rope)``: keys (normed, rotated) and values ``(B, heads, T,
      head_dim)`` of ``x (B, T, dim)`` -- views of ``(B, T, heads, head_dim)`` rows, as
      the reference returns them;
    - ``forward(x, rope, keys, values)``: ``o_proj`` of the attention of ``x``'s queries
      onto ``keys``/``values (B, heads, L, head_dim)`` (any strides with unit channel
      stride), the query prologue inside the attention kernel;
    - ``attend_block(x, rope)``: ``forward(x, rope, *project_kv(x, rope))`` for blocks of
      at most 16 tokens as one fused launch.
    """

    def __init__(self, config):
        super().__init__()
        dim = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.head_dim = dim // self.num_heads
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.k_proj = nn.Linear(dim, dim, bias=False)
        self.v_proj = nn.Linear(dim, dim, bias=False)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self.q_norm = FlashMapRMSNorm(self.head_dim, config.qk_norm_eps)
        self.k_norm = FlashMapRMSNorm(self.head_dim, config.qk_norm_eps)
        self._qkv = _Joined()

    def _split_heads(self, y: torch.Tensor) -> torch.Tensor:
        return y.view(y.shape[0], y.shape[1], self.num_heads, self.head_dim)

    def project_kv(self, x: torch.Tensor, rope):
        b, t, _ = x.shape
        k = self.k_proj(x).view(b * t, self.num_heads, self.head_dim)
        keys = ops.rms_norm_rope(k, self.k_norm.weight, _token_rope(rope, b, t), None, self.k_norm.eps)
        values = self._split_heads(self.v_proj(x))
        return keys.view(b, t, self.num_heads, self.head_dim).transpose(1, 2), values.transpose(1, 2)

    def forward(self, x: torch.Tensor, rope, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        b, t, _ = x.shape
        queries = self._split_heads(self.q_proj(x))
        prologue = ops.Prologue(self.q_norm.weight, _token_rope(rope, b, t), None, self.q_norm.eps)
        out = ops.block_attention_contig(queries, keys, values, prologue=prologue)
        return self.o_proj(out.view(b, t, -1))

    def attend_block(self, x: torch.Tensor, rope) -> torch.Tensor:
        b, t, _ = x.shape
        if t > 16:
            return self(x, rope, *self.project_kv(x, rope))
        if self.q_norm.eps != self.k_norm.eps:
            raise ValueError("the fused block attention takes one eps for the q and k norms")
        qkv = F.linear(x, self._qkv((self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)))
        qkv = qkv.view(b, t, 3, self.num_heads, self.head_dim)
        out = ops.block_self_attention(qkv, self.q_norm.weight, self.k_norm.weight, _token_rope(rope, b, t), None,
                                       self.q_norm.eps)
        return self.o_proj(out.view(b, t, -1))


class FlashMapMLP(nn.Module):
    """``fc2(gelu(fc1(x)))`` for "gelu"; ``down_proj(silu(gate) * up)`` with ``gate, up``
    the halves of ``gate_up_proj(x)`` for "swiglu" (flashmap/modeling_flashmap.py:150-170)."""

    def __init__(self, config):
        super().__init__()
        self.mlp_type = getattr(config, "mlp_type", "gelu")
        dim, hidden = config.hidden_size, config.intermediate_size
        if self.mlp_type == "swiglu":
            self.gate_up_proj = nn.Linear(dim, 2 * hidden, bias=False)
            self.down_proj = nn.Linear(hidden, dim, bias=False)
        else:
            self.fc1 = nn.Linear(dim, hidden)
            self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.mlp_type != "swiglu":
            return self.fc2(F.gelu(self.fc1(x)))
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class FlashMapLayer(nn.Module):
    """A DiT block (flashmap/modeling_flashmap.py:173-192): self-attention across the
    block's slots, cross-attention to the context and an MLP, each behind a modulated
    LayerNorm and a gated residual. ``run`` threads the residual stream through
    ``fm_adaln_residual``: each sublayer's residual is fused with the next norm,
    the last one with the norm that follows the layer (``next_norm``)."""

    def __init__(self, config):
        super().__init__()
        self.self_attn_adaln = FlashMapAdaLayerNorm(config)
        self.self_attn = FlashMapAttention(config)
        self.cross_attn_adaln = FlashMapAdaLayerNorm(config)
        self.cross_attn = FlashMapAttention(config)
        self.mlp_adaln = FlashMapAdaLayerNorm(config)
        self.mlp = FlashMapMLP(config)

    def run(self, x, h, modulations, rope: ops.Rope, context, next_norm=None, x_out=None):
        """``x`` the residual stream and ``h`` its self-attention norm (already
        modulated); returns the stream after the layer and, for ``next_norm = (scale,
        shift, eps)``, its next norm (else None). ``x_out`` (may be ``x``) receives
        the stream."""
        (_, _, self_gate), (c_scale, c_shift, cross_gate), (m_scale, m_shift, mlp_gate) = modulations
        y = self.self_attn.attend_block(h, rope)
        x, h = ops.adaln_residual(x, y, self_gate, (c_scale, c_shift), self.cross_attn_adaln.eps, x_out=x_out)
        y = self.cross_attn(h, rope, *context)
        x, h = ops.adaln_residual(x, y, cross_gate, (m_scale, m_shift), self.mlp_adaln.eps, x_out=x)
        y = self.mlp(h)
        follow = None if next_norm is None else tuple(next_norm[:2])
        return ops.adaln_residual(x, y, mlp_gate, follow, 0.0 if next_norm is None else next_norm[2], x_out=x)

    def forward(self, x, modulations, rope, context) -> torch.Tensor:
        rows = _token_rope(rope, x.shape[0], x.shape[1])
        scale, shift, _ = modulations[0]
        h = ops.adaln_residual(x, None, None, (scale, shift), self.self_attn_adaln.eps)[1]
        return self.run(x, h, modulations, rows, context)[0]


class FlashMapCache:
    """The context's cross-attention keys and values for every DiT layer
    (flashmap/modeling_flashmap.py:195-219): ``kv (layers, 2, B, heads, max_length,
    head_dim)``, positions ``[0, length)`` holding the target's features and position
    ``length`` the anchor of the block being drafted. The kernels read it through
    strides; the context writer addresses it as a paged cache whose page is a sequence
    (page size ``max_length``, page ``b``, value offset ``kv.stride(1)``)."""

    def __init__(self, config, batch_size: int, max_length: int, device=None, dtype=None):
        cfg = drafter_config(config)
        head_dim = cfg.hidden_size // cfg.num_attention_heads
        self.kv = torch.zeros((cfg.num_hidden_layers, 2, batch_size, cfg.num_attention_heads, max_length, head_dim),
                              device=device, dtype=dtype)
        self.length = 0
        self._layout = None
        self._rope = {}

    def write(self, layer: int, start: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Store ``keys``/``values (B, heads, n, head_dim)`` at positions ``start ..
        start + n`` of ``layer``."""
        stop, capacity = start + keys.shape[2], self.kv.shape[4]
        if stop > capacity:
            raise ValueError(f"this cache ends at position {capacity}; the write reaches {stop}")
        self.kv[layer, :, :, :, start:stop].copy_(torch.stack((keys, values)))

    def context(self, end: int) -> list:
        """Per layer, ``(keys, values)`` views of positions ``[0, end)``."""
        window = self.kv[..., :end, :]
        return list(zip(window[:, 0].unbind(0), window[:, 1].unbind(0)))

    def writer_layout(self):
        """``(per-layer base addresses (layers,) int64 on the device, (block, head,
        token, value) strides, page size)``: the cache as fm_write_context_kv addresses
        a paged cache, position ``p`` of sequence ``b`` at slot ``b * max_length + p``."""
        if self._layout is None or self._layout[0].device != self.kv.device:
            kv = self.kv
            if kv.stride(-1) != 1:
                raise ValueError("the cache needs unit channel stride")
            bases = torch.tensor([kv[i].data_ptr() for i in range(kv.shape[0])], dtype=torch.int64, device=kv.device)
            self._layout = (bases, (kv.stride(2), kv.stride(3), kv.stride(4), kv.stride(1)), kv.shape[4])
        return self._layout

    def rope_rows(self, head_dim: int, theta: float) -> ops.Rope:
        """Rotary rows of positions ``0 .. max_length - 1`` (built once per cache)."""
        key = (head_dim, float(theta))
        if key not in self._rope:
            cos, sin = rope_tables(torch.arange(self.kv.shape[4], device=self.kv.device)[None], head_dim, theta)
            self._rope[key] = ops.rope_from_split(cos.reshape(-1, head_dim // 2), sin.reshape(-1, head_dim // 2))
        return self._rope[key]


@dataclass
class FlashMapGenerateOutput:
    """What ``spec_generate`` returns (flashmap/modeling_flashmap.py:222-236):
    ``sequences (1, length)`` = prompt + generated tokens, ``num_new_tokens``, and per
    target pass the tokens it committed (``acceptance_lengths``; a final pass that
    overshoots ``max_new_tokens`` still counts whole)."""

    sequences: torch.LongTensor
    num_new_tokens: int
    acceptance_lengths: list = field(default_factory=list)

    @property
    def acceptance_length(self) -> float:
        """Mean tokens committed per target pass."""
        passes = self.acceptance_lengths
        return sum(passes) / len(passes) if passes else 0.0


class _FeatureTap:
    """Forward hooks on the target's decoder layers ``ids`` keeping each one's latest
    output; calling the tap concatenates them along the hidden dimension."""

    def __init__(self, layers, ids):
        self.ids = list(ids)
        self.latest = {}
        self.handles = [layers[i].register_forward_hook(self._keeper(i)) for i in self.ids]

    def _keeper(self, i):
        def keep(_module, _inputs, output):
            self.latest[i] = output[0] if isinstance(output, tuple) else output

        return keep

    def __call__(self) -> torch.Tensor:
        return torch.cat([self.latest[i] for i in self.ids], dim=-1)

    def close(self) -> None:
        while self.handles:
            self.handles.pop().remove()


class _Acceptance:
    """Token choice and the accept/reject rule of one lossless speculative decode
    (flashmap/modeling_flashmap.py:566-597): greedy at temperature 0, else sampling
    with rejection against the draft's per-slot distributions. The generator is drawn
    in the reference's order (draft sample, uniforms, bonus token)."""

    def __init__(self, temperature: float, generator):
        self.temperature, self.generator = temperature, generator
        self.greedy = temperature <= 0

    def pick(self, logits: torch.Tensor):
        """``(1, n, V)`` logits -> tokens ``(1, n)`` and their distributions (None when greedy)."""
        if self.greedy:
            return logits.argmax(dim=-1), None
        probs = (logits.float() / self.temperature).softmax(dim=-1)
        return torch.multinomial(probs[0], 1, generator=self.generator).T, probs

    def verify(self, proposal: torch.Tensor, proposal_probs, target_logits: torch.Tensor):
        """How many of the ``(1, block)`` proposed tokens the target keeps, and its own
        next token, from the target's ``(1, block + 1, V)`` logits."""
        if self.greedy:
            choice = target_logits.argmax(dim=-1)
            kept = int((proposal == choice[:, :-1]).cumprod(dim=1).sum())
            return kept, choice[:, kept]
        p_all = (target_logits.float() / self.temperature).softmax(dim=-1)[0]
        idx = proposal[0, :, None]
        p = p_all[:-1].gather(-1, idx)[:, 0]
        q = proposal_probs[0].gather(-1, idx)[:, 0]
        u = torch.rand(q.shape, device=q.device, generator=self.generator)
        kept = int((u * q < p).cumprod(dim=0).sum())
        dist = p_all[kept]
        if kept < proposal.shape[1]:  # the rejected slot draws from max(p - q, 0)
            leftover = (dist - proposal_probs[0, kept]).clamp_min(0)
            if leftover.sum() > 0:
                dist = leftover
        return kept, torch.multinomial(dist, 1, generator=self.generator)


def _cut_at_stop(tokens: torch.Tensor, stops: torch.Tensor) -> torch.Tensor:
    hits = torch.isin(tokens[0], stops).nonzero()
    return tokens[:, : int(hits[0]) + 1] if len(hits) else tokens


class FlashMapDraftModel(nn.Module):
    """The FlashMap drafter (flashmap/modeling_flashmap.py:239-612) on the gfx950
    kernels. Build it with :meth:`from_pretrained` (a local checkpoint folder),
    :meth:`from_reference` (a live reference model) or from a config, then move it to
    the GPU in bfloat16."""

    def __init__(self, config=None, **overrides):
        super().__init__()
        cfg = self.config = drafter_config(config, **overrides)
        dim, target_dim = cfg.hidden_size, cfg.target_hidden_size
        self.head_dim = dim // cfg.num_attention_heads
        # context features: the target's hidden states at target_layer_ids, and the anchor
        self.fc = nn.Linear(len(cfg.target_layer_ids) * target_dim, dim, bias=False)
        self.hidden_norm = FlashMapRMSNorm(dim, cfg.rms_norm_eps)
        self.anchor_proj = nn.Linear(target_dim, dim)
        self.anchor_norm = FlashMapRMSNorm(dim, cfg.rms_norm_eps)
        # state featurization
        self.state_norm = FlashMapRMSNorm(target_dim, cfg.rms_norm_eps)
        self.noise_norm = FlashMapRMSNorm(target_dim, cfg.rms_norm_eps)
        self.noise_gate = nn.Parameter(torch.ones(1))
        # the DiT
        self.x_embed = nn.Linear(target_dim, dim)
        self.time_embed = FlashMapTimeEmbedding(cfg)
        self.jump_embed = FlashMapTimeEmbedding(cfg)
        self.layers = nn.ModuleList(FlashMapLayer(cfg) for _ in range(cfg.num_hidden_layers))
        self.final_adaln = FlashMapAdaLayerNorm(cfg)
        self.head = nn.Linear(dim, target_dim)
        if cfg.state_vocab_size is not None:
            self.register_buffer("draft_ids", torch.arange(cfg.state_vocab_size))
        self._kv_weight, self._k_norms = _Joined(), _Joined()
        self._derived = {}

    # -- construction ----------------------------------------------------------------

    @classmethod
    def from_pretrained(cls, path: str, device=None, dtype=torch.bfloat16) -> "FlashMapDraftModel":
        """A local checkpoint folder: ``config.json`` plus ``*.safetensors``."""
        from safetensors.torch import load_file

        with open(os.path.join(path, "config.json")) as f:
            model = cls(json.load(f))
        shards = sorted(n for n in os.listdir(path) if n.endswith(".safetensors"))
        state = {}
        for name in shards:
            state.update(load_file(os.path.join(path, name)))
        model.load_state_dict(state)
        return model.to(device=device, dtype=dtype)

    @classmethod
    def from_reference(cls, reference: nn.Module) -> "FlashMapDraftModel":
        """The same drafter as a live reference ``FlashMapDraftModel`` (weights copied),
        on its device and in its dtype."""
        model = cls(reference.config)
        model.load_state_dict(reference.state_dict())
        first = next(reference.parameters())
        return model.to(device=first.device, dtype=first.dtype)

    # Values derived from the weights (each jump's modulations, the state vocabulary's
    # rows, the target embedding's constants) are kept until the weights move or reload.

    def _apply(self, fn, *args, **kwargs):
        self._derived = {}
        return super()._apply(fn, *args, **kwargs)

    def load_state_dict(self, *args, **kwargs):
        self._derived = {}
        return super().load_state_dict(*args, **kwargs)

    @property
    def device(self) -> torch.device:
        return self.head.weight.device

    @property
    def dtype(self) -> torch.dtype:
        return self.head.weight.dtype

    # -- the network -----------------------------------------------------------------

    @torch.no_grad()
    def time_conditioning(self, s: float, t: float):
        """The AdaLN modulations of the jump ``s -> t``: per layer ``(self, cross,
        MLP)``, then the final norm's (flashmap/modeling_flashmap.py:287-300). They
        depend on the two times only and are computed once per jump."""
        table = self._derived.setdefault("time", {})
        if (s, t) not in table:
            times = torch.tensor([s, t], device=self.device)
            cond = (self.time_embed(times[:1]) + self.jump_embed(times[1:]))[None]
            per_layer = [
                tuple(norm.modulation(cond) for norm in (layer.self_attn_adaln, layer.cross_attn_adaln,
                                                          layer.mlp_adaln))
                for layer in self.layers
            ]
            table[(s, t)] = (per_layer, self.final_adaln.modulation(cond))
        return table[(s, t)]

    def forward(self, inputs_embeds, s: float, t: float, position_ids, context) -> torch.Tensor:
        """The jump ``s -> t`` of the featurized state ``inputs_embeds (B, K,
        target_hidden)`` of blocks at ``position_ids (B, K)`` -> hidden states ``(B, K,
        target_hidden)``, each layer attending to its ``context`` ``(keys, values)``
        (flashmap/modeling_flashmap.py:302-313). The residual stream runs through one
        fused kernel per sublayer boundary, in place."""
        per_layer, final = self.time_conditioning(s, t)
        b, k = position_ids.shape
        rope = _token_rope(rope_tables(position_ids, self.head_dim, self.config.rope_theta), b, k)
        x = self.x_embed(inputs_embeds)
        if not self.layers:
            return self.head(self.final_adaln(x, final)[0])
        scale, shift, _ = per_layer[0][0]
        h = ops.adaln_residual(x, None, None, (scale, shift), self.layers[0].self_attn_adaln.eps)[1]
        follow = [(m[0][0], m[0][1], layer.self_attn_adaln.eps) for m, layer in zip(per_layer[1:], self.layers[1:])]
        follow.append((final[0], final[1], self.final_adaln.eps))
        for layer, mods, ctx, nxt in zip(self.layers, per_layer, context, follow):
            x, h = layer.run(x, h, mods, rope, ctx, nxt, x_out=x)
        return self.head(h)

    # -- context ---------------------------------------------------------------------

    def select_target_hidden(self, hidden_states) -> torch.Tensor:
        """The drafter's features from a target forward's ``hidden_states`` tuple
        (outputs of layers ``target_layer_ids``; entry 0 is the embedding)."""
        return torch.cat([hidden_states[i + 1] for i in self.config.target_layer_ids], dim=-1)

    @contextmanager
    def target_features(self, target: nn.Module):
        """Hooks keeping the outputs of the target's layers ``target_layer_ids``; yields
        a callable concatenating them for the target's last forward
        (flashmap/modeling_flashmap.py:321-339)."""
        tap = _FeatureTap(target.get_decoder().layers, self.config.target_layer_ids)
        try:
            yield tap
        finally:
            tap.close()

    def _store_context(self, cache: FlashMapCache, start: int, context: torch.Tensor) -> None:
        """Every layer's keys and values of ``context (B, n, dim)`` at positions ``start
        ..``: one GEMM over the layers' concatenated k/v weights gives rows ``(tokens,
        layers, 2, heads, head_dim)``, one writer launch k-norms, rotates and stores them
        (flashmap/modeling_flashmap.py:139-142, 211-216 per layer in the reference)."""
        b, n, dim = context.shape
        if cache.kv.dtype != torch.bfloat16:
            raise TypeError(f"the context writer stores bfloat16 caches, got {cache.kv.dtype}")
        if start + n > cache.kv.shape[4]:
            raise ValueError(f"this cache ends at position {cache.kv.shape[4]}; the write reaches {start + n}")
        layers = self.layers
        weight = self._kv_weight([p for layer in layers for p in (layer.cross_attn.k_proj.weight,
                                                                   layer.cross_attn.v_proj.weight)])
        k_norms = self._k_norms([layer.cross_attn.k_norm.weight for layer in layers], torch.float32)
        rows = F.linear(context.reshape(b * n, dim), weight)
        bases, strides, page = cache.writer_layout()
        pos = torch.arange(start, start + n, device=context.device)
        slots = (torch.arange(b, device=context.device)[:, None] * page + pos).reshape(-1)
        heads = self.config.num_attention_heads
        eps = layers[0].cross_attn.k_norm.eps if len(layers) else 0.0
        ops.write_context_kv(rows.view(b * n, len(layers), 2, heads, self.head_dim), pos.repeat(b), slots, k_norms,
                             cache.rope_rows(self.head_dim, self.config.rope_theta), bases, strides, page, eps,
                             heads_per_cache=heads)

    @torch.no_grad()
    def extend_context(self, cache: FlashMapCache, target_hidden: torch.Tensor) -> None:
        """Append the target's features ``(B, n, ...)`` at the next ``n`` verified
        positions (flashmap/modeling_flashmap.py:342-351)."""
        context = self.hidden_norm(self.fc(target_hidden.to(self.dtype)))
        self._store_context(cache, cache.length, context)
        cache.length += target_hidden.shape[1]

    # -- state -----------------------------------------------------------------------

    @torch.no_grad()
    def state_vocab(self, embed_tokens: nn.Module, lm_head: nn.Module):
        """``(embedding, head weight, head bias)`` restricted to the state vocabulary
        (all rows without one; ``draft_ids``' rows, copied once, with one)."""
        embedding, weight, bias = embed_tokens.weight, lm_head.weight, getattr(lm_head, "bias", None)
        if self.config.state_vocab_size is None:
            return embedding, weight, bias
        key = (embedding.data_ptr(), weight.data_ptr(), embedding.device, embedding.dtype)
        held = self._derived.get("vocab")
        if held is None or held[0] != key:
            ids = self.draft_ids.to(embedding.device)
            held = (key, (embedding[ids], weight[ids], None if bias is None else bias[ids]))
            self._derived["vocab"] = held
        return held[1]

    def token_logits(self, logits: torch.Tensor) -> torch.Tensor:
        """State-vocabulary logits scattered over the target's vocabulary, ``-inf``
        elsewhere (unchanged without a state vocabulary)."""
        if self.config.state_vocab_size is None:
            return logits
        full = logits.new_full((*logits.shape[:-1], self.config.vocab_size), float("-inf"))
        full[..., self.draft_ids.to(logits.device)] = logits
        return full

    @torch.no_grad()
    def target_constants(self, embedding: torch.Tensor):
        """``(uniform posterior @ E, L)`` for the state vocabulary's embedding ``E (V,
        H)``, ``L L^T = E^T E`` (flashmap/modeling_flashmap.py:396-418): the Gram matrix
        in float32 over 16384-row slices, its Cholesky factor in float64 on the CPU."""
        key = (embedding.data_ptr(), tuple(embedding.shape), embedding.device, embedding.dtype)
        held = self._derived.get("target")
        if held is None or held[0] != key:
            slices = embedding.split(16384)
            gram = slices[0].float().T @ slices[0].float()
            for rows in slices[1:]:
                gram = gram + rows.float().T @ rows.float()
            factor = torch.linalg.cholesky(gram.cpu().double())
            uniform = torch.full((1, embedding.shape[0]), 1.0 / embedding.shape[0], device=embedding.device)
            held = (key, (uniform.to(embedding.dtype) @ embedding, factor.to(self.device, self.dtype)))
            self._derived["target"] = held
        return held[1]

    def mix_state(self, posterior_embeds, state_embeds, s: float, t: float) -> torch.Tensor:
        """The DiT input from the state's two projections onto the embedding: the
        normed posterior plus the gated normed linear term (flashmap/modeling_flashmap.py:388-394)."""
        jump = 1.0 if self.config.noise_gate == "constant" else t - s
        gate = (self.noise_gate.float() * jump).to(self.dtype)
        return self.state_norm(posterior_embeds.to(self.dtype)) + gate * self.noise_norm(state_embeds.to(self.dtype))

    def embed_state(self, state, s: float, t: float, embedding: torch.Tensor) -> torch.Tensor:
        """DiT input for a vocabulary-sized state ``(B, K, V)`` at ``s`` jumping to ``t``
        (flashmap/modeling_flashmap.py:370-386): its sharpened posterior and the state
        itself, both through the embedding."""
        if s == 0:
            posterior_embeds = self.target_constants(embedding)[0]
        else:
            sharpness = s / max(1.0 - s, 1e-3) ** 2
            posterior_embeds = (state.float() * sharpness).softmax(dim=-1).to(embedding.dtype) @ embedding
        return self.mix_state(posterior_embeds, state.to(embedding.dtype) @ embedding, s, t)

    # -- drafting --------------------------------------------------------------------

    def _jump_grid(self, steps: int) -> list:
        grids = self.config.jump_grids
        if str(steps) not in grids:
            known = ", ".join(sorted(grids, key=int))
            raise ValueError(f"no jump grid for num_steps={steps}; this drafter's config defines {known}")
        return grids[str(steps)]

    def _open_block(self, cache: FlashMapCache, anchor_ids: torch.Tensor, embed_tokens: nn.Module) -> torch.Tensor:
        """Store the anchor's embedding features at position ``cache.length`` and return
        the block's positions ``(B, block_size)`` after it."""
        at = cache.length
        feats = self.anchor_norm(self.anchor_proj(embed_tokens(anchor_ids[:, None]).to(self.dtype)))
        self._store_context(cache, at, feats)
        slots = torch.arange(self.config.block_size, device=anchor_ids.device)
        return (at + 1 + slots).expand(anchor_ids.shape[0], -1)

    def _start(self, noise, steps: int, batch: int, embedding: torch.Tensor, t1: float, generator):
        """``(state, inputs)`` before the first jump: the given or drawn noise as the
        state, or, for one jump without given noise, the DiT input directly from noise
        drawn in the embedding's span (``z @ L^T``, see ``target_constants``)."""
        shape = (batch, self.config.block_size)
        if noise is not None:
            return noise, None
        if steps == 1:
            uniform_embeds, factor = self.target_constants(embedding)
            z = torch.randn(shape + (factor.shape[0],), device=embedding.device, dtype=factor.dtype,
                            generator=generator)
            return None, self.mix_state(uniform_embeds, z @ factor.T, 0.0, t1)
        return torch.randn(shape + (embedding.shape[0],), device=embedding.device, generator=generator), None

    @torch.no_grad()
    def draft(self, anchor_ids, cache: FlashMapCache, embed_tokens, lm_head, num_steps: Optional[int] = None,
              noise: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """Draft logits ``(B, block_size, V)`` for the block after ``anchor_ids (B,)``
        (flashmap/modeling_flashmap.py:420-479). ``cache`` holds the target's features
        before the anchor; ``embed_tokens``/``lm_head`` are the target's; ``noise (B,
        block_size, S)`` is the starting state (drawn when None)."""
        steps = num_steps or self.config.num_steps
        grid = self._jump_grid(steps)
        embedding, head_weight, head_bias = self.state_vocab(embed_tokens, lm_head)
        positions = self._open_block(cache, anchor_ids, embed_tokens)
        context = cache.context(cache.length + 1)
        state, inputs = self._start(noise, steps, anchor_ids.shape[0], embedding, grid[1], generator)
        logits = None
        for s, t, nxt in jump_times(grid):
            if state is not None:
                inputs = self.embed_state(state, s, t, embedding)
            logits = F.linear(self(inputs, s, t, positions, context).to(head_weight.dtype), head_weight, head_bias)
            if nxt < 1.0:  # the state moves to the next grid time (eq. 19 of arXiv:2602.16813)
                state = ((1.0 - nxt) * state + (nxt - s) * logits.float().softmax(dim=-1)) / (1.0 - s)
        return self.token_logits(logits)

    # -- speculative decoding --------------------------------------------------------

    def check_target(self, target) -> None:
        """Raise unless ``target`` can serve this drafter: its vocabulary and hidden size,
        enough layers for ``target_layer_ids``, attention layers only (a rejected draft
        is undone by cropping the target's cache) and one device with the drafter; warn
        when it is not the model the drafter was trained for
        (flashmap/modeling_flashmap.py:483-512)."""
        cfg = self.config
        text = target.config.get_text_config() if hasattr(target.config, "get_text_config") else target.config
        embedding, lm_head = target.get_input_embeddings().weight, target.get_output_embeddings().weight
        want = (cfg.vocab_size, cfg.target_hidden_size)
        for what, w in (("input embedding", embedding), ("lm_head", lm_head)):
            if tuple(w.shape) != want:
                raise ValueError(f"the target's {what} is {tuple(w.shape)}; this drafter ({cfg.target_model}) "
                                 f"reads a vocabulary of {want[0]} at hidden size {want[1]}")
        deepest, layers = max(cfg.target_layer_ids), text.num_hidden_layers
        if deepest >= layers - 1:
            raise ValueError(f"the drafter reads target layer {deepest}; a target of {layers} layers has none "
                             f"past layer {layers - 2} to read")
        kinds = sorted({k for k in (getattr(text, "layer_types", None) or ()) if k not in _CROPPABLE})
        name = (getattr(text, "_name_or_path", None) or "").rstrip("/")
        if kinds:
            raise ValueError(f"{name or 'the target'} has {', '.join(kinds)} layers, whose state cannot be rolled "
                             "back after a rejected draft; spec_generate would not be lossless (serve it with "
                             "the vLLM or SGLang plugin)")
        if name and name.split("/")[-1] != cfg.target_model.split("/")[-1]:
            warnings.warn(f"{name} is not {cfg.target_model}, the target this drafter was trained for")
        devices = {self.device, embedding.device, lm_head.device}
        if len(devices) > 1:
            raise ValueError(f"the drafter, the target's embedding and its lm_head sit on {sorted(map(str, devices))}; "
                             "they must share one device")

    def _check_generator(self, generator) -> None:
        if generator is None:
            return
        dev = generator.device
        if dev.type == "cuda" and dev.index is None:  # an index-less "cuda" generator is the current device's
            dev = torch.device("cuda", torch.cuda.current_device())
        if (dev.type, dev.index or 0) != (self.device.type, self.device.index or 0):
            raise ValueError(f"the generator lives on {generator.device}; spec_generate draws on {self.device}")

    @torch.no_grad()
    def spec_generate(self, target, input_ids: torch.LongTensor, max_new_tokens: int = 256, temperature: float = 0.0,
                      num_steps: Optional[int] = None, stop_token_ids: Optional[list] = None,
                      generator: Optional[torch.Generator] = None) -> FlashMapGenerateOutput:
        """Lossless speculative decoding of a transformers causal LM ``target`` from the
        prompt ``input_ids (1, P)`` (flashmap/modeling_flashmap.py:514-612): every pass
        drafts a block after the last token, scores it with one target forward, and
        commits the accepted prefix plus one token of the target's own. Greedy at
        ``temperature`` 0 (the target's greedy decoding exactly), rejection sampling
        above it; stops after ``max_new_tokens`` or a token of ``stop_token_ids``
        (default: the target's ``eos_token_id``)."""
        from transformers import DynamicCache

        if input_ids.shape[0] != 1:
            raise ValueError(f"spec_generate takes one prompt, input_ids (1, P); got {input_ids.shape[0]} rows")
        self.check_target(target)
        self._check_generator(generator)
        if stop_token_ids is None:
            eos = target.generation_config.eos_token_id
            stop_token_ids = [] if eos is None else [eos] if isinstance(eos, int) else list(eos)
        dev, block = self.device, self.config.block_size
        prompt = input_ids.to(dev)
        stops = torch.tensor(stop_token_ids, device=dev, dtype=torch.long)
        rule = _Acceptance(temperature, generator)
        embed_tokens, lm_head = target.get_input_embeddings(), target.get_output_embeddings()

        with self.target_features(target) as features:
            past = DynamicCache()
            first = target(prompt, past_key_values=past, use_cache=True, logits_to_keep=1)
            tokens = rule.pick(first.logits[:, -1:])[0]
            # the last pass may commit a whole block past max_new_tokens
            cache = FlashMapCache(self.config, 1, prompt.shape[1] + max_new_tokens + block + 1, device=dev,
                                  dtype=self.dtype)
            self.extend_context(cache, features())
            committed_per_pass = []
            while tokens.shape[1] < max_new_tokens and not bool(torch.isin(tokens[0, -1], stops)):
                anchor = tokens[:, -1]
                proposal, proposal_probs = rule.pick(self.draft(anchor, cache, embed_tokens, lm_head, num_steps,
                                                                generator=generator))
                at = prompt.shape[1] + tokens.shape[1] - 1  # the anchor's position
                scored = target(torch.cat([anchor[:, None], proposal], dim=1),
                                position_ids=torch.arange(at, at + block + 1, device=dev)[None],
                                past_key_values=past, use_cache=True)
                kept, bonus = rule.verify(proposal, proposal_probs, scored.logits)
                fresh = _cut_at_stop(torch.cat([proposal[:, :kept], bonus.view(1, 1)], dim=1), stops)
                tokens = torch.cat([tokens, fresh], dim=1)
                committed_per_pass.append(fresh.shape[1])
                # the target keeps the anchor and the accepted drafts; the bonus is the next anchor
                surplus = past.get_seq_length() - (at + kept + 1)
                if surplus > 0:
                    past.crop(-surplus)
                self.extend_context(cache, features()[:, : kept + 1])

        tokens = tokens[:, :max_new_tokens]
        return FlashMapGenerateOutput(sequences=torch.cat([prompt, tokens], dim=1), num_new_tokens=tokens.shape[1],
                                      acceptance_lengths=committed_per_pass)
