"""Drop-in FlashMap drafter for the transformers path, with its attention on the gfx950
kernels.

The module tree and parameter names are those of the reference's
``FlashMapDraftModel`` (flashmap/modeling_flashmap.py:241-313), so a reference checkpoint
(its ``config.json`` and safetensors, or a live model's ``state_dict()``) loads as is;
``draft`` and ``spec_generate`` keep the reference's signatures and results. What runs
differently is the attention of every DiT layer:

- self-attention across the block's slots: q/k RMSNorm + RoPE and the unmasked
  16 x 16 attention in one launch (``fm_block_self_attention``, row a8);
- cross-attention to the context: the query prologue fused into the split-KV block
  attention over the cache (``fm_block_attn_contig``, rows a3 + a5);
- the context's keys: RMSNorm + RoPE by ``fm_rms_norm_rope`` before the cache write
  (row a4).

The rest of the DiT (time embeddings, adaptive LayerNorms, MLPs, projections) is plain
torch, as in the reference. The kernels are bf16 and GPU-only: the model must live on a
ROCm device in bfloat16, and every attention call fails loudly otherwise.
"""

from __future__ import annotations

import json
import math
import os
from contextlib import contextmanager
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import ops

__all__ = ["FlashMapCache", "FlashMapDraftModel", "FlashMapGenerateOutput", "drafter_config", "jump_times"]

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


def drafter_config(config=None, **overrides) -> SimpleNamespace:
    """A drafter configuration from a reference ``FlashMapConfig``, a ``config.json``
    dict or keyword arguments (missing fields take the reference's defaults)."""
    if config is None:
        src = {}
    elif isinstance(config, dict):
        src = dict(config)
    else:
        src = {k: getattr(config, k) for k in _DEFAULTS if hasattr(config, k)}
    cfg = {**_DEFAULTS, **{k: v for k, v in src.items() if k in _DEFAULTS}, **overrides}
    cfg["target_layer_ids"] = list(cfg["target_layer_ids"])
    cfg["jump_grids"] = dict(_JUMP_GRIDS if cfg["jump_grids"] is None else cfg["jump_grids"])
    if cfg["mlp_type"] not in ("gelu", "swiglu"):
        raise ValueError(f"mlp_type must be gelu or swiglu, got {cfg['mlp_type']!r}")
    return SimpleNamespace(**cfg)


def jump_times(grid) -> list:
    """``(s, t, next)`` per jump over ``grid``: the network jumps from ``s`` to ``t``
    and the state then moves to ``next``; each jump lands where the next starts, so
    ``t == next`` (flashmap/configuration_flashmap.py:23-31)."""
    times = [float(v) for v in grid]
    return [(a, b, b) for a, b in zip(times, times[1:])]


def _rope_rows(positions: torch.Tensor, head_dim: int, theta: float) -> ops.Rope:
    """Rotary rows of ``positions (B, T)``, one row per token in ``b * T + t`` order,
    computed with the torch expression of flashmap/modeling_flashmap.py:53-58."""
    inv_freq = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=positions.device).float() / head_dim)
    angles = positions.reshape(-1).float()[:, None] * inv_freq
    return ops.rope_from_split(angles.cos(), angles.sin())


class _RMSNorm(nn.Module):
    """RMSNorm with the scale ``w / rms(x)`` rounded to ``x``'s dtype before the
    multiply (flashmap/modeling_flashmap.py:69-80)."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        inv_rms = torch.rsqrt(x.float().square().mean(-1, keepdim=True) + self.eps)
        return x * (self.weight.float() * inv_rms).to(x.dtype)


class _TimeEmbedding(nn.Module):
    """Sinusoidal features of a time in [0, 1], then a two-layer MLP
    (flashmap/modeling_flashmap.py:83-99)."""

    def __init__(self, cfg):
        super().__init__()
        self.dim, self.scale = cfg.time_embed_dim, cfg.time_scale
        self.linear_1 = nn.Linear(cfg.time_embed_dim, cfg.cond_dim)
        self.linear_2 = nn.Linear(cfg.cond_dim, cfg.cond_dim)

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        half = self.dim // 2
        freqs = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device).float() / half)
        phase = (t.float() * self.scale)[..., None] * freqs
        feats = torch.cat([phase.cos(), phase.sin()], dim=-1).to(self.linear_1.weight.dtype)
        return self.linear_2(F.silu(self.linear_1(feats)))


class _AdaLN(nn.Module):
    """LayerNorm modulated by the time conditioning: ``(scale, shift, gate)`` from one
    linear map of ``silu(cond)`` (flashmap/modeling_flashmap.py:102-117)."""

    def __init__(self, cfg):
        super().__init__()
        self.linear = nn.Linear(cfg.cond_dim, 3 * cfg.hidden_size)
        self.eps = cfg.layer_norm_eps

    def modulation(self, cond: torch.Tensor):
        return self.linear(F.silu(cond)).chunk(3, dim=-1)

    def forward(self, x: torch.Tensor, modulation):
        scale, shift, gate = modulation
        return F.layer_norm(x, x.shape[-1:], eps=self.eps) * (1 + scale) + shift, gate


class _Attention(nn.Module):
    """Projections and q/k norm weights of one attention (parameter names of
    flashmap/modeling_flashmap.py:118-134); the attention itself runs on the kernels."""

    def __init__(self, cfg):
        super().__init__()
        dim = cfg.hidden_size
        self.heads = cfg.num_attention_heads
        self.head_dim = dim // self.heads
        self.eps = cfg.qk_norm_eps
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.k_proj = nn.Linear(dim, dim, bias=False)
        self.v_proj = nn.Linear(dim, dim, bias=False)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self.q_norm = _RMSNorm(self.head_dim, cfg.qk_norm_eps)
        self.k_norm = _RMSNorm(self.head_dim, cfg.qk_norm_eps)

    def _split(self, y: torch.Tensor) -> torch.Tensor:
        return y.view(*y.shape[:2], self.heads, self.head_dim)

    def project_kv(self, x: torch.Tensor, rope: ops.Rope):
        """Keys (k-normed and rotated) and values ``(B, T, heads, head_dim)`` of ``x (B,
        T, dim)``; ``rope`` has one row per token (flashmap/modeling_flashmap.py:139-142)."""
        b, t, _ = x.shape
        k = self.k_proj(x).view(b * t, self.heads, self.head_dim)
        keys = ops.rms_norm_rope(k, self.k_norm.weight, rope, None, self.eps)
        return keys.view(b, t, self.heads, self.head_dim), self._split(self.v_proj(x))

    def self_attend(self, x: torch.Tensor, rope: ops.Rope) -> torch.Tensor:
        """Attention across the block's slots, queries and keys both from ``x``
        (flashmap/modeling_flashmap.py:188): one fused launch."""
        b, t, _ = x.shape
        qkv = torch.stack([self._split(p(x)) for p in (self.q_proj, self.k_proj, self.v_proj)], dim=2)
        out = ops.block_self_attention(qkv, self.q_norm.weight, self.k_norm.weight, rope, None, self.eps)
        return self.o_proj(out.view(b, t, -1))

    def cross_attend(self, x: torch.Tensor, rope: ops.Rope, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """Attention of ``x``'s queries onto ``keys``/``values (B, heads, L, head_dim)``
        with the query prologue fused (flashmap/modeling_flashmap.py:144-147)."""
        q = self._split(self.q_proj(x))
        prologue = ops.Prologue(self.q_norm.weight, rope, None, self.eps)
        out = ops.block_attention_contig(q, keys, values, prologue=prologue)
        return self.o_proj(out.flatten(2))


class _MLP(nn.Module):
    """``fc2(gelu(fc1(x)))`` or, for "swiglu", ``down_proj(silu(gate) * up)``
    (flashmap/modeling_flashmap.py:150-170)."""

    def __init__(self, cfg):
        super().__init__()
        self.swiglu = cfg.mlp_type == "swiglu"
        dim, hidden = cfg.hidden_size, cfg.intermediate_size
        if self.swiglu:
            self.gate_up_proj = nn.Linear(dim, 2 * hidden, bias=False)
            self.down_proj = nn.Linear(hidden, dim, bias=False)
        else:
            self.fc1 = nn.Linear(dim, hidden)
            self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.swiglu:
            gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
            return self.down_proj(F.silu(gate) * up)
        return self.fc2(F.gelu(self.fc1(x)))


class _Layer(nn.Module):
    """A DiT block: self-attention, cross-attention, MLP, each behind a modulated
    LayerNorm and a gated residual (flashmap/modeling_flashmap.py:173-192)."""

    def __init__(self, cfg):
        super().__init__()
        self.self_attn_adaln = _AdaLN(cfg)
        self.self_attn = _Attention(cfg)
        self.cross_attn_adaln = _AdaLN(cfg)
        self.cross_attn = _Attention(cfg)
        self.mlp_adaln = _AdaLN(cfg)
        self.mlp = _MLP(cfg)

    def forward(self, x, modulations, rope: ops.Rope, context) -> torch.Tensor:
        m_self, m_cross, m_mlp = modulations
        h, gate = self.self_attn_adaln(x, m_self)
        x = x + gate * self.self_attn.self_attend(h, rope)
        h, gate = self.cross_attn_adaln(x, m_cross)
        x = x + gate * self.cross_attn.cross_attend(h, rope, *context)
        h, gate = self.mlp_adaln(x, m_mlp)
        return x + gate * self.mlp(h)


class FlashMapCache:
    """Every DiT layer's cross-attention keys and values of the context: positions
    ``[0, length)`` hold the target's features, position ``length`` the anchor while a
    block is drafted (flashmap/modeling_flashmap.py:195-219). Same tensor layout,
    ``(layers, 2, B, heads, max_length, head_dim)``, read by the kernels through strides."""

    def __init__(self, config, batch_size: int, max_length: int, device=None, dtype=None):
        cfg = config if isinstance(config, SimpleNamespace) else drafter_config(config)
        head_dim = cfg.hidden_size // cfg.num_attention_heads
        shape = (cfg.num_hidden_layers, 2, batch_size, cfg.num_attention_heads, max_length, head_dim)
        self.kv = torch.zeros(shape, device=device, dtype=dtype)
        self.length = 0

    def write(self, layer: int, start: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Store ``keys``/``values (B, heads, n, head_dim)`` at positions ``start ..``."""
        end = start + keys.shape[2]
        if end > self.kv.shape[4]:
            raise ValueError(f"FlashMapCache holds {self.kv.shape[4]} positions, writing up to {end}")
        self.kv[layer, 0, :, :, start:end] = keys
        self.kv[layer, 1, :, :, start:end] = values

    def context(self, end: int) -> list:
        """Per layer, the (keys, values) views of positions ``[0, end)``."""
        return [(layer_kv[0, :, :, :end], layer_kv[1, :, :, :end]) for layer_kv in self.kv]


@dataclass
class FlashMapGenerateOutput:
    """Prompt plus generated tokens ``(1, length)``, the number generated and the tokens
    committed per target forward pass (flashmap/modeling_flashmap.py:222-236)."""

    sequences: torch.LongTensor
    num_new_tokens: int
    acceptance_lengths: list = field(default_factory=list)

    @property
    def acceptance_length(self) -> float:
        return sum(self.acceptance_lengths) / max(len(self.acceptance_lengths), 1)


class FlashMapDraftModel(nn.Module):
    """The FlashMap drafter (flashmap/modeling_flashmap.py:239-612) with its attention
    on the gfx950 kernels. Build it with :meth:`from_pretrained` (a local checkpoint
    folder), :meth:`from_reference` (a live reference model) or from a config, then
    move it to the GPU in bfloat16."""

    def __init__(self, config=None, **overrides):
        super().__init__()
        cfg = self.config = drafter_config(config, **overrides)
        dim, target_dim = cfg.hidden_size, cfg.target_hidden_size
        self.head_dim = dim // cfg.num_attention_heads
        self.fc = nn.Linear(len(cfg.target_layer_ids) * target_dim, dim, bias=False)
        self.hidden_norm = _RMSNorm(dim, cfg.rms_norm_eps)
        self.anchor_proj = nn.Linear(target_dim, dim)
        self.anchor_norm = _RMSNorm(dim, cfg.rms_norm_eps)
        self.state_norm = _RMSNorm(target_dim, cfg.rms_norm_eps)
        self.noise_norm = _RMSNorm(target_dim, cfg.rms_norm_eps)
        self.noise_gate = nn.Parameter(torch.ones(1))
        self.x_embed = nn.Linear(target_dim, dim)
        self.time_embed = _TimeEmbedding(cfg)
        self.jump_embed = _TimeEmbedding(cfg)
        self.layers = nn.ModuleList(_Layer(cfg) for _ in range(cfg.num_hidden_layers))
        self.final_adaln = _AdaLN(cfg)
        self.head = nn.Linear(dim, target_dim)
        if cfg.state_vocab_size is not None:
            self.register_buffer("draft_ids", torch.arange(cfg.state_vocab_size))
        self._memo = {}

    # -- construction ----------------------------------------------------------------

    @classmethod
    def from_pretrained(cls, path: str, device=None, dtype=torch.bfloat16) -> "FlashMapDraftModel":
        """A local checkpoint folder: ``config.json`` plus ``*.safetensors``."""
        from safetensors.torch import load_file

        with open(os.path.join(path, "config.json")) as f:
            model = cls(json.load(f))
        state = {}
        for name in sorted(os.listdir(path)):
            if name.endswith(".safetensors"):
                state.update(load_file(os.path.join(path, name)))
        model.load_state_dict(state)
        return model.to(device=device, dtype=dtype)

    @classmethod
    def from_reference(cls, reference: nn.Module) -> "FlashMapDraftModel":
        """The same drafter as a live reference ``FlashMapDraftModel`` (weights copied),
        on its device and in its dtype."""
        model = cls(reference.config)
        model.load_state_dict(reference.state_dict())
        p = next(reference.parameters())
        return model.to(device=p.device, dtype=p.dtype)

    def _apply(self, fn, *args, **kwargs):
        self._memo = {}
        return super()._apply(fn, *args, **kwargs)

    def load_state_dict(self, *args, **kwargs):
        self._memo = {}
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
        """AdaLN modulations of the jump ``s -> t`` for every norm (per layer: self,
        cross, MLP; then the final norm), memoized per ``(s, t)``
        (flashmap/modeling_flashmap.py:271-284)."""
        key = ("time", s, t)
        if key not in self._memo:
            st = torch.tensor([s, t], device=self.device)
            cond = (self.time_embed(st[:1]) + self.jump_embed(st[1:]))[None]
            per_layer = [
                [n.modulation(cond) for n in (blk.self_attn_adaln, blk.cross_attn_adaln, blk.mlp_adaln)]
                for blk in self.layers
            ]
            self._memo[key] = (per_layer, self.final_adaln.modulation(cond))
        return self._memo[key]

    def forward(self, inputs_embeds, s: float, t: float, position_ids, context) -> torch.Tensor:
        """One jump ``s -> t`` of the featurized state ``(B, K, target_hidden)`` of blocks
        at ``position_ids (B, K)``, with each layer's context ``(keys, values)``
        (flashmap/modeling_flashmap.py:286-298)."""
        per_layer, final = self.time_conditioning(s, t)
        rope = _rope_rows(position_ids, self.head_dim, self.config.rope_theta)
        h = self.x_embed(inputs_embeds)
        for blk, mods, ctx in zip(self.layers, per_layer, context):
            h = blk(h, mods, rope, ctx)
        h, _ = self.final_adaln(h, final)
        return self.head(h)

    # -- context ---------------------------------------------------------------------

    @contextmanager
    def target_features(self, target: nn.Module):
        """Hooks keeping the outputs of the target's layers ``target_layer_ids``; yields
        a function concatenating them for the last target forward
        (flashmap/modeling_flashmap.py:321-339)."""
        layers, kept = target.get_decoder().layers, {}

        def hook_for(i):
            def hook(_module, _args, output):
                kept[i] = output[0] if isinstance(output, tuple) else output

            return hook

        handles = [layers[i].register_forward_hook(hook_for(i)) for i in self.config.target_layer_ids]
        try:
            yield lambda: torch.cat([kept[i] for i in self.config.target_layer_ids], dim=-1)
        finally:
            for h in handles:
                h.remove()

    def _write_context(self, cache: FlashMapCache, start: int, feats: torch.Tensor) -> None:
        b, n, _ = feats.shape
        pos = torch.arange(start, start + n, device=feats.device).expand(b, -1)
        rope = _rope_rows(pos, self.head_dim, self.config.rope_theta)
        for i, blk in enumerate(self.layers):
            keys, values = blk.cross_attn.project_kv(feats, rope)
            cache.write(i, start, keys.transpose(1, 2), values.transpose(1, 2))

    @torch.no_grad()
    def extend_context(self, cache: FlashMapCache, target_hidden: torch.Tensor) -> None:
        """Append the target's features ``(B, n, ...)`` at the next ``n`` positions
        (flashmap/modeling_flashmap.py:342-351)."""
        feats = self.hidden_norm(self.fc(target_hidden.to(self.dtype)))
        self._write_context(cache, cache.length, feats)
        cache.length += target_hidden.shape[1]

    # -- drafting --------------------------------------------------------------------

    @torch.no_grad()
    def state_vocab(self, embed_tokens: nn.Module, lm_head: nn.Module):
        """``(embedding, head weight, head bias)`` over the state vocabulary
        (flashmap/modeling_flashmap.py:355-368)."""
        emb, w, bias = embed_tokens.weight, lm_head.weight, getattr(lm_head, "bias", None)
        if self.config.state_vocab_size is None:
            return emb, w, bias
        key = ("vocab", emb.data_ptr(), w.data_ptr(), emb.device, emb.dtype)
        if key not in self._memo:
            ids = self.draft_ids.to(emb.device)
            self._memo = {k: v for k, v in self._memo.items() if k[0] != "vocab"}
            self._memo[key] = (emb[ids], w[ids], None if bias is None else bias[ids])
        return self._memo[key]

    def token_logits(self, logits: torch.Tensor) -> torch.Tensor:
        """Logits over the target's vocabulary (``-inf`` outside the state vocabulary)."""
        if self.config.state_vocab_size is None:
            return logits
        full = logits.new_full((*logits.shape[:-1], self.config.vocab_size), float("-inf"))
        full[..., self.draft_ids.to(logits.device)] = logits
        return full

    @torch.no_grad()
    def target_constants(self, embedding: torch.Tensor):
        """The embedded uniform posterior and ``L`` with ``L L^T = E^T E`` (float64
        Cholesky on the CPU) for the target embedding ``E``
        (flashmap/modeling_flashmap.py:396-418)."""
        key = ("target", embedding.data_ptr(), tuple(embedding.shape), embedding.device, embedding.dtype)
        if key not in self._memo:
            vocab = embedding.shape[0]
            gram = None
            for rows in embedding.split(16384):
                part = rows.float().T @ rows.float()
                gram = part if gram is None else gram + part
            factor = torch.linalg.cholesky(gram.cpu().double())
            uniform = torch.full((1, vocab), 1.0 / vocab, device=embedding.device)
            self._memo = {k: v for k, v in self._memo.items() if k[0] != "target"}
            self._memo[key] = (uniform.to(embedding.dtype) @ embedding, factor.to(self.device, self.dtype))
        return self._memo[key]

    def mix_state(self, posterior_embeds, state_embeds, s: float, t: float) -> torch.Tensor:
        """State embedding from its posterior and linear projections
        (flashmap/modeling_flashmap.py:388-394)."""
        weight = 1.0 if self.config.noise_gate == "constant" else t - s
        gate = (self.noise_gate.float() * weight).to(self.dtype)
        return self.state_norm(posterior_embeds.to(self.dtype)) + gate * self.noise_norm(state_embeds.to(self.dtype))

    def embed_state(self, state, s: float, t: float, embedding: torch.Tensor) -> torch.Tensor:
        """DiT input for the state ``(B, K, V)`` at ``s`` jumping to ``t``
        (flashmap/modeling_flashmap.py:370-386)."""
        if s == 0:
            posterior_embeds = self.target_constants(embedding)[0]
        else:
            sharpen = s / max(1.0 - s, 1e-3) ** 2
            posterior_embeds = (state.float() * sharpen).softmax(dim=-1).to(embedding.dtype) @ embedding
        return self.mix_state(posterior_embeds, state.to(embedding.dtype) @ embedding, s, t)

    @torch.no_grad()
    def draft(self, anchor_ids, cache: FlashMapCache, embed_tokens, lm_head, num_steps: Optional[int] = None,
              noise: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """Draft logits ``(B, block_size, V)`` for the block after ``anchor_ids (B,)``,
        as flashmap/modeling_flashmap.py:420-479: the anchor's embedding is written to
        the cache at its position, then the jumps of the step grid run over the
        context ``[0, anchor]``."""
        cfg = self.config
        steps = num_steps or cfg.num_steps
        if str(steps) not in cfg.jump_grids:
            raise ValueError(f"num_steps must be one of {', '.join(sorted(cfg.jump_grids, key=int))} "
                             f"(the config's jump_grids), got {steps}")
        grid = cfg.jump_grids[str(steps)]
        batch, block = anchor_ids.shape[0], cfg.block_size
        dev = anchor_ids.device
        embedding, head_w, head_b = self.state_vocab(embed_tokens, lm_head)

        anchor = cache.length
        anchor_feats = self.anchor_norm(self.anchor_proj(embed_tokens(anchor_ids[:, None]).to(self.dtype)))
        self._write_context(cache, anchor, anchor_feats)
        context = cache.context(anchor + 1)
        positions = anchor + 1 + torch.arange(block, device=dev).expand(batch, -1)

        state, inputs = noise, None
        if state is None and steps == 1:  # one jump reads its noise only through x0 @ E
            uniform_embeds, factor = self.target_constants(embedding)
            z = torch.randn((batch, block, factor.shape[0]), device=dev, dtype=factor.dtype, generator=generator)
            inputs = self.mix_state(uniform_embeds, z @ factor.T, 0.0, grid[1])
        elif state is None:
            state = torch.randn((batch, block, embedding.shape[0]), device=dev, generator=generator)

        logits = None
        for s, t, nxt in jump_times(grid):
            if state is not None:
                inputs = self.embed_state(state, s, t, embedding)
            hidden = self(inputs, s, t, positions, context).to(head_w.dtype)
            logits = F.linear(hidden, head_w, head_b)
            if nxt < 1.0:  # the state moves to the next grid time
                state = ((1.0 - nxt) * state + (nxt - s) * logits.float().softmax(dim=-1)) / (1.0 - s)
        return self.token_logits(logits)

    # -- speculative decoding --------------------------------------------------------

    def check_target(self, target) -> None:
        """Raise if ``target``'s embedding / lm_head do not match the drafter's vocabulary
        and target hidden size, or it has too few layers for ``target_layer_ids``
        (flashmap/modeling_flashmap.py:483-512, the shape checks)."""
        want = (self.config.vocab_size, self.config.target_hidden_size)
        emb, head = target.get_input_embeddings().weight, target.get_output_embeddings().weight
        if tuple(emb.shape) != want or tuple(head.shape) != want:
            raise ValueError(f"this drafter needs a target with vocabulary {want[0]} and hidden size {want[1]}, "
                             f"got an embedding of shape {tuple(emb.shape)}")
        layers = len(target.get_decoder().layers)
        if max(self.config.target_layer_ids) >= layers - 1:
            raise ValueError(f"target_layer_ids {self.config.target_layer_ids} need more than {layers} target layers")
        if emb.device != self.device:
            raise ValueError(f"the drafter and the target's embedding must share a device, got {self.device} "
                             f"and {emb.device}")

    @torch.no_grad()
    def spec_generate(self, target, input_ids: torch.LongTensor, max_new_tokens: int = 256, temperature: float = 0.0,
                      num_steps: Optional[int] = None, stop_token_ids: Optional[list] = None,
                      generator: Optional[torch.Generator] = None) -> FlashMapGenerateOutput:
        """Lossless speculative decoding of a transformers causal LM ``target`` from the
        prompt ``input_ids (1, P)``: per round, draft a block after the last token,
        score it with one target pass, keep the accepted prefix plus the target's own
        token (flashmap/modeling_flashmap.py:514-612). Greedy at ``temperature`` 0,
        rejection sampling above it."""
        from transformers import DynamicCache

        if input_ids.shape[0] != 1:
            raise ValueError("spec_generate decodes one sequence at a time")
        self.check_target(target)
        if stop_token_ids is None:
            eos = target.generation_config.eos_token_id
            stop_token_ids = [] if eos is None else [eos] if isinstance(eos, int) else list(eos)
        dev = self.device
        input_ids = input_ids.to(dev)
        stop = torch.tensor(stop_token_ids, device=dev, dtype=torch.long)
        embed_tokens, lm_head = target.get_input_embeddings(), target.get_output_embeddings()
        block, prompt_len = self.config.block_size, input_ids.shape[1]

        def pick(logits):  # (1, n, V) -> tokens (1, n), distributions
            if temperature <= 0:
                return logits.argmax(dim=-1), None
            probs = (logits.float() / temperature).softmax(dim=-1)
            return torch.multinomial(probs[0], 1, generator=generator).T, probs

        with self.target_features(target) as features:
            kv = DynamicCache()
            out = target(input_ids, past_key_values=kv, use_cache=True, logits_to_keep=1)
            tokens = pick(out.logits[:, -1:])[0]
            cache = FlashMapCache(self.config, 1, prompt_len + max_new_tokens + block + 1, device=dev, dtype=self.dtype)
            self.extend_context(cache, features())
            accepted_per_pass = []
            while tokens.shape[1] < max_new_tokens and not torch.isin(tokens[0, -1], stop):
                anchor = tokens[:, -1]
                draft, draft_probs = pick(self.draft(anchor, cache, embed_tokens, lm_head, num_steps,
                                                     generator=generator))
                pos = prompt_len + tokens.shape[1] - 1  # the anchor's position
                out = target(torch.cat([anchor[:, None], draft], dim=1),
                             position_ids=torch.arange(pos, pos + block + 1, device=dev)[None],
                             past_key_values=kv, use_cache=True)
                if temperature <= 0:
                    tt = out.logits.argmax(dim=-1)
                    n_ok = int((draft == tt[:, :-1]).cumprod(dim=1).sum())
                    bonus = tt[:, n_ok]
                else:
                    p_t = (out.logits.float() / temperature).softmax(dim=-1)[0]
                    p = p_t[:-1].gather(-1, draft[0, :, None])[:, 0]
                    q = draft_probs[0].gather(-1, draft[0, :, None])[:, 0]
                    u = torch.rand(q.shape, device=q.device, generator=generator)
                    n_ok = int((u * q < p).cumprod(dim=0).sum())
                    residual = p_t[n_ok]
                    if n_ok < block:
                        residual = (residual - draft_probs[0, n_ok]).clamp_min(0)
                        if residual.sum() <= 0:
                            residual = p_t[n_ok]
                    bonus = torch.multinomial(residual, 1, generator=generator)
                new = torch.cat([draft[:, :n_ok], bonus.view(1, 1)], dim=1)
                hit = torch.isin(new[0], stop).nonzero()
                if len(hit):
                    new = new[:, : int(hit[0]) + 1]
                tokens = torch.cat([tokens, new], dim=1)
                accepted_per_pass.append(new.shape[1])
                extra = kv.get_seq_length() - (pos + n_ok + 1)
                if extra > 0:
                    kv.crop(-extra)
                self.extend_context(cache, features()[:, : n_ok + 1])
        tokens = tokens[:, :max_new_tokens]
        return FlashMapGenerateOutput(torch.cat([input_ids, tokens], dim=1), tokens.shape[1], accepted_per_pass)
