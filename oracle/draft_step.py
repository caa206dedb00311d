"""CPU restatement of the vLLM plugin's one-jump draft step.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Restates flashmap/vllm/model.py:
779-809 (``_prologue``: the anchors' context rows), 915-925 (``_one_jump``: the folded
noise read-out), 813-903 (``_dit``) and 1039-1041 (``compute_draft_logits``) on bf16 CPU
tensors, each op rounding as the reference's eager op does; the kernels' parts are the
pinned oracle functions of ``oracle.attention`` (self-attention, Q prologue, paged
attention, context write) and ``oracle.dit`` (the residual stream). Weights come in as a
dict of plain tensors (keys below); the folds (``flashmap_amd.fold``) are pinned by their
own identities.

Pinned by: composition of pinned functions; against the unfolded transformers
composition for the noise read-out (tests/test_gpu_draft_step.py).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import attention as ref
from . import dit


def _rms(x, w, eps):
    return ref.rms_norm(x, w, eps)


def write_anchor_rows(w: dict, anchors, positions, slots, caches, page):
    """``_prologue`` + ``_write`` for the anchors: embedding -> anchor_proj -> anchor_norm ->
    the layers' K/V projection -> k-norm + RoPE -> the caches (modified in place)."""
    rows = _rms(F.linear(w["embed"][anchors], w["anchor_proj.weight"], w["anchor_proj.bias"]),
                w["anchor_norm.weight"], w["anchor_norm.eps"])
    kv = F.linear(rows, w["context_kv_weight"])
    layers = len(caches)
    ref.write_context_kv_vllm(kv.view(rows.shape[0], layers, 2, w["heads"], -1), positions, slots,
                              w["context_k_norm"], w["cos_sin"], caches, page, w["k_eps"])


def one_jump(w: dict, anchors, anchor_positions, z, caches, block_table):
    """The final AdaLN output ``(B K, dim)`` bf16 of one jump (after the anchors are
    written): folded noise read-out, then the DiT layers over the paged caches."""
    k = w["block"]
    batch = anchors.shape[0]
    tokens, heads = batch * k, w["heads"]
    slot_pos = (anchor_positions[:, None] + 1 + torch.arange(k)).reshape(-1)
    seqused = anchor_positions + 1
    cu = torch.arange(0, tokens + 1, k, dtype=torch.int32)
    rms = torch.rsqrt((z * z) @ w["noise_eigvals"] + w["noise_eps"])
    noise = F.linear(z.to(torch.bfloat16), w["noise_embed"])
    hidden = w["first_hidden"] + (w["gain"] * rms)[:, None].to(torch.bfloat16) * noise
    cs = w["cos_sin"][slot_pos]
    cos, sin = cs[..., 0], cs[..., 1]
    for i, lw in enumerate(w["layers"]):
        (s_sc, s_sh, s_g), (c_sc, c_sh, c_g), (m_sc, m_sh, m_g) = lw["mods"]
        h = dit.adaln_residual(hidden, None, None, s_sc, s_sh, w["ln_eps"])[1]
        qkv = F.linear(h, lw["self_qkv"]).view(batch, k, 3, heads, -1)
        att = ref.block_self_attention(qkv, lw["self_q_norm"], lw["self_k_norm"], cos.view(batch, k, -1),
                                       sin.view(batch, k, -1), lw["qk_eps"]).to(torch.bfloat16)
        hidden = dit.adaln_residual(hidden, F.linear(att.reshape(tokens, -1), lw["self_o"]), s_g, None, None, 0)[0]
        h = dit.adaln_residual(hidden, None, None, c_sc, c_sh, w["ln_eps"])[1]
        q = ref.rms_norm_rope_vllm(F.linear(h, lw["cross_q"]).view(tokens, heads, -1), lw["cross_q_norm"],
                                   w["cos_sin"], slot_pos, lw["qk_eps"])
        ctx = ref.block_attention_paged_vllm(q, caches[i], cu, seqused, block_table).to(torch.bfloat16)
        hidden = dit.adaln_residual(hidden, F.linear(ctx.reshape(tokens, -1), lw["cross_o"]), c_g, None, None, 0)[0]
        h = dit.adaln_residual(hidden, None, None, m_sc, m_sh, w["ln_eps"])[1]
        if "fc1.weight" in lw:
            y = F.linear(F.gelu(F.linear(h, lw["fc1.weight"], lw["fc1.bias"])), lw["fc2.weight"], lw["fc2.bias"])
        else:
            gate, up = F.linear(h, lw["gate_up_proj.weight"]).chunk(2, dim=-1)
            y = F.linear(F.silu(gate) * up, lw["down_proj.weight"])
        hidden = dit.adaln_residual(hidden, y, m_g, None, None, 0)[0]
    return dit.adaln_residual(hidden, None, None, w["final_mod"][0], w["final_mod"][1], w["ln_eps"])[1]


def draft_logits(w: dict, hidden):
    """``compute_draft_logits``: the folded head over the draft vocabulary."""
    return F.linear(hidden, w["head_weight"], w["head_bias"])
