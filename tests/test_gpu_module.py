"""The module-level drop-in (flashmap/modeling_flashmap.py:118-147): ``FlashMapAttention``
with the reference's ``project_kv(x, rope)`` and ``forward(x, rope, keys, values)``, the
``(cos, sin)`` pair of ``rope_tables`` as ``rope``, and a caller shaped like the
reference's ``FlashMapLayer.forward`` (flashmap/modeling_flashmap.py:185-192) holding it
unchanged.

The oracle composes the same module in float32 on the CPU from the same bf16 weights:
projections rounded to bf16 as a bf16 GEMM's output is, oracle rms_norm + apply_rope for
queries and keys, fp32 attention, o_proj. Bar: max-abs 2e-2 and mean-abs 2e-3 of the
fp32 result for the bf16 outputs; keys and values within two bf16 ulps per element."""

from types import SimpleNamespace

import pytest
import torch

from _inputs import check_close
from flashmap_amd import drafter as d
from oracle import attention as ref

pytestmark = pytest.mark.gpu


def _config(hidden, heads):
    return SimpleNamespace(hidden_size=hidden, num_attention_heads=heads, qk_norm_eps=1e-6, cond_dim=32,
                           layer_norm_eps=1e-6, intermediate_size=2 * hidden, mlp_type="gelu")


def _attention(cfg, dev, seed):
    torch.manual_seed(seed)
    attn = d.FlashMapAttention(cfg)
    with torch.no_grad():
        for name, p in attn.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(0.75 + 0.5 * torch.rand(p.shape))
            else:
                p.normal_(0.0, 0.02)
    return attn.to(dev, torch.bfloat16)


def _oracle_module(attn, x, ctx, pos_q, pos_k, theta):
    """The reference module's math in float32 from the bf16 weights (CPU)."""
    w = {n: p.detach().float().cpu() for n, p in attn.named_parameters()}
    heads, hd = attn.num_heads, attn.head_dim

    def proj(name, t):  # bf16 GEMM output: fp32 accumulate, bf16 result
        return (t.float() @ w[name].T).bfloat16()

    cq, sq = ref.rope_tables(pos_q, hd, theta)
    ck, sk = ref.rope_tables(pos_k, hd, theta)
    b, t, _ = x.shape
    q = ref.apply_rope(ref.rms_norm(proj("q_proj.weight", x).view(b, t, heads, hd), w["q_norm.weight"], 1e-6), cq, sq)
    L = ctx.shape[1]
    k = ref.apply_rope(ref.rms_norm(proj("k_proj.weight", ctx).view(b, L, heads, hd), w["k_norm.weight"], 1e-6), ck, sk)
    v = proj("v_proj.weight", ctx).view(b, L, heads, hd)
    o = ref.attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    return k.transpose(1, 2), v.transpose(1, 2), o.bfloat16().float().reshape(b, t, -1) @ w["o_proj.weight"].T


@pytest.mark.parametrize("hidden,heads,batch,ctx_len", [
    (1024, 16, 1, 512),   # the CPU-plumbing configuration's shape (MHA: the module has one head count)
    (4096, 32, 2, 2048),  # 32 heads of 128 over 2048 positions
    (256, 2, 3, 37),      # a ragged context length
])
def test_project_kv_and_forward_match_the_oracle(dev, hidden, heads, batch, ctx_len):
    print(f"FlashMapAttention hidden={hidden} heads={heads} B={batch} L={ctx_len}", flush=True)
    cfg = _config(hidden, heads)
    attn = _attention(cfg, dev, hidden + ctx_len)
    g = torch.Generator().manual_seed(ctx_len)
    x = torch.randn(batch, 16, hidden, generator=g).bfloat16()
    ctx = torch.randn(batch, ctx_len, hidden, generator=g).bfloat16()
    pos_k = torch.arange(ctx_len).expand(batch, -1)
    pos_q = ctx_len + torch.arange(16).expand(batch, -1)
    theta = 1e6
    keys, values = attn.project_kv(ctx.to(dev), d.rope_tables(pos_k.to(dev), attn.head_dim, theta))
    out = attn(x.to(dev), d.rope_tables(pos_q.to(dev), attn.head_dim, theta), keys, values)
    torch.cuda.synchronize()
    want_k, want_v, want_o = _oracle_module(attn, x, ctx, pos_q, pos_k, theta)
    assert keys.shape == (batch, heads, ctx_len, attn.head_dim) and values.shape == keys.shape
    assert out.shape == (batch, 16, hidden) and out.dtype == torch.bfloat16
    for name, got, want in (("keys", keys, want_k), ("values", values, want_v)):
        # One ulp of a projection (GPU and CPU sum in different orders) can flip the
        # bf16-rounded norm scale by an ulp as well, and the rotation mixes each (even,
        # odd) pair: the bar is two bf16 ulps of the pair's magnitude per element.
        w = want.float()
        pair = w.unflatten(-1, (-1, 2)).norm(dim=-1, keepdim=True).expand(*w.shape[:-1], -1, 2).flatten(-2)
        err = (got.float().cpu() - w).abs()
        bad = err > 2.0 ** -6 * pair + 1e-3
        i = int(((err - 2.0 ** -6 * pair) if bad.any() else err).argmax())
        assert not bad.any(), (f"{name}: {int(bad.sum())} elements off, worst got "
                               f"{got.float().flatten()[i]:.5f} want {w.flatten()[i]:.5f} pair {pair.flatten()[i]:.4f}")
        assert err.mean() <= 2e-3
    check_close(out.float().cpu(), want_o)


class _ReferenceShapedLayer(torch.nn.Module):
    """A caller written against the reference module interface: the reference's
    ``FlashMapLayer.forward`` call pattern, with the modules swapped in."""

    def __init__(self, layer):
        super().__init__()
        self.self_attn_adaln, self.self_attn = layer.self_attn_adaln, layer.self_attn
        self.cross_attn_adaln, self.cross_attn = layer.cross_attn_adaln, layer.cross_attn
        self.mlp_adaln, self.mlp = layer.mlp_adaln, layer.mlp

    def forward(self, x, modulations, rope, context):
        self_mod, cross_mod, mlp_mod = modulations
        h, gate = self.self_attn_adaln(x, self_mod)
        x = x + gate * self.self_attn(h, rope, *self.self_attn.project_kv(h, rope))
        h, gate = self.cross_attn_adaln(x, cross_mod)
        x = x + gate * self.cross_attn(h, rope, *context)
        h, gate = self.mlp_adaln(x, mlp_mod)
        return x + gate * self.mlp(h)


def test_reference_shaped_layer_holds_the_modules(dev):
    """The same weights through the reference's call pattern (eager residuals, the
    self-attention as project_kv + forward) and through FlashMapLayer.forward (fused
    residual kernel, one-launch self-attention): equal within the bf16 bar."""
    hidden, heads, batch, ctx_len = 256, 2, 3, 200
    cfg = _config(hidden, heads)
    torch.manual_seed(3)
    layer = d.FlashMapLayer(cfg)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(0.75 + 0.5 * torch.rand(p.shape))
            elif name.endswith("adaln.linear.weight"):
                p.normal_(0.0, 0.05)
            else:
                p.normal_(0.0, 0.05 if p.dim() > 1 else 0.02)
    layer = layer.to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(batch, 16, hidden, generator=g).bfloat16().to(dev)
    cond = torch.randn(1, 1, 32, generator=g).bfloat16().to(dev)
    mods = [n.modulation(cond) for n in (layer.self_attn_adaln, layer.cross_attn_adaln, layer.mlp_adaln)]
    ctx = torch.randn(batch, ctx_len, hidden, generator=g).bfloat16().to(dev)
    pos_k = torch.arange(ctx_len, device=dev).expand(batch, -1)
    pos_q = ctx_len + torch.arange(16, device=dev).expand(batch, -1)
    rope_q = d.rope_tables(pos_q, hidden // heads, 1e6)
    context = layer.cross_attn.project_kv(ctx, d.rope_tables(pos_k, hidden // heads, 1e6))
    got = layer(x, mods, rope_q, context)
    want = _ReferenceShapedLayer(layer)(x, mods, rope_q, context)
    torch.cuda.synchronize()
    check_close(got.float().cpu(), want.float().cpu())
