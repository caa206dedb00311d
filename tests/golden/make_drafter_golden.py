"""Writes tests/golden/drafter_tiny.safetensors: inputs and outputs of the reference
drafter's ``draft`` on two tiny random-init configurations, the composition that no
closed form pins (AdaLN-zero ordering, gated residuals, time conditioning, state mixing,
the jump loop). Run once, in the development container where the reference source is
present (never where the GPU tests run, and never as part of the tests):

    python tests/golden/make_drafter_golden.py /root/reference

Reference: flashmap/modeling_flashmap.py (FlashMapDraftModel.extend_context, draft),
imported from the given checkout with a random-init FlashMapConfig; nothing is
downloaded. For each case the fixture holds the drafter's state dict, the target's
embedding and lm_head, the context features, the anchor ids, the noise, and the draft
logits the reference returns (fp32 math of a bf16 model on the CPU).
"""

import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

CASES = {
    # name: (config overrides, batch, context positions, num_steps)
    "gelu_full_vocab_1step": (dict(mlp_type="gelu"), 3, 37, 1),
    "swiglu_state_vocab_2step": (dict(mlp_type="swiglu", state_vocab_size=200), 2, 20, 2),
}
BASE = dict(target_hidden_size=128, vocab_size=512, target_layer_ids=[0, 1], block_size=16, hidden_size=128,
            num_hidden_layers=2, num_attention_heads=2, intermediate_size=256, cond_dim=32, time_embed_dim=32)


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    from flashmap.configuration_flashmap import FlashMapConfig
    from flashmap.modeling_flashmap import FlashMapCache, FlashMapDraftModel

    out, meta = {}, {}
    for name, (over, batch, ctx, steps) in CASES.items():
        torch.manual_seed(1234)
        cfg = FlashMapConfig(**BASE, **over)
        model = FlashMapDraftModel(cfg).eval()
        with torch.no_grad():  # non-trivial norm weights, gates and biases
            for pname, p in model.named_parameters():
                if pname.endswith("norm.weight") or pname == "noise_gate":
                    p.copy_(0.75 + 0.5 * torch.rand(p.shape))
                elif pname.endswith(".bias"):
                    p.copy_(0.02 * torch.randn(p.shape))
                elif pname.endswith("adaln.linear.weight"):
                    p.copy_(0.05 * torch.randn(p.shape))
        model = model.to(torch.bfloat16)
        g = torch.Generator().manual_seed(99)
        embed = torch.nn.Embedding(cfg.vocab_size, cfg.target_hidden_size).to(torch.bfloat16)
        head = torch.nn.Linear(cfg.target_hidden_size, cfg.vocab_size, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            embed.weight.copy_(torch.randn(embed.weight.shape, generator=g))
            head.weight.copy_(0.05 * torch.randn(head.weight.shape, generator=g))
        feats = torch.randn(batch, ctx, len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g)
        feats = feats.to(torch.bfloat16)
        anchors = torch.randint(0, cfg.vocab_size, (batch,), generator=g)
        svocab = cfg.state_vocab_size or cfg.vocab_size
        noise = torch.randn(batch, cfg.block_size, svocab, generator=g)
        cache = FlashMapCache(cfg, batch, ctx + 1, dtype=torch.bfloat16)
        model.extend_context(cache, feats)
        logits = model.draft(anchors, cache, embed, head, num_steps=steps, noise=noise)
        for k, v in model.state_dict().items():
            out[f"{name}/model/{k}"] = v.contiguous()
        out[f"{name}/embed"] = embed.weight.detach().contiguous()
        out[f"{name}/lm_head"] = head.weight.detach().contiguous()
        out[f"{name}/features"] = feats
        out[f"{name}/anchors"] = anchors
        out[f"{name}/noise"] = noise
        out[f"{name}/logits"] = logits.float().contiguous()
        meta[name] = dict(config={**BASE, **over}, batch=batch, context=ctx, num_steps=steps,
                          state_keys=sorted(model.state_dict().keys()))
    here = Path(__file__).resolve().parent
    save_file(out, str(here / "drafter_tiny.safetensors"), metadata={"cases": json.dumps(meta)})
    print("wrote", here / "drafter_tiny.safetensors")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
