"""The drop-in drafter's structure on the CPU: its parameter names and shapes are the
reference checkpoint's (recorded by tests/golden/make_drafter_golden.py from the
reference's FlashMapDraftModel), the config defaults and jump times follow the
reference's configuration module, and the model refuses to run its attention off the GPU."""

import json
from pathlib import Path

import pytest
import torch
from safetensors import safe_open

from flashmap_amd import drafter as d

GOLDEN = Path(__file__).resolve().parent / "golden" / "drafter_tiny.safetensors"


def _cases():
    with safe_open(str(GOLDEN), "pt") as f:
        return json.loads(f.metadata()["cases"]), {k: f.get_tensor(k) for k in f.keys()}


def test_state_dict_matches_reference_checkpoint():
    meta, tensors = _cases()
    for name, case in meta.items():
        model = d.FlashMapDraftModel(case["config"])
        ours = model.state_dict()
        assert sorted(ours) == case["state_keys"], name
        for k in ours:
            assert tuple(ours[k].shape) == tuple(tensors[f"{name}/model/{k}"].shape), (name, k)
        model.load_state_dict({k: tensors[f"{name}/model/{k}"] for k in ours})  # strict


def test_config_defaults_and_jump_times():
    cfg = d.drafter_config()
    assert (cfg.hidden_size, cfg.num_attention_heads, cfg.block_size, cfg.num_steps) == (2048, 16, 16, 1)
    assert cfg.jump_grids["2"] == [0.0, 0.8172569274902344, 1.0]
    assert d.jump_times([0.0, 0.5, 1.0]) == [(0.0, 0.5, 0.5), (0.5, 1.0, 1.0)]
    assert d.drafter_config({"hidden_size": 64, "unknown": 1}).hidden_size == 64
    with pytest.raises(ValueError):
        d.drafter_config(mlp_type="relu")


def test_cache_layout_and_bounds():
    cfg = d.drafter_config(hidden_size=128, num_attention_heads=2, num_hidden_layers=3)
    cache = d.FlashMapCache(cfg, batch_size=2, max_length=10)
    assert tuple(cache.kv.shape) == (3, 2, 2, 2, 10, 64)
    k = torch.randn(2, 2, 4, 64)
    cache.write(1, 3, k, -k)
    keys, values = cache.context(7)[1]
    assert torch.equal(keys[:, :, 3:7], k) and torch.equal(values[:, :, 3:7], -k)
    with pytest.raises(ValueError):
        cache.write(0, 8, k, k)


def test_attention_refuses_cpu_tensors():
    meta, _ = _cases()
    model = d.FlashMapDraftModel(meta["gelu_full_vocab_1step"]["config"]).to(torch.bfloat16)
    cache = d.FlashMapCache(model.config, 1, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        model.extend_context(cache, torch.zeros(1, 2, 256, dtype=torch.bfloat16))
