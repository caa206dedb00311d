"""Packaging: the engine entry points declared in pyproject.toml resolve to this
package's plugin functions (the reference declares its plugins the same way,
pyproject.toml:36-40 of the reference), which register the ops under the reference
namespaces once and leave a taken namespace alone."""

import importlib
from pathlib import Path

import torch

try:
    import tomllib
except ModuleNotFoundError:  # Python 3.10
    import tomli as tomllib

ROOT = Path(__file__).resolve().parents[1]


def test_entry_points_resolve_and_register():
    meta = tomllib.loads((ROOT / "pyproject.toml").read_text())
    eps = meta["project"]["entry-points"]
    targets = [eps["vllm.general_plugins"]["flashmap_amd"], eps["sglang.srt.plugins"]["flashmap_amd"]]
    for target in targets:
        mod, fn = target.split(":")
        plugin = getattr(importlib.import_module(mod), fn)
        plugin()
        plugin()  # idempotent
    assert callable(torch.ops.flashmap_vllm.paged_cross_attention)
    assert callable(torch.ops.flashmap_sglang.paged_cross_attention)
