"""The drop-in op layer on the CPU: the vLLM / SGLang plugin ops register under a
namespace with the reference signatures, their fake implementations give the shapes
and dtypes the reference's do (so torch.compile and graph capture can trace them), and
unsupported variants fail loudly."""

import pytest
import torch

from flashmap_amd import sglang as fs
from flashmap_amd import vllm as fv

META = torch.device("meta")


def _e(*shape, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device=META)


@pytest.fixture(scope="module")
def ns():
    fv.register("fm_cpu_test_vllm")
    fs.register("fm_cpu_test_sglang")
    return torch.ops.fm_cpu_test_vllm, torch.ops.fm_cpu_test_sglang


def test_register_is_idempotent():
    a = fv.register("fm_cpu_test_vllm_idem")
    assert fv.register("fm_cpu_test_vllm_idem") is a
    assert set(a) == {"rms_norm_rope", "block_self_attention", "paged_cross_attention",
                      "paged_cross_attention_runs"}


def test_vllm_fake_shapes(ns):
    v, _ = ns
    q = _e(64 * 16, 32, 128, dtype=torch.bfloat16)
    kv = _e(100, 8, 16, 256, dtype=torch.bfloat16)
    out = v.paged_cross_attention(q, kv, _e(65, dtype=torch.int32), _e(64, dtype=torch.int32),
                                  _e(64, 10, dtype=torch.int32), None, None, 16, 8192, 0.088, 3)
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    x = _e(10, 4, 128, dtype=torch.bfloat16)
    assert v.rms_norm_rope(x, _e(128), _e(100, 64, 2), _e(10, dtype=torch.long), 1e-6).shape == x.shape
    qkv = _e(3, 16, 3, 4, 128, dtype=torch.bfloat16)
    got = v.block_self_attention(qkv, _e(128), _e(128), _e(100, 64, 2), _e(48, dtype=torch.long), 1e-6)
    assert got.shape == (48, 512) and got.dtype == torch.bfloat16
    caches = [_e(100, 8, 16, 256, dtype=torch.bfloat16) for _ in range(3)]
    runs = v.paged_cross_attention_runs(q[:, :20], caches, [0, 0, 8, 0, 1, 0, 8, 8, 2, 0, 4, 16],
                                        _e(65, dtype=torch.int32), _e(64, dtype=torch.int32),
                                        _e(64, 10, dtype=torch.int32), None, 16, 8192, 0.088)
    assert runs.shape == (64 * 16, 20, 128) and runs.dtype == torch.bfloat16


def test_sglang_fake_shapes(ns):
    _, s = ns
    qkv = _e(3, 16, 3, 4, 128, dtype=torch.bfloat16)
    assert s.block_self_attention(qkv, _e(128), _e(128), _e(3, 16, 64, 2), 1e-6).shape == (3, 16, 4, 128)
    q = _e(8, 16, 32, 128, dtype=torch.bfloat16)
    kb = _e(1000, 8, 128, dtype=torch.bfloat16)
    out = s.paged_cross_attention(q, kb, kb, _e(8, dtype=torch.int32), _e(8, 300, dtype=torch.int32), None)
    assert out.shape == q.shape
    x = _e(2, 16, 8, 128, dtype=torch.bfloat16)
    assert s.rms_norm_rope(x, _e(128), _e(2, 16, 64, 2), 1e-6).shape == x.shape
    kb8 = _e(1000, 8, 128, dtype=torch.float8_e4m3fn)
    out8 = s.paged_cross_attention_fp8(q, kb8, kb8, _e(8, dtype=torch.int32), _e(8, 300, dtype=torch.int32), None)
    assert out8.shape == q.shape and out8.dtype == q.dtype


def test_unsupported_variants_raise():
    q = torch.zeros(16, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        fs.fused_kv_norm_rope_write(q, q, q, q, q, q, 1, 256, 64, 1e-6, is_neox_style=True)


def test_fp8_variants_route_to_the_kernels():
    """The fp8 variants (vLLM descales / scales, SGLang's _fp8 ops) reach the fp8 kernel
    wrappers, which refuse CPU tensors (no CPU fallback)."""
    q8 = torch.zeros(16, 4, 64, dtype=torch.float8_e4m3fn)
    cache8 = torch.zeros(2, 4, 16, 128, dtype=torch.uint8)
    i32 = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        fv.paged_cross_attention(q8, cache8, i32, i32[:1], torch.zeros(1, 2, dtype=torch.int32), None,
                                 torch.ones(3, 1, 4), 16, 64, 0.125, 3)
    kv = torch.zeros(3, 1, 2, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        fv.write_context_kv(kv, torch.zeros(3, dtype=torch.long), torch.zeros(3, dtype=torch.long),
                            torch.ones(1, 64), torch.zeros(8, 32, 2), torch.zeros(1, dtype=torch.long),
                            (1, 1, 1, 1), 16, 1e-6, scales=torch.ones(1, 2))
    qb = torch.zeros(1, 16, 4, 64, dtype=torch.bfloat16)
    pool8 = torch.zeros(10, 4, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="GPU"):
        fs.paged_cross_attention_fp8(qb, pool8, pool8, i32[:1], torch.zeros(1, 4, dtype=torch.int32), None)


def test_rope_freqs_matches_oracle_table():
    from oracle import attention as ref

    pos = torch.arange(77)
    assert torch.equal(fs.rope_freqs(pos, 128, 1e6), ref.rope_freqs(pos, 128, 1e6))
