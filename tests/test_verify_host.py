"""SplitKVVerify's host logic on the CPU: the cases it declines (returning False having
done nothing, as flashmap/sglang/verify_attention.py:382-402 does), the QLEN_ONLY
refusal, and its extend_attention_fwd call signature. No GPU calls: every case here is
decided before the kernels are reached."""

import inspect

import pytest
import torch


def _args(dtype=torch.bfloat16, bs=2, length=3, hq=8, hkv=2, d=128, pool=50):
    q = torch.zeros(bs * length, hq, d, dtype=dtype)
    k = torch.zeros(bs * length, hkv, d, dtype=dtype)
    o = torch.zeros(bs * length, hq * d, dtype=dtype)
    kb = torch.zeros(pool, hkv, d, dtype=dtype)
    qo = torch.arange(0, bs * length + 1, length, dtype=torch.int32)
    indptr = torch.zeros(bs + 1, dtype=torch.int32)
    indices = torch.zeros(0, dtype=torch.int32)
    return [q, k, k.clone(), o, kb, kb.clone(), qo, indptr, indices, None, True, None, length]


@pytest.mark.parametrize(
    "change",
    [
        dict(logit_cap=30.0),
        dict(sinks=torch.zeros(8)),
        dict(sliding_window_size=128),
        dict(xai_temperature_len=4),
        dict(k_scale=None),
        dict(v_scale=torch.ones(1)),
    ],
)
def test_declines_like_the_reference(change):
    from flashmap_amd.verify_attention import SplitKVVerify

    args = _args()
    assert SplitKVVerify()(*args, **change) is False
    assert bool((args[3] == 0).all())


def test_declines_shapes_the_kernels_do_not_take():
    from flashmap_amd.verify_attention import SplitKVVerify

    fwd = SplitKVVerify()
    args = _args()
    args[10] = False  # non-causal without a mask
    assert fwd(*args) is False
    assert fwd(*_args(dtype=torch.float16)) is False  # bf16 kernels
    assert fwd(*_args(d=96)) is False  # head_dim 64 / 128
    assert fwd(*_args(hq=6, hkv=4)) is False  # grouped heads must divide
    args = _args()
    args[12] = 4  # q does not hold bs * L tokens
    assert fwd(*args) is False


def test_qlen_mask_decline_raises():
    from flashmap_amd.verify_attention import SplitKVVerify

    fwd = SplitKVVerify()
    fwd.qlen_mask = True
    args = _args()
    args[9] = torch.ones(2 * 9, dtype=torch.bool)
    with pytest.raises(RuntimeError, match="L x L masks"):
        fwd(*args, logit_cap=30.0)


def test_signature_is_extend_attention_fwd():
    from flashmap_amd.verify_attention import SplitKVVerify

    names = list(inspect.signature(SplitKVVerify.__call__).parameters)
    assert names[:14] == ["self", "q", "k", "v", "o", "k_buffer", "v_buffer", "qo_indptr", "kv_indptr",
                          "kv_indices", "custom_mask", "is_causal", "mask_indptr", "max_len_extend"]
    assert SplitKVVerify.qlen_mask is False and SplitKVVerify.MAX_SCRATCH_BYTES == 512 << 20


def test_functional_op_refuses_cpu_tensors():
    from flashmap_amd import ops

    q, k, v, _, kb, vb, _, indptr, indices, *_ = _args()
    with pytest.raises(ValueError, match="GPU"):
        ops.verify_attention(q, k, v, kb, vb, indptr, indices)
