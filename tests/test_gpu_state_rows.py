"""The several-jump draft's state kernels (fm_state_embed_rows, fm_state_update;
flashmap/vllm/model.py:944-956 and 1031-1036) against the same formulas in float64 on
the CPU: the posterior softmax(evidence * state) and the state rounded to bf16, every
element within one bf16 ulp of the correctly rounded float64 value (and almost all equal
to it); the updated state ((1 - end) state + (end - start) softmax(logits)) / (1 - start)
within 1e-5 relative of the float64 value (the sum of up to 151936 exponentials in
float32). Row widths with a tail (not a multiple
of 4), the 151936-token vocabulary, strided rows, and the wrappers' checks."""

import pytest
import torch

from _inputs import gen
from flashmap_amd import ops

pytestmark = pytest.mark.gpu


def _bf16_ulps(got, want64):
    """|got - want| in units of the bf16 ulp at want (float64 reference)."""
    w = want64.float()
    ulp = torch.where(w == 0, torch.full_like(w, 2.0 ** -133),
                      2.0 ** (torch.floor(torch.log2(w.abs().clamp_min(1e-38))) - 7))
    return ((got.double() - want64).abs() / ulp.double())


def _state(rows, vocab, g, scale=3.0):
    return (scale * torch.randn(rows, vocab, generator=g)).float()


def _rows(x, dev):
    """x on the device in rows padded to a multiple of 4 values (the kernels' layout)."""
    buf = torch.zeros(x.shape[0], -(-x.shape[1] // 4) * 4, dtype=x.dtype, device=dev)
    return buf[:, :x.shape[1]].copy_(x)


@pytest.mark.parametrize("rows,vocab,evidence", [(3, 200, 0.0), (17, 1003, 1.7), (64, 4096, 0.4),
                                                 (16, 151936, 2.5)])
def test_state_embed_rows(dev, rows, vocab, evidence):
    print(f"state_embed_rows rows={rows} vocab={vocab} evidence={evidence}", flush=True)
    g = gen(rows + vocab)
    state = _state(rows, vocab, g)
    got = ops.state_embed_rows(_rows(state, dev), evidence).cpu()
    post64 = torch.softmax(state.double() * evidence, dim=-1)
    ulps = _bf16_ulps(got[:rows], post64)
    exact = float((got[:rows].double() == post64.bfloat16().double()).float().mean())
    print(f"  posterior: max {float(ulps.max()):.3f} bf16 ulps, {exact:.4f} equal to the rounded float64", flush=True)
    assert float(ulps.max()) <= 1.0 and exact >= 0.99
    assert torch.equal(got[rows:], state.bfloat16()), "the state rows are the state rounded to bf16"
    assert torch.allclose(got[:rows].double().sum(-1), torch.ones(rows, dtype=torch.float64), atol=0.02)
    alone = ops.state_embed_rows(_rows(state, dev), evidence, posterior=False).cpu()
    assert torch.equal(alone, state.bfloat16()), "posterior=False: the state rows alone"


@pytest.mark.parametrize("rows,vocab,start,end", [(3, 200, 0.0, 0.5), (17, 1003, 0.25, 0.75),
                                                  (64, 4096, 0.5, 1.0), (16, 151936, 0.1, 0.6)])
def test_state_update(dev, rows, vocab, start, end):
    print(f"state_update rows={rows} vocab={vocab} start={start} end={end}", flush=True)
    g = gen(7 * rows + vocab)
    state = torch.softmax(_state(rows, vocab, g), dim=-1)  # a distribution, as between jumps
    logits = (2 * torch.randn(rows, vocab, generator=g)).bfloat16()
    s_dev = _rows(state, dev)
    out = ops.state_update(s_dev, logits.to(dev), start, end)
    assert out.data_ptr() == s_dev.data_ptr(), "in place"
    want = ((1.0 - end) * state.double() + (end - start) * torch.softmax(logits.double(), -1)) / (1.0 - start)
    rel = ((out.cpu().double() - want).abs() / want.abs().clamp_min(1e-30))
    print(f"  max relative error {float(rel.max()):.3e}", flush=True)
    # float32 with the sum of up to 151936 exponentials in another order: ~1e-6 typical
    assert float(rel.max()) <= 1e-5
    assert torch.allclose(out.cpu().double().sum(-1), torch.ones(rows, dtype=torch.float64), atol=1e-4)


def test_state_kernels_strided_rows(dev):
    """Rows inside a wider buffer (the draft step's padded state), and the state update
    against torch's float32 expression on the same device."""
    g = gen(99)
    base = torch.zeros(8, 1008, device=dev)
    state = base[:, :1001]
    state.copy_(torch.softmax(_state(8, 1001, g), -1).to(dev))
    logits = torch.randn(8, 1001, generator=g).bfloat16().to(dev)
    want = ((1.0 - 0.8) * state + (0.8 - 0.3) * logits.float().softmax(-1)) / (1.0 - 0.3)
    ops.state_update(state, logits, 0.3, 0.8)
    assert torch.allclose(state, want, rtol=1e-6, atol=0)
    assert torch.count_nonzero(base[:, 1001:]) == 0, "the padding is left alone"
    both = ops.state_embed_rows(state, 1.0)
    assert both.shape == (16, 1001) and torch.equal(both[8:], state.bfloat16())


def test_state_wrapper_checks(dev):
    with pytest.raises(ValueError, match="float32"):
        ops.state_embed_rows(torch.zeros(2, 8, dtype=torch.bfloat16, device=dev), 1.0)
    with pytest.raises(ValueError, match="row stride"):
        ops.state_embed_rows(torch.zeros(2, 9, device=dev)[:, :5], 1.0)
    with pytest.raises(ValueError, match="jump times"):
        ops.state_update(torch.zeros(2, 8, device=dev), torch.zeros(2, 8, dtype=torch.bfloat16, device=dev), 1.0, 1.0)
    with pytest.raises(ValueError, match="logits must be bf16"):
        ops.state_update(torch.zeros(2, 8, device=dev), torch.zeros(2, 8, device=dev), 0.0, 0.5)
