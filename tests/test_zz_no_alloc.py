"""fm_block_attn_paged_static, the attention entry point that allocates nothing (its
split-KV scratch is the library's static per-GPU array), against fm_block_attn_paged on
the same inputs: identical bits, since both run the same kernels on the same grid. Two
calls in a row, the second with a smaller batch (the array keeps the first call's
contents), with the query prologue and with the step plan; and a call whose scratch would
not fit the array fails with FM_ERR_WORKSPACE before anything is launched."""

import pytest
import torch

from _inputs import check_close, paged_layout
from oracle import attention as ref

pytestmark = pytest.mark.gpu

D, PAGE, K_ROWS = 128, 16, 16


def _case(dev, batch, hq, hkv, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    bt, total = paged_layout(lens.tolist(), PAGE, g)
    cache = torch.randn(total, hkv, PAGE, 2 * D, generator=g).bfloat16()
    q = torch.randn(batch * K_ROWS, hq, D, generator=g).bfloat16()
    table = ref.rope_table(hi + K_ROWS + 1, D, 1e6)
    pos = torch.cat([int(n) + torch.arange(K_ROWS) for n in lens])
    cu = torch.arange(batch + 1, dtype=torch.int32) * K_ROWS
    return dict(lens=lens, bt=bt, cache=cache, q=q, table=table, pos=pos, cu=cu, hi=hi)


def _both(dev, c, with_plan):
    from flashmap_amd import ops

    w = torch.ones(D, device=dev)
    pro = ops.Prologue(w, ops.rope_from_table(c["table"].to(dev)), c["pos"].to(dev), 1e-6)
    lens = c["lens"].to(dev, torch.int32)
    args = (c["q"].to(dev), c["cache"].to(dev), c["cu"].to(dev), lens, c["bt"].to(dev), K_ROWS, c["hi"], D ** -0.5)
    plan = ops.attention_plan(lens) if with_plan else None
    want = ops.block_attention_paged(*args, prologue=pro, plan=plan)
    out = torch.full_like(want, float("nan"))
    got = ops.block_attention_paged_static(*args, prologue=pro, plan=plan, out=out)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    return got, want


def test_static_scratch_matches_workspace_call_twice(dev):
    print("static scratch: C3-like batch 64, then batch 5", flush=True)
    big = _case(dev, 64, 32, 8, 256, 8192, 3)
    got, want = _both(dev, big, with_plan=True)
    assert torch.equal(got, want)
    b = 7  # one sequence against the oracle
    n = int(big["lens"][b])
    k, v = ref.gather_vllm(big["cache"], big["bt"], n, b)
    qn = ref.rms_norm_rope_vllm(big["q"][b * K_ROWS:(b + 1) * K_ROWS], torch.ones(D), big["table"],
                                big["pos"][b * K_ROWS:(b + 1) * K_ROWS], 1e-6)
    check_close(got[b * K_ROWS:(b + 1) * K_ROWS].cpu(), ref.attention(qn.float().transpose(0, 1), k, v).transpose(0, 1))
    small = _case(dev, 5, 32, 8, 1, 700, 4)  # smaller input, the array still holds the first call's data
    got, want = _both(dev, small, with_plan=False)
    assert torch.equal(got, want)


def test_static_scratch_too_small_raises(dev):
    from flashmap_amd import _native, ops

    limit = _native.lib().fm_static_scratch_bytes()
    assert limit == 32 << 20
    batch, hq, hkv = 600, 32, 8  # 4800 units of 64 rows: ~90 MB of partials
    lens = torch.full((batch,), 64, dtype=torch.int32, device=dev)
    bt = torch.arange(batch * 4, dtype=torch.int32, device=dev).view(batch, 4)
    cache = torch.zeros(batch * 4, hkv, PAGE, 2 * D, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(batch * K_ROWS, hq, D, dtype=torch.bfloat16, device=dev)
    cu = torch.arange(batch + 1, dtype=torch.int32, device=dev) * K_ROWS
    out = torch.zeros_like(q)
    with pytest.raises(_native.NativeError, match="static scratch") as e:
        ops.block_attention_paged_static(q, cache, cu, lens, bt, K_ROWS, 64, D ** -0.5, out=out)
    assert e.value.code == _native.FM_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert (out == 0).all()  # nothing was launched


_CAPTURED_FIRST_CALL = r"""
import sys
import torch
sys.path.insert(0, sys.argv[1])
from flashmap_amd import ops
from oracle import attention as ref

dev = torch.device("cuda", 0)
g = torch.Generator().manual_seed(8)
D, PAGE, K = 128, 16, 16
lens = torch.randint(100, 3000, (9,), generator=g)
pages = [(int(n) + PAGE - 1) // PAGE for n in lens]
perm = torch.randperm(sum(pages), generator=g)
bt = torch.zeros(9, max(pages), dtype=torch.int32)
o = 0
for b, n in enumerate(pages):
    bt[b, :n] = perm[o:o + n].int()
    o += n
cache = torch.randn(sum(pages), 8, PAGE, 2 * D, generator=g).bfloat16().to(dev)
q = torch.randn(9 * K, 32, D, generator=g).bfloat16().to(dev)
pos = torch.cat([int(n) + torch.arange(K) for n in lens]).to(dev)
pro = ops.Prologue(torch.ones(D, device=dev), ops.rope_from_table(ref.rope_table(3100, D, 1e6).to(dev)), pos, 1e-6)
cu = (torch.arange(10, dtype=torch.int32) * K).to(dev)
lens_d, bt_d = lens.to(dev, torch.int32), bt.to(dev)
args = (q, cache, cu, lens_d, bt_d, K, 3000, D ** -0.5)
out = torch.zeros_like(q)
ops.static_scratch_init()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first static call
    ops.block_attention_paged_static(*args, prologue=pro, out=out)
want = ops.block_attention_paged(*args, prologue=pro)
for i in range(3):
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {i} differs from the workspace call"
    q.mul_(-1.0)  # new queries between replays (eager work), the same shapes
    want = ops.block_attention_paged(*args, prologue=pro)
    torch.cuda.synchronize()
print("captured first call ok", flush=True)
"""


def test_static_first_call_under_capture(dev):
    """A fresh process whose first fm_block_attn_paged_static call is captured into a HIP
    graph (after fm_static_scratch_init): every replay equals the workspace call."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    print("static scratch: first call under graph capture, fresh process", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CAPTURED_FIRST_CALL, root], capture_output=True, text=True,
                          timeout=110)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "captured first call ok" in proc.stdout
