"""GPU parity of the draft step's token selection and noise (csrc/sampling.hip) through
the C ABI, against the CPU oracle (oracle/sampling.py):

- argmax per row: exact (int64 indices) for bf16 / fp16 / fp32 logits, ties to the first
  index, all -inf rows, NaN rows, strided rows, vocabularies that end mid-chunk or on a
  whole number of tiles, a 151936-entry vocabulary;
- the fused sampler: greedy rows exact; sampled rows equal the oracle's tokens wherever
  the oracle's winning key beats the runner-up by more than 1e-4 (the random words are
  exact, the logs may differ in the last ulp); int32 offset wraparound past 2^31;
- seeded normals: within 2e-5 (relative, at least 1 absolute unit) of the oracle, for
  int32 and int64 rows / positions, unseeded rows, seeds with high words.
"""

import numpy as np
import pytest
import torch

from _inputs import gen
from flashmap_amd import ops
from oracle import sampling as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,vocab,stride", [(1, 1, 1), (3, 100, 100), (17, 8193, 8200), (5, 24581, 24581),
                                               (3, 32768, 32768), (64, 151936, 151936)])
def test_argmax_rows(dev, dtype, rows, vocab, stride):
    g = gen(rows + vocab)
    x = torch.randn(rows, stride, generator=g).to(dtype)[:, :vocab]
    if vocab > 10:  # planted ties: the row max at three places, the first must win
        m = x.float().max(dim=1).values + 1
        for r in range(rows):
            cols = torch.randperm(vocab, generator=g)[:3]
            x[r, cols] = m[r].to(dtype)
    got = ops.argmax_rows(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.from_numpy(S.argmax_first(x.float().numpy())))
    assert torch.equal(got.cpu(), x.float().argmax(dim=1))


def test_argmax_special_rows(dev):
    x = torch.randn(4, 20000).bfloat16()
    x[0] = -float("inf")
    x[1, 777] = float("nan")
    x[1, 19999] = float("nan")
    x[2] = 0
    x[3, 12345] = float("inf")
    got = ops.argmax_rows(x.to(dev)).cpu()
    assert got.tolist() == [0, 777, 0, 12345]


def test_sample_rows(dev):
    g = gen(5)
    rows, vocab = 40, 50000
    x = (torch.randn(rows, vocab, generator=g) * 3).bfloat16()
    temps = torch.rand(rows, generator=g) + 0.3
    greedy = torch.zeros(rows, dtype=torch.bool)
    greedy[::3] = True
    seed = torch.tensor(0x1234_5678_9ABC, dtype=torch.int64)
    got = ops.sample_rows(x.to(dev), temps.to(dev), greedy.to(dev), seed.to(dev)).cpu().numpy()
    keys = S.sample_keys(x.float().numpy(), temps.numpy(), greedy.numpy(), int(seed))
    want = S.argmax_first(keys)
    gr = greedy.numpy()
    assert (got[gr] == want[gr]).all()
    top2 = np.sort(keys[~gr], axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-4
    assert clear.sum() >= (~gr).sum() - 2
    assert (got[~gr][clear] == want[~gr][clear]).all()
    # the sampled rows are not the argmax (noise applied) for most rows
    assert (got[~gr] != x.float().argmax(1).numpy()[~gr]).mean() > 0.5


def test_sample_rows_offsets_wrap_past_int32(dev):
    """row * V + col passes 2^31 for the last rows: int32 arithmetic, as the reference's."""
    rows, vocab = 300, 7_300_000
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(rows, vocab, generator=g, device=dev, dtype=torch.bfloat16)
    temps = torch.ones(rows)
    greedy = torch.zeros(rows, dtype=torch.bool)
    seed = torch.tensor(77, dtype=torch.int64)
    got = ops.sample_rows(x, temps.to(dev), greedy.to(dev), seed.to(dev)).cpu().numpy()
    row0 = rows - 3
    assert row0 * vocab > 2 ** 31
    tail = x[row0:].float().cpu().numpy()
    del x
    keys = S.sample_keys(tail, temps[row0:].numpy(), greedy[row0:].numpy(), 77, row0=row0)
    top2 = np.sort(keys, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-4
    assert (got[row0:][clear] == S.argmax_first(keys)[clear]).all()


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_seeded_normal(dev, idx_dtype):
    g = gen(7)
    seeds = torch.tensor([3, (1 << 40) + 7, -5, 123456789012345], dtype=torch.int64)
    rows = torch.tensor([0, 1, -1, 2, 3, 3, -2, 1], dtype=idx_dtype)
    pos = torch.randint(0, 10000, (8,), generator=g).to(idx_dtype)
    n_cols = 3000
    got = ops.seeded_normal(seeds.to(dev), rows.to(dev), pos.to(dev), n_cols, 0.7).cpu().numpy()
    want = S.seeded_normal(seeds.numpy(), rows.numpy(), pos.numpy(), n_cols, 0.7)
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert err.max() < 2e-5


def test_plugin_entry_points(dev):
    from flashmap_amd import sglang as fs
    from flashmap_amd import vllm as fv

    x = torch.randn(6, 1000).float().to(dev)
    assert torch.equal(fv.split_argmax(x), x.argmax(dim=1))
    seed = torch.tensor(9, dtype=torch.int64, device=dev)
    t = torch.ones(6, device=dev)
    greedy = torch.ones(6, dtype=torch.bool, device=dev)
    assert torch.equal(fs.sample_rows(x, t, greedy, seed), x.argmax(dim=1))
    z = fv.seeded_normal(torch.tensor([1, 2], device=dev), torch.tensor([0, 1], device=dev),
                         torch.tensor([5, 6], device=dev), 10, 2.0)
    assert z.shape == (2, 10) and z.dtype == torch.float32
