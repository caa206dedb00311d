"""The wrappers' host-side extent checks (flashmap_amd/ops.py): every tensor a kernel
indexes without a bounds check (per-request tensors, rotary tables, norm weights,
positions, descales, pool-writer metadata) is sized on the host before a launch, and a
short one raises ValueError instead of reaching the GPU. CPU only: the checks read
shapes, never device memory."""

import pytest
import torch

from flashmap_amd import ops


def _table(rows=10, pairs=64):
    return torch.zeros(rows, pairs, 2)


def test_rope_tables_know_their_pairs():
    assert ops.rope_from_table(_table(10, 64)).pairs == 64
    assert ops.rope_from_split(torch.zeros(10, 32), torch.zeros(10, 32)).pairs == 32
    assert ops.rope_from_cat(torch.zeros(10, 128)).pairs == 64
    ops.rope_from_table(_table(10, 64)).check(128)
    with pytest.raises(ValueError, match="head_dim 64"):
        ops.rope_from_table(_table(10, 64)).check(64)  # more pairs than the head has
    with pytest.raises(ValueError, match="head_dim 128"):
        ops.rope_from_cat(torch.zeros(10, 64)).check(128)  # too few
    with pytest.raises(ValueError, match="0 rows"):
        ops.rope_from_table(_table(0, 64)).check(128)  # empty: no row to clamp to
    with pytest.raises(ValueError, match="share one shape"):
        ops.rope_from_split(torch.zeros(10, 64), torch.zeros(9, 64))


def test_prologue_extents():
    rope = ops.rope_from_table(_table(100, 64))
    ops.Prologue(torch.ones(128), rope, torch.zeros(48, dtype=torch.int64), 1e-6).check(48, 128)
    ops.Prologue(torch.ones(128), rope, None, 1e-6).check(48, 128)
    with pytest.raises(ValueError, match="weight"):
        ops.Prologue(torch.ones(64), rope, None, 1e-6).check(48, 128)
    with pytest.raises(ValueError, match="positions has 47 rows"):
        ops.Prologue(torch.ones(128), rope, torch.zeros(47, dtype=torch.int64), 1e-6).check(48, 128)
    assert ops._prologue_args(None, 48, 128) is ops._NO_PROLOGUE


def test_request_extents():
    table = torch.zeros(4, 10, dtype=torch.int32)
    cu = torch.arange(0, 5 * 16, 16, dtype=torch.int32)
    ops._check_requests(4, cu, 64, 16, table, "block_table", torch.zeros(10, dtype=torch.int32))
    ops._check_requests(4, None, 64, 16, table, "block_table", None)
    with pytest.raises(ValueError, match="cu_seqlens_q has 4 rows"):
        ops._check_requests(4, cu[:4], 64, 16, table, "block_table", None)
    with pytest.raises(ValueError, match="batch x max_seqlen_q = 64"):
        ops._check_requests(4, None, 63, 16, table, "block_table", None)
    with pytest.raises(ValueError, match="block_table has 3 rows"):
        ops._check_requests(4, cu, 64, 16, table[:3], "block_table", None)
    with pytest.raises(ValueError, match="must be \\(requests, columns\\)"):
        ops._check_requests(4, cu, 64, 16, table.view(-1), "block_table", None)
    with pytest.raises(ValueError, match="plan has 9 rows"):
        ops._check_requests(4, cu, 64, 16, table, "block_table", torch.zeros(9, dtype=torch.int32))


def test_descale_extents():
    full = torch.ones(3)[:, None, None].expand(3, 5, 8)
    assert ops._descale_args(full, 5, 8)[0] == full.data_ptr()
    assert ops._descale_args(None, 5, 8) == [None, 0, 0, 0]
    for bad in (torch.ones(2, 5, 8), torch.ones(3, 4, 8), torch.ones(3, 5, 7), torch.ones(3, 40)):
        with pytest.raises(ValueError, match="descales"):
            ops._descale_args(bad, 5, 8)


def test_pool_writer_extents():
    rope = ops.rope_from_cat(torch.zeros(100, 128))
    meta = torch.zeros(2, 4, dtype=torch.int64)
    w = torch.ones(2, 128)
    pos, locs = torch.zeros(12, dtype=torch.int64), torch.zeros(3, 4, dtype=torch.int64)
    ops._check_pool_write(meta, w, rope, pos, locs, 2, 128, 12, torch.zeros(3, dtype=torch.int32), 4)
    ops._check_pool_write(meta, w, rope, pos, locs, 2, 128, 12, None, None)
    bad = [
        (dict(meta=torch.zeros(2, 3, dtype=torch.int64)), "meta must be"),
        (dict(meta=meta[:1]), "meta has 1 rows"),
        (dict(w=w[:1]), "k_norm_weights holds 128"),
        (dict(pos=pos[:11]), "positions holds 11"),
        (dict(locs=locs[:2]), "locs holds 8"),
        (dict(commit=torch.zeros(2, dtype=torch.int32)), "commit_lens holds 2"),
        (dict(width=None), "needs locs_row_width"),
    ]
    for change, message in bad:
        args = dict(meta=meta, w=w, pos=pos, locs=locs, commit=torch.zeros(3, dtype=torch.int32), width=4)
        args.update(change)
        with pytest.raises(ValueError, match=message):
            ops._check_pool_write(args["meta"], args["w"], rope, args["pos"], args["locs"], 2, 128, 12,
                                  args["commit"], args["width"])


def test_need_helpers():
    ops._need_rows(None, 5, "x")
    ops._need_numel(None, 5, "x")
    with pytest.raises(ValueError, match="x has 0 rows"):
        ops._need_rows(torch.tensor(3), 1, "x")
    with pytest.raises(ValueError, match="x holds 4 values"):
        ops._need_numel(torch.zeros(2, 2), 5, "x")
