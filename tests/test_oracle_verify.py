"""Pins the verify-attention oracle (oracle.attention.verify_attention /
verify_visibility, restating flashmap/sglang/verify_attention.py:35-233, 360-474)
against what the mathematics fixes: a float64 brute force over explicit (score, value)
lists, the reference's own split form (context and verify-token partials merged by
their LSE), the textbook attention it reduces to, scale and GQA identities, and the
mask layouts. Each check is chosen so that a plausible slip (k_scale on the verify
tokens, v_scale dropped, the mask transposed, context columns read, a wrong KV head)
fails one of them."""

import math

import torch

from _inputs import tree_visibility, verify_case
from oracle import attention as ref


def _brute(case, sm_scale, k_scale, v_scale):
    """float64, one (b, t, head) at a time, from explicit lists of (score, value)."""
    q, k, v = case["q"].double(), case["k"].double(), case["v"].double()
    kb, vb = case["key_buffer"].double(), case["value_buffer"].double()
    indptr, indices = case["kv_indptr"].tolist(), case["kv_indices"].tolist()
    bs = len(indptr) - 1
    tokens, hq, d = q.shape
    length, hkv = tokens // bs, kb.shape[1]
    mask = None if case["custom_mask"] is None else case["custom_mask"].tolist()
    out = torch.zeros(tokens, hq, d, dtype=torch.float64)
    for b in range(bs):
        ctx = indptr[b + 1] - indptr[b]
        for t in range(length):
            for h in range(hq):
                kh = h * hkv // hq
                qr = q[b * length + t, h]
                pairs = []
                for p in range(ctx):
                    slot = indices[indptr[b] + p]
                    pairs.append((float(qr @ kb[slot, kh]) * sm_scale * k_scale, vb[slot, kh] * v_scale))
                for j in range(length):
                    if mask is None:
                        seen = j <= t
                    elif case["qlen_mask"]:
                        seen = bool(mask[b * length * length + t * length + j])
                    else:
                        seen = bool(mask[int(case["mask_indptr"][b]) + t * (ctx + length) + ctx + j])
                    if seen:
                        pairs.append((float(qr @ k[b * length + j, kh]) * sm_scale, v[b * length + j, kh]))
                if not pairs:
                    continue
                m = max(s for s, _ in pairs)
                w = [math.exp(s - m) for s, _ in pairs]
                out[b * length + t, h] = sum(wi * x for wi, (_, x) in zip(w, pairs)) / sum(w)
    return out


def _oracle(case, **kw):
    return ref.verify_attention(case["q"], case["k"], case["v"], case["key_buffer"], case["value_buffer"],
                                case["kv_indptr"], case["kv_indices"], case["custom_mask"], case["mask_indptr"],
                                case["qlen_mask"], **kw)


def test_float64_brute_force_tree_rows_layout():
    case = verify_case(3, 4, 4, 2, 8, [5, 0, 3], mask="rows", seed=1, dtype=torch.float32)
    got = _oracle(case, sm_scale=0.4, k_scale=0.7, v_scale=1.3)
    want = _brute(case, 0.4, 0.7, 1.3)
    assert torch.allclose(got.double(), want, atol=1e-5, rtol=1e-5)


def test_float64_brute_force_causal_and_qlen():
    for mask in ("causal", "qlen"):
        case = verify_case(2, 5, 6, 3, 16, [7, 2], mask=mask, seed=2, dtype=torch.float32)
        got = _oracle(case, sm_scale=0.25)
        want = _brute(case, 0.25, 1.0, 1.0)
        assert torch.allclose(got.double(), want, atol=1e-5, rtol=1e-5), mask


def test_equals_reference_split_form():
    """The reference's structure: a context partial (scores * sm_scale * k_scale, values
    * v_scale) and a verify-token partial per row, each (out, lse), merged by LSE."""
    case = verify_case(2, 6, 4, 2, 16, [9, 4], mask="qlen", seed=3, dtype=torch.float32)
    sm, ks, vs = 0.3, 0.8, 1.7
    got = _oracle(case, sm_scale=sm, k_scale=ks, v_scale=vs)
    q, k, v = case["q"], case["k"], case["v"]
    kb, vb = case["key_buffer"], case["value_buffer"]
    ip, idx = case["kv_indptr"], case["kv_indices"].long()
    length = 6
    for b in range(2):
        rows = idx[int(ip[b]):int(ip[b + 1])]
        vis = case["custom_mask"][b * 36:(b + 1) * 36].reshape(6, 6)
        for t in range(length):
            qr = q[b * length + t][:, None]  # (Hq, 1, D)
            oc, lc = ref.attention_lse(qr, kb[rows].transpose(0, 1) * ks, vb[rows].transpose(0, 1) * vs, sm)
            j = vis[t].nonzero().flatten() + b * length
            ot, lt = ref.attention_lse(qr, k[j].transpose(0, 1), v[j].transpose(0, 1), sm)
            want = ref.lse_merge([oc, ot], [lc, lt])[:, 0]
            assert torch.allclose(got[b * length + t], want, atol=1e-5), (b, t)


def test_single_token_causal_is_attention_onto_context_plus_token():
    case = verify_case(2, 1, 8, 2, 32, [11, 6], seed=4, dtype=torch.float32)
    got = _oracle(case)
    ip, idx = case["kv_indptr"], case["kv_indices"].long()
    for b in range(2):
        rows = idx[int(ip[b]):int(ip[b + 1])]
        keys = torch.cat([case["key_buffer"][rows], case["k"][b:b + 1]]).transpose(0, 1)
        vals = torch.cat([case["value_buffer"][rows], case["v"][b:b + 1]]).transpose(0, 1)
        want = ref.attention(case["q"][b][:, None], keys, vals)[:, 0]
        assert torch.allclose(got[b], want, atol=1e-5)


def test_scales_equal_prescaled_pool():
    case = verify_case(2, 3, 4, 4, 16, [8, 5], seed=5, dtype=torch.float64)
    got = _oracle(case, k_scale=0.6, v_scale=2.5)
    scaled = dict(case, key_buffer=case["key_buffer"] * 0.6, value_buffer=case["value_buffer"] * 2.5)
    want = _oracle(scaled)
    assert torch.allclose(got, want, atol=1e-6)
    # and the scales touch the context only: with no context they change nothing
    empty = verify_case(2, 3, 4, 4, 16, [0, 0], seed=5, dtype=torch.float64)
    assert torch.allclose(_oracle(empty, k_scale=0.6, v_scale=2.5), _oracle(empty), atol=1e-6)


def test_gqa_equals_mha_on_repeated_kv():
    case = verify_case(2, 4, 8, 2, 16, [6, 3], mask="qlen", seed=6, dtype=torch.float32)
    got = _oracle(case)
    rep = dict(case, k=case["k"].repeat_interleave(4, 1), v=case["v"].repeat_interleave(4, 1),
               key_buffer=case["key_buffer"].repeat_interleave(4, 1),
               value_buffer=case["value_buffer"].repeat_interleave(4, 1))
    assert torch.allclose(got, _oracle(rep), atol=1e-5)


def test_mask_layouts_agree_and_context_columns_are_ignored():
    g = torch.Generator().manual_seed(7)
    causal = verify_case(3, 5, 4, 2, 16, [4, 0, 9], seed=8, dtype=torch.float32)
    tril = torch.ones(5, 5, dtype=torch.bool).tril()
    qlen = dict(causal, custom_mask=tril.reshape(-1).repeat(3), qlen_mask=True)
    rows, starts = [], [0]
    for ctx in (4, 0, 9):
        junk = torch.randint(0, 2, (5, ctx), generator=g).bool()
        rows.append(torch.cat([junk, tril], 1).reshape(-1))
        starts.append(starts[-1] + 5 * (ctx + 5))
    full = dict(causal, custom_mask=torch.cat(rows), mask_indptr=torch.tensor(starts))
    want = _oracle(causal)
    assert torch.allclose(_oracle(qlen), want, atol=0)
    assert torch.allclose(_oracle(full), want, atol=0)


def test_row_that_sees_nothing_is_zero_and_context_only_otherwise():
    case = verify_case(2, 3, 4, 2, 16, [0, 6], mask="qlen", seed=9, dtype=torch.float32)
    mask = case["custom_mask"].clone()
    mask[0:3] = False  # request 0, token 0 sees no token (and has no context)
    mask[9 + 3:9 + 6] = False  # request 1, token 1 sees only its context
    case = dict(case, custom_mask=mask)
    got = _oracle(case)
    assert torch.count_nonzero(got[0]) == 0
    rows = case["kv_indices"].long()[0:6]
    want = ref.attention(case["q"][4][:, None], case["key_buffer"][rows].transpose(0, 1),
                         case["value_buffer"][rows].transpose(0, 1))[:, 0]
    assert torch.allclose(got[4], want, atol=1e-5)


def test_tree_visibility_is_ancestors():
    g = torch.Generator().manual_seed(10)
    vis = tree_visibility(12, g)
    assert vis.diagonal().all() and vis[:, 0].all()  # every node sees itself and the root
    assert not vis.triu(1).any()  # parents precede children
    for j in range(1, 12):  # exactly one parent: the deepest proper ancestor
        anc = vis[j].nonzero().flatten().tolist()
        parent = anc[-2]
        assert vis[parent].nonzero().flatten().tolist() == anc[:-1]
