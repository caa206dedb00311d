"""Torch-facing wrappers of the gfx950 kernels (``include/flashmap_amd.h``).

Every function takes CUDA (ROCm) tensors, checks the contract the kernels rely on
(dtype, alignment, strides), and enqueues the kernel on torch's current stream. The
wrappers allocate only their outputs and, outside graph capture, the persistent
split-KV workspace. There is no other code path: without the built library every
call raises.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _native
from ._native import call

__all__ = [
    "Rope",
    "adaln_residual",
    "noise_rows",
    "argmax_rows",
    "attention_plan",
    "block_attention_contig",
    "block_attention_paged",
    "block_attention_paged_fp8",
    "block_attention_paged_runs",
    "block_attention_token_paged",
    "block_attention_token_paged_fp8",
    "block_self_attention",
    "rms_norm_rope",
    "rope_from_cat",
    "rope_from_split",
    "rope_from_table",
    "sample_rows",
    "seeded_normal",
    "verify_attention",
    "verify_workspace_bytes",
    "workspace_for",
    "write_context_kv",
    "write_context_kv_fp8",
    "write_context_kv_pool",
    "write_context_kv_pool_fp8",
]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_cuda(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"flashmap_amd kernels run on the GPU; got a tensor on {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    return device


def _bf16_rows(x: torch.Tensor, name: str) -> torch.Tensor:
    """``x`` as bf16 with unit channel stride, 16-byte aligned rows (copied if needed)."""
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    ok = x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in x.stride()[:-1])
    return x if ok else x.contiguous()


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.float32 and t.is_contiguous()) else t.float().contiguous()


def _i64(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int64 and t.is_contiguous()) else t.to(torch.int64).contiguous()


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int32 and t.is_contiguous()) else t.to(torch.int32).contiguous()


def _need_rows(t: torch.Tensor | None, n: int, what: str) -> None:
    """Raise unless ``t`` has at least ``n`` entries along its first dimension: the
    kernels index it that far without bounds checks."""
    have = None if t is None else (t.shape[0] if t.dim() else 0)
    if have is not None and have < n:
        raise ValueError(f"{what} has {have} rows; the call reads {n}")


def _need_numel(t: torch.Tensor | None, n: int, what: str) -> None:
    """Raise unless ``t`` holds at least ``n`` values (read flat by the kernels)."""
    if t is not None and t.numel() < n:
        raise ValueError(f"{what} holds {t.numel()} values; the call reads {n}")


# ---------------------------------------------------------------------------- rope


@dataclass(frozen=True)
class Rope:
    """A float32 rotary table as the kernels read it: cos/sin of pair ``i`` at row ``r``
    are ``cos[r * row_stride + i * pair_stride]`` (same for ``sin``)."""

    cos: torch.Tensor
    sin_ptr: int
    row_stride: int
    pair_stride: int
    rows: int
    pairs: int
    keep: tuple = ()

    def args(self) -> list:
        return [self.cos.data_ptr(), self.sin_ptr, self.row_stride, self.pair_stride, self.rows]

    def check(self, head_dim: int) -> None:
        """The kernels read pairs ``[0, head_dim / 2)`` of rows ``[0, rows)`` (positions
        are clamped to the rows)."""
        if 2 * self.pairs != head_dim or self.rows < 1:
            raise ValueError(f"rotary table of {self.rows} rows x {self.pairs} pairs does not serve "
                             f"head_dim {head_dim}")


def rope_from_table(cos_sin: torch.Tensor) -> Rope:
    """vLLM's ``rope_table`` / SGLang's ``rope_freqs``: ``(..., D/2, 2)`` float32 with
    (cos, sin) interleaved per pair (flashmap/vllm/kernels.py:26-33,
    flashmap/sglang/model.py:116-123). Rows are the leading dims flattened."""
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.shape[-1] != 2:
        raise ValueError("rotary table must be contiguous float32 (..., head_dim/2, 2)")
    half = cos_sin.shape[-2] if cos_sin.dim() >= 2 else 0
    rows = cos_sin.numel() // (2 * half) if half else 0
    return Rope(cos_sin, cos_sin.data_ptr() + 4, 2 * half, 2, rows, half, (cos_sin,))


def rope_from_split(cos: torch.Tensor, sin: torch.Tensor) -> Rope:
    """transformers' ``rope_tables``: separate ``cos`` and ``sin`` ``(..., D/2)``
    (flashmap/modeling_flashmap.py:53-58)."""
    if cos.shape != sin.shape or cos.dim() == 0:
        raise ValueError(f"cos and sin tables must share one shape (..., head_dim/2), got "
                         f"{tuple(cos.shape)} and {tuple(sin.shape)}")
    cos, sin = _f32(cos), _f32(sin)
    half = cos.shape[-1]
    return Rope(cos, sin.data_ptr(), half, 1, cos.numel() // half if half else 0, half, (cos, sin))


def rope_from_cat(table: torch.Tensor) -> Rope:
    """SGLang's writer table ``(P, D)`` = ``[cos(D/2) | sin(D/2)]`` per row
    (flashmap/sglang/model.py:814-817)."""
    if table.dtype != torch.float32 or not table.is_contiguous() or table.dim() == 0:
        raise ValueError("rotary table must be contiguous float32 (P, head_dim)")
    d = table.shape[-1]
    return Rope(table, table.data_ptr() + 4 * (d // 2), d, 1, table.numel() // d if d else 0, d // 2, (table,))


# ------------------------------------------------------------------------ prologue


def rms_norm_rope(
    x: torch.Tensor,
    weight: torch.Tensor,
    rope: Rope,
    positions: torch.Tensor | None,
    eps: float,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """QK-RMSNorm + interleaved RoPE of ``x (tokens, heads, head_dim)`` bf16: the rope
    row of token ``t`` is ``positions[t]`` (or ``t`` without positions)."""
    if x.dim() != 3:
        raise ValueError(f"x must be (tokens, heads, head_dim), got {tuple(x.shape)}")
    _check_cuda(x, weight, rope.cos, positions)
    x = _bf16_rows(x, "x")
    tokens, heads, head_dim = x.shape
    rope.check(head_dim)
    _need_numel(weight, head_dim, "weight")
    _need_rows(positions, tokens, "positions")
    if out is None:
        out = torch.empty((tokens, heads, head_dim), dtype=torch.bfloat16, device=x.device)
    if tokens == 0:
        return out
    weight = _f32(weight)
    pos = None if positions is None else _i64(positions)
    call(
        "fm_rms_norm_rope",
        x.data_ptr(), out.data_ptr(), tokens, heads, head_dim,
        x.stride(0), x.stride(1), out.stride(0), out.stride(1),
        weight.data_ptr(), *rope.args(), _ptr(pos), float(eps), _stream(x),
    )
    return out


# ----------------------------------------------------------------------- attention


class _WorkspacePool:
    """One persistent split-KV workspace per device, grown outside graph capture.
    A replaced buffer is kept alive, since captured graphs may still point at it.
    Every call on the device uses it: calls on one stream are ordered, calls on two
    streams that may overlap in time would race on it."""

    def __init__(self):
        self.buffers: dict[torch.device, torch.Tensor] = {}
        self.retired: list[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        buf = self.buffers.get(device)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"the attention workspace ({nbytes} bytes) must grow outside graph capture: "
                    "run the call once (warm-up) before capturing"
                )
            if buf is not None:
                self.retired.append(buf)
            size = max(nbytes, 1 << 20)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self.buffers[device] = buf
        return buf


_WORKSPACES = _WorkspacePool()
_WS_BYTES: dict[tuple, int] = {}


def workspace_for(batch: int, max_seqlen_q: int, hq: int, hkv: int, head_dim: int, max_seqlen_k: int,
                  device: torch.device) -> torch.Tensor:
    """The device's persistent workspace, large enough for an attention call of these
    sizes (fm_attn_workspace_bytes)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (batch, max_seqlen_q, hq, hkv, head_dim, max_seqlen_k, index)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_native.lib().fm_attn_workspace_bytes(batch, max_seqlen_q, hq, hkv, head_dim, max_seqlen_k, index))
        if nbytes == 0:
            raise RuntimeError(f"fm_attn_workspace_bytes failed: {_native.last_error()}")
        _WS_BYTES[key] = nbytes
    return _WORKSPACES.get(torch.device("cuda", index), nbytes)


def attention_plan(seqlens: torch.Tensor) -> torch.Tensor:
    """The split-KV plan of one step (int32 ``(2 (batch + 1),)``: the tile prefixes for
    bf16 and for e4m3 K/V), shared by every layer that attends with these context
    lengths; the analogue of FlashAttention's ``get_scheduler_metadata``
    (flashmap/vllm/model.py:967-989)."""
    _check_cuda(seqlens)
    seqlens = _i32(seqlens)
    batch = seqlens.shape[0]
    plan = torch.empty(2 * (batch + 1), dtype=torch.int32, device=seqlens.device)
    call("fm_attn_plan", seqlens.data_ptr(), batch, plan.data_ptr(), _stream(seqlens))
    return plan


@dataclass
class Prologue:
    """Fused QK-RMSNorm + RoPE of the queries inside the attention kernel."""

    weight: torch.Tensor
    rope: Rope
    positions: torch.Tensor | None
    eps: float

    def args(self) -> list:
        w = _f32(self.weight)
        self._keep = (w, None if self.positions is None else _i64(self.positions))
        return [w.data_ptr(), *self.rope.args(), _ptr(self._keep[1]), float(self.eps)]

    def check(self, tokens: int, head_dim: int) -> None:
        """Extents the kernels rely on: ``head_dim`` weights, the table's pairs, one
        position per query row."""
        self.rope.check(head_dim)
        if self.weight.numel() < head_dim:
            raise ValueError(f"q_norm weight holds {self.weight.numel()} values, head_dim is {head_dim}")
        _need_rows(self.positions, tokens, "prologue positions")


_NO_PROLOGUE = [None, None, None, 0, 0, 0, None, 0.0]


def _prologue_args(prologue: Prologue | None, tokens: int, head_dim: int) -> list:
    if prologue is None:
        return _NO_PROLOGUE
    prologue.check(tokens, head_dim)
    return prologue.args()


def _check_requests(batch: int, cu_seqlens_q: torch.Tensor | None, tokens: int, max_seqlen_q: int,
                    table: torch.Tensor, table_name: str, plan: torch.Tensor | None) -> None:
    """Extents of a call's per-request tensors (the kernels index them by request
    without bounds checks; the table's columns and the cache's pages are clamped)."""
    if cu_seqlens_q is None:
        if tokens < batch * max_seqlen_q:
            raise ValueError(f"without cu_seqlens_q the query holds batch x max_seqlen_q = "
                             f"{batch * max_seqlen_q} rows; got {tokens}")
    else:
        _need_rows(cu_seqlens_q, batch + 1, "cu_seqlens_q")
    if table.dim() != 2:
        raise ValueError(f"{table_name} must be (requests, columns), got {tuple(table.shape)}")
    _need_rows(table, batch, table_name)
    _need_rows(plan, 2 * (batch + 1), "plan")
MAX_RUNS = 8  # runs of KV heads per fm_block_attn_paged_runs call


def _q_out(query: torch.Tensor, out: torch.Tensor | None, varlen: bool):
    query = _bf16_rows(query, "query")
    if out is None:
        out = torch.empty(query.shape, dtype=torch.bfloat16, device=query.device)
    if varlen:  # (tokens, heads, D)
        qs = [0, query.stride(0), query.stride(1)]
        os_ = [0, out.stride(0), out.stride(1)]
    else:  # (batch, q_len, heads, D)
        qs = [query.stride(0), query.stride(1), query.stride(2)]
        os_ = [out.stride(0), out.stride(1), out.stride(2)]
    return query, out, qs, os_


def block_attention_contig(
    query: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    softmax_scale: float | None = None,
    seqlens_k: torch.Tensor | None = None,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Non-causal attention of ``query (B, T, Hq, D)`` onto ``keys``/``values`` ``(B, Hkv,
    L, D)`` (FlashMapCache.context views; any strides with unit channel stride).
    ``seqlens_k (B,)`` limits each sequence to its first positions (default all L)."""
    _check_cuda(query, keys, values, seqlens_k)
    batch, q_len, hq, d = query.shape
    if keys.dim() != 4 or keys.shape != values.shape or keys.shape[0] < batch or keys.shape[3] != d:
        raise ValueError(f"keys and values must both be (batch >= {batch}, kv_heads, positions, {d}); got "
                         f"{tuple(keys.shape)} and {tuple(values.shape)}")
    _need_rows(seqlens_k, batch, "seqlens_k")
    _need_rows(plan, 2 * (batch + 1), "plan")
    _, hkv, kv_len, _ = keys.shape
    keys, values = _bf16_rows(keys, "keys"), _bf16_rows(values, "values")
    query, out, qs, os_ = _q_out(query, out, varlen=False)
    if batch == 0 or q_len == 0:
        return out
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    sl = None if seqlens_k is None else _i32(seqlens_k)
    ws = workspace_for(batch, q_len, hq, hkv, d, kv_len, query.device)
    call(
        "fm_block_attn_contig",
        query.data_ptr(), *qs, out.data_ptr(), *os_, None,
        keys.data_ptr(), keys.stride(0), keys.stride(1), keys.stride(2),
        values.data_ptr(), values.stride(0), values.stride(1), values.stride(2),
        _ptr(sl), kv_len, batch, q_len, hq, hkv, d, float(scale),
        *_prologue_args(prologue, batch * q_len, d),
        _ptr(plan), ws.data_ptr(), ws.numel(), _stream(query),
    )
    return out


def block_attention_paged(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor | None,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Non-causal attention of ``query (tokens, Hq, D)`` (rows of request ``b`` from
    ``cu_seqlens_q``) onto vLLM's paged cache ``(num_blocks, Hkv, page, 2D)`` (K then V
    in every token row), each request reading its first ``seqused_k[b]`` positions
    through ``block_table`` (flashmap/vllm/model.py:93-134)."""
    prep = _paged_call(query, kv_cache, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
                       softmax_scale, prologue, plan, out)
    if prep.args is None:
        return prep.out
    ws = workspace_for(prep.batch, max_seqlen_q, prep.hq, prep.hkv, prep.d, max_seqlen_k, query.device)
    call("fm_block_attn_paged", *prep.args, ws.data_ptr(), ws.numel(), _stream(query))
    return prep.out


def static_scratch_init() -> None:
    """Sets up :func:`block_attention_paged_static` on the current device (the scratch
    array's address and the host-side caches its first call would fill); call it before
    capturing that first call into a graph."""
    call("fm_static_scratch_init")


def block_attention_paged_static(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor | None,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`block_attention_paged` through ``fm_block_attn_paged_static``: no workspace,
    the library's per-GPU static scratch instead (for callers that cannot allocate
    device memory). Pass ``out`` to allocate nothing at all. Calls that may overlap in
    time on one GPU race on the scratch; a call needing more than
    ``fm_static_scratch_bytes()`` raises."""
    prep = _paged_call(query, kv_cache, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
                       softmax_scale, prologue, plan, out)
    if prep.args is not None:
        call("fm_block_attn_paged_static", *prep.args, _stream(query))
    return prep.out


@dataclass
class _PagedCall:
    out: torch.Tensor
    args: list | None  # None: nothing to launch
    batch: int = 0
    hq: int = 0
    hkv: int = 0
    d: int = 0


def _paged_call(query, kv_cache, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k, softmax_scale,
                prologue, plan, out) -> _PagedCall:
    """Checks of a vLLM-layout call and its C arguments up to the plan (the entry points
    differ only in what follows: a workspace, or none)."""
    _check_cuda(query, kv_cache, cu_seqlens_q, seqused_k, block_table)
    if kv_cache.dtype != torch.bfloat16:
        raise TypeError(f"kv_cache must be bfloat16, got {kv_cache.dtype}")
    tokens, hq, d = query.shape
    num_blocks, hkv, page, two_d = kv_cache.shape
    if two_d != 2 * d:
        raise ValueError(f"kv_cache rows hold {two_d} values, expected 2 * {d}")
    if kv_cache.stride(-1) != 1:
        raise ValueError("kv_cache must have unit channel stride")
    batch = seqused_k.shape[0]
    _check_requests(batch, cu_seqlens_q, tokens, max_seqlen_q, block_table, "block_table", plan)
    query, out, qs, os_ = _q_out(query, out, varlen=True)
    if batch == 0 or tokens == 0:
        return _PagedCall(out, None)
    cu = None if cu_seqlens_q is None else _i32(cu_seqlens_q)
    if cu is None:
        qs[0], os_[0] = max_seqlen_q * qs[1], max_seqlen_q * os_[1]
    bt = block_table if (block_table.dtype == torch.int32 and block_table.stride(-1) == 1) else _i32(block_table)
    sk = _i32(seqused_k)
    args = [
        query.data_ptr(), *qs, out.data_ptr(), *os_, _ptr(cu),
        kv_cache.data_ptr(), num_blocks, kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), d, page,
        bt.data_ptr(), bt.stride(0), bt.shape[1], sk.data_ptr(), batch, max_seqlen_q, max_seqlen_k,
        hq, hkv, d, float(softmax_scale),
        *_prologue_args(prologue, tokens, d),
        _ptr(plan),
    ]
    # Tensors converted above (int32 copies, contiguous rows) must outlive the launch.
    prep = _PagedCall(out, args, batch, hq, hkv, d)
    prep.keep = (query, cu, bt, sk)
    return prep


def block_attention_paged_runs(
    query: torch.Tensor,
    caches: list[torch.Tensor] | tuple[torch.Tensor, ...],
    runs: list[tuple[int, int, int, int]],
    cu_seqlens_q: torch.Tensor | None,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`block_attention_paged` for a layer whose KV heads lie in runs over several
    vLLM caches of one geometry (the virtual context-cache layout,
    flashmap/vllm/context_cache.py:33-73): ``runs`` lists ``(cache, first slot, count,
    first head)`` in head order (a layer's ``ContextCachePlan.segments``), KV head
    ``first head + i`` of the run at slot ``first slot + i`` of ``caches[cache]``. One
    launch for all runs, where attend_by_segments makes one call per run and
    concatenates (flashmap/vllm/context_cache.py:120-139)."""
    if not runs:
        raise ValueError("runs must list at least one (cache, first slot, count, first head)")
    if len(runs) > MAX_RUNS:
        raise ValueError(f"at most {MAX_RUNS} runs per call, got {len(runs)}")
    c0 = caches[runs[0][0]]
    tokens, hq, d = query.shape
    num_blocks, hpc, page, two_d = c0.shape
    head = 0
    for cache_id, first_slot, count, first_head in runs:
        c = caches[cache_id]
        if c.dtype != torch.bfloat16:
            raise TypeError(f"kv caches must be bfloat16, got {c.dtype}")
        if c.device != c0.device or c.shape != c0.shape or c.stride() != c0.stride():
            raise ValueError("the runs' caches must share one device, shape and strides")
        if first_head != head or count <= 0 or first_slot < 0 or first_slot + count > hpc:
            raise ValueError(f"run {(cache_id, first_slot, count, first_head)} does not continue the heads at {head} "
                             f"within a cache of {hpc} heads")
        head += count
    hkv = head
    if two_d != 2 * d:
        raise ValueError(f"kv caches' rows hold {two_d} values, expected 2 * {d}")
    if c0.stride(-1) != 1:
        raise ValueError("kv caches must have unit channel stride")
    _check_cuda(query, c0, cu_seqlens_q, seqused_k, block_table)
    batch = seqused_k.shape[0]
    _check_requests(batch, cu_seqlens_q, tokens, max_seqlen_q, block_table, "block_table", plan)
    query, out, qs, os_ = _q_out(query, out, varlen=True)
    if batch == 0 or tokens == 0:
        return out
    cu = None if cu_seqlens_q is None else _i32(cu_seqlens_q)
    if cu is None:
        qs[0], os_[0] = max_seqlen_q * qs[1], max_seqlen_q * os_[1]
    bt = block_table if (block_table.dtype == torch.int32 and block_table.stride(-1) == 1) else _i32(block_table)
    sk = _i32(seqused_k)
    n = len(runs)
    ptrs = (ctypes.c_void_p * n)(*[caches[r[0]].data_ptr() for r in runs])
    slots = (ctypes.c_int32 * n)(*[r[1] for r in runs])
    counts = (ctypes.c_int32 * n)(*[r[2] for r in runs])
    ws = workspace_for(batch, max_seqlen_q, hq, hkv, d, max_seqlen_k, query.device)
    call(
        "fm_block_attn_paged_runs",
        query.data_ptr(), *qs, out.data_ptr(), *os_, _ptr(cu),
        ctypes.addressof(ptrs), ctypes.addressof(slots), ctypes.addressof(counts), n, hpc,
        num_blocks, c0.stride(0), c0.stride(1), c0.stride(2), d, page,
        bt.data_ptr(), bt.stride(0), bt.shape[1], sk.data_ptr(), batch, max_seqlen_q, max_seqlen_k,
        hq, hkv, d, float(softmax_scale),
        *_prologue_args(prologue, tokens, d),
        _ptr(plan), ws.data_ptr(), ws.numel(), _stream(query),
    )
    return out


def block_attention_token_paged(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    cache_seqlens: torch.Tensor,
    page_table: torch.Tensor,
    softmax_scale: float | None = None,
    max_seqlen_k: int | None = None,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Non-causal attention of ``query (bs, q_len, Hq, D)`` onto SGLang's token pool
    ``key_buffer``/``value_buffer (pool, Hkv, D)``: request ``b`` reads pool rows
    ``page_table[b, :cache_seqlens[b]]`` (flashmap/sglang/model.py:127-146)."""
    _check_cuda(query, key_buffer, value_buffer, cache_seqlens, page_table)
    batch, q_len, hq, d = query.shape
    if key_buffer.dim() != 3 or key_buffer.shape != value_buffer.shape or key_buffer.shape[2] != d:
        raise ValueError(f"key_buffer and value_buffer must both be (pool, kv_heads, {d}); got "
                         f"{tuple(key_buffer.shape)} and {tuple(value_buffer.shape)}")
    _need_rows(cache_seqlens, batch, "cache_seqlens")
    _check_requests(batch, None, batch * q_len, q_len, page_table, "page_table", plan)
    pool, hkv, _ = key_buffer.shape
    key_buffer, value_buffer = _bf16_rows(key_buffer, "key_buffer"), _bf16_rows(value_buffer, "value_buffer")
    query, out, qs, os_ = _q_out(query, out, varlen=False)
    if batch == 0 or q_len == 0:
        return out
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    pt = page_table if (page_table.dtype == torch.int32 and page_table.stride(-1) == 1) else _i32(page_table)
    sl = _i32(cache_seqlens)
    max_k = pt.shape[1] if max_seqlen_k is None else max_seqlen_k
    ws = workspace_for(batch, q_len, hq, hkv, d, max_k, query.device)
    call(
        "fm_block_attn_token_paged",
        query.data_ptr(), *qs, out.data_ptr(), *os_, None,
        key_buffer.data_ptr(), value_buffer.data_ptr(), pool,
        key_buffer.stride(0), key_buffer.stride(1), value_buffer.stride(0), value_buffer.stride(1),
        pt.data_ptr(), pt.stride(0), pt.shape[1], sl.data_ptr(), batch, q_len, max_k,
        hq, hkv, d, float(scale),
        *_prologue_args(prologue, batch * q_len, d),
        _ptr(plan), ws.data_ptr(), ws.numel(), _stream(query),
    )
    return out


# ------------------------------------------------------------------- fp8 (e4m3) KV


def _fp8_query(query: torch.Tensor, out: torch.Tensor | None, varlen: bool):
    """(query, out, query strides, out strides, q_fp8) of an fp8-cache call: e4m3 (or
    uint8) queries are passed as bytes, bf16 ones are quantized in the call."""
    if query.element_size() == 1:
        ok = query.stride(-1) == 1 and query.data_ptr() % 16 == 0 and all(st % 8 == 0 for st in query.stride()[:-1])
        q = query if ok else query.contiguous()
        if out is None:
            out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        if varlen:
            qs, os_ = [0, q.stride(0), q.stride(1)], [0, out.stride(0), out.stride(1)]
        else:
            qs, os_ = [q.stride(0), q.stride(1), q.stride(2)], [out.stride(0), out.stride(1), out.stride(2)]
        return q, out, qs, os_, 1
    q, out, qs, os_ = _q_out(query, out, varlen)
    return q, out, qs, os_, 0


def _descale_args(descales: torch.Tensor | None, batch: int, hkv: int) -> list:
    """(pointer, kind, batch, head strides) of FlashAttention-style descales (3, batch,
    kv_heads) float32 (expanded views allowed)."""
    if descales is None:
        return [None, 0, 0, 0]
    if descales.dim() != 3 or descales.shape[0] < 3 or descales.shape[1] < batch or descales.shape[2] < hkv:
        raise ValueError(f"descales must be (3, {batch}, {hkv}) (query, key, value); got {tuple(descales.shape)}")
    d = descales if descales.dtype == torch.float32 else descales.float()
    return [d.data_ptr(), d.stride(0), d.stride(1), d.stride(2)]


def block_attention_paged_fp8(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor | None,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    descales: torch.Tensor | None = None,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`block_attention_paged` onto an e4m3 cache ``(num_blocks, Hkv, page, 2D)``
    (one byte per element): ``query`` e4m3 (quantized by the caller, ``descales[0]`` its
    descale) or bf16 (quantized per (request, query head) in the call); ``descales (3,
    requests, Hkv)`` = query, key, value descales (flashmap/vllm/model.py:93-134, 863-873).
    Returns bf16."""
    _check_cuda(query, kv_cache, cu_seqlens_q, seqused_k, block_table, descales)
    _fp8_cache(kv_cache, "kv_cache")
    tokens, hq, d = query.shape
    num_blocks, hkv, page, two_d = kv_cache.shape
    if two_d != 2 * d or kv_cache.stride(-1) != 1:
        raise ValueError(f"kv_cache must be (blocks, heads, page, 2 * {d}) with unit channel stride")
    batch = seqused_k.shape[0]
    _check_requests(batch, cu_seqlens_q, tokens, max_seqlen_q, block_table, "block_table", plan)
    query, out, qs, os_, q_fp8 = _fp8_query(query, out, varlen=True)
    if batch == 0 or tokens == 0:
        return out
    cu = None if cu_seqlens_q is None else _i32(cu_seqlens_q)
    if cu is None:
        qs[0], os_[0] = max_seqlen_q * qs[1], max_seqlen_q * os_[1]
    bt = block_table if (block_table.dtype == torch.int32 and block_table.stride(-1) == 1) else _i32(block_table)
    sk = _i32(seqused_k)
    ws = workspace_for(batch, max_seqlen_q, hq, hkv, d, max_seqlen_k, query.device)
    call(
        "fm_block_attn_paged_fp8",
        query.data_ptr(), q_fp8, *qs, out.data_ptr(), *os_, _ptr(cu),
        kv_cache.data_ptr(), num_blocks, kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), d, page,
        bt.data_ptr(), bt.stride(0), bt.shape[1], sk.data_ptr(), batch, max_seqlen_q, max_seqlen_k,
        hq, hkv, d, float(softmax_scale), *_descale_args(descales, batch, hkv),
        *_prologue_args(prologue, tokens, d),
        _ptr(plan), ws.data_ptr(), ws.numel(), _stream(query),
    )
    return out


def block_attention_token_paged_fp8(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    cache_seqlens: torch.Tensor,
    page_table: torch.Tensor,
    softmax_scale: float | None = None,
    descales: torch.Tensor | None = None,
    max_seqlen_k: int | None = None,
    prologue: Prologue | None = None,
    plan: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`block_attention_token_paged` onto e4m3 pools: ``query (bs, q_len, Hq, D)``
    bf16 is quantized per (request, query head) with scale amax / 448 and every operand
    descaled, as flashmap_sglang::paged_cross_attention_fp8 does
    (flashmap/sglang/model.py:154-181); an e4m3 ``query`` takes ``descales[0]``."""
    _check_cuda(query, key_buffer, value_buffer, cache_seqlens, page_table, descales)
    _fp8_cache(key_buffer, "key_buffer")
    _fp8_cache(value_buffer, "value_buffer")
    batch, q_len, hq, d = query.shape
    if key_buffer.dim() != 3 or key_buffer.shape != value_buffer.shape or key_buffer.shape[2] != d:
        raise ValueError(f"key_buffer and value_buffer must both be (pool, kv_heads, {d}); got "
                         f"{tuple(key_buffer.shape)} and {tuple(value_buffer.shape)}")
    _need_rows(cache_seqlens, batch, "cache_seqlens")
    _check_requests(batch, None, batch * q_len, q_len, page_table, "page_table", plan)
    pool, hkv, _ = key_buffer.shape
    query, out, qs, os_, q_fp8 = _fp8_query(query, out, varlen=False)
    if batch == 0 or q_len == 0:
        return out
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    pt = page_table if (page_table.dtype == torch.int32 and page_table.stride(-1) == 1) else _i32(page_table)
    sl = _i32(cache_seqlens)
    max_k = pt.shape[1] if max_seqlen_k is None else max_seqlen_k
    ws = workspace_for(batch, q_len, hq, hkv, d, max_k, query.device)
    call(
        "fm_block_attn_token_paged_fp8",
        query.data_ptr(), q_fp8, *qs, out.data_ptr(), *os_, None,
        key_buffer.data_ptr(), value_buffer.data_ptr(), pool,
        key_buffer.stride(0), key_buffer.stride(1), value_buffer.stride(0), value_buffer.stride(1),
        pt.data_ptr(), pt.stride(0), pt.shape[1], sl.data_ptr(), batch, q_len, max_k,
        hq, hkv, d, float(scale), *_descale_args(descales, batch, hkv),
        *_prologue_args(prologue, batch * q_len, d),
        _ptr(plan), ws.data_ptr(), ws.numel(), _stream(query),
    )
    return out


# ------------------------------------------------------------------ verify attention

_VERIFY_WS_BYTES: dict[tuple, int] = {}


def verify_workspace_bytes(batch: int, verify_len: int, hq: int, hkv: int, head_dim: int, max_context: int,
                           pool_size: int, device: torch.device) -> int:
    """Workspace bytes of a verify call of these sizes (fm_verify_workspace_bytes)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (batch, verify_len, hq, hkv, head_dim, max_context, pool_size, index)
    nbytes = _VERIFY_WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_native.lib().fm_verify_workspace_bytes(batch, verify_len, hq, hkv, head_dim, max_context,
                                                             pool_size, index))
        if nbytes == 0:
            raise RuntimeError(f"fm_verify_workspace_bytes failed: {_native.last_error()}")
        _VERIFY_WS_BYTES[key] = nbytes
    return nbytes


def _verify_rows(x: torch.Tensor, name: str) -> bool:
    """Whether ``x`` is bf16 with unit channel stride, 16-byte aligned, other strides
    multiples of 8 elements: the layout the verify kernels read in place."""
    return (x.dtype == torch.bfloat16 and x.stride(-1) == 1 and x.data_ptr() % 16 == 0
            and all(st % 8 == 0 for st in x.stride()[:-1]))


def verify_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    custom_mask: torch.Tensor | None = None,
    mask_indptr: torch.Tensor | None = None,
    qlen_mask: bool = False,
    sm_scale: float | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    out: torch.Tensor | None = None,
    max_context: int | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Target verify attention (flashmap/sglang/verify_attention.py:35-233, 360-474):
    ``q (bs * L, Hq, D)`` -- L verify tokens per request -- attends to request b's
    context, pool rows ``kv_indices[kv_indptr[b]:kv_indptr[b + 1]]`` of
    ``key_buffer/value_buffer (pool, Hkv, D)``, and to the verify tokens' own keys and
    values ``k, v (bs * L, Hkv, D)`` causally (``custom_mask`` None), under sglang's
    custom mask (rows of context + L entries at ``mask_indptr[b]``, the last L of which
    apply) or, with ``qlen_mask``, under each request's L x L block at ``b * L * L``.
    Context scores are scaled by ``sm_scale * k_scale``, context values by
    ``v_scale``. Returns ``out (bs * L, Hq, D)`` bf16. ``workspace`` (uint8, at least
    :func:`verify_workspace_bytes`) defaults to the device's persistent one."""
    _check_cuda(q, k, v, key_buffer, value_buffer, kv_indptr, kv_indices, custom_mask, mask_indptr)
    bs = kv_indptr.shape[0] - 1
    tokens, hq, d = q.shape
    pool, hkv, _ = key_buffer.shape
    if bs < 1 or tokens == 0:
        return torch.empty_like(q) if out is None else out
    if tokens % bs:
        raise ValueError(f"q holds {tokens} tokens, not a multiple of the {bs} requests")
    length = tokens // bs
    if key_buffer.shape != value_buffer.shape or key_buffer.shape[2] != d:
        raise ValueError(f"key_buffer and value_buffer must both be (pool, kv_heads, {d}); got "
                         f"{tuple(key_buffer.shape)} and {tuple(value_buffer.shape)}")
    q = _bf16_rows(q, "q")
    k = _bf16_rows(k.view(-1, hkv, d), "k")
    v = _bf16_rows(v.view(-1, hkv, d), "v")
    _need_rows(k, tokens, "k")
    _need_rows(v, tokens, "v")
    key_buffer, value_buffer = _bf16_rows(key_buffer, "key_buffer"), _bf16_rows(value_buffer, "value_buffer")
    if out is None:
        out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    elif not _verify_rows(out, "out"):
        raise ValueError("out must be bf16 with unit channel stride, 16-byte aligned, strides multiples of 8")
    indptr = _i32(kv_indptr)
    if kv_indices.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"kv_indices must be int32 or int64, got {kv_indices.dtype}")
    indices = kv_indices.contiguous()
    mode, mask, mptr = 0, None, None
    if custom_mask is not None:
        if custom_mask.element_size() != 1:
            raise TypeError(f"custom_mask must hold one byte per entry (bool/uint8), got {custom_mask.dtype}")
        mask = custom_mask.contiguous()
        if qlen_mask:
            mode = 2
            _need_numel(mask, bs * length * length, "custom_mask")
        else:
            if mask_indptr is None:
                raise ValueError("a custom mask in sglang's layout needs mask_indptr")
            mode, mptr = 1, _i64(mask_indptr)
            _need_rows(mptr, bs, "mask_indptr")
    scale = d ** -0.5 if sm_scale is None else float(sm_scale)
    ctx = 0 if max_context is None else int(max_context)
    nbytes = verify_workspace_bytes(bs, length, hq, hkv, d, ctx, pool, q.device)
    if workspace is None:
        index = q.device.index if q.device.index is not None else torch.cuda.current_device()
        workspace = _WORKSPACES.get(torch.device("cuda", index), nbytes)
    elif workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace of {workspace.numel() * workspace.element_size()} bytes, need {nbytes}")
    call(
        "fm_verify_attention",
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
        key_buffer.data_ptr(), value_buffer.data_ptr(), pool,
        key_buffer.stride(0), key_buffer.stride(1), value_buffer.stride(0), value_buffer.stride(1),
        indptr.data_ptr(), indices.data_ptr(), indices.element_size(),
        _ptr(mask), _ptr(mptr), mode, bs, length, hq, hkv, d,
        scale, float(k_scale), float(v_scale), ctx,
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(q),
    )
    return out


# ------------------------------------------------------------------ self-attention


def block_self_attention(
    qkv: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    rope: Rope,
    positions: torch.Tensor | None,
    eps: float,
    softmax_scale: float | None = None,
) -> torch.Tensor:
    """Unmasked attention within each block of ``qkv (blocks, T, 3, heads, D)`` after
    q/k RMSNorm + RoPE; returns ``(blocks, T, heads, D)`` bf16."""
    _check_cuda(qkv, q_norm, k_norm, rope.cos, positions)
    if qkv.dtype != torch.bfloat16:
        raise TypeError(f"qkv must be bfloat16, got {qkv.dtype}")
    qkv = qkv.contiguous()
    blocks, t, three, heads, d = qkv.shape
    if three != 3:
        raise ValueError(f"qkv must be (blocks, T, 3, heads, head_dim), got {tuple(qkv.shape)}")
    rope.check(d)
    _need_numel(q_norm, d, "q_norm")
    _need_numel(k_norm, d, "k_norm")
    _need_rows(positions, blocks * t, "positions")
    out = torch.empty((blocks, t, heads, d), dtype=torch.bfloat16, device=qkv.device)
    if blocks == 0:
        return out
    qn, kn = _f32(q_norm), _f32(k_norm)
    pos = None if positions is None else _i64(positions)
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    call(
        "fm_block_self_attention",
        qkv.data_ptr(), out.data_ptr(), blocks, t, heads, d, qn.data_ptr(), kn.data_ptr(),
        *rope.args(), _ptr(pos), float(eps), float(scale), _stream(qkv),
    )
    return out


# ------------------------------------------------------------------------ writers


def write_context_kv(
    kv: torch.Tensor,
    positions: torch.Tensor,
    slots: torch.Tensor,
    k_norm: torch.Tensor,
    rope: Rope,
    cache_ptrs: torch.Tensor,
    cache_strides: tuple[int, int, int, int],
    block_size: int,
    eps: float,
    heads_per_cache: int | None = None,
) -> None:
    """k-norm + RoPE + store of ``kv (tokens, layers, 2, heads, D)`` into vLLM-layout
    bf16 caches at ``slots`` (negative = skip); see fm_write_context_kv."""
    _check_cuda(kv, positions, slots, k_norm, cache_ptrs)
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"kv must be bfloat16, got {kv.dtype}")
    kv = kv.contiguous()
    tokens, layers, _, heads, d = kv.shape
    if tokens == 0:
        return
    hpc = heads_per_cache or heads
    if cache_ptrs.numel() * hpc < layers * heads:
        raise ValueError(f"{cache_ptrs.numel()} caches of {hpc} heads cannot hold {layers} x {heads} heads")
    rope.check(d)
    _need_numel(k_norm, layers * d, "k_norm")
    _need_rows(positions, tokens, "positions")
    _need_rows(slots, tokens, "slots")
    sb, sh, st, voff = cache_strides
    kn = _f32(k_norm)
    call(
        "fm_write_context_kv",
        kv.data_ptr(), tokens, layers, heads, d, _i64(positions).data_ptr(), _i64(slots).data_ptr(),
        kn.data_ptr(), *rope.args(), _i64(cache_ptrs).data_ptr(), cache_ptrs.numel(), hpc,
        sb, sh, st, voff, block_size, float(eps), _stream(kv),
    )


def write_context_kv_pool(
    kv: torch.Tensor,
    meta: torch.Tensor,
    k_norm_weights: torch.Tensor,
    rope: Rope,
    positions: torch.Tensor,
    locs: torch.Tensor,
    num_layers: int,
    kv_size: int,
    head_dim: int,
    eps: float,
    commit_lens: torch.Tensor | None = None,
    locs_row_width: int | None = None,
) -> None:
    """k-norm + RoPE + store of ``kv (tokens, layers * 2 * kv_size)`` into SGLang pools
    described by ``meta (layers, 4)``; see fm_write_context_kv_pool."""
    _check_cuda(kv, meta, k_norm_weights, positions, locs, commit_lens)
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"kv must be bfloat16, got {kv.dtype}")
    kv = kv.contiguous()
    tokens = kv.shape[0]
    if tokens == 0:
        return
    heads = kv_size // head_dim
    if kv.numel() != tokens * num_layers * 2 * kv_size:
        raise ValueError("kv must be (tokens, layers * 2 * kv_size)")
    _check_pool_write(meta, k_norm_weights, rope, positions, locs, num_layers, head_dim, tokens, commit_lens,
                      locs_row_width)
    cl = None if commit_lens is None else _i32(commit_lens)
    call(
        "fm_write_context_kv_pool",
        kv.data_ptr(), tokens, num_layers, heads, head_dim, _i64(meta).data_ptr(),
        _f32(k_norm_weights).data_ptr(), *rope.args(), _i64(positions).data_ptr(), _i64(locs).data_ptr(),
        _ptr(cl), int(locs_row_width or 0), float(eps), _stream(kv),
    )


def _check_pool_write(meta, k_norm_weights, rope, positions, locs, layers, head_dim, tokens, commit_lens,
                      locs_row_width) -> None:
    """Extents the pool writers read: meta rows per layer, weights, one position and
    one location per token, one commit length per row of ``locs_row_width`` tokens."""
    rope.check(head_dim)
    if meta.dim() != 2 or meta.shape[1] != 4:
        raise ValueError(f"meta must be (layers, 4), got {tuple(meta.shape)}")
    _need_rows(meta, layers, "meta")
    _need_numel(k_norm_weights, layers * head_dim, "k_norm_weights")
    _need_numel(positions, tokens, "positions")
    _need_numel(locs, tokens, "locs")
    if commit_lens is not None:
        if not locs_row_width:
            raise ValueError("commit_lens needs locs_row_width")
        _need_numel(commit_lens, -(-tokens // locs_row_width), "commit_lens")


def _fp8_cache(t: torch.Tensor, name: str) -> None:
    if t.element_size() != 1:
        raise TypeError(f"{name} must be an fp8 (e4m3) or uint8 tensor, got {t.dtype}")


def write_context_kv_fp8(
    kv: torch.Tensor,
    positions: torch.Tensor,
    slots: torch.Tensor,
    k_norm: torch.Tensor,
    rope: Rope,
    cache_ptrs: torch.Tensor,
    cache_strides: tuple[int, int, int, int],
    block_size: int,
    eps: float,
    scales: torch.Tensor,
    heads_per_cache: int | None = None,
) -> None:
    """:func:`write_context_kv` into e4m3 caches (one byte per element, strides in
    elements) with per-layer ``scales (layers, 2)`` (key, value); see
    fm_write_context_kv_fp8 (flashmap/vllm/kernels.py:292-299)."""
    _check_cuda(kv, positions, slots, k_norm, cache_ptrs, scales)
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"kv must be bfloat16, got {kv.dtype}")
    kv = kv.contiguous()
    tokens, layers, _, heads, d = kv.shape
    if tokens == 0:
        return
    hpc = heads_per_cache or heads
    if cache_ptrs.numel() * hpc < layers * heads:
        raise ValueError(f"{cache_ptrs.numel()} caches of {hpc} heads cannot hold {layers} x {heads} heads")
    rope.check(d)
    _need_numel(k_norm, layers * d, "k_norm")
    _need_rows(positions, tokens, "positions")
    _need_rows(slots, tokens, "slots")
    if scales.numel() < 2 * layers:
        raise ValueError(f"scales must hold (layers, 2) = {2 * layers} values, got {scales.numel()}")
    sb, sh, st, voff = cache_strides
    kn, sc = _f32(k_norm), _f32(scales)
    call(
        "fm_write_context_kv_fp8",
        kv.data_ptr(), tokens, layers, heads, d, _i64(positions).data_ptr(), _i64(slots).data_ptr(),
        kn.data_ptr(), *rope.args(), _i64(cache_ptrs).data_ptr(), cache_ptrs.numel(), hpc,
        sb, sh, st, voff, block_size, sc.data_ptr(), float(eps), _stream(kv),
    )


def write_context_kv_pool_fp8(
    kv: torch.Tensor,
    meta: torch.Tensor,
    k_norm_weights: torch.Tensor,
    rope: Rope,
    positions: torch.Tensor,
    locs: torch.Tensor,
    num_layers: int,
    kv_size: int,
    head_dim: int,
    eps: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    commit_lens: torch.Tensor | None = None,
    locs_row_width: int | None = None,
) -> None:
    """:func:`write_context_kv_pool` into e4m3 pools with static scales and the pool
    writer's norm rounding; see fm_write_context_kv_pool_fp8
    (flashmap/sglang/kernels.py:283-357)."""
    _check_cuda(kv, meta, k_norm_weights, positions, locs, commit_lens)
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"kv must be bfloat16, got {kv.dtype}")
    kv = kv.contiguous()
    tokens = kv.shape[0]
    if tokens == 0:
        return
    heads = kv_size // head_dim
    if kv.numel() != tokens * num_layers * 2 * kv_size:
        raise ValueError("kv must be (tokens, layers * 2 * kv_size)")
    _check_pool_write(meta, k_norm_weights, rope, positions, locs, num_layers, head_dim, tokens, commit_lens,
                      locs_row_width)
    cl = None if commit_lens is None else _i32(commit_lens)
    call(
        "fm_write_context_kv_pool_fp8",
        kv.data_ptr(), tokens, num_layers, heads, head_dim, _i64(meta).data_ptr(),
        _f32(k_norm_weights).data_ptr(), *rope.args(), _i64(positions).data_ptr(), _i64(locs).data_ptr(),
        _ptr(cl), int(locs_row_width or 0), float(k_scale), float(v_scale), float(eps), _stream(kv),
    )


# ------------------------------------------------------------ token selection and noise

_LOGIT_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _logits(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() != 2:
        raise ValueError(f"logits must be (rows, vocab), got {tuple(logits.shape)}")
    if logits.dtype not in _LOGIT_DTYPES:
        raise TypeError(f"logits must be bfloat16, float16 or float32, got {logits.dtype}")
    return logits if logits.stride(-1) == 1 else logits.contiguous()


def _select(name: str, logits: torch.Tensor, *extra) -> torch.Tensor:
    rows, vocab = logits.shape
    out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    if rows == 0:
        return out
    if vocab == 0:
        raise ValueError("an empty vocabulary has no argmax")
    ws = torch.empty(max(int(_native.lib().fm_select_workspace_bytes(rows, vocab)), 1), dtype=torch.uint8,
                     device=logits.device)
    call(name, logits.data_ptr(), _LOGIT_DTYPES[logits.dtype], rows, vocab, logits.stride(0), *extra,
         out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(logits))
    return out


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """Per row of ``logits (rows, vocab)`` (bf16, fp16 or fp32) the int64 index of the
    largest value, the first among equals, a NaN counting as the largest: ``argmax(-1)``
    as flashmap/vllm/fold.py:117-128 (split_argmax) computes it."""
    _check_cuda(logits)
    return _select("fm_argmax_rows", _logits(logits))


def sample_rows(
    logits: torch.Tensor, temperatures: torch.Tensor, greedy: torch.Tensor, seed: torch.Tensor
) -> torch.Tensor:
    """A token per row of ``logits (rows, V)``: the argmax for rows where ``greedy`` is
    set, else a sample of softmax(logits / temperature) by Gumbel-max with Triton's
    Philox noise ``tl.rand(seed, row * V + col)`` (flashmap/sglang/kernels.py:195-247);
    ``seed`` is an int64 scalar tensor (advance it between calls for fresh noise)."""
    _check_cuda(logits, temperatures, greedy, seed)
    logits = _logits(logits)
    rows = logits.shape[0]
    if temperatures.numel() != rows or greedy.numel() != rows:
        raise ValueError(f"temperatures and greedy must hold one entry per row ({rows})")
    if seed.dtype != torch.int64 or seed.numel() != 1:
        raise TypeError("seed must be an int64 scalar tensor")
    g = greedy if (greedy.dtype in (torch.bool, torch.uint8) and greedy.is_contiguous()) else (greedy != 0)
    g = g.view(torch.uint8) if g.dtype == torch.bool else g
    return _select("fm_sample_rows", logits, _f32(temperatures).data_ptr(), g.contiguous().data_ptr(),
                   seed.data_ptr())


def seeded_normal(
    seeds: torch.Tensor, rows: torch.Tensor, positions: torch.Tensor, n_cols: int, scale: float = 1.0
) -> torch.Tensor:
    """Standard normals ``(len(rows), n_cols)`` in float32 times ``scale``, row ``i``
    keyed by ``seeds[rows[i]] * 1000003 + positions[i]`` (seed 0 where ``rows[i] < 0``),
    column ``j`` at offset ``j``: Triton's ``tl.randn`` stream as
    flashmap/vllm/kernels.py:367-410 draws it. ``rows[i]`` must index ``seeds``."""
    _check_cuda(seeds, rows, positions)
    n = rows.shape[0]
    out = torch.empty(n, n_cols, dtype=torch.float32, device=rows.device)
    if n == 0 or n_cols == 0:
        return out
    if positions.shape[0] != n:
        raise ValueError("positions must hold one entry per row")
    r = rows if (rows.dtype in (torch.int32, torch.int64) and rows.is_contiguous()) else _i64(rows)
    p = positions if (positions.dtype in (torch.int32, torch.int64) and positions.is_contiguous()) else _i64(positions)
    call("fm_seeded_normal", _i64(seeds).data_ptr(), r.data_ptr(), int(r.dtype == torch.int64), p.data_ptr(),
         int(p.dtype == torch.int64), n, n_cols, float(scale), out.data_ptr(), out.stride(0), _stream(rows))
    return out


# --------------------------------------------------------------------- DiT stream


def _rows2d(t: torch.Tensor, dim: int, name: str) -> torch.Tensor:
    """``t (..., dim)`` bf16 as ``(rows, dim)`` rows with unit channel stride (a view
    when the leading dims flatten to one row stride, else a copy)."""
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.shape[-1] != dim:
        raise ValueError(f"{name} rows hold {t.shape[-1]} values, expected {dim}")
    r = t.reshape(-1, dim)
    if r.stride(-1) != 1 or r.stride(0) % 8 or r.data_ptr() % 16:
        r = r.contiguous()
    return r


def _vec(t: torch.Tensor, dim: int, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.numel() != dim:
        raise ValueError(f"{name} holds {t.numel()} values, expected {dim} (one per channel)")
    v = t.reshape(dim)
    return v if (v.stride(0) == 1 and v.data_ptr() % 16 == 0) else v.contiguous()


def adaln_residual(
    x: torch.Tensor,
    y: torch.Tensor | None,
    gate: torch.Tensor | None,
    modulation: tuple[torch.Tensor, torch.Tensor] | None,
    eps: float,
    x_out: torch.Tensor | None = None,
    gate_per_row: bool = False,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """The DiT's residual stream in one pass: ``x' = x + gate * y`` (skipped when ``y``
    is None), then ``h = LN(x') * (1 + scale) + shift`` for ``modulation = (scale,
    shift)`` (skipped when None), each op rounded to bf16 like torch's eager ops
    (flashmap/modeling_flashmap.py:114-117, 185-192). ``x``/``y (..., dim)`` bf16, or
    ``x (dim,)``: one row shared by every row of ``y``; ``gate``, ``scale``, ``shift``:
    ``dim`` values shared by every row (``gate_per_row``: one gate value per row).
    ``x_out`` (may be ``x``) receives ``x'``, else a new tensor does. Returns ``(x',
    h)``, ``x'`` None without a residual."""
    _check_cuda(x, y, gate, x_out, *(modulation or ()))
    dim = x.shape[-1]
    if dim % 8 or not 0 < dim <= 8192:
        raise ValueError(f"rows of {dim} values: the kernel takes a multiple of 8, at most 8192")
    shared = x.dim() == 1 and y is not None
    shape = y.shape if shared else x.shape
    xr = _vec(x, dim, "x")[None] if shared else _rows2d(x, dim, "x")
    x_stride = 0 if shared else xr.stride(0)
    rows = math.prod(shape[:-1])
    yr = g = xo = None
    if y is not None:
        if gate is None:
            raise ValueError("a residual needs its gate")
        if y.shape[-1] != dim or (not shared and y.numel() != x.numel()):
            raise ValueError(f"y {tuple(y.shape)} does not match x {tuple(x.shape)}")
        yr = _rows2d(y, dim, "y")
        g = _vec(gate, rows, "gate (one per row)") if gate_per_row else _vec(gate, dim, "gate")
        if x_out is None:
            x_out = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
        if x_out.numel() != rows * dim:
            raise ValueError(f"x_out holds {x_out.numel()} values, the stream {rows * dim}")
        xo = x_out.view(rows, dim)  # raises unless x_out's rows are one strided view
        if xo.stride(-1) != 1 or xo.stride(0) % 8 or xo.data_ptr() % 16:
            raise ValueError("x_out must hold 16-byte aligned rows with unit channel stride")
    h = sc = sh = None
    if modulation is not None:
        sc, sh = (_vec(m, dim, n) for m, n in zip(modulation, ("scale", "shift")))
        h = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
    if rows == 0 or (yr is None and h is None):
        return x_out, h
    hr = None if h is None else h.view(rows, dim)
    call(
        "fm_adaln_residual",
        xr.data_ptr(), x_stride, _ptr(yr), 0 if yr is None else yr.stride(0), _ptr(g), int(gate_per_row),
        _ptr(sc), _ptr(sh), _ptr(xo), 0 if xo is None else xo.stride(0), _ptr(hr), 0 if hr is None else hr.stride(0),
        rows, dim, float(eps), _stream(y if shared else x),
    )
    return x_out, h


def noise_rows(z: torch.Tensor, eigvals: torch.Tensor, eps: float, gain: float,
               z_bf16: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The folded noise read-out's row pass (flashmap/vllm/model.py:915-925): for ``z
    (rows, H)`` float32, ``(z in bf16, bf16(gain * rsqrt(z^2 @ eigvals + eps)) (rows,))``."""
    _check_cuda(z, eigvals, z_bf16)
    if z.dtype != torch.float32 or z.dim() != 2 or z.stride(-1) != 1:
        raise ValueError("z must be float32 (rows, H) with unit channel stride")
    rows, hidden = z.shape
    if z.stride(0) % 4 or z.data_ptr() % 16:
        z = z.contiguous()
    lam = _f32(eigvals)
    _need_numel(lam, hidden, "eigvals")
    if z_bf16 is None:
        z_bf16 = torch.empty(rows, hidden, dtype=torch.bfloat16, device=z.device)
    elif (z_bf16.dtype != torch.bfloat16 or tuple(z_bf16.shape) != (rows, hidden) or z_bf16.stride(-1) != 1
          or z_bf16.stride(0) % 4 or z_bf16.data_ptr() % 8):
        raise ValueError(f"z_bf16 must be bf16 ({rows}, {hidden}) with unit channel stride, a row stride "
                         f"of a multiple of 4 and 8-byte alignment; got {z_bf16.dtype} {tuple(z_bf16.shape)} "
                         f"strides {z_bf16.stride()}")
    scale = torch.empty(rows, dtype=torch.bfloat16, device=z.device)
    if rows:
        call("fm_noise_rows", z.data_ptr(), rows, hidden, z.stride(0), lam.data_ptr(), float(eps), float(gain),
             z_bf16.data_ptr(), z_bf16.stride(0), scale.data_ptr(), _stream(z))
    return z_bf16, scale


def _state_rows(state: torch.Tensor) -> None:
    if state.dtype != torch.float32 or state.dim() != 2 or state.stride(-1) != 1:
        raise ValueError("the state must be float32 (rows, vocab) with unit column stride")
    if state.stride(0) % 4 or state.data_ptr() % 16:
        raise ValueError("the state's row stride must be a multiple of 4 and its data 16-byte aligned")


def state_embed_rows(state: torch.Tensor, evidence: float, out: torch.Tensor | None = None,
                     posterior: bool = True) -> torch.Tensor:
    """``torch.cat([softmax(evidence * state), state]).to(bf16)`` for the several-jump
    draft's state ``(rows, vocab)`` float32 (flashmap/vllm/model.py:944-956): one kernel
    reading each row twice, ``(2 rows, vocab)`` bf16, the operand of the state
    embedding's GEMM. ``posterior=False``: the state rows alone ``(rows, vocab)`` (one
    read), for a jump whose posterior is uniform."""
    _check_cuda(state, out)
    _state_rows(state)
    rows, vocab = state.shape
    n = 2 * rows if posterior else rows
    if out is None:  # rows padded to a multiple of 4 values
        out = torch.empty(n, -(-vocab // 4) * 4, dtype=torch.bfloat16, device=state.device)[:, :vocab]
    elif (out.dtype != torch.bfloat16 or tuple(out.shape) != (n, vocab) or out.stride(-1) != 1
          or out.stride(0) % 4 or out.data_ptr() % 8):
        raise ValueError(f"out must be bf16 ({n}, {vocab}) with unit column stride, a row stride of a "
                         f"multiple of 4 and 8-byte alignment; got {out.dtype} {tuple(out.shape)} {out.stride()}")
    if rows:
        call("fm_state_embed_rows", state.data_ptr(), rows, vocab, state.stride(0), float(evidence),
             int(posterior), out.data_ptr(), out.stride(0), _stream(state))
    return out


def state_update(state: torch.Tensor, logits: torch.Tensor, start: float, end: float) -> torch.Tensor:
    """The state update between two jumps, in place (flashmap/vllm/model.py:1031-1036):
    ``state = ((1 - end) state + (end - start) softmax(logits)) / (1 - start)`` with
    ``logits (rows, vocab)`` bf16, in float32 with torch's rounding points."""
    _check_cuda(state, logits)
    _state_rows(state)
    rows, vocab = state.shape
    if logits.dtype != torch.bfloat16 or tuple(logits.shape) != (rows, vocab):
        raise ValueError(f"logits must be bf16 ({rows}, {vocab}); got {logits.dtype} {tuple(logits.shape)}")
    if logits.stride(-1) != 1 or logits.stride(0) % 4 or logits.data_ptr() % 8:  # into rows of 4k values
        padded = torch.empty(rows, -(-vocab // 4) * 4, dtype=torch.bfloat16, device=logits.device)[:, :vocab]
        logits = padded.copy_(logits)
    if not (start < 1.0 and end >= start):
        raise ValueError(f"jump times must satisfy start <= end and start < 1, got {start}, {end}")
    if rows:
        call("fm_state_update", state.data_ptr(), rows, vocab, state.stride(0), logits.data_ptr(),
             logits.stride(0), float(start), float(end), _stream(state))
    return state


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
