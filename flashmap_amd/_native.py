"""ctypes binding of the C ABI in ``include/flashmap_amd.h``.

The library is loaded once, from the package's ``_lib`` directory. There is no
fallback: a missing or stale library raises, so nothing silently runs elsewhere.
"""

from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libflashmap_amd.so"
ABI_VERSION = 1

FM_OK = 0
FM_ERR_INVALID = 1
FM_ERR_UNSUPPORTED = 2
FM_ERR_WORKSPACE = 3
FM_ERR_HIP = 4

P = c_void_p
I32 = c_int32
I64 = c_int64
F32 = c_float

_ROPE = [P, P, I64, I64, I64]  # cos, sin, row stride, pair stride, rows
_Q = [P, I64, I64, I64, P, I64, I64, I64, P]  # q + strides, out + strides, cu_seqlens_q
_PROLOGUE = [P, *_ROPE, P, F32]  # q_norm_weight, rope, q_positions, eps
_SPLIT = [P, P, c_size_t, P]  # plan, workspace, workspace bytes, stream

# name -> (restype, argtypes), in header order.
SIGNATURES: dict[str, tuple] = {
    "fm_last_error": (ctypes.c_char_p, []),
    "fm_abi_version": (c_int, []),
    "fm_device_cus": (c_int, [c_int, ctypes.POINTER(c_int)]),
    "fm_rms_norm_rope": (c_int, [P, P, I64, I32, I32, I64, I64, I64, I64, P, *_ROPE, P, F32, P]),
    "fm_attn_plan_bytes": (c_size_t, [I32]),
    "fm_attn_plan": (c_int, [P, I32, P, P]),
    "fm_attn_workspace_bytes": (c_size_t, [I32, I32, I32, I32, I32, I32, c_int]),
    "fm_block_attn_contig": (
        c_int,
        [*_Q, P, I64, I64, I64, P, I64, I64, I64, P, I32, I32, I32, I32, I32, I32, F32,
         *_PROLOGUE, *_SPLIT],
    ),
    "fm_block_attn_paged": (
        c_int,
        [*_Q, P, I64, I64, I64, I64, I64, I32, P, I64, I64, P, I32, I32, I32, I32, I32, I32, F32,
         *_PROLOGUE, *_SPLIT],
    ),
    "fm_static_scratch_bytes": (c_size_t, []),
    "fm_static_scratch_init": (c_int, []),
    "fm_block_attn_paged_static": (
        c_int,
        [*_Q, P, I64, I64, I64, I64, I64, I32, P, I64, I64, P, I32, I32, I32, I32, I32, I32, F32,
         *_PROLOGUE, P, P],
    ),
    "fm_block_attn_paged_runs": (
        c_int,
        [*_Q, P, P, P, I32, I32, I64, I64, I64, I64, I64, I32, P, I64, I64, P, I32, I32, I32, I32, I32, I32,
         F32, *_PROLOGUE, *_SPLIT],
    ),
    "fm_block_attn_token_paged": (
        c_int,
        [*_Q, P, P, I64, I64, I64, I64, I64, P, I64, I64, P, I32, I32, I32, I32, I32, I32, F32,
         *_PROLOGUE, *_SPLIT],
    ),
    "fm_block_attn_paged_fp8": (
        c_int,
        [P, I32, I64, I64, I64, P, I64, I64, I64, P, P, I64, I64, I64, I64, I64, I32, P, I64, I64, P,
         I32, I32, I32, I32, I32, I32, F32, P, I64, I64, I64, *_PROLOGUE, *_SPLIT],
    ),
    "fm_block_attn_token_paged_fp8": (
        c_int,
        [P, I32, I64, I64, I64, P, I64, I64, I64, P, P, P, I64, I64, I64, I64, I64, P, I64, I64, P,
         I32, I32, I32, I32, I32, I32, F32, P, I64, I64, I64, *_PROLOGUE, *_SPLIT],
    ),
    "fm_verify_workspace_bytes": (c_size_t, [I32, I32, I32, I32, I32, I32, I64, c_int]),
    "fm_verify_attention": (
        c_int,
        [P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, P, I64, I64, I64, I64, I64, P, P, I32,
         P, P, I32, I32, I32, I32, I32, I32, F32, F32, F32, I32, P, c_size_t, P],
    ),
    "fm_block_self_attention": (
        c_int, [P, P, I64, I32, I32, I32, P, P, *_ROPE, P, F32, F32, P]
    ),
    "fm_write_context_kv": (
        c_int,
        [P, I64, I32, I32, I32, P, P, P, *_ROPE, P, I32, I32, I64, I64, I64, I64, I32, F32, P],
    ),
    "fm_write_context_kv_pool": (
        c_int, [P, I64, I32, I32, I32, P, P, *_ROPE, P, P, P, I64, F32, P]
    ),
    "fm_write_context_kv_fp8": (
        c_int,
        [P, I64, I32, I32, I32, P, P, P, *_ROPE, P, I32, I32, I64, I64, I64, I64, I32, P, F32, P],
    ),
    "fm_write_context_kv_pool_fp8": (
        c_int, [P, I64, I32, I32, I32, P, P, *_ROPE, P, P, P, I64, F32, F32, F32, P]
    ),
    "fm_select_workspace_bytes": (c_size_t, [I64, I64]),
    "fm_argmax_rows": (c_int, [P, I32, I64, I64, I64, P, P, c_size_t, P]),
    "fm_sample_rows": (c_int, [P, I32, I64, I64, I64, P, P, P, P, P, c_size_t, P]),
    "fm_seeded_normal": (c_int, [P, P, I32, P, I32, I64, I64, F32, P, I64, P]),
    "fm_adaln_residual": (c_int, [P, I64, P, I64, P, I32, P, P, P, I64, P, I64, I64, I32, F32, P]),
    "fm_noise_rows": (c_int, [P, I64, I32, I64, P, F32, F32, P, I64, P, P]),
    "fm_state_embed_rows": (c_int, [P, I64, I64, I64, F32, I32, P, I64, P]),
    "fm_state_update": (c_int, [P, I64, I64, I64, P, I64, c_double, c_double, P]),
    "fm_profile_enable": (c_int, [c_int]),
    "fm_clock_probe": (c_int, [P, ctypes.c_uint64, P]),
    "fm_profile_read": (c_int, [ctypes.POINTER(c_double), ctypes.POINTER(c_int64)]),
    "fm_tuning_reload": (c_int, []),
}

_lib = None


class NativeError(RuntimeError):
    """A FM_ERR_* status from the library, with its fm_last_error() text."""

    def __init__(self, code: int, name: str, message: str):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python -m flashmap_amd._build`"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        version = handle.fm_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {version}, this package expects {ABI_VERSION}")
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise NativeError on failure."""
    handle = lib()
    rc = getattr(handle, name)(*args)
    if rc != FM_OK:
        raise NativeError(rc, name, handle.fm_last_error().decode(errors="replace"))


def last_error() -> str:
    return lib().fm_last_error().decode(errors="replace")
