"""The C-ABI library on the CPU (no GPU calls): it loads, exports every function
``include/flashmap_amd.h`` declares with the signature the ctypes binding uses, and
rejects bad arguments with the documented status codes before touching the device.
The torch wrappers refuse CPU tensors (there is no CPU fallback)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashmap_amd.h"


def _declared():
    text = HEADER.read_text()
    body = text[text.index('extern "C"'):]
    return re.findall(r"^[A-Za-z_][\w\s\*]*?\b(fm_\w+)\s*\(", body, re.M)


@pytest.fixture(scope="module")
def lib():
    from flashmap_amd import _native

    if not _native.LIB_PATH.exists():  # the driver builds first; build here otherwise
        from flashmap_amd import _build

        _build.build()
    return _native.lib()


def test_header_declarations_are_bound():
    from flashmap_amd import _native

    names = _declared()
    assert len(names) >= 15
    assert names == list(_native.SIGNATURES), "ctypes bindings must follow the header, in order"


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"{name} is declared but not exported"


def test_abi_version(lib):
    from flashmap_amd import _native

    want = int(re.search(r"#define FM_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.fm_abi_version() == want == _native.ABI_VERSION


def _err(lib):
    return lib.fm_last_error().decode()


def test_prologue_argument_errors(lib):
    from flashmap_amd import _native as n

    x = ctypes.c_void_p(16)  # never dereferenced: the checks return first
    rope = [x, x, 64, 1, 0]
    rc = lib.fm_rms_norm_rope(x, x, -1, 8, 128, 1024, 128, 1024, 128, x, *rope, None, ctypes.c_float(1e-6), None)
    assert rc == n.FM_ERR_INVALID and "bad sizes" in _err(lib)
    rc = lib.fm_rms_norm_rope(x, x, 4, 8, 96, 1024, 128, 1024, 128, x, *rope, None, ctypes.c_float(1e-6), None)
    assert rc == n.FM_ERR_UNSUPPORTED and "head_dim 96" in _err(lib)
    rc = lib.fm_rms_norm_rope(x, None, 4, 8, 128, 1024, 128, 1024, 128, x, *rope, None, ctypes.c_float(1e-6), None)
    assert rc == n.FM_ERR_INVALID and "NULL" in _err(lib)
    rc = lib.fm_rms_norm_rope(x, x, 4, 8, 128, 1020, 128, 1024, 128, x, *rope, None, ctypes.c_float(1e-6), None)
    assert rc == n.FM_ERR_INVALID and "multiples of 8" in _err(lib)
    # zero tokens is a no-op
    assert lib.fm_rms_norm_rope(None, None, 0, 8, 128, 0, 0, 0, 0, None, None, None, 0, 0, 0, None,
                                ctypes.c_float(1e-6), None) == n.FM_OK


def test_attention_argument_errors(lib):
    from flashmap_amd import _native as n

    x = ctypes.c_void_p(16)
    f = ctypes.c_float
    common_q = [x, 0, 4096, 128, x, 0, 4096, 128, None]
    pro = [None, None, None, 0, 0, 0, None, f(1e-6)]
    split = [None, None, 0, None]
    # paged: a NULL block table is rejected before anything else
    rc = lib.fm_block_attn_paged(*common_q, x, 10, 65536, 4096, 256, 128, 16, None, 8, 8, x, 2, 16, 128,
                                 32, 8, 128, f(0.088), *pro, *split)
    assert rc == n.FM_ERR_INVALID and "NULL" in _err(lib)
    # self-attention: blocks of more than 16 slots are unsupported
    rc = lib.fm_block_self_attention(x, x, 4, 17, 8, 128, x, x, x, x, 64, 1, 0, None, f(1e-6), f(0.088), None)
    assert rc == n.FM_ERR_UNSUPPORTED and "block_size 17" in _err(lib)
    rc = lib.fm_block_self_attention(x, x, 4, 16, 8, 80, x, x, x, x, 64, 1, 0, None, f(1e-6), f(0.088), None)
    assert rc == n.FM_ERR_UNSUPPORTED and "head_dim 80" in _err(lib)


def test_residual_stream_argument_errors(lib):
    from flashmap_amd import _native as n

    x = ctypes.c_void_p(16)
    f = ctypes.c_float(1e-6)
    rc = lib.fm_adaln_residual(x, 16, x, 16, x, 0, x, x, x, 16, x, 16, 4, 12, f, None)
    assert rc == n.FM_ERR_UNSUPPORTED and "dim 12" in _err(lib)
    rc = lib.fm_adaln_residual(x, 16384, x, 16384, x, 0, x, x, x, 16384, x, 16384, 4, 16384, f, None)
    assert rc == n.FM_ERR_UNSUPPORTED and "at most 8192" in _err(lib)
    rc = lib.fm_adaln_residual(x, 64, x, 64, None, 0, x, x, x, 64, x, 64, 4, 64, f, None)
    assert rc == n.FM_ERR_INVALID and "gate" in _err(lib)
    rc = lib.fm_adaln_residual(x, 64, None, 0, None, 0, None, None, None, 0, None, 0, 4, 64, f, None)
    assert rc == n.FM_ERR_INVALID and "nothing to write" in _err(lib)
    rc = lib.fm_adaln_residual(x, 60, None, 0, None, 0, x, x, None, 0, x, 64, 4, 64, f, None)
    assert rc == n.FM_ERR_INVALID and "multiples of 8" in _err(lib)
    rc = lib.fm_adaln_residual(x, 0, x, 64, x, 1, x, x, x, 64, x, 64, 4, 64, f, None)
    assert rc == n.FM_ERR_INVALID and "shared x row" in _err(lib)
    assert lib.fm_adaln_residual(None, 0, None, 0, None, 0, None, None, None, 0, None, 0, 0, 64, f, None) == n.FM_OK
    rc = lib.fm_noise_rows(x, 4, 30, 32, x, f, f, x, 32, x, None)
    assert rc == n.FM_ERR_UNSUPPORTED and "hidden 30" in _err(lib)
    rc = lib.fm_noise_rows(x, 4, 32, 30, x, f, f, x, 32, x, None)
    assert rc == n.FM_ERR_INVALID and "row strides" in _err(lib)
    rc = lib.fm_state_embed_rows(x, 4, 30, 30, f, 1, x, 32, None)
    assert rc == n.FM_ERR_INVALID and "state must be 16-byte aligned" in _err(lib)
    rc = lib.fm_state_embed_rows(x, 4, 32, 32, f, 1, ctypes.c_void_p(20), 32, None)
    assert rc == n.FM_ERR_INVALID and "out must be 8-byte aligned" in _err(lib)
    assert lib.fm_state_embed_rows(None, 0, 32, 32, f, 1, None, 32, None) == n.FM_OK
    rc = lib.fm_state_update(x, 4, 32, 32, x, 32, 1.0, 1.0, None)
    assert rc == n.FM_ERR_INVALID and "jump times" in _err(lib)
    rc = lib.fm_state_update(x, 4, 32, 32, x, 30, 0.0, 0.5, None)
    assert rc == n.FM_ERR_INVALID and "logits must be 8-byte aligned" in _err(lib)


def test_plan_and_workspace_sizes_without_device(lib):
    assert lib.fm_attn_plan_bytes(5) == 2 * 4 * 6  # the bf16 and e4m3 tile prefixes
    assert lib.fm_attn_plan_bytes(-3) == 2 * 4
    # invalid shapes answer with a minimal size instead of querying the device
    assert lib.fm_attn_workspace_bytes(4, 16, 30, 8, 128, 1024, 0) == 256
    assert lib.fm_attn_workspace_bytes(4, 16, 32, 8, 96, 1024, 0) == 256


def test_wrappers_refuse_cpu_tensors():
    from flashmap_amd import ops

    x = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    table = torch.zeros(16, 64, 2)
    with pytest.raises(ValueError, match="GPU"):
        ops.rms_norm_rope(x, torch.ones(128), ops.rope_from_table(table), None, 1e-6)


def test_verify_argument_errors(lib):
    from flashmap_amd import _native as n

    x = ctypes.c_void_p(16)
    f = ctypes.c_float
    qkvo = [x, 4096, 128, x, 1024, 128, x, 1024, 128, x, 4096, 128]
    pool = [x, x, 100, 1024, 128, 1024, 128]
    tail = [4, 17, 32, 8, 128, f(0.088), f(1.0), f(1.0), 0, None, 0, None]
    # zero requests or tokens: nothing to do
    assert lib.fm_verify_attention(*qkvo, *pool, x, x, 4, None, None, 0, 0, *tail[1:]) == n.FM_OK
    # NULL indptr
    rc = lib.fm_verify_attention(*qkvo, *pool, None, x, 4, None, None, 0, *tail)
    assert rc == n.FM_ERR_INVALID and "NULL" in _err(lib)
    # index width
    rc = lib.fm_verify_attention(*qkvo, *pool, x, x, 2, None, None, 0, *tail)
    assert rc == n.FM_ERR_INVALID and "int32 or int64" in _err(lib)
    # mask modes and their arrays
    rc = lib.fm_verify_attention(*qkvo, *pool, x, x, 4, None, None, 3, *tail)
    assert rc == n.FM_ERR_INVALID and "mask_mode 3" in _err(lib)
    rc = lib.fm_verify_attention(*qkvo, *pool, x, x, 4, None, None, 2, *tail)
    assert rc == n.FM_ERR_INVALID and "custom_mask" in _err(lib)
    rc = lib.fm_verify_attention(*qkvo, *pool, x, x, 4, x, None, 1, *tail)
    assert rc == n.FM_ERR_INVALID and "mask_indptr" in _err(lib)
    # verify-token strides
    bad = list(qkvo)
    bad[4] = 1020
    rc = lib.fm_verify_attention(*bad, *pool, x, x, 4, None, None, 0, *tail)
    assert rc == n.FM_ERR_INVALID and "multiples of 8" in _err(lib)
    # invalid shapes answer the workspace query with a minimal size
    assert lib.fm_verify_workspace_bytes(4, 17, 30, 8, 128, 0, 1000, 0) == 256
    assert lib.fm_verify_workspace_bytes(4, 17, 32, 8, 96, 0, 1000, 0) == 256


def test_tuning_reload(lib):
    # host only: re-reads the FLASHMAP_* overrides, touches no device
    assert lib.fm_tuning_reload() == 0
