"""The C-ABI library loads and exports every function ``include/*.h`` declares (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    names: list[str] = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ss_\w+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("ss_reshape_and_cache", "ss_paged_attention", "ss_paged_attention_varlen",
                     "ss_paged_attention_workspace_size", "ss_status_string", "ss_last_error",
                     "ss_w4a16_gemm", "ss_w4a16_workspace_size", "ss_copy_blocks", "ss_rope_and_cache",
                     "ss_build_step_metadata", "ss_rmsnorm", "ss_swiglu", "ss_attention_status"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _ffi.SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings_without_gpu():
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    assert lib.ss_status_string(0) == b"ok"
    assert b"invalid" in lib.ss_status_string(1)
    assert lib.ss_version() >= 100


def test_argument_errors_need_no_device():
    """Shape checks run on the host before any HIP call; a GQA error is SS_ERR_INVALID."""
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    z = _ffi.i64_array([0, 0, 0])
    st = lib.ss_paged_attention(None, None, None, None, None, None, 1, 6, 4, 128, 1, 1, 16, 1,
                                z, z, z, 0, 1.0, _ffi.SS_DTYPE_BF16, None, 0, None)
    assert st == _ffi.SS_ERR_INVALID
    assert b"GQA" in lib.ss_last_error()
    # head_dim above 256 (the reference's Triton bound, triton_paged.py:22) and unknown
    # dtypes are unsupported; every head_dim up to 256 and fp32 are served
    st = lib.ss_paged_attention(None, None, None, None, None, None, 1, 8, 8, 320, 1, 1, 16, 1,
                                z, z, z, 0, 1.0, _ffi.SS_DTYPE_BF16, None, 0, None)
    assert st == _ffi.SS_ERR_UNSUPPORTED
    st = lib.ss_paged_attention(None, None, None, None, None, None, 1, 8, 8, 96, 1, 1, 16, 1,
                                z, z, z, 0, 1.0, 9, None, 0, None)
    assert st == _ffi.SS_ERR_UNSUPPORTED
    st = lib.ss_paged_attention(None, None, None, None, None, None, 1, 8, 8, 96, 1, 1, 12, 1,
                                z, z, z, 0, 1.0, _ffi.SS_DTYPE_F32, None, 0, None)
    assert st == _ffi.SS_ERR_INVALID and b"null" in lib.ss_last_error()
    for dt in (_ffi.SS_DTYPE_F32, _ffi.SS_DTYPE_BF16):
        out = ctypes.c_int64(-1)
        assert lib.ss_paged_attention_workspace_size(4, 8, 2, 80, 1, dt, ctypes.byref(out)) == _ffi.SS_OK
        assert out.value > 0
    with pytest.raises(ValueError):
        _ffi.check(_ffi.SS_ERR_INVALID, "probe")
    with pytest.raises(RuntimeError):
        _ffi.check(_ffi.SS_ERR_UNSUPPORTED, "probe")
    # empty work is a no-op that touches no pointer
    st = lib.ss_reshape_and_cache(None, None, None, None, None, 0, 0, 8, 128, 16, 0, z, z, z, 2, None)
    assert st == _ffi.SS_OK
    assert isinstance(ctypes.c_int(st).value, int)


def test_w4a16_argument_errors_need_no_device():
    """Format checks of quant_ref.py:38-42 happen on the host: bad group sizes are SS_ERR_INVALID."""
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    out = ctypes.c_int64(-1)
    assert lib.ss_w4a16_workspace_size(4, 64, 256, 12, _ffi.SS_DTYPE_BF16, ctypes.byref(out)) == _ffi.SS_ERR_INVALID
    assert b"multiple of 8" in lib.ss_last_error()
    assert lib.ss_w4a16_workspace_size(4, 64, 100, 32, _ffi.SS_DTYPE_BF16, ctypes.byref(out)) == _ffi.SS_ERR_INVALID
    assert lib.ss_w4a16_workspace_size(1, 4096, 4096, 128, _ffi.SS_DTYPE_BF16, ctypes.byref(out)) == _ffi.SS_OK
    assert out.value == 0  # batch 1: the GEMV, no scratch
    # the tiled kernel splits K over workgroups: fp32 partials [ranges][m][n]
    assert lib.ss_w4a16_workspace_size(64, 4096, 14336, 128, _ffi.SS_DTYPE_BF16, ctypes.byref(out)) == _ffi.SS_OK
    # fp32 partials of two or more K ranges, then one 8-byte arrival word per output tile
    ranges, words = divmod(out.value, 64 * 4096 * 4)
    assert ranges >= 2 and 0 < words <= 8 * 4096 and words % 8 == 0
    assert lib.ss_w4a16_workspace_size(64, 4096, 14336, 128, _ffi.SS_DTYPE_F32, ctypes.byref(out)) == _ffi.SS_OK
    assert out.value == 0  # fp32 activations take the scalar kernel
    st = lib.ss_w4a16_gemm(None, None, None, None, None, 0, 8, 256, 128, 256, 8, _ffi.SS_DTYPE_BF16,
                           _ffi.SS_DTYPE_F16, None, 0, None)
    assert st == _ffi.SS_OK  # empty batch touches nothing
    st = lib.ss_w4a16_gemm(None, None, None, None, None, 1, 8, 256, 128, 256, 8, _ffi.SS_DTYPE_BF16,
                           7, None, 0, None)
    assert st == _ffi.SS_ERR_UNSUPPORTED


def test_copy_blocks_argument_errors_need_no_device():
    """Empty copies touch nothing; negative extents and null pointers are SS_ERR_INVALID."""
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    assert lib.ss_copy_blocks(None, None, 2, 0, 0, 0, 0, 0, 0, 32768, None, 0, None) == _ffi.SS_OK
    assert lib.ss_copy_blocks(None, None, -1, 0, 0, 0, 0, 0, 0, 32768, None, 1, None) == _ffi.SS_ERR_INVALID
    assert lib.ss_copy_blocks(None, None, 2, 0, 0, 4, 0, 0, 4, 32768, None, 1, None) == _ffi.SS_ERR_INVALID
    assert b"null pointer" in lib.ss_last_error()


def test_rope_and_cache_argument_errors_need_no_device():
    """Odd head_dim and unknown dtypes are rejected on the host; no tokens is a no-op."""
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    st3 = _ffi.i64_array([0, 0, 0])
    st2 = _ffi.i64_array([0, 0])
    args = lambda n, d, dt: (None, None, None, None, None, None, None, None, None, 1, n, 4, 2, d, 16, 64,  # noqa: E731
                             st3, st3, st3, st3, st2, st2, st3, dt, None)
    assert lib.ss_rope_and_cache(*args(0, 128, _ffi.SS_DTYPE_BF16)) == _ffi.SS_OK
    assert lib.ss_rope_and_cache(*args(4, 7, _ffi.SS_DTYPE_BF16)) == _ffi.SS_ERR_INVALID
    assert b"even" in lib.ss_last_error()
    assert lib.ss_rope_and_cache(*args(4, 128, 9)) == _ffi.SS_ERR_UNSUPPORTED
    assert lib.ss_rope_and_cache(*args(4, 128, _ffi.SS_DTYPE_BF16)) == _ffi.SS_ERR_INVALID  # null pointers


def test_build_step_metadata_argument_errors_need_no_device():
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    assert lib.ss_build_step_metadata(None, 0, 0, None, None, 0, 16, None, None, None, 0, None) == _ffi.SS_OK
    assert lib.ss_build_step_metadata(None, 0, 0, None, None, 2, 0, None, None, None, 0, None) == _ffi.SS_ERR_INVALID
    assert lib.ss_build_step_metadata(None, 0, 0, None, None, 2, 16, None, None, None, 0, None) == _ffi.SS_ERR_INVALID
    assert b"null pointer" in lib.ss_last_error()


def test_attention_workspace_holds_the_prefill_work_list():
    """Decode-only launches need an occupancy-sized workspace whatever the batch; with
    prefill rows the workspace also holds the prefill work list (a count plus one int32
    per sequence and 128-row query tile), and a workspace without room for it is
    SS_ERR_WORKSPACE before any HIP call."""
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    d = ctypes.c_int64(0)

    def size(batch, max_query_len):
        assert lib.ss_paged_attention_workspace_size(batch, 32, 8, 128, max_query_len, _ffi.SS_DTYPE_BF16,
                                                     ctypes.byref(d)) == _ffi.SS_OK
        return d.value

    assert size(1, 1) == size(256, 1) > 0
    assert size(196, 512) - size(4, 512) == 4 * (196 - 4) * (512 * 4 // 128)
    assert lib.ss_paged_attention_workspace_size(-1, 32, 8, 128, 512, _ffi.SS_DTYPE_BF16,
                                                 ctypes.byref(d)) == _ffi.SS_ERR_INVALID
    # a padded prefill launch (Tq = 512 rows per sequence) whose workspace only fits the decode part
    fake = 1 << 20  # 16-byte aligned, never dereferenced on the host
    q_str = _ffi.i64_array([512 * 32 * 128, 128, 32 * 128])
    o_str = _ffi.i64_array([512 * 32 * 128, 32 * 128, 128])
    c_str = _ffi.i64_array([16 * 8 * 128, 8 * 128, 128])
    st = lib.ss_paged_attention(fake, fake, fake, fake, fake, fake, 4, 32, 8, 128, 512, 64, 16, 1024,
                                q_str, o_str, c_str, 64, 1.0, _ffi.SS_DTYPE_BF16, fake, size(4, 1), None)
    assert st == _ffi.SS_ERR_WORKSPACE, lib.ss_last_error()
    assert b"work list" in lib.ss_last_error()


def test_shared_prefix_argument_errors_need_no_device():
    """The shared-prefix entry checks GQA, batch and prefix_blocks on the host; an empty
    batch returns SS_OK before any HIP call; the Python wrapper refuses CPU tensors."""
    import torch

    from slipstream_amd import _ffi
    from slipstream_amd.kernels import paged_attention_shared_prefix

    lib = _ffi.lib()
    out = ctypes.c_int64(0)
    bf16 = _ffi.SS_DTYPE_BF16
    size = lib.ss_paged_attention_shared_prefix_workspace_size
    assert size(-1, 28, 4, 128, 16, 8, bf16, ctypes.byref(out)) == _ffi.SS_ERR_INVALID
    assert size(4, 28, 4, 128, 16, -1, bf16, ctypes.byref(out)) == _ffi.SS_ERR_INVALID
    assert size(4, 6, 4, 128, 16, 8, bf16, ctypes.byref(out)) == _ffi.SS_ERR_INVALID
    z2, z3 = _ffi.i64_array([0, 0]), _ffi.i64_array([0, 0, 0])

    def call(batch, n_q, n_kv, max_blocks, prefix_blocks):
        return lib.ss_paged_attention_shared_prefix(None, None, None, None, None, None, batch, n_q, n_kv, 128,
                                                    max_blocks, 16, 64, prefix_blocks, z2, z2, z3, max_blocks,
                                                    1.0, bf16, None, 0, None)

    assert call(4, 28, 4, 8, 9) == _ffi.SS_ERR_INVALID
    assert b"prefix_blocks" in lib.ss_last_error()
    assert call(4, 28, 4, 8, -1) == _ffi.SS_ERR_INVALID
    assert call(4, 6, 4, 8, 2) == _ffi.SS_ERR_INVALID
    assert b"GQA" in lib.ss_last_error()
    assert call(0, 28, 4, 8, 2) == _ffi.SS_OK
    q = torch.zeros(4, 28, 1, 128, dtype=torch.bfloat16)
    kv = torch.zeros(1, 2, 64, 16, 4, 128, dtype=torch.bfloat16)
    bt = torch.zeros(4, 8, dtype=torch.int32)
    lens = torch.full((4,), 64, dtype=torch.int32)
    with pytest.raises(ValueError, match="prefix_blocks"):
        paged_attention_shared_prefix(q, kv, bt, lens, 0, 0.1, 16, 9)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        paged_attention_shared_prefix(q, kv, bt, lens, 0, 0.1, 16, 2)


def test_attention_status_null_pointer_needs_no_device():
    from slipstream_amd import _ffi

    lib = _ffi.lib()
    assert lib.ss_attention_status(None, 1, None) == _ffi.SS_ERR_INVALID
    assert b"null" in lib.ss_last_error()


def test_debug_checks_of_a_packed_step_run_on_the_host(monkeypatch):
    """SLIPSTREAM_DEBUG: a slot count that is not the step's token count, or a query
    longer than max_query_len, raises ValueError before any device work (the reference
    raises for queries it cannot attend, attention.py:44-45)."""
    import torch

    from slipstream_amd.kernels.paged_attention import _check_stream
    from slipstream_amd.paged_cache import build_packed_step

    monkeypatch.setenv("SLIPSTREAM_DEBUG", "1")
    bt = torch.zeros((2, 4), dtype=torch.int32)
    prior = torch.tensor([3, 0], dtype=torch.int32)
    ql = torch.tensor([1, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="total_tokens"):
        build_packed_step(bt, prior, ql, 16, 9, 5)
    with pytest.raises(ValueError, match="max_query_len"):
        build_packed_step(bt, prior, ql, 16, 6, 4)
    cu = torch.tensor([0, 1, 6], dtype=torch.int32)
    _check_stream(cu, 6, 5)
    with pytest.raises(ValueError, match="max_query_len"):
        _check_stream(cu, 6, 4)
    with pytest.raises(ValueError, match="query tokens"):
        _check_stream(cu, 5, 5)
    with pytest.raises(ValueError, match="non-decreasing"):
        _check_stream(torch.tensor([0, 4, 2], dtype=torch.int32), 6, 5)
