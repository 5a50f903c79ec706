"""The no-alloc packed attention entry point (ss_paged_attention_varlen_noalloc): its
scratch is a static device array, so it must give exactly what the workspace entry
point (ss_paged_attention_varlen) gives on the same inputs -- same kernels, same
split -- on two calls in a row, the second smaller (the array keeps the first call's
contents), and refuse a call whose scratch need exceeds the array, before any device
work. Calls the C ABI directly."""

from __future__ import annotations

import ctypes

import pytest
import torch

from slipstream_amd import _ffi, workloads

pytestmark = pytest.mark.gpu


def _args(b, out):
    kc, vc = b.kv_cache[0, 0], b.kv_cache[0, 1]
    return [b.q.data_ptr(), out.data_ptr(), kc.data_ptr(), vc.data_ptr(), b.block_tables.data_ptr(),
            b.cu_seqlens.data_ptr(), b.context_lens.data_ptr(), b.batch, b.q.shape[0], b.n_q, b.n_kv,
            b.head_dim, b.max_query_len, b.block_tables.shape[1], b.block_size, b.kv_cache.shape[2],
            _ffi.i64_array([b.q.stride(0), b.q.stride(1)]), _ffi.i64_array([out.stride(0), out.stride(1)]),
            _ffi.i64_array([kc.stride(0), kc.stride(1), kc.stride(2)]), b.block_tables.stride(0), b.scale,
            _ffi.dtype_code(b.q.dtype)]


def _with_workspace(b, device):
    lib = _ffi.lib()
    need = ctypes.c_int64(0)
    _ffi.check(lib.ss_paged_attention_workspace_size(b.batch, b.n_q, b.n_kv, b.head_dim, max(1, b.max_query_len),
                                                     _ffi.dtype_code(b.q.dtype), ctypes.byref(need)), "ws")
    ws = torch.empty(max(need.value, 16), dtype=torch.uint8, device=device)
    out = torch.full_like(b.q, float("nan"))
    _ffi.check(lib.ss_paged_attention_varlen(*_args(b, out), ws.data_ptr(), ws.numel(), _ffi.stream_ptr(device)),
               "varlen")
    return out


def _no_alloc(b, device):
    out = torch.full_like(b.q, float("nan"))
    _ffi.check(_ffi.lib().ss_paged_attention_varlen_noalloc(*_args(b, out), _ffi.stream_ptr(device)), "noalloc")
    return out


def _batch(device, seed, n_prefill, chunk, n_decode):
    ctx, ql = workloads.mixed_step_lengths(seed=seed, n_prefill=n_prefill, chunk=chunk, n_decode=n_decode)
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device=device, seed=seed)
    b.cu_seqlens = b.cu_seqlens.to(torch.int32)
    b.context_lens = b.context_lens.to(torch.int32)
    return b


def test_no_alloc_equals_workspace_entry_on_two_calls(device):
    big = _batch(device, 3, n_prefill=4, chunk=512, n_decode=192)  # the C3 step shape
    small = _batch(device, 4, n_prefill=1, chunk=40, n_decode=9)
    for b in (big, small):
        want = _with_workspace(b, device)
        got = _no_alloc(b, device)
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        assert torch.equal(got, want)


def test_no_alloc_decode_only_and_empty(device):
    b = workloads.build_batch([17, 300, 1000, 64, 5000], [1] * 5, n_q=32, n_kv=8, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device=device, seed=5)
    b.cu_seqlens = b.cu_seqlens.to(torch.int32)
    b.context_lens = b.context_lens.to(torch.int32)
    got = _no_alloc(b, device)
    want = _with_workspace(b, device)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    args = _args(b, got)
    args[7] = 0  # batch 0: nothing to attend, returns at once
    assert _ffi.lib().ss_paged_attention_varlen_noalloc(*args, _ffi.stream_ptr(device)) == _ffi.SS_OK


def test_no_alloc_refuses_a_scratch_need_beyond_the_array(device):
    """A packed description whose scratch need passes the array's 64 MiB: refused with
    SS_ERR_WORKSPACE and a message, nothing launched (the pointers are never read)."""
    lib = _ffi.lib()
    batch, mq = 30000, 16384  # 30000 x 512 query tiles x 4 B = 61 MB of work list + decode partials
    need = ctypes.c_int64(0)
    _ffi.check(lib.ss_paged_attention_workspace_size(batch, 32, 8, 128, mq, _ffi.SS_DTYPE_BF16, ctypes.byref(need)),
               "ws")
    assert need.value > 64 << 20
    z2, z3 = _ffi.i64_array([4096, 128]), _ffi.i64_array([16384, 1024, 128])
    st = lib.ss_paged_attention_varlen_noalloc(16, 16, 16, 16, 16, 16, 16, batch, 1 << 20, 32, 8, 128, mq, 512, 16,
                                               100000, z2, z2, z3, 512, 0.088, _ffi.SS_DTYPE_BF16,
                                               _ffi.stream_ptr(device))
    assert st == _ffi.SS_ERR_WORKSPACE
    assert b"static scratch" in lib.ss_last_error()
