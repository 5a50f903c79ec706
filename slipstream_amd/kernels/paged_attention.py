"""Paged attention (decode, prefill, packed varlen) on HIP, gfx950.

Drop-in for ``slipstream/kernels/paged_attention.py:21-52``:
``paged_attention_decode`` and ``paged_attention_prefill`` keep the reference
signature ``(q, kv_cache, block_tables, seq_lens, layer_idx, scale, block_size)``
with ``q`` ``[B, n_q, Tq, D]`` and return ``[B, Tq, n_q, D]`` in ``q``'s dtype
(``slipstream/models/layers/attention.py:88``, ``triton_paged.py:293``).
Semantics are those of ``paged_attention_ref`` (``attention_ref.py:68-89``) with
the Triton kernel's edge rules (``triton_paged.py:133-206``): negative table
entries are masked, a query row with no visible key returns zeros.

``paged_attention_varlen`` is the packed entry the reference lacks: one token
stream described by ``cu_seqlens`` / ``context_lens`` (decode and prefill rows
mixed), equal to the per-sequence calls concatenated.

Shapes: bf16, fp16 and fp32 caches, any head_dim up to 256 and any block size up to
1024 -- the range the reference's Triton decode serves (``triton_paged.py:22-23,283-284``).
bf16/fp16 with head_dim 64, 128 or 256 and power-of-two blocks of at least 4 tokens
take the MFMA kernels; every other shape takes the general kernel
(``csrc/paged_general.hip``).

There is no CPU path and no fallback: non-device tensors raise, and an
unsupported shape raises ``RuntimeError`` from the HIP library.
"""

from __future__ import annotations

import os

import torch

from slipstream_amd import _ffi
from slipstream_amd.kernels._common import cache_planes, require_device, unit_last_stride

_SUPPORTED = (torch.bfloat16, torch.float16, torch.float32)
_WS_BYTES: dict[tuple, int] = {}


def _debug() -> bool:
    """``SLIPSTREAM_DEBUG`` as read by ``slipstream/core/debug.py:7``."""
    return os.environ.get("SLIPSTREAM_DEBUG", "0") not in {"0", "false", "False", ""}


def _strides(x: torch.Tensor, dims: tuple[int, ...]) -> list[int]:
    """Element strides of ``dims``; a size-1 dim is never indexed, so it reports 0."""
    st, sh = x.stride(), x.shape
    return [st[d] if sh[d] > 1 else 0 for d in dims]


def _check_cache(kv_cache: torch.Tensor, layer_idx: int, block_size: int, head_dim: int) -> None:
    if kv_cache.ndim != 6:
        raise ValueError("kv_cache must be [num_layers, 2, num_blocks, block_size, n_kv, head_dim]")
    if kv_cache.shape[3] != block_size:
        raise ValueError(f"kv_cache block_size {kv_cache.shape[3]} != block_size {block_size}")
    if head_dim != kv_cache.shape[5]:
        raise ValueError(f"q head_dim {head_dim} != cache {kv_cache.shape[5]}")
    if not 0 <= layer_idx < kv_cache.shape[0]:
        raise ValueError(f"layer_idx {layer_idx} out of range for {kv_cache.shape[0]} layers")


def _workspace(device: torch.device, batch: int, n_q: int, n_kv: int, head_dim: int,
               max_query_len: int, dtype_code: int) -> torch.Tensor:
    """Scratch sized by the library: the decode split-K partials (by occupancy) and,
    when some sequence has prefill rows, the prefill work list (by batch and query tiles)."""
    mq = max(1, max_query_len)
    rows = mq * (n_q // n_kv)
    # decode-only launches need the same bytes for every batch; prefill ones scale with it
    key = (device.index, n_q, n_kv, head_dim, min(16, rows), dtype_code) + ((batch, mq) if rows > 16 else ())
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        out = _ffi.ctypes.c_int64(0)
        status = _ffi.lib().ss_paged_attention_workspace_size(
            batch, n_q, n_kv, head_dim, max(1, max_query_len), dtype_code, _ffi.ctypes.byref(out)
        )
        _ffi.check(status, "paged attention workspace")
        if len(_WS_BYTES) > 4096:  # many distinct prefill batch shapes: start over
            _WS_BYTES.clear()
        nbytes = _WS_BYTES[key] = max(int(out.value), 16)
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _planes(kv_cache: torch.Tensor, layer_idx: int, who: str) -> tuple[int, int, tuple[int, int, int]]:
    """K/V plane addresses and strides; the kernels index head_dim with unit stride
    (16-byte alignment only decides between the MFMA and the general kernels)."""
    if kv_cache.stride(5) != 1:
        raise _ffi.KernelError(f"{who}: kv_cache must have unit head_dim stride")
    return cache_planes(kv_cache, layer_idx, who, aligned=False)


def _int32(x: torch.Tensor) -> torch.Tensor:
    return (x if x.dtype == torch.int32 else x.to(torch.int32)).contiguous()


def paged_attention(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer_idx: int,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """Attention of ``q`` ``[B, n_q, Tq, D]`` (the last Tq tokens of each sequence)
    over the paged KV of ``seq_lens[b]`` tokens; returns ``[B, Tq, n_q, D]``."""
    if q.ndim != 4:
        raise ValueError(f"q must be [B, n_q, Tq, D], got {tuple(q.shape)}")
    batch, n_q, tq, head_dim = q.shape
    _check_cache(kv_cache, layer_idx, block_size, head_dim)
    n_kv = int(kv_cache.shape[4])
    if n_kv == 0 or n_q % n_kv != 0:
        raise ValueError(f"GQA requires n_q % n_kv == 0, got n_q={n_q} n_kv={n_kv}")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError(f"block_tables must be [B={batch}, max_blocks], got {tuple(block_tables.shape)}")
    if seq_lens.numel() != batch:
        raise ValueError(f"seq_lens has {seq_lens.numel()} entries for batch {batch}")
    if batch == 0 or n_q == 0 or tq == 0:
        return q.new_empty((batch, tq, n_q, head_dim))
    require_device("paged_attention", q, kv_cache, block_tables, seq_lens)
    if q.dtype not in _SUPPORTED or kv_cache.dtype != q.dtype:
        raise _ffi.KernelError(
            f"unsupported dtypes q={q.dtype} kv_cache={kv_cache.dtype} (bf16/fp16/fp32, equal)"
        )
    q = unit_last_stride(q)
    block_tables = _int32(block_tables)
    seq_lens = _int32(seq_lens.reshape(-1))
    k_ptr, v_ptr, c_str = _planes(kv_cache, layer_idx, "paged_attention")
    out = torch.empty((batch, tq, n_q, head_dim), device=q.device, dtype=q.dtype)
    code = _ffi.dtype_code(q.dtype)
    ws = _workspace(q.device, batch, n_q, n_kv, head_dim, tq, code)
    status = _ffi.lib().ss_paged_attention(
        q.data_ptr(),
        out.data_ptr(),
        k_ptr,
        v_ptr,
        block_tables.data_ptr(),
        seq_lens.data_ptr(),
        batch,
        n_q,
        n_kv,
        head_dim,
        tq,
        block_tables.shape[1],
        block_size,
        kv_cache.shape[2],
        _ffi.i64x3(*_strides(q, (0, 1, 2))),
        _ffi.i64x3(*_strides(out, (0, 1, 2))),
        _ffi.i64x3(*c_str),
        block_tables.stride(0),
        float(scale),
        code,
        ws.data_ptr(),
        ws.numel(),
        _ffi.stream_ptr(q.device),
    )
    _ffi.check(status, "paged_attention")
    return out


def paged_attention_decode(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer_idx: int,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """Gathers KV through the block table. ``q`` is ``[B, n_q, 1, D]`` typically.

    Mirrors ``slipstream/kernels/paged_attention.py:21-40``; any ``Tq`` is
    accepted (the causal rule of ``attention.py:46-48`` applies).
    """
    return paged_attention(q, kv_cache, block_tables, seq_lens, layer_idx, scale, block_size)


_PREFIX_WS: dict[tuple, int] = {}


def paged_attention_shared_prefix(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer_idx: int,
    scale: float,
    block_size: int,
    prefix_blocks: int,
) -> torch.Tensor:
    """Decode of ``q`` ``[B, n_q, 1, D]`` for a batch whose block tables all begin with
    the same ``prefix_blocks`` blocks (a prefix-cache hit: ``prefix_cache.py:37-56``
    shares full blocks, ``block_manager.py:91-98`` attaches them). Returns what
    ``paged_attention_decode`` (``kernels/paged_attention.py:21-40``) returns, up to
    rounding, while reading the shared prefix once for the batch instead of once per
    sequence. The caller promises ``block_tables[:, :prefix_blocks]`` equal to row 0 in
    every row (the prefix pass reads row 0) and ``seq_lens >= prefix_blocks *
    block_size`` (a shorter sequence sets ``SS_STATUS_PREFIX_SHORT`` in
    ``attention_status``); ``SLIPSTREAM_DEBUG`` checks both on the host."""
    if q.ndim != 4 or q.shape[2] != 1:
        raise ValueError(f"q must be [B, n_q, 1, D], got {tuple(q.shape)}")
    batch, n_q, _, head_dim = q.shape
    _check_cache(kv_cache, layer_idx, block_size, head_dim)
    n_kv = int(kv_cache.shape[4])
    if n_kv == 0 or n_q % n_kv != 0:
        raise ValueError(f"GQA requires n_q % n_kv == 0, got n_q={n_q} n_kv={n_kv}")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError(f"block_tables must be [B={batch}, max_blocks], got {tuple(block_tables.shape)}")
    if seq_lens.numel() != batch:
        raise ValueError(f"seq_lens has {seq_lens.numel()} entries for batch {batch}")
    if not 0 <= prefix_blocks <= block_tables.shape[1]:
        raise ValueError(f"prefix_blocks {prefix_blocks} outside [0, {block_tables.shape[1]}]")
    if batch == 0 or n_q == 0:
        return q.new_empty((batch, 1, n_q, head_dim))
    require_device("paged_attention_shared_prefix", q, kv_cache, block_tables, seq_lens)
    if q.dtype not in _SUPPORTED or kv_cache.dtype != q.dtype:
        raise _ffi.KernelError(
            f"unsupported dtypes q={q.dtype} kv_cache={kv_cache.dtype} (bf16/fp16/fp32, equal)"
        )
    q = unit_last_stride(q)
    block_tables = _int32(block_tables)
    seq_lens = _int32(seq_lens.reshape(-1))
    if _debug() and prefix_blocks > 0:
        if not bool((block_tables[:, :prefix_blocks] == block_tables[:1, :prefix_blocks]).all()):
            raise ValueError("block_tables rows differ inside the shared prefix")
        if int(seq_lens.min()) < prefix_blocks * block_size:
            raise ValueError("a sequence is shorter than the shared prefix")
    k_ptr, v_ptr, c_str = _planes(kv_cache, layer_idx, "paged_attention_shared_prefix")
    out = torch.empty((batch, 1, n_q, head_dim), device=q.device, dtype=q.dtype)
    code = _ffi.dtype_code(q.dtype)
    key = (q.device.index, batch, n_q, n_kv, head_dim, block_size, prefix_blocks, code)
    nbytes = _PREFIX_WS.get(key)
    if nbytes is None:
        size = _ffi.ctypes.c_int64(0)
        status = _ffi.lib().ss_paged_attention_shared_prefix_workspace_size(
            batch, n_q, n_kv, head_dim, block_size, prefix_blocks, code, _ffi.ctypes.byref(size)
        )
        _ffi.check(status, "shared-prefix attention workspace")
        if len(_PREFIX_WS) > 4096:
            _PREFIX_WS.clear()
        nbytes = _PREFIX_WS[key] = max(int(size.value), 16)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    status = _ffi.lib().ss_paged_attention_shared_prefix(
        q.data_ptr(),
        out.data_ptr(),
        k_ptr,
        v_ptr,
        block_tables.data_ptr(),
        seq_lens.data_ptr(),
        batch,
        n_q,
        n_kv,
        head_dim,
        block_tables.shape[1],
        block_size,
        kv_cache.shape[2],
        prefix_blocks,
        _ffi.i64x2(*_strides(q, (0, 1))),
        _ffi.i64x2(*_strides(out, (0, 2))),
        _ffi.i64x3(*c_str),
        block_tables.stride(0),
        float(scale),
        code,
        ws.data_ptr(),
        ws.numel(),
        _ffi.stream_ptr(q.device),
    )
    _ffi.check(status, "paged_attention_shared_prefix")
    return out


def paged_attention_prefill(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer_idx: int,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """Prefill chunk: mirrors ``slipstream/kernels/paged_attention.py:43-52``.

    With ``SLIPSTREAM_DEBUG`` set, a query longer than its KV (``Tq > seq_len``)
    raises ``ValueError`` as the reference's ``packed_causal_mask`` does
    (``attention.py:44-45``); that check reads ``seq_lens`` on the host, so it is
    off by default and such rows then follow the Triton rule (rows with no
    visible key are zero).
    """
    if _debug() and q.ndim == 4 and q.shape[2] > 1 and seq_lens.numel() > 0:
        shortest = int(seq_lens.min().item())
        if q.shape[2] > shortest:
            raise ValueError(f"query_len {q.shape[2]} > key_len {shortest}")
    return paged_attention(q, kv_cache, block_tables, seq_lens, layer_idx, scale, block_size)


def _check_stream(cu: torch.Tensor, total: int, max_query_len: int) -> None:
    """Host check of a packed description (reads ``cu_seqlens`` back: debug only).

    The reference raises ``ValueError`` for queries it cannot attend
    (``attention.py:44-45``); without this check the device kernels write zeros for
    rows past ``max_query_len`` and clamp a stream that runs past ``q``, and report
    both through :func:`attention_status`."""
    c = cu.cpu()
    lens = c[1:] - c[:-1]
    if int(c[0]) < 0 or bool((lens < 0).any()):
        raise ValueError("cu_seqlens must start at >= 0 and be non-decreasing")
    if int(c[-1]) > total:
        raise ValueError(f"cu_seqlens[-1] = {int(c[-1])} > {total} query tokens")
    if lens.numel() and int(lens.max()) > max_query_len:
        raise ValueError(f"query_len {int(lens.max())} > max_query_len {max_query_len}")


def attention_status(device: torch.device | int | None = None, clear: bool = True) -> int:
    """The device status word (``ss_attention_status``) after the current stream's work:
    ``SS_STATUS_QUERY_TOO_LONG`` (a packed sequence longer than ``max_query_len``, its
    extra rows written as zeros), ``SS_STATUS_STREAM_OVERRUN`` (``cu_seqlens`` past
    the token count, clamped) and ``SS_STATUS_PREFIX_SHORT`` (a shared-prefix call
    whose prefix is longer than a sequence). Synchronises the stream; 0 means no
    promise was broken."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else
                       (device if isinstance(device, int) else device.index or 0))
    flags = _ffi.ctypes.c_int(0)
    with torch.cuda.device(dev):
        status = _ffi.lib().ss_attention_status(_ffi.ctypes.byref(flags), int(bool(clear)), _ffi.stream_ptr(dev))
    _ffi.check(status, "attention_status")
    return int(flags.value)


def paged_attention_varlen(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens: torch.Tensor,
    context_lens: torch.Tensor,
    layer_idx: int,
    scale: float,
    block_size: int,
    max_query_len: int,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Packed step: ``q`` ``[T, n_q, D]`` holds every sequence's new tokens back to back.

    Sequence ``b`` owns tokens ``cu_seqlens[b]:cu_seqlens[b+1]`` and has
    ``context_lens[b]`` KV tokens (after this step's tokens were written), i.e.
    ``cu_seqlens = [0] + cumsum(query_lens)`` and ``context_lens = seq_lens`` of
    ``PagedForward`` (``slipstream/memory/paged_cache.py:35-54``).
    ``max_query_len`` must bound every ``query_len`` (host-known, no sync) and
    ``cu_seqlens[-1] <= T``. A sequence longer than ``max_query_len`` gets zeros in its
    uncovered rows and a stream past ``T`` is clamped; both set a bit that
    :func:`attention_status` reports, and ``SLIPSTREAM_DEBUG`` raises ``ValueError`` for
    them on the host before the launch. Returns ``[T, n_q, D]`` (written into ``out``
    when given: same shape and dtype as ``q``, unit head_dim stride).
    """
    if q.ndim != 3:
        raise ValueError(f"q must be [T, n_q, D], got {tuple(q.shape)}")
    total, n_q, head_dim = q.shape
    _check_cache(kv_cache, layer_idx, block_size, head_dim)
    n_kv = int(kv_cache.shape[4])
    if n_kv == 0 or n_q % n_kv != 0:
        raise ValueError(f"GQA requires n_q % n_kv == 0, got n_q={n_q} n_kv={n_kv}")
    batch = context_lens.numel()
    if cu_seqlens.numel() != batch + 1:
        raise ValueError(f"cu_seqlens must have batch+1={batch + 1} entries, got {cu_seqlens.numel()}")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError(f"block_tables must be [B={batch}, max_blocks], got {tuple(block_tables.shape)}")
    if max_query_len < 0:
        raise ValueError("max_query_len must be >= 0")
    if out is None:
        out = torch.empty((total, n_q, head_dim), device=q.device, dtype=q.dtype)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(2) != 1:
        raise ValueError(f"out must be {tuple(q.shape)} {q.dtype} on {q.device} with unit last stride")
    if batch == 0 or total == 0 or n_q == 0:
        return out
    require_device("paged_attention_varlen", q, kv_cache, block_tables, cu_seqlens, context_lens)
    if q.dtype not in _SUPPORTED or kv_cache.dtype != q.dtype:
        raise _ffi.KernelError(
            f"unsupported dtypes q={q.dtype} kv_cache={kv_cache.dtype} (bf16/fp16/fp32, equal)"
        )
    q = unit_last_stride(q)
    block_tables = _int32(block_tables)
    cu = _int32(cu_seqlens.reshape(-1))
    ctx = _int32(context_lens.reshape(-1))
    if _debug():
        _check_stream(cu, total, max_query_len)
    k_ptr, v_ptr, c_str = _planes(kv_cache, layer_idx, "paged_attention_varlen")
    code = _ffi.dtype_code(q.dtype)
    ws = _workspace(q.device, batch, n_q, n_kv, head_dim, max(1, max_query_len), code)
    status = _ffi.lib().ss_paged_attention_varlen(
        q.data_ptr(),
        out.data_ptr(),
        k_ptr,
        v_ptr,
        block_tables.data_ptr(),
        cu.data_ptr(),
        ctx.data_ptr(),
        batch,
        total,
        n_q,
        n_kv,
        head_dim,
        max_query_len,
        block_tables.shape[1],
        block_size,
        kv_cache.shape[2],
        _ffi.i64x2(*_strides(q, (0, 1))),
        _ffi.i64x2(*_strides(out, (0, 1))),
        _ffi.i64x3(*c_str),
        block_tables.stride(0),
        float(scale),
        code,
        ws.data_ptr(),
        ws.numel(),
        _ffi.stream_ptr(q.device),
    )
    _ffi.check(status, "paged_attention_varlen")
    return out
