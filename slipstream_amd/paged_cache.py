"""Paged KV tensor and per-step metadata (layout contract of the reference).

Restates ``slipstream/memory/paged_cache.py:13-68`` (``allocate_kv_cache``,
``slots_from_pairs``, ``PagedForward``, ``pad_block_tables``) so callers of the
HIP kernels build the same tensors the reference engine builds, and adds the
packed description (``cu_seqlens`` / ``context_lens``) of one mixed step.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

# slipstream/core/types.py:23-29
KV_CACHE_LAYOUT = "num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim"


def allocate_kv_cache(
    num_layers: int,
    num_blocks: int,
    block_size: int,
    num_kv_heads: int,
    head_dim: int,
    *,
    dtype: torch.dtype,
    device: torch.device,
) -> torch.Tensor:
    """Zeros ``[L, 2, num_blocks, block_size, n_kv, D]`` (``paged_cache.py:13-28``)."""
    return torch.zeros(
        (num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim), dtype=dtype, device=device
    )


def slots_from_pairs(pairs: list[tuple[int, int]], block_size: int) -> list[int]:
    """``block * block_size + offset`` (``paged_cache.py:31-32``)."""
    return [block_id * block_size + offset for block_id, offset in pairs]


def pad_block_tables(tables: list[list[int]], max_blocks: int, device: torch.device) -> torch.Tensor:
    """``[B, max_blocks]`` int32 padded with -1 (``paged_cache.py:57-68``), one upload."""
    out = torch.full((len(tables), max_blocks), -1, dtype=torch.int32)
    for i, table in enumerate(tables):
        n = min(len(table), max_blocks)
        if n:
            out[i, :n] = torch.tensor(table[:n], dtype=torch.int32)
    return out.to(device)


@dataclass
class PagedForward:
    """What attention sees for one paged step (``paged_cache.py:35-54``).

    ``slot_mapping`` indexes the new tokens written this step (``N = sum query_lens``),
    ``seq_lens`` are KV lengths after those tokens were reserved, and the queries
    of sequence ``b`` are its last ``query_lens[b]`` tokens.
    """

    kv: torch.Tensor
    block_tables: torch.Tensor  # [B, max_blocks] int32, -1 padded
    seq_lens: torch.Tensor  # [B] int32
    slot_mapping: torch.Tensor  # [N] int64
    query_lens: torch.Tensor  # [B] int32
    block_size: int
    write_kv: bool = True

    @property
    def batch(self) -> int:
        return int(self.seq_lens.shape[0])


@dataclass
class PackedStep:
    """Packed description of one mixed step: the varlen kernel's metadata.

    ``cu_seqlens = [0] + cumsum(query_lens)``; ``context_lens = seq_lens``.
    """

    cu_seqlens: torch.Tensor  # [B+1] int32
    context_lens: torch.Tensor  # [B] int32
    block_tables: torch.Tensor  # [B, max_blocks] int32
    slot_mapping: torch.Tensor  # [T] int64
    max_query_len: int
    total_tokens: int


def pack_step(fwd: PagedForward, query_lens: list[int]) -> PackedStep:
    """Packed metadata for ``fwd``; ``query_lens`` is the host copy of ``fwd.query_lens``."""
    cu = [0]
    for n in query_lens:
        cu.append(cu[-1] + int(n))
    device = fwd.seq_lens.device
    return PackedStep(
        cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device),
        context_lens=fwd.seq_lens.to(torch.int32),
        block_tables=fwd.block_tables,
        slot_mapping=fwd.slot_mapping,
        max_query_len=max(query_lens) if query_lens else 0,
        total_tokens=cu[-1],
    )


def build_packed_step(
    block_tables: torch.Tensor,
    prior_lens: torch.Tensor,
    query_lens: torch.Tensor,
    block_size: int,
    total_tokens: int,
    max_query_len: int,
) -> PackedStep:
    """Packed metadata of one step built on the device (``ss_build_step_metadata``).

    Replaces the host-list building of ``build_paged_forward`` (``paged_cache.py:71-109``):
    ``block_tables [B, max_blocks]``, ``prior_lens [B]`` (KV tokens before the step) and
    ``query_lens [B]`` stay on the device; the new tokens' slots are those
    ``append_slot`` hands out (``block_manager.py:141-159``). ``total_tokens`` and
    ``max_query_len`` are the host's own copies (the scheduler chose the lengths); no
    value is read back from the device.
    """
    from slipstream_amd import _ffi

    if block_tables.ndim != 2 or block_tables.dtype != torch.int32:
        raise ValueError(f"block_tables must be [B, max_blocks] int32, got {tuple(block_tables.shape)} "
                         f"{block_tables.dtype}")
    batch = block_tables.shape[0]
    for t, name in ((prior_lens, "prior_lens"), (query_lens, "query_lens")):
        if t.shape != (batch,) or t.dtype != torch.int32 or t.device != block_tables.device:
            raise ValueError(f"{name} must be [{batch}] int32 on {block_tables.device}, got {tuple(t.shape)} "
                             f"{t.dtype} on {t.device}")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    device = block_tables.device
    if os.environ.get("SLIPSTREAM_DEBUG", "0") not in {"0", "false", "False", ""} and batch:
        ql = query_lens.cpu().clamp_min(0)
        if int(ql.sum()) != total_tokens:
            raise ValueError(f"total_tokens {total_tokens} != sum(query_lens) {int(ql.sum())}")
        if int(ql.max()) > max_query_len:
            raise ValueError(f"query_len {int(ql.max())} > max_query_len {max_query_len}")
    # every entry is written by the kernel (no fill: the step may be graph-captured);
    # slots past sum(query_lens) get -1, so a padded slot_mapping never scatters
    cu = torch.empty(batch + 1, dtype=torch.int32, device=device) if batch else torch.zeros(1, dtype=torch.int32)
    ctx = torch.empty(batch, dtype=torch.int32, device=device)
    slots = torch.empty(max(total_tokens, 0), dtype=torch.int64, device=device)
    if not batch:
        slots.fill_(-1)
    if batch:
        if device.type != "cuda":
            raise _ffi.KernelError(f"build_packed_step: slipstream_amd runs on HIP devices only; got {device}")
        lib = _ffi.lib()
        status = lib.ss_build_step_metadata(
            block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1], prior_lens.contiguous().data_ptr(),
            query_lens.contiguous().data_ptr(), batch, block_size, cu.data_ptr(), ctx.data_ptr(),
            slots.data_ptr(), slots.numel(), _ffi.stream_ptr(device))
        _ffi.check(status, "build_step_metadata")
    return PackedStep(cu_seqlens=cu, context_lens=ctx, block_tables=block_tables, slot_mapping=slots,
                      max_query_len=max_query_len, total_tokens=total_tokens)
