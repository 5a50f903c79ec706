"""Paged KV tensor and per-step metadata (layout contract of the reference).

Restates ``slipstream/memory/paged_cache.py:13-68`` (``allocate_kv_cache``,
``slots_from_pairs``, ``PagedForward``, ``pad_block_tables``) so callers of the
HIP kernels build the same tensors the reference engine builds, and adds the
packed description (``cu_seqlens`` / ``context_lens``) of one mixed step.
"""

from __future__ import annotations

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
