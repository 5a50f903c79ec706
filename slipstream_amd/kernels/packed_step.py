"""One packed attention step of a layer (HIP, gfx950): what ``Attention.forward`` does for
a paged step (``slipstream/models/layers/attention.py:163-184``: rotary embedding, KV
scatter, then decode or prefill attention per call), for every sequence of a mixed
step at once. Built from ``rope_and_cache`` (RoPE fused with the scatter) and
``paged_attention_varlen``; with the step's metadata from
``slipstream_amd.paged_cache.build_packed_step`` nothing is read back to the host, so
a decode step captures into a graph and replays with new lengths.
"""

from __future__ import annotations

import torch

from slipstream_amd.kernels.paged_attention import paged_attention_varlen
from slipstream_amd.kernels.rope_cache import rope_and_cache
from slipstream_amd.paged_cache import PackedStep


def packed_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    kv_cache: torch.Tensor,
    step: PackedStep,
    layer_idx: int,
    scale: float,
    block_size: int,
    write_kv: bool = True,
) -> torch.Tensor:
    """``q [T, n_q, D]``, ``k``/``v [T, n_kv, D]``, ``cos``/``sin [T, D]`` for the step's T
    tokens (sequence-major, as ``cu_seqlens``); returns the attention output
    ``[T, n_q, D]``. ``write_kv=False`` (the reference's replay mode, ``PagedForward``)
    rotates Q only and leaves the cache as it is."""
    if write_kv:
        q_rot = rope_and_cache(q, k, v, cos, sin, kv_cache, step.slot_mapping, layer_idx, block_size)
    else:
        q_rot = _rope_only(q, cos, sin, kv_cache, layer_idx, block_size)
    return paged_attention_varlen(q_rot, kv_cache, step.block_tables, step.cu_seqlens, step.context_lens,
                                  layer_idx, scale, block_size, step.max_query_len)


def _rope_only(q: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, kv_cache: torch.Tensor, layer_idx: int,
               block_size: int) -> torch.Tensor:
    """Q rotation without touching the cache: the fused kernel with every slot skipped."""
    n_kv, d = kv_cache.shape[4], kv_cache.shape[5]
    dummy = torch.empty((q.shape[0], n_kv, d), dtype=q.dtype, device=q.device)
    skip = torch.full((q.shape[0],), -1, dtype=torch.int64, device=q.device)
    return rope_and_cache(q, dummy, dummy, cos, sin, kv_cache, skip, layer_idx, block_size)
