"""Scatter K/V into the paged cache via slot_mapping (HIP, gfx950).

Drop-in for ``slipstream/kernels/reshape_and_cache.py:10-27``: same signature,
same argument checks and messages as ``_flatten_kv`` / ``reshape_and_cache_ref``
(``slipstream/kernels/attention_ref.py:8-39``), same skip of negative slots as
the Triton kernel (``slipstream/kernels/triton_paged.py:70-71``). The reference's
``[B, n_kv, T, D]`` input is read through its strides; no permuted copy is made.
Device tensors only: there is no CPU or fallback path.
"""

from __future__ import annotations

import torch

from slipstream_amd import _ffi
from slipstream_amd.kernels._common import cache_planes, require_device


def _token_view(x: torch.Tensor) -> tuple[int, int, list[int], torch.Tensor]:
    """(n_outer, n_inner, [outer, inner, head] strides, tensor with unit dim stride)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    if x.ndim == 4:  # [B, n_kv, T, D]: token n = b*T + t
        return x.shape[0], x.shape[2], [x.stride(0), x.stride(2), x.stride(1)], x
    return 1, x.shape[0], [0, x.stride(0), x.stride(1)], x


def reshape_and_cache(
    k: torch.Tensor,
    v: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layer_idx: int,
    block_size: int,
) -> None:
    """Write new K/V into ``kv_cache[layer_idx, 0/1, slot // block_size, slot % block_size]``.

    ``k``/``v`` are ``[N, n_kv, D]`` or ``[B, n_kv, T, D]`` (token order b-major,
    as ``_flatten_kv``); ``slot_mapping`` is ``[N]`` int64. Negative slots are
    skipped; so are slots past the pool (the reference would raise, a GPU write
    there would corrupt memory).
    """
    if k.shape != v.shape:
        raise ValueError(f"k/v shape mismatch {tuple(k.shape)} vs {tuple(v.shape)}")
    if k.ndim not in (3, 4):
        raise ValueError(f"k must be [N,n_kv,D] or [B,n_kv,T,D], got {tuple(k.shape)}")
    n_kv = k.shape[1]
    head_dim = k.shape[-1]
    n_tok = k.shape[0] * k.shape[2] if k.ndim == 4 else k.shape[0]
    if slot_mapping.numel() != n_tok:
        raise ValueError(f"slot_mapping {slot_mapping.numel()} != tokens {n_tok}")
    if n_tok == 0:
        return
    require_device("reshape_and_cache", k, v, kv_cache, slot_mapping)
    if kv_cache.ndim != 6:
        raise ValueError("kv_cache must be [num_layers, 2, num_blocks, block_size, n_kv, head_dim]")
    if kv_cache.shape[3] != block_size:
        raise ValueError(f"kv_cache block_size {kv_cache.shape[3]} != block_size {block_size}")
    if kv_cache.shape[4] != n_kv or kv_cache.shape[5] != head_dim:
        raise ValueError(
            f"k rows [n_kv={n_kv}, D={head_dim}] do not match the cache "
            f"[{kv_cache.shape[4]}, {kv_cache.shape[5]}]"
        )
    if k.dtype != kv_cache.dtype or v.dtype != kv_cache.dtype:
        raise ValueError(f"k/v dtype {k.dtype} != kv_cache dtype {kv_cache.dtype}")
    if not 0 <= layer_idx < kv_cache.shape[0]:
        raise ValueError(f"layer_idx {layer_idx} out of range for {kv_cache.shape[0]} layers")
    if kv_cache.stride(5) != 1:
        raise ValueError("kv_cache must have a unit head_dim stride")
    if slot_mapping.dtype != torch.int64:
        slot_mapping = slot_mapping.to(torch.int64)
    slot_mapping = slot_mapping.reshape(-1).contiguous()

    n_outer, n_inner, k_str, k = _token_view(k)
    _, _, v_str, v = _token_view(v)
    k_ptr, v_ptr, c_str = cache_planes(kv_cache, layer_idx, "reshape_and_cache", aligned=False)
    num_slots = kv_cache.shape[2] * block_size
    lib = _ffi.lib()
    status = lib.ss_reshape_and_cache(
        k.data_ptr(),
        v.data_ptr(),
        k_ptr,
        v_ptr,
        slot_mapping.data_ptr(),
        n_outer,
        n_inner,
        n_kv,
        head_dim,
        block_size,
        num_slots,
        _ffi.i64x3(*k_str),
        _ffi.i64x3(*v_str),
        _ffi.i64x3(*c_str),
        kv_cache.element_size(),
        _ffi.stream_ptr(kv_cache.device),
    )
    _ffi.check(status, "reshape_and_cache")
