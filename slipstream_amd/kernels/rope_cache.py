"""Rotary embedding of Q and K fused with the KV scatter (HIP, gfx950).

Replaces, in one launch, what ``Attention.forward`` runs before paged attention
(``slipstream/models/layers/attention.py:163,171-174``): ``apply_rotary_pos_emb``
(``slipstream/models/layers/rope.py:20-36``) on Q and K, then ``reshape_and_cache`` of
the rotated K and of V (``slipstream/kernels/reshape_and_cache.py:10-27``). The rotated K
is written only into the cache (the reference materialises ``k_embed`` and reads it back).
The arithmetic is the reference's, rounding for rounding: bit identical outputs.
Device tensors only: there is no CPU or fallback path.
"""

from __future__ import annotations

import torch

from slipstream_amd import _ffi
from slipstream_amd.kernels._common import cache_planes, require_device


def _token_layout(x: torch.Tensor, unsqueeze_dim: int) -> tuple[int, int, list[int]]:
    """(n_outer, n_inner, [outer, inner, head] strides) of a Q/K/V tensor."""
    if x.ndim == 3:  # packed [N, H, D]
        return 1, x.shape[0], [0, x.stride(0), x.stride(1)]
    if unsqueeze_dim == 1:  # [B, H, T, D]
        return x.shape[0], x.shape[2], [x.stride(0), x.stride(2), x.stride(1)]
    return x.shape[0], x.shape[1], [x.stride(0), x.stride(1), x.stride(2)]  # [B, T, H, D]


def _cs_strides(c: torch.Tensor, x: torch.Tensor) -> list[int]:
    """(outer, inner) token strides of cos/sin: ``[B, T, D]`` (or ``[N, D]`` packed)."""
    if x.ndim == 3:
        if c.ndim != 2:
            raise ValueError(f"packed q/k take cos/sin [N, head_dim], got {tuple(c.shape)}")
        return [0, c.stride(0)]
    if c.ndim != 3:
        raise ValueError(f"cos/sin must be [B, T, head_dim], got {tuple(c.shape)}")
    return [c.stride(0) if c.shape[0] > 1 else 0, c.stride(1)]


def rope_and_cache(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layer_idx: int,
    block_size: int,
    unsqueeze_dim: int = 1,
) -> torch.Tensor:
    """Return ``q_embed`` and write ``k_embed`` and ``v`` into
    ``kv_cache[layer_idx, 0/1, slot // block_size, slot % block_size]``.

    Layouts as the reference's: ``q [B, n_q, T, D]``, ``k``/``v [B, n_kv, T, D]`` with
    ``cos``/``sin [B, T, D]`` (``unsqueeze_dim=1``, ``rope.py:20-36``), or ``[B, T, H, D]``
    with ``unsqueeze_dim=2``; or a packed token stream ``q [N, n_q, D]``, ``k``/``v
    [N, n_kv, D]`` with ``cos``/``sin [N, D]``. ``slot_mapping`` is ``[N]`` int64 in token
    order (b-major); negative slots are skipped. ``cos``/``sin`` may broadcast over B
    (size 1). ``q_embed`` has q's shape and strides.
    """
    if unsqueeze_dim not in (1, 2):
        raise ValueError(f"unsqueeze_dim must be 1 or 2, got {unsqueeze_dim}")
    if q.ndim not in (3, 4) or k.ndim != q.ndim or v.shape != k.shape:
        raise ValueError(f"q/k/v must all be [B,H,T,D] / [B,T,H,D] or packed [N,H,D]; got "
                         f"{tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    head_dim = q.shape[-1]
    if k.shape[-1] != head_dim or head_dim % 2:
        raise ValueError(f"head_dim must be even and shared by q/k/v, got {head_dim} and {k.shape[-1]}")
    heads_dim = 1 if q.ndim == 3 else (1 if unsqueeze_dim == 1 else 2)
    n_q, n_kv = q.shape[heads_dim], k.shape[heads_dim]
    n_outer, n_inner, q_str = _token_layout(q, unsqueeze_dim)
    ko, ki, k_str = _token_layout(k, unsqueeze_dim)
    _, _, v_str = _token_layout(v, unsqueeze_dim)
    if (ko, ki) != (n_outer, n_inner):
        raise ValueError(f"q and k token counts differ: {tuple(q.shape)} vs {tuple(k.shape)}")
    n_tok = n_outer * n_inner
    if slot_mapping.numel() != n_tok:
        raise ValueError(f"slot_mapping {slot_mapping.numel()} != tokens {n_tok}")
    for c, name in ((cos, "cos"), (sin, "sin")):
        if c.shape[-1] != head_dim:
            raise ValueError(f"{name} last dim {c.shape[-1]} != head_dim {head_dim}")
        want = (n_inner,) if q.ndim == 3 else (n_outer, n_inner)
        got = tuple(c.shape[:-1])
        if q.ndim == 4 and got[0] == 1:
            got = (n_outer, got[1])
        if got != want:
            raise ValueError(f"{name} {tuple(c.shape)} does not cover the {n_tok} tokens of q {tuple(q.shape)}")
    dtypes = {t.dtype for t in (q, k, v, cos, sin, kv_cache)}
    if len(dtypes) != 1:
        raise ValueError(f"q, k, v, cos, sin and kv_cache must share one dtype, got {sorted(map(str, dtypes))}")
    if kv_cache.ndim != 6 or kv_cache.shape[3] != block_size:
        raise ValueError("kv_cache must be [num_layers, 2, num_blocks, block_size, n_kv, head_dim]")
    if kv_cache.shape[4] != n_kv or kv_cache.shape[5] != head_dim:
        raise ValueError(f"k rows [n_kv={n_kv}, D={head_dim}] do not match the cache "
                         f"[{kv_cache.shape[4]}, {kv_cache.shape[5]}]")
    if not 0 <= layer_idx < kv_cache.shape[0]:
        raise ValueError(f"layer_idx {layer_idx} out of range for {kv_cache.shape[0]} layers")
    out = torch.empty_like(q)
    if n_tok == 0:
        return out
    require_device("rope_and_cache", q, k, v, cos, sin, kv_cache, slot_mapping)
    unit = [t.stride(-1) == 1 for t in (q, k, v, cos, sin, out)] + [kv_cache.stride(5) == 1]
    if not all(unit):
        raise ValueError("q, k, v, cos, sin and kv_cache need a unit head_dim stride")
    if slot_mapping.dtype != torch.int64:
        slot_mapping = slot_mapping.to(torch.int64)
    slot_mapping = slot_mapping.reshape(-1).contiguous()
    _, _, o_str = _token_layout(out, unsqueeze_dim)
    k_ptr, v_ptr, c_str = cache_planes(kv_cache, layer_idx, "rope_and_cache", aligned=False)
    lib = _ffi.lib()
    status = lib.ss_rope_and_cache(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(),
        k_ptr, v_ptr, slot_mapping.data_ptr(), n_outer, n_inner, n_q, n_kv, head_dim,
        block_size, kv_cache.shape[2] * block_size,
        _ffi.i64_array(q_str), _ffi.i64_array(k_str), _ffi.i64_array(v_str), _ffi.i64_array(o_str),
        _ffi.i64_array(_cs_strides(cos, q)), _ffi.i64_array(_cs_strides(sin, q)),
        _ffi.i64x3(*c_str),
        _ffi.dtype_code(q.dtype), _ffi.stream_ptr(q.device),
    )
    _ffi.check(status, "rope_and_cache")
    return out
