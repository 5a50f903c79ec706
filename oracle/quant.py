"""numpy oracle of the W4A16 format and linear (test infrastructure).

Restates slipstream/kernels/quant_ref.py:38-133: group-wise asymmetric int4,
``qweight[o, j]`` holds ``q[o, 8j + n]`` in bits ``4n .. 4n+3`` (stored as int32
two's complement), ``scales``/``qzeros`` are ``[out, in // group_size]``, and
``w_hat = (q - zero) * scale``.
"""

from __future__ import annotations

import numpy as np

_LEVELS = 15


def check_shapes(in_features: int, group_size: int) -> None:
    """quant_ref.py:38-42."""
    if group_size % 8 != 0:
        raise ValueError(f"group_size must be a multiple of 8, got {group_size}")
    if in_features % group_size != 0:
        raise ValueError(f"in_features {in_features} not divisible by group_size {group_size}")


def pack_int4(q: np.ndarray) -> np.ndarray:
    """``[out, in]`` nibbles -> ``[out, in // 8]`` int32 (quant_ref.py:45-60)."""
    q = np.asarray(q)
    if q.ndim != 2:
        raise ValueError(f"q must be 2-D [out, in], got {q.shape}")
    out, in_features = q.shape
    if in_features % 8 != 0:
        raise ValueError(f"in_features {in_features} not divisible by 8")
    q64 = (q.astype(np.uint64) & 0xF).reshape(out, in_features // 8, 8)
    word = np.zeros((out, in_features // 8), dtype=np.uint64)
    for n in range(8):
        word |= q64[:, :, n] << np.uint64(4 * n)
    return word.astype(np.uint32).view(np.int32)


def unpack_int4(qweight: np.ndarray, in_features: int) -> np.ndarray:
    """Inverse of :func:`pack_int4`: int32 words -> ``[out, in]`` int64 in 0..15 (quant_ref.py:63-69)."""
    w = np.asarray(qweight).astype(np.int64) & 0xFFFFFFFF
    shifts = (np.arange(8, dtype=np.int64) * 4)[None, None, :]
    nib = (w[:, :, None] >> shifts) & 0xF
    return nib.reshape(w.shape[0], in_features)


def quantize_w4a16(weight: np.ndarray, group_size: int):
    """``weight [out, in]`` -> ``(qweight, scales float32, qzeros int32)`` (quant_ref.py:72-100).

    Float32 arithmetic and round-half-to-even, the range widened to include 0.
    """
    weight = np.asarray(weight)
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2-D [out, in], got {weight.shape}")
    out, in_features = weight.shape
    check_shapes(in_features, group_size)
    g = in_features // group_size
    w = weight.reshape(out, g, group_size).astype(np.float32)
    wmin = np.minimum(w.min(axis=-1, keepdims=True), np.float32(0))
    wmax = np.maximum(w.max(axis=-1, keepdims=True), np.float32(0))
    scale = np.maximum(wmax - wmin, np.float32(1e-12)) / np.float32(_LEVELS)
    zero = np.clip(np.round(-wmin / scale), 0, _LEVELS)
    q = np.clip(np.round(w / scale) + zero, 0, _LEVELS).reshape(out, in_features)
    return pack_int4(q.astype(np.int64)), scale[..., 0].astype(np.float32), zero[..., 0].astype(np.int32)


def dequantize_w4a16(qweight: np.ndarray, scales: np.ndarray, qzeros: np.ndarray,
                     group_size: int) -> np.ndarray:
    """Exact ``(q - zero) * scale`` in float64, ``[out, in]`` (quant_ref.py:103-116 before its cast)."""
    out, g = scales.shape
    in_features = g * group_size
    q = unpack_int4(qweight, in_features).reshape(out, g, group_size).astype(np.float64)
    s = np.asarray(scales, dtype=np.float64).reshape(out, g, 1)
    z = np.asarray(qzeros, dtype=np.float64).reshape(out, g, 1)
    return ((q - z) * s).reshape(out, in_features)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32 (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def dequantize_faithful(qweight: np.ndarray, scales: np.ndarray, qzeros: np.ndarray,
                        group_size: int, scale_dtype=np.float16, act_is_bf16: bool = True) -> np.ndarray:
    """The reference's rounding chain: fp32 ``(q - z) * s`` -> ``scales.dtype`` -> activation dtype.

    quant_ref.py:112-116 then ``.to(x.dtype)`` at :132.
    """
    w = dequantize_w4a16(qweight, scales, qzeros, group_size).astype(np.float32)
    w = w.astype(scale_dtype).astype(np.float32)
    return round_to_bf16(w) if act_is_bf16 else w


def w4a16_gemm(x: np.ndarray, qweight: np.ndarray, scales: np.ndarray, qzeros: np.ndarray,
               group_size: int) -> np.ndarray:
    """``x [..., in] @ dequant(W).T`` in float64 with the exact dequantised weight (quant_ref.py:119-133)."""
    w = dequantize_w4a16(qweight, scales, qzeros, group_size)
    return np.asarray(x, dtype=np.float64) @ w.T
