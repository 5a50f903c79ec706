"""numpy oracle of the rotary embedding fused with the KV scatter (test infrastructure).

Restates slipstream/models/layers/rope.py:13-36 (``rotate_half``,
``apply_rotary_pos_emb``) with the rounding of the reference's torch ops: every
elementwise op on bf16/fp16 tensors computes in fp32 and rounds to the tensor dtype
(nearest even), and fp32 ops round each product and sum separately. So for x with
halves (x1, x2) and cos/sin halves (c1, c2), (s1, s2):
    out1 = r(r(x1 * c1) + r(-x2 * s1)),  out2 = r(r(x2 * c2) + r(x1 * s2)),
where a product of two bf16/fp16 values is exact in fp32 and a sum is rounded to
fp32 first (then to the dtype), as torch does. The scatter is
``paged_attention.reshape_and_cache`` of this package.
"""

from __future__ import annotations

import numpy as np

from oracle.quant import round_to_bf16


def rotate_half(x: np.ndarray) -> np.ndarray:
    """rope.py:13-17: ``cat(-x[..., D/2:], x[..., :D/2])``."""
    half = x.shape[-1] // 2
    return np.concatenate((-x[..., half:], x[..., :half]), axis=-1)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float64 values -> the nearest ``dtype`` value via fp32 (as torch rounds an op's
    fp32 result), returned as float64."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == "bf16":
        return round_to_bf16(f).astype(np.float64)
    if dtype == "f16":
        return f.astype(np.float16).astype(np.float64)
    if dtype == "f32":
        return f.astype(np.float64)
    raise ValueError(dtype)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """``x * cos + rotate_half(x) * sin`` with the reference's rounding (rope.py:33-35).

    ``x``, ``cos``, ``sin`` hold values exactly representable in ``dtype`` (float64
    arrays, broadcastable). For fp32 the products are rounded to fp32 before the sum.
    """
    r = lambda a: round_to(a, dtype)  # noqa: E731
    return r(r(x * cos) + r(rotate_half(x) * sin))


def rope_cos_sin(positions: np.ndarray, head_dim: int, theta: float, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """Default RoPE tables (rope.py:39-42,96-106) in float64, rounded to ``dtype``:
    inv_freq[i] = theta^(-2i/D), emb = cat(pos * inv_freq, pos * inv_freq). (The
    reference forms them in fp32; tests feed the kernels whatever tables they use.)"""
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    freqs = np.asarray(positions, dtype=np.float64)[..., None] * inv
    emb = np.concatenate((freqs, freqs), axis=-1)
    return round_to(np.cos(emb), dtype), round_to(np.sin(emb), dtype)
