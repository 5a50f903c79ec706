"""RMSNorm and SwiGLU (HIP, gfx950) behind the reference's fused-kernel seams.

Drop-ins for ``fused_rmsnorm(x, weight, residual=None, eps=1e-6)``
(``slipstream/kernels/fused_rmsnorm.py:125-137``) and ``fused_swiglu(gate, up)``
(``slipstream/kernels/fused_swiglu.py:72-79``) with the rounding of the reference's
eager paths (``rmsnorm.py:30-33``, ``mlp.py:37-40``): the residual is added in the
tensor dtype, the variance is fp32, ``x_hat`` is rounded to the dtype before the weight;
``silu(gate)`` is rounded before the product. Device tensors only.
"""

from __future__ import annotations

import torch

from slipstream_amd import _ffi
from slipstream_amd.kernels._common import require_device


def _rows(t: torch.Tensor, cols: int) -> tuple[torch.Tensor, int]:
    """2-D ``[rows, cols]`` view with a unit column stride (copied only when needed)."""
    t2 = t.reshape(-1, cols) if cols else t.reshape(-1, 1)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < cols):
        t2 = t2.contiguous()
    return t2, t2.stride(0)


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None = None,
                  eps: float = 1e-6) -> torch.Tensor:
    """``rms(x) * w``, or ``rms(x + residual) * w`` when ``residual`` is set."""
    cols = x.shape[-1]
    if weight.numel() != cols:
        raise ValueError(f"weight numel {weight.numel()} != hidden {cols}")
    if residual is not None and residual.shape != x.shape:
        raise ValueError(f"residual {tuple(residual.shape)} != x {tuple(x.shape)}")
    dtypes = {x.dtype, weight.dtype} | ({residual.dtype} if residual is not None else set())
    if len(dtypes) != 1:
        raise ValueError(f"x, weight and residual must share a dtype, got {sorted(map(str, dtypes))}")
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if x.numel() == 0:
        return out
    require_device("fused_rmsnorm", x, weight, *([residual] if residual is not None else []))
    x2, xs = _rows(x, cols)
    r2, rs = _rows(residual, cols) if residual is not None else (None, 0)
    w = weight.reshape(cols).contiguous()
    o2 = out.view(-1, cols)
    status = _ffi.lib().ss_rmsnorm(x2.data_ptr(), r2.data_ptr() if r2 is not None else None, w.data_ptr(),
                                   o2.data_ptr(), x2.shape[0], cols, xs, rs, o2.stride(0), float(eps),
                                   _ffi.dtype_code(x.dtype), _ffi.stream_ptr(x.device))
    _ffi.check(status, "fused_rmsnorm")
    return out


def fused_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up``."""
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate/up must share shape and dtype")
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    if gate.numel() == 0:
        return out
    require_device("fused_swiglu", gate, up)
    cols = gate.shape[-1]
    g2, gs = _rows(gate, cols)
    u2, us = _rows(up, cols)
    o2 = out.view(-1, cols)
    status = _ffi.lib().ss_swiglu(g2.data_ptr(), u2.data_ptr(), o2.data_ptr(), g2.shape[0], cols, gs, us,
                                  o2.stride(0), _ffi.dtype_code(gate.dtype), _ffi.stream_ptr(gate.device))
    _ffi.check(status, "fused_swiglu")
    return out
