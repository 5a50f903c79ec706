"""Shared host-side checks for the HIP entry points."""

from __future__ import annotations

import torch


def require_device(who: str, *tensors: torch.Tensor) -> None:
    """Every tensor must live on the same HIP device (ROCm reports ``type == "cuda"``).

    The reference routes CPU tensors to its PyTorch path
    (``slipstream/kernels/paged_attention.py:31``,
    ``slipstream/kernels/reshape_and_cache.py:19``); this package is the device
    path only and refuses CPU tensors loudly instead of computing elsewhere.
    """
    dev = None
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{who}: slipstream_amd runs on HIP devices only; got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{who}: tensors on different devices ({dev} vs {t.device})")


def unit_last_stride(x: torch.Tensor) -> torch.Tensor:
    """Return ``x`` itself when its rows are 16-byte aligned and unit-strided, else a contiguous copy."""
    elem = x.element_size()
    ok = x.stride(-1) == 1 and x.data_ptr() % 16 == 0
    if ok:
        for d in range(x.ndim - 1):
            if x.shape[d] > 1 and (x.stride(d) * elem) % 16 != 0:
                ok = False
                break
    return x if ok else x.contiguous()
