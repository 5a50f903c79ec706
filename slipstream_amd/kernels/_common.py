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
    st = x.stride()
    ok = st[-1] == 1 and x.data_ptr() % 16 == 0
    if ok:
        shape = x.shape
        for d in range(x.ndim - 1):
            if shape[d] > 1 and (st[d] * elem) % 16 != 0:
                ok = False
                break
    return x if ok else x.contiguous()


def cache_planes(kv_cache: torch.Tensor, layer_idx: int, who: str,
                 aligned: bool = True) -> tuple[int, int, tuple[int, int, int]]:
    """Device addresses of layer ``layer_idx``'s K and V planes of a
    ``[L, 2, NB, bs, n_kv, D]`` pool and the planes' (block, offset, head) element
    strides, computed from the pool's strides (no view tensors). With ``aligned`` the
    planes must have a unit head_dim stride and 16-byte alignment (the attention
    kernels' condition; the scatter kernels choose their vector width themselves)."""
    st = kv_cache.stride()
    elem = kv_cache.element_size()
    base = kv_cache.data_ptr() + layer_idx * st[0] * elem
    k_ptr, v_ptr = base, base + st[1] * elem
    if aligned and (st[5] != 1 or k_ptr % 16 or v_ptr % 16):
        raise _kernel_error(f"{who}: kv_cache planes must have unit head_dim stride and 16-byte alignment")
    return k_ptr, v_ptr, (st[2], st[3], st[4])


def _kernel_error(msg: str) -> Exception:
    from slipstream_amd._ffi import KernelError

    return KernelError(msg)
