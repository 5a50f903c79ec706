"""W4A16 int4-weight linear on HIP, gfx950.

Drop-in for ``slipstream/kernels/quant_gemm.py:23-42``: same signature
``w4a16_gemm(x, qweight, scales, qzeros, group_size)``, same format
(``slipstream/kernels/quant_ref.py:8-20``): ``qweight [out, in/8]`` int32 with
nibble ``n`` of word ``j`` holding ``q[:, 8j+n]`` at bit ``4n``; ``scales`` and
``qzeros`` ``[out, in/group_size]``; ``w = (q - zero) * scale``. ``x`` is
``[..., in]``; the result is ``[..., out]`` in ``x``'s dtype, no bias.

Device tensors only. The kernel accumulates in fp32 with the exact dequantised
weight; the reference rounds the weight to ``scales.dtype`` and then ``x.dtype``
before a 16-bit matmul, so results agree within the W4A16 tolerance
(1e-2 relative), not bit for bit.
"""

from __future__ import annotations

import torch

from slipstream_amd import _ffi
from slipstream_amd.kernels._common import require_device

# Split-K partials of the tiled kernel, one buffer per (device, stream): every call writes
# the partials it reads, so the buffer needs no initialisation and keeps no state.
_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}
# Workspace bytes the library asks for, by shape (a plan depends on the shape and the
# device's CU count only).
_WS_NEED: dict[tuple, int] = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def check_w4a16_args(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                     group_size: int) -> tuple[int, int]:
    """Shape checks of the format (``quant_ref.py:38-42``); returns ``(out, in)``."""
    if group_size <= 0 or group_size % 8 != 0:
        raise ValueError(f"group_size must be a multiple of 8, got {group_size}")
    if scales.ndim != 2 or qweight.ndim != 2:
        raise ValueError("qweight and scales must be 2-D [out, in/8] and [out, in/group_size]")
    out_features, n_groups = scales.shape
    in_features = n_groups * group_size
    if tuple(qweight.shape) != (out_features, in_features // 8):
        raise ValueError(f"qweight {tuple(qweight.shape)} does not match [out={out_features}, in/8={in_features // 8}]")
    if tuple(qzeros.shape) != tuple(scales.shape):
        raise ValueError(f"qzeros {tuple(qzeros.shape)} != scales {tuple(scales.shape)}")
    if x.shape[-1] != in_features:
        raise ValueError(f"x has {x.shape[-1]} input features, weight expects {in_features}")
    if qweight.dtype != torch.int32:
        raise ValueError(f"qweight must be int32, got {qweight.dtype}")
    return out_features, in_features


def w4a16_gemm(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
) -> torch.Tensor:
    """W4A16 linear ``x @ dequantize(W).T`` (no bias); ``[..., in] -> [..., out]`` in x's dtype."""
    out_features, in_features = check_w4a16_args(x, qweight, scales, qzeros, group_size)
    lead = x.shape[:-1]
    out = torch.empty((*lead, out_features), dtype=x.dtype, device=x.device)
    m = out.numel() // out_features if out_features else 0
    if m == 0 or out_features == 0:
        return out
    require_device("w4a16_gemm", x, qweight, scales, qzeros)
    x2 = x.reshape(m, in_features)
    if x2.stride(-1) != 1 or (in_features and x2.data_ptr() % 16):
        x2 = x2.contiguous()
    qweight = qweight.contiguous()
    scales = scales.contiguous()
    qzeros = (qzeros if qzeros.dtype == torch.int32 else qzeros.to(torch.int32)).contiguous()
    act = _ffi.dtype_code(x.dtype)
    sdt = _ffi.dtype_code(scales.dtype)
    lib = _ffi.lib()
    key = (x.device.index, m, out_features, in_features, group_size, act)
    need = _WS_NEED.get(key)
    if need is None:
        out_b = _ffi.ctypes.c_int64(0)
        _ffi.check(lib.ss_w4a16_workspace_size(m, out_features, in_features, group_size, act,
                                               _ffi.ctypes.byref(out_b)), "w4a16 workspace")
        if len(_WS_NEED) > 4096:  # many distinct shapes: start over
            _WS_NEED.clear()
        need = _WS_NEED[key] = int(out_b.value)
    stream = _ffi.stream_ptr(x.device)
    ws = _workspace(x.device, stream, need)
    o2 = out.view(m, out_features)
    status = lib.ss_w4a16_gemm(
        x2.data_ptr(),
        o2.data_ptr(),
        qweight.data_ptr(),
        scales.data_ptr(),
        qzeros.data_ptr(),
        m,
        out_features,
        in_features,
        group_size,
        x2.stride(0),
        o2.stride(0),
        act,
        sdt,
        ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0,
        stream,
    )
    _ffi.check(status, "w4a16_gemm")
    return out
