"""W4A16 linear and SwiGLU MLP modules on the HIP kernels: the quantized decode path.

``W4A16Linear`` holds a weight in the reference's format (``quant_ref.py:8-20``: packed
int32 nibbles ``[N, K/8]``, scales ``[N, K/g]``, int32 zero points ``[N, K/g]``) and runs
``w4a16_gemm`` in place of ``nn.Linear``; ``W4A16MLP`` is the reference's SwiGLU MLP
(``slipstream/models/layers/mlp.py:12-40``, ``down(silu(gate(x)) * up(x))``) on three of
them with ``fused_swiglu`` between. ``from_linear`` / ``from_mlp`` quantize dense
modules once, at load, with the reference's quantizer (``quant_ref.py:72-100``,
restated below with torch ops on the weight's device); the forward passes are the
HIP kernels only.
"""

from __future__ import annotations

import torch
from torch import nn

from slipstream_amd.kernels.norm_act import fused_swiglu
from slipstream_amd.kernels.quant_gemm import w4a16_gemm

_LEVELS = 15


def quantize_weight(weight: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``quantize_w4a16`` (``quant_ref.py:72-100``): per group of ``group_size`` inputs,
    the range [min(w, 0), max(w, 0)] in 15 steps, ``zero = round(-min / scale)``,
    ``q = clamp(round(w / scale) + zero, 0, 15)`` (round half to even), packed so that
    nibble n of word j is ``q[8j + n]`` (``quant_ref.py:45-60``). Returns
    ``(qweight int32 [N, K/8], scales [N, K/g] in weight's dtype, qzeros int32 [N, K/g])``."""
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2-D [out, in], got {tuple(weight.shape)}")
    out, k = weight.shape
    if group_size <= 0 or group_size % 8 or k % group_size:
        raise ValueError(f"group_size {group_size} must be a multiple of 8 dividing in_features {k}")
    w = weight.reshape(out, k // group_size, group_size).float()
    zero_t = torch.zeros_like(w[..., :1])
    wmin = torch.minimum(w.amin(dim=-1, keepdim=True), zero_t)
    wmax = torch.maximum(w.amax(dim=-1, keepdim=True), zero_t)
    scale = (wmax - wmin).clamp_min(1e-12) / _LEVELS
    zero = torch.round(-wmin / scale).clamp_(0, _LEVELS)
    q = torch.clamp(torch.round(w / scale) + zero, 0, _LEVELS).reshape(out, k).to(torch.int64)
    shifts = torch.arange(0, 32, 4, device=weight.device, dtype=torch.int64)
    packed = (q.view(out, k // 8, 8) << shifts).sum(dim=-1)
    qweight = packed.to(torch.int32)  # the 32-bit pattern, two's complement (quant_ref.py:57-60)
    return qweight, scale.squeeze(-1).to(weight.dtype), zero.squeeze(-1).to(torch.int32)


class W4A16Linear(nn.Module):
    """``y = x @ dequant(W).T (+ bias)`` through ``w4a16_gemm``."""

    def __init__(self, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, group_size: int,
                 bias: torch.Tensor | None = None) -> None:
        super().__init__()
        self.group_size = group_size
        self.out_features, n_groups = scales.shape
        self.in_features = n_groups * group_size
        self.register_buffer("qweight", qweight)
        self.register_buffer("scales", scales)
        self.register_buffer("qzeros", qzeros)
        self.register_buffer("bias", bias)

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 128) -> "W4A16Linear":
        qweight, scales, qzeros = quantize_weight(linear.weight.detach(), group_size)
        bias = linear.bias.detach().clone() if linear.bias is not None else None
        return cls(qweight, scales, qzeros, group_size, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = w4a16_gemm(x, self.qweight, self.scales, self.qzeros, self.group_size)
        return y + self.bias if self.bias is not None else y

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, group_size={self.group_size}"


class W4A16MLP(nn.Module):
    """SwiGLU MLP (``mlp.py:12-40``) on W4A16 linears: ``down(silu(gate(x)) * up(x))``."""

    def __init__(self, gate_proj: W4A16Linear, up_proj: W4A16Linear, down_proj: W4A16Linear) -> None:
        super().__init__()
        self.gate_proj = gate_proj
        self.up_proj = up_proj
        self.down_proj = down_proj

    @classmethod
    def from_mlp(cls, mlp: nn.Module, group_size: int = 128) -> "W4A16MLP":
        """Quantize a module with ``gate_proj`` / ``up_proj`` / ``down_proj`` linears (the
        reference's ``MLP``, HF names)."""
        return cls(W4A16Linear.from_linear(mlp.gate_proj, group_size),
                   W4A16Linear.from_linear(mlp.up_proj, group_size),
                   W4A16Linear.from_linear(mlp.down_proj, group_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(fused_swiglu(self.gate_proj(x), self.up_proj(x)))
