"""W4A16 linear and SwiGLU MLP modules on the HIP kernels: the quantized decode path.

``W4A16Linear`` holds a weight in the reference's format (``quant_ref.py:8-20``: packed
int32 nibbles ``[N, K/8]``, scales ``[N, K/g]``, int32 zero points ``[N, K/g]``) and runs
``w4a16_gemm`` in place of ``nn.Linear``; ``W4A16MLP`` is the reference's SwiGLU MLP
(``slipstream/models/layers/mlp.py:12-40``, ``down(silu(gate(x)) * up(x))``) on three of
them with ``fused_swiglu`` between. ``from_linear`` / ``from_mlp`` quantize dense
modules once, at load, with the reference's quantizer (``quant_ref.py:72-100``,
restated below with torch ops on the weight's device); ``from_awq`` / ``from_gptq`` /
``from_state_dict`` re-lay out the tensors of AWQ and GPTQ checkpoints into the reference
format at load (the quantized-model loading the reference plans, ``MASTERPLAN.md:620-627``).
The forward passes are the HIP kernels only.
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
    # A 0-d tensor divisor, not the Python number: on the GPU torch divides by a scalar
    # as a multiplication by its reciprocal, which differs from the reference's
    # (CPU) division in the last bit of about one scale in a few hundred.
    levels = torch.full((), float(_LEVELS), dtype=w.dtype, device=w.device)
    scale = (wmax - wmin).clamp_min(1e-12) / levels
    zero = torch.round(-wmin / scale).clamp_(0, _LEVELS)
    q = torch.clamp(torch.round(w / scale) + zero, 0, _LEVELS).reshape(out, k).to(torch.int64)
    shifts = torch.arange(0, 32, 4, device=weight.device, dtype=torch.int64)
    packed = (q.view(out, k // 8, 8) << shifts).sum(dim=-1)
    qweight = packed.to(torch.int32)  # the 32-bit pattern, two's complement (quant_ref.py:57-60)
    return qweight, scale.squeeze(-1).to(weight.dtype), zero.squeeze(-1).to(torch.int32)


# AutoAWQ's GEMM layout packs eight output columns per int32 word in this order: nibble i
# (bits 4i..4i+3) of word j holds column 8j + _AWQ_ORDER[i].
_AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _nibbles(words: torch.Tensor) -> torch.Tensor:
    """int32 words [..., w] -> int64 nibbles [..., w, 8], nibble i = bits 4i..4i+3."""
    if words.dtype != torch.int32:
        raise ValueError(f"packed int4 tensors must be int32, got {words.dtype}")
    shifts = torch.arange(0, 32, 4, device=words.device, dtype=torch.int64)
    return (words.to(torch.int64).unsqueeze(-1) >> shifts) & 0xF


def _pack_rows(q: torch.Tensor) -> torch.Tensor:
    """int64 [N, K] values 0..15 -> the reference's int32 [N, K/8] (nibble n = q[8j+n])."""
    n, k = q.shape
    shifts = torch.arange(0, 32, 4, device=q.device, dtype=torch.int64)
    return (q.view(n, k // 8, 8) << shifts).sum(dim=-1).to(torch.int32)


def _check_group_layout(k: int, n: int, scales: torch.Tensor, group_size: int, who: str) -> None:
    if group_size <= 0 or group_size % 8 or k % group_size:
        raise ValueError(f"{who}: group_size {group_size} must be a multiple of 8 dividing in_features {k}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"{who}: scales {tuple(scales.shape)} != [in/group_size={k // group_size}, out={n}]")


def awq_to_reference(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                     group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """AutoAWQ GEMM checkpoint tensors -> the reference format (``quant_ref.py:8-20``).

    AWQ stores ``qweight`` int32 ``[in, out/8]`` and ``qzeros`` int32 ``[in/g, out/8]``
    with eight output columns per word in the order of ``_AWQ_ORDER``, and ``scales``
    ``[in/g, out]``; the weight is ``W[o, i] = (q[i, o] - z[i/g, o]) * s[i/g, o]``, the
    reference's affine form. Returns ``(qweight [out, in/8], scales [out, in/g],
    qzeros [out, in/g])``, a pure re-layout (the dequantised weight is unchanged)."""
    if qweight.ndim != 2 or qzeros.ndim != 2 or scales.ndim != 2:
        raise ValueError("awq: qweight, qzeros and scales must be 2-D")
    k, n = qweight.shape[0], qweight.shape[1] * 8
    _check_group_layout(k, n, scales, group_size, "awq")
    if tuple(qzeros.shape) != (k // group_size, n // 8):
        raise ValueError(f"awq: qzeros {tuple(qzeros.shape)} != [in/group_size, out/8]")
    inv = torch.tensor(_AWQ_ORDER, device=qweight.device).argsort()  # column c%8 -> nibble
    q = _nibbles(qweight)[..., inv].reshape(k, n)
    z = _nibbles(qzeros)[..., inv.to(qzeros.device)].reshape(k // group_size, n)
    return _pack_rows(q.t().contiguous()), scales.t().contiguous(), z.t().contiguous().to(torch.int32)


def gptq_to_reference(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
                      g_idx: torch.Tensor | None = None,
                      checkpoint_format: str = "gptq") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """GPTQ checkpoint tensors (AutoGPTQ / GPTQModel layout) -> the reference format.

    GPTQ stores ``qweight`` int32 ``[in/8, out]`` (nibble i of word ``[j, o]`` is input
    row 8j+i), ``qzeros`` int32 ``[in/g, out/8]`` (nibble i of word ``[r, j]`` is output
    column 8j+i), ``scales`` ``[in/g, out]`` and ``g_idx`` (each input row's group). The
    ``"gptq"`` (v1) format stores each zero point minus one and its dequantisation adds
    the one back (``z = stored + 1``, so a stored 15 means 16); ``"gptq_v2"`` stores the
    zero point itself. Checkpoints quantized with act-order (``g_idx`` other than
    ``i // group_size``) group inputs out of order, which the reference format cannot
    express: they raise ``ValueError``."""
    if checkpoint_format not in ("gptq", "gptq_v2"):
        raise ValueError(f"gptq: checkpoint_format must be 'gptq' or 'gptq_v2', got {checkpoint_format!r}")
    if qweight.ndim != 2 or qzeros.ndim != 2 or scales.ndim != 2:
        raise ValueError("gptq: qweight, qzeros and scales must be 2-D")
    k, n = qweight.shape[0] * 8, qweight.shape[1]
    _check_group_layout(k, n, scales, group_size, "gptq")
    if tuple(qzeros.shape) != (k // group_size, n // 8):
        raise ValueError(f"gptq: qzeros {tuple(qzeros.shape)} != [in/group_size, out/8]")
    if g_idx is not None:
        want = torch.arange(k, device=g_idx.device, dtype=torch.int64) // group_size
        if g_idx.numel() != k or not torch.equal(g_idx.reshape(-1).to(torch.int64), want):
            raise ValueError("gptq: act-order g_idx (inputs grouped out of order) is not supported")
    q = _nibbles(qweight).permute(0, 2, 1).reshape(k, n)  # [in/8, out, 8] -> rows 8j+i
    z = _nibbles(qzeros).reshape(k // group_size, n)
    if checkpoint_format == "gptq":
        z = z + 1
    return _pack_rows(q.t().contiguous()), scales.t().contiguous(), z.t().contiguous().to(torch.int32)


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

    @classmethod
    def from_awq(cls, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
                 bias: torch.Tensor | None = None) -> "W4A16Linear":
        """From the tensors of an AutoAWQ GEMM checkpoint (``awq_to_reference``)."""
        return cls(*awq_to_reference(qweight, qzeros, scales, group_size), group_size, bias)

    @classmethod
    def from_gptq(cls, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
                  g_idx: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                  checkpoint_format: str = "gptq") -> "W4A16Linear":
        """From the tensors of a GPTQ checkpoint (``gptq_to_reference``)."""
        return cls(*gptq_to_reference(qweight, qzeros, scales, group_size, g_idx, checkpoint_format),
                   group_size, bias)

    @classmethod
    def from_state_dict(cls, state: dict, prefix: str, group_size: int, checkpoint_format: str = "awq",
                        device: torch.device | str | None = None) -> "W4A16Linear":
        """Load ``prefix.{qweight,qzeros,scales[,g_idx][,bias]}`` from a checkpoint's tensors
        (e.g. ``safetensors.torch.load_file``); ``checkpoint_format`` is ``"awq"``, ``"gptq"``
        or ``"gptq_v2"``."""
        def get(name: str, required: bool = True):
            t = state.get(f"{prefix}.{name}")
            if t is None and required:
                raise KeyError(f"{prefix}.{name} missing from the checkpoint")
            return t if t is None or device is None else t.to(device)
        if checkpoint_format == "awq":
            return cls.from_awq(get("qweight"), get("qzeros"), get("scales"), group_size, get("bias", False))
        return cls.from_gptq(get("qweight"), get("qzeros"), get("scales"), group_size, get("g_idx", False),
                             get("bias", False), checkpoint_format)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = w4a16_gemm(x, self.qweight, self.scales, self.qzeros, self.group_size)
        return y + self.bias if self.bias is not None else y

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, group_size={self.group_size}"


class W4A16MLP(nn.Module):
    """SwiGLU MLP (``mlp.py:12-40``) on W4A16 linears: ``down(silu(gate(x)) * up(x))``.

    The gate and up projections are held as one linear of ``2 * intermediate`` output
    rows (gate rows first): both read the same ``x``, so one launch streams both weights
    and stages ``x`` once, and ``fused_swiglu`` reads the two halves of its output in
    place. Quantization is per output row, so the fused weight is exactly the two
    weights stacked.
    """

    def __init__(self, gate_proj: W4A16Linear, up_proj: W4A16Linear, down_proj: W4A16Linear) -> None:
        super().__init__()
        if (gate_proj.in_features, gate_proj.out_features, gate_proj.group_size) != (
                up_proj.in_features, up_proj.out_features, up_proj.group_size):
            raise ValueError("gate_proj and up_proj must share in/out features and group size")
        bias = None
        if gate_proj.bias is not None or up_proj.bias is not None:
            zeros = lambda lin: torch.zeros(lin.out_features, dtype=lin.scales.dtype, device=lin.scales.device)
            bias = torch.cat([gate_proj.bias if gate_proj.bias is not None else zeros(gate_proj),
                              up_proj.bias if up_proj.bias is not None else zeros(up_proj)])
        self.intermediate = gate_proj.out_features
        self.gate_up_proj = W4A16Linear(torch.cat([gate_proj.qweight, up_proj.qweight]),
                                        torch.cat([gate_proj.scales, up_proj.scales]),
                                        torch.cat([gate_proj.qzeros, up_proj.qzeros]), gate_proj.group_size, bias)
        self.down_proj = down_proj

    @classmethod
    def from_mlp(cls, mlp: nn.Module, group_size: int = 128) -> "W4A16MLP":
        """Quantize a module with ``gate_proj`` / ``up_proj`` / ``down_proj`` linears (the
        reference's ``MLP``, HF names)."""
        return cls(W4A16Linear.from_linear(mlp.gate_proj, group_size),
                   W4A16Linear.from_linear(mlp.up_proj, group_size),
                   W4A16Linear.from_linear(mlp.down_proj, group_size))

    @classmethod
    def from_state_dict(cls, state: dict, prefix: str, group_size: int, checkpoint_format: str = "awq",
                        device: torch.device | str | None = None) -> "W4A16MLP":
        """Load ``prefix.{gate,up,down}_proj`` quantized linears from a checkpoint's tensors."""
        return cls(*(W4A16Linear.from_state_dict(state, f"{prefix}.{name}", group_size, checkpoint_format, device)
                     for name in ("gate_proj", "up_proj", "down_proj")))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gu = self.gate_up_proj(x)
        i = self.intermediate
        return self.down_proj(fused_swiglu(gu[..., :i], gu[..., i:]))
