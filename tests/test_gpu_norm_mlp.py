"""RMSNorm / SwiGLU kernels against the reference's eager arithmetic (torch ops on the
device, rmsnorm.py:30-33, fused_rmsnorm.py:73-82, mlp.py:37-40), and the quantized SwiGLU
MLP (W4A16 linears + fused SwiGLU) against a fp32 dequantise-then-matmul reference."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from slipstream_amd.kernels import fused_rmsnorm, fused_swiglu
from slipstream_amd.quantized import W4A16Linear, W4A16MLP

pytestmark = pytest.mark.gpu

# bf16/fp16: one unit in the last place. fp32: the reference's own fused-kernel
# tolerance (test_fused_kernels.py:19, 1e-5), since there the fp32 sum order and
# rsqrt / exp differences are not hidden by a final rounding.
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 1e-5}


def _close_within_one_ulp(got: torch.Tensor, want: torch.Tensor, what: str) -> None:
    """Equal, except where the reference's fp32 sum order / rsqrt / exp make the value
    before the final rounding differ in its last bits: then one unit in the last place
    (16-bit), and at least 99 % of the elements bit-identical."""
    g, w = got.float(), want.float()
    tol = ULP[got.dtype] * w.abs() + (1e-6 if got.dtype == torch.float32 else 1e-30)
    bad = (g - w).abs() > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of tolerance"
    if got.dtype != torch.float32:
        exact = (g == w).float().mean().item()
        assert exact > 0.99, f"{what}: only {exact:.4f} of the elements bit-identical"


def _eager_rmsnorm(x, w, residual, eps):
    if residual is not None:
        x = x + residual
    x32 = x.float()
    return w * (x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)).to(x.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 7, 4096), (5, 896), (3, 16), (2, 14336), (3, 40960)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_matches_eager(device, dtype, shape, with_residual):
    """Rows past 2048 16-byte pieces (fp32 above 8192 columns, 16-bit above 16384) take
    the two-pass kernel."""
    g = torch.Generator(device=device).manual_seed(shape[-1])
    x = torch.randn(shape, generator=g, device=device).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g, device=device)).to(dtype)
    r = torch.randn(shape, generator=g, device=device).to(dtype) if with_residual else None
    _close_within_one_ulp(fused_rmsnorm(x, w, r, 1e-6), _eager_rmsnorm(x, w, r, 1e-6), f"rmsnorm {shape} {dtype}")


def test_rmsnorm_reference_test_shape(device):
    """test_fused_kernels.py:13-19: x [2, 8, 16], unit weight, fp32 -- atol/rtol 1e-5."""
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(2, 8, 16, generator=g, device=device)
    w = torch.ones(16, device=device)
    torch.testing.assert_close(fused_rmsnorm(x, w, eps=1e-6), _eager_rmsnorm(x, w, None, 1e-6), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(3, 14336), (64, 4864), (1, 8)])
def test_swiglu_matches_eager(device, dtype, shape):
    g = torch.Generator(device=device).manual_seed(shape[0])
    gate = (3 * torch.randn(shape, generator=g, device=device)).to(dtype)
    up = torch.randn(shape, generator=g, device=device).to(dtype)
    _close_within_one_ulp(fused_swiglu(gate, up), F.silu(gate) * up, f"swiglu {shape} {dtype}")


def test_strided_rows(device):
    """Row views of wider buffers (a fused gate/up projection's halves)."""
    g = torch.Generator(device=device).manual_seed(3)
    gu = torch.randn(6, 2 * 4096, generator=g, device=device).to(torch.bfloat16)
    gate, up = gu[:, :4096], gu[:, 4096:]
    _close_within_one_ulp(fused_swiglu(gate, up), F.silu(gate) * up, "swiglu strided")
    w = torch.ones(4096, device=device, dtype=torch.bfloat16)
    _close_within_one_ulp(fused_rmsnorm(gate, w), _eager_rmsnorm(gate, w, None, 1e-6), "rmsnorm strided")


@pytest.mark.parametrize("m", [1, 16, 64])
def test_quantized_mlp_matches_dense_dequant(device, m):
    """Qwen2.5-0.5B MLP shape (896 -> 4864 -> 896), g = 128: the W4A16 MLP (gate and up
    fused into one launch) equals the separately quantized gate / up / down weights
    dequantised and run densely in fp32 (1e-2 relative)."""
    torch.manual_seed(m)
    hid, inter = 896, 4864
    mlp = torch.nn.Module()
    mlp.gate_proj = torch.nn.Linear(hid, inter, bias=False)
    mlp.up_proj = torch.nn.Linear(hid, inter, bias=False)
    mlp.down_proj = torch.nn.Linear(inter, hid, bias=False)
    mlp = mlp.to(device=device, dtype=torch.bfloat16)
    q = W4A16MLP.from_mlp(mlp, 128)
    parts = [W4A16Linear.from_linear(lin, 128) for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj)]
    x = torch.randn(m, hid, device=device, dtype=torch.bfloat16)
    y = q(x)

    def deq(lin: W4A16Linear) -> torch.Tensor:
        shifts = torch.arange(0, 32, 4, device=device)
        nib = (lin.qweight.to(torch.int64)[..., None] >> shifts) & 15
        qv = nib.reshape(lin.out_features, lin.in_features).float()
        s = lin.scales.float().repeat_interleave(lin.group_size, dim=1)
        z = lin.qzeros.float().repeat_interleave(lin.group_size, dim=1)
        return (qv - z) * s

    g = x.float() @ deq(parts[0]).T
    u = x.float() @ deq(parts[1]).T
    h = (F.silu(g.to(torch.bfloat16)) * u.to(torch.bfloat16)).float()
    ref = h @ deq(parts[2]).T
    rel = ((y.float() - ref).norm() / ref.norm()).item()
    assert rel < 1e-2, rel


@pytest.mark.parametrize("fmt", ["awq", "gptq"])
def test_checkpoint_linear_matches_checkpoint_weight(device, fmt):
    """A linear loaded from AWQ / GPTQ tensors (4096 -> 1024, g = 128, every zero point
    0..15, so GPTQ v1 also reads 16) equals x @ W.T with the weight the checkpoint
    describes, W[o, i] = (q[i, o] - z[i/g, o]) * s[i/g, o], in fp32 (1e-2 relative)."""
    from slipstream_amd.quantized import _AWQ_ORDER
    k, n, g, m = 4096, 1024, 128, 16
    gen = torch.Generator().manual_seed(7)
    q = torch.randint(0, 16, (k, n), generator=gen)
    z = torch.randint(0, 16, (k // g, n), generator=gen)
    s = (torch.rand(k // g, n, generator=gen) * 0.015 + 0.005).half()
    shifts = torch.arange(0, 32, 4)

    def pack(v: torch.Tensor) -> torch.Tensor:  # [..., 8] nibbles -> int32 words
        return ((v & 15) << shifts).sum(-1).to(torch.int64).sub(
            ((v & 15) << shifts).sum(-1).ge(1 << 31).to(torch.int64) << 32).to(torch.int32)

    if fmt == "awq":
        order = torch.tensor(_AWQ_ORDER)
        state = {"p.qweight": pack(q.view(k, n // 8, 8)[..., order]),
                 "p.qzeros": pack(z.view(k // g, n // 8, 8)[..., order]), "p.scales": s}
        zt = z
    else:
        state = {"p.qweight": pack(q.view(k // 8, 8, n).permute(0, 2, 1)),
                 "p.qzeros": pack((z - 1).view(k // g, n // 8, 8)), "p.scales": s,
                 "p.g_idx": torch.arange(k, dtype=torch.int32) // g}
        zt = torch.where(z == 0, torch.full_like(z, 16), z)  # v1: stored z-1, read back + 1
    lin = W4A16Linear.from_state_dict(state, "p", g, fmt, device=device)
    w = ((q - zt.repeat_interleave(g, 0)).float() * s.float().repeat_interleave(g, 0)).T.to(device)
    x = torch.randn(m, k, device=device, dtype=torch.bfloat16)
    ref = x.float() @ w.T
    y = lin(x)
    rel = ((y.float() - ref).norm() / ref.norm()).item()
    assert rel < 1e-2, rel
