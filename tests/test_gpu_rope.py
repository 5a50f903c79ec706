"""GPU parity of the fused rotary embedding + KV scatter against the numpy oracle:
bit exact (``oracle.rope.apply_rope`` then ``oracle.paged_attention.reshape_and_cache``;
rope.py:20-36, attention_ref.py:21-39)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from oracle import rope as orope
from slipstream_amd.kernels import reshape_and_cache, rope_and_cache

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _bits(t) -> np.ndarray:
    if isinstance(t, np.ndarray):
        return t.view(np.uint32) if t.dtype.itemsize == 4 else t.view(np.uint16)
    t = t.detach().cpu().contiguous()
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()]).numpy().view(
        np.uint16 if t.element_size() == 2 else np.uint32)


def _as_dtype_array(x: np.ndarray, tdt) -> np.ndarray:
    """float64 values exactly representable in tdt -> that dtype's raw array."""
    return torch.from_numpy(x).to(tdt).contiguous().view(
        {2: torch.int16, 4: torch.int32}[torch.empty(0, dtype=tdt).element_size()]).numpy()


def _case(b, t, n_q, n_kv, d, tdt, seed, nb=64, bs=16, layout="bhtd"):
    g = torch.Generator().manual_seed(seed)
    qs = torch.randn(b, t, n_q, d, generator=g).to(tdt)
    ks = torch.randn(b, t, n_kv, d, generator=g).to(tdt)
    vs = torch.randn(b, t, n_kv, d, generator=g).to(tdt)
    cos = torch.randn(b, t, d, generator=g).to(tdt)
    sin = torch.randn(b, t, d, generator=g).to(tdt)
    kv = torch.randn(2, 2, nb, bs, n_kv, d, generator=g).to(tdt)
    slots = torch.from_numpy(np.random.default_rng(seed).permutation(nb * bs)[: b * t].astype(np.int64))
    if layout == "bhtd":  # the attention layer's transposed views (attention.py:146-160)
        q, k, v = qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2)
    elif layout == "bthd":
        q, k, v = qs, ks, vs
    else:  # packed token stream
        q, k, v = qs.reshape(b * t, n_q, d), ks.reshape(b * t, n_kv, d), vs.reshape(b * t, n_kv, d)
        cos, sin = cos.reshape(b * t, d), sin.reshape(b * t, d)
    return q, k, v, cos, sin, kv, slots


def _expected(q, k, v, cos, sin, kv, slots, layer, bs, tdt, layout):
    """oracle: q_embed and the cache after the scatter of (k_embed, v), as raw bits"""
    dt = DT[tdt]
    f = lambda x: x.double().numpy()  # noqa: E731
    if layout == "bhtd":
        c, s = f(cos)[:, None], f(sin)[:, None]
    elif layout == "bthd":
        c, s = f(cos)[:, :, None], f(sin)[:, :, None]
    else:
        c, s = f(cos)[:, None], f(sin)[:, None]
    q_emb = orope.apply_rope(f(q), c, s, dt)
    k_emb = orope.apply_rope(f(k), c, s, dt)
    if layout == "bthd":  # the scatter takes [B, n_kv, T, D] or [N, n_kv, D]
        k_emb, vv = k_emb.transpose(0, 2, 1, 3), f(v).transpose(0, 2, 1, 3)
    else:
        vv = f(v)
    cache = _as_dtype_array(kv.double().numpy(), tdt).copy()
    ora.reshape_and_cache(_as_dtype_array(k_emb, tdt), _as_dtype_array(vv, tdt), cache, slots.numpy(), layer, bs)
    return _as_dtype_array(q_emb, tdt), cache


@pytest.mark.parametrize("tdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["bhtd", "bthd", "packed"])
def test_rope_and_cache_bit_exact(device, tdt, layout):
    print(f"rope_and_cache {tdt} {layout}", flush=True)
    q, k, v, cos, sin, kv, slots = _case(3, 7, 32, 8, 128, tdt, seed=5, layout=layout)
    want_q, want_cache = _expected(q, k, v, cos, sin, kv, slots, 1, 16, tdt, layout)
    dev = [x.to(device) for x in (q, k, v, cos, sin, kv, slots)]
    qd, kd, vd, cd, sd, kvd, sld = dev
    out = rope_and_cache(qd, kd, vd, cd, sd, kvd, sld, 1, 16, unsqueeze_dim=2 if layout == "bthd" else 1)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == tdt
    assert np.array_equal(_bits(out), _bits(want_q))
    assert np.array_equal(_bits(kvd), _bits(want_cache))


@pytest.mark.parametrize("d,n_q,n_kv", [(64, 14, 2), (256, 8, 2), (6, 3, 1), (40, 4, 4)])
def test_rope_and_cache_head_dims_and_skipped_slots(device, d, n_q, n_kv):
    """Qwen (14/2, D 64), D 256, head dims whose halves are not 16-byte pieces (6, 40:
    the element-wise path), negative slots skipped."""
    tdt = torch.bfloat16
    q, k, v, cos, sin, kv, slots = _case(2, 5, n_q, n_kv, d, tdt, seed=d, nb=8, bs=4)
    slots[1] = -1
    slots[6] = -5
    want_q, want_cache = _expected(q, k, v, cos, sin, kv, slots, 0, 4, tdt, "bhtd")
    qd, kd, vd, cd, sd, kvd, sld = [x.to(device) for x in (q, k, v, cos, sin, kv, slots)]
    out = rope_and_cache(qd, kd, vd, cd, sd, kvd, sld, 0, 4)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), _bits(want_q))
    assert np.array_equal(_bits(kvd), _bits(want_cache))


def test_rope_and_cache_equals_unfused_torch_rope_then_scatter(device):
    """The decode step's shapes (Llama 32/8 heads, one token per sequence, cos/sin of
    real positions shared over the batch): the fused op equals torch's
    apply_rotary_pos_emb arithmetic on the device followed by this package's scatter."""
    tdt = torch.bfloat16
    b, n_q, n_kv, d = 64, 32, 8, 128
    g = torch.Generator().manual_seed(9)
    q = torch.randn(b, n_q, 1, d, generator=g).to(tdt).to(device)
    k = torch.randn(b, n_kv, 1, d, generator=g).to(tdt).to(device)
    v = torch.randn(b, n_kv, 1, d, generator=g).to(tdt).to(device)
    c64, s64 = orope.rope_cos_sin(np.arange(100, 100 + b)[:, None], d, 500000.0, "bf16")
    cos = torch.from_numpy(c64).to(tdt).to(device)  # [B, 1, D]
    sin = torch.from_numpy(s64).to(tdt).to(device)
    kv = torch.zeros(1, 2, 40, 16, n_kv, d, dtype=tdt, device=device)
    slots = torch.randperm(640, generator=g)[:b].to(device)
    kv_ref = kv.clone()
    cu, su = cos.unsqueeze(1), sin.unsqueeze(1)
    rot = lambda x: torch.cat((-x[..., d // 2:], x[..., : d // 2]), dim=-1)  # noqa: E731
    q_ref = q * cu + rot(q) * su
    k_ref = k * cu + rot(k) * su
    reshape_and_cache(k_ref, v, kv_ref, slots, 0, 16)
    out = rope_and_cache(q, k, v, cos, sin, kv, slots, 0, 16)
    torch.cuda.synchronize()
    assert torch.equal(out, q_ref) and torch.equal(kv, kv_ref)


def test_rope_and_cache_argument_errors(device):
    q, k, v, cos, sin, kv, slots = [x.to(device) for x in _case(1, 4, 4, 2, 16, torch.bfloat16, seed=1, nb=4, bs=4)]
    with pytest.raises(ValueError):
        rope_and_cache(q, k, v, cos, sin, kv, slots[:3], 0, 4)
    with pytest.raises(ValueError):
        rope_and_cache(q, k, v, cos.float(), sin, kv, slots, 0, 4)
    with pytest.raises(ValueError):
        rope_and_cache(q, k, v, cos, sin, kv, slots, 2, 4)
    with pytest.raises(ValueError):
        rope_and_cache(q, k, v, cos[:, :, :8], sin, kv, slots, 0, 4)
