"""Pins of ``oracle/reference_path.py``, the reference's own CPU path restated in torch
(``slipstream/kernels/attention_ref.py:21-89``, ``models/layers/attention.py:20-88``):
the timed CPU baseline and the dtype-faithful secondary check of the GPU tests.

Each check is chosen so that a plausible slip fails it: the scatter bit for bit
against the numpy oracle (a swapped block/offset or K/V plane), the gather in closed
form (truncation to the table, the reference's negative-index hole), attention in
float32 against the float64 oracle and torch's SDPA (a wrong GQA head map, mask
offset or scale), and in bf16 / fp16 within those types' rounding bounds.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_attention as ora
from oracle import reference_path as ref
from slipstream_amd import workloads

# bf16 keeps 8 significant bits, fp16 11: the reference's path rounds the scores, the
# scaled scores, the softmax weights and the output to the dtype, a few units of
# 2^-8 (2^-11) of the output's scale. Measured: 2.3e-3 (bf16) and 1.9e-4 (fp16)
# worst over the shapes below.
TOL = {torch.bfloat16: (6e-3, 2e-2), torch.float16: (1e-3, 4e-3), torch.float32: (1e-5, 1e-5)}


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().numpy().astype(np.float64)


def _tables(b) -> torch.Tensor:
    t = torch.full((len(b.tables_host), b.block_tables.shape[1]), -1, dtype=torch.int32)
    for i, row in enumerate(b.tables_host):
        t[i, : len(row)] = torch.tensor(row, dtype=torch.int32)
    return t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["flat", "bnhd"])
def test_scatter_bit_exact_against_oracle(dtype, layout):
    g = torch.Generator().manual_seed(1)
    nb, bs, n_kv, d = 40, 16, 4, 64
    kv = torch.randn(2, 2, nb, bs, n_kv, d, generator=g).to(dtype)
    if layout == "flat":
        k = torch.randn(37, n_kv, d, generator=g).to(dtype)
    else:  # the reference's [B, n_kv, T, D] input, token b*T + t
        k = torch.randn(5, n_kv, 7, d, generator=g).to(dtype)
    v = torch.randn(k.shape, generator=g).to(dtype)
    n = k.shape[0] if layout == "flat" else 35
    slots = torch.randperm(nb * bs, generator=g)[:n]
    want = kv.view(torch.int16).numpy().copy()
    kb, vb = k.view(torch.int16).numpy(), v.view(torch.int16).numpy()
    ora.reshape_and_cache(kb, vb, want, slots.numpy(), 1, bs)
    ref.scatter(k, v, kv, slots, 1, bs)
    assert np.array_equal(kv.view(torch.int16).numpy(), want)


def test_scatter_length_errors():
    kv = torch.zeros(1, 2, 4, 16, 2, 8)
    with pytest.raises(ValueError, match="slot_mapping"):
        ref.scatter(torch.zeros(3, 2, 8), torch.zeros(3, 2, 8), kv, torch.zeros(2, dtype=torch.long), 0, 16)
    with pytest.raises(ValueError, match="mismatch"):
        ref.scatter(torch.zeros(3, 2, 8), torch.zeros(2, 2, 8), kv, torch.zeros(3, dtype=torch.long), 0, 16)
    ref.scatter(torch.zeros(0, 2, 8), torch.zeros(0, 2, 8), kv, torch.zeros(0, dtype=torch.long), 0, 16)


def test_gather_copies_pages_in_table_order():
    g = torch.Generator().manual_seed(2)
    kv = torch.randn(1, 2, 30, 16, 2, 8, generator=g).to(torch.bfloat16)
    table = torch.tensor([7, 3, 22, 0], dtype=torch.int32)
    k, v = ref.gather(kv, 0, table, 50, 16)
    assert k.shape == (1, 2, 50, 8)
    ok, ov, valid = ora.gather_kv(kv.view(torch.int16).numpy(), 0, table.numpy(), 50, 16)
    assert valid.all()
    assert np.array_equal(k[0].permute(1, 0, 2).contiguous().view(torch.int16).numpy(), ok)
    assert np.array_equal(v[0].permute(1, 0, 2).contiguous().view(torch.int16).numpy(), ov)


def test_gather_truncates_to_the_table_and_reads_a_hole_from_the_last_block():
    """attention_ref.py:50-51: n_blocks = min(ceil(len / bs), #entries >= 0), then the
    first n_blocks entries as they are -- a -1 among them is Python's last block."""
    kv = torch.arange(6 * 4, dtype=torch.float32).reshape(1, 1, 6, 4, 1, 1).expand(1, 2, 6, 4, 1, 1).contiguous()
    k, _ = ref.gather(kv, 0, torch.tensor([2, 4], dtype=torch.int32), 13, 4)  # table covers 8 of 13
    assert k.flatten().tolist() == [8, 9, 10, 11, 16, 17, 18, 19]
    k, _ = ref.gather(kv, 0, torch.tensor([2, -1, 3, 1], dtype=torch.int32), 13, 4)
    # 3 valid entries -> 3 blocks: 2, then -1 (= block 5), then 3; 12 tokens of the 13
    assert k.flatten().tolist() == [8, 9, 10, 11, 20, 21, 22, 23, 12, 13, 14, 15]
    k, v = ref.gather(kv, 0, torch.tensor([-1, -1], dtype=torch.int32), 5, 4)
    assert k.shape == (1, 1, 0, 1) and v.shape == (1, 1, 0, 1)
    k, _ = ref.gather(kv, 0, torch.tensor([1], dtype=torch.int32), 0, 4)
    assert k.shape[2] == 0


def test_eager_raises_for_a_query_longer_than_its_keys():
    q = torch.zeros(1, 2, 3, 8)
    kv = torch.zeros(1, 1, 2, 8)
    with pytest.raises(ValueError, match="query_len 3 > key_len 2"):
        ref.eager(q, kv, kv, 1.0)


SHAPES = [  # (n_q, n_kv, D, Tq): C1, Llama-3-8B, Qwen2.5-7B, MHA with a causal chunk
    (14, 2, 64, 1), (32, 8, 128, 1), (28, 4, 128, 3), (8, 8, 64, 9),
]


@pytest.mark.parametrize("n_q,n_kv,d,tq", SHAPES)
def test_paged_attention_float32_equals_oracle_and_sdpa(n_q, n_kv, d, tq):
    """The same code in float32: its indexing (GQA map, causal offset, scale, table walk)
    against the float64 oracle and, independently, torch's SDPA in float64."""
    ctx = [40, 300, 17, 129, 64]
    b = workloads.build_batch(ctx, [tq] * len(ctx), n_q=n_q, n_kv=n_kv, head_dim=d, block_size=16,
                              dtype=torch.float32, device="cpu", seed=n_q + d + tq)
    tables = _tables(b)
    got = ref.paged_attention(b.padded_q(), b.kv_cache, tables, b.context_lens, 0, b.scale, 16)
    want = ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables.numpy(), np.array(ctx), 0, b.scale, 16)
    atol, rtol = TOL[torch.float32]
    np.testing.assert_allclose(f64(got), want, atol=atol, rtol=rtol)
    for i, c in enumerate(ctx):
        k, v = ref.gather(b.kv_cache.double(), 0, tables[i], c, 16)
        k = k.repeat_interleave(n_q // n_kv, dim=1)
        v = v.repeat_interleave(n_q // n_kv, dim=1)
        mask = torch.arange(c)[None, :] <= torch.arange(c - tq, c)[:, None]
        sd = F.scaled_dot_product_attention(b.padded_q()[i : i + 1].double(), k, v, attn_mask=mask, scale=b.scale)
        np.testing.assert_allclose(f64(got[i]), sd[0].transpose(0, 1).numpy(), atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n_q,n_kv,d,tq", SHAPES)
def test_paged_attention_half_precision_within_rounding_of_oracle(dtype, n_q, n_kv, d, tq):
    ctx = [40, 300, 511, 1000, 17, 64]
    b = workloads.build_batch(ctx, [tq] * len(ctx), n_q=n_q, n_kv=n_kv, head_dim=d, block_size=16,
                              dtype=dtype, device="cpu", seed=3)
    tables = _tables(b)
    got = ref.paged_attention(b.padded_q(), b.kv_cache, tables, b.context_lens, 0, b.scale, 16)
    assert got.dtype == dtype and got.shape == (len(ctx), tq, n_q, d)
    want = ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables.numpy(), np.array(ctx), 0, b.scale, 16)
    atol, rtol = TOL[dtype]
    np.testing.assert_allclose(f64(got), want, atol=atol, rtol=rtol)


def test_paged_attention_order_and_block_relabelling():
    """Output row b belongs to sequence b, and relabelling the pool's blocks (tables
    remapped to match) changes nothing, bit for bit."""
    ctx = [300, 40, 129]
    b = workloads.build_batch(ctx, [1] * 3, n_q=8, n_kv=2, head_dim=64, block_size=16, dtype=torch.bfloat16,
                              device="cpu", seed=5)
    tables = _tables(b)
    out = ref.paged_attention(b.padded_q(), b.kv_cache, tables, b.context_lens, 0, b.scale, 16)
    perm = torch.randperm(b.kv_cache.shape[2], generator=torch.Generator().manual_seed(0))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    kv2 = b.kv_cache[:, :, perm]  # new block i holds old block perm[i]
    t2 = torch.where(tables >= 0, inv[tables.clamp_min(0).long()].to(torch.int32), tables)
    out2 = ref.paged_attention(b.padded_q(), kv2, t2, b.context_lens, 0, b.scale, 16)
    assert torch.equal(out, out2)
    one = ref.paged_attention(b.padded_q()[1:2], b.kv_cache, tables[1:2], b.context_lens[1:2], 0, b.scale, 16)
    assert torch.equal(out[1:2], one)
