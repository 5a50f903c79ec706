"""GPU parity of the general paged-attention kernel (``csrc/paged_general.hip``): the
shapes outside the MFMA kernels' tiles that the reference's Triton decode still serves
(``triton_paged.py:22-23,283-284``: any float dtype, head_dim <= 256, block_size <= 128)
-- fp32 caches, head_dim 8 / 80 / 96 / 112 / 5, block sizes that are not a power of two,
rows without 16-byte alignment -- against the float64 numpy oracle of
``paged_attention_ref`` (``attention_ref.py:68-89``).

The general kernel computes in fp32 from the cache's values and rounds the output once,
so fp32 caches are held to the reference's own fp32 bar (``atol = rtol = 1e-5``,
``tests/kernels/test_paged_attention.py:70``) and 16-bit caches to the attention
tolerance (2e-3 abs + 1e-2 rel).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from slipstream_amd import workloads
from slipstream_amd._ffi import SS_STATUS_QUERY_TOO_LONG
from slipstream_amd.kernels import (
    attention_status,
    paged_attention_decode,
    paged_attention_prefill,
    paged_attention_shared_prefix,
    paged_attention_varlen,
    reshape_and_cache,
)
from tests._helpers import assert_attn_close, f64, record_error, tables_array

pytestmark = pytest.mark.gpu


def _assert_fp32_close(got: torch.Tensor, ref: np.ndarray, what: str, atol=1e-5, rtol=1e-5) -> None:
    g = f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    record_error(what, g, ref)
    err = np.abs(g - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} elements off, max err {err.max():.3e}"


def _close(got, ref, what):
    if got.dtype == torch.float32:
        _assert_fp32_close(got, ref, what)
    else:
        assert_attn_close(got, ref, what)


def _oracle_padded(b: workloads.PagedBatch) -> np.ndarray:
    tables = tables_array(b.tables_host, b.block_tables.shape[1])
    return ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables, np.array(b.ctx_host), 0, b.scale,
                               b.block_size)


def _oracle_varlen(b: workloads.PagedBatch) -> np.ndarray:
    tables = tables_array(b.tables_host, b.block_tables.shape[1])
    cu = np.concatenate([[0], np.cumsum(b.query_lens)])
    return ora.paged_attention_varlen(f64(b.q), f64(b.kv_cache), tables, cu, np.array(b.ctx_host), 0, b.scale,
                                      b.block_size)


@pytest.mark.parametrize("tq", [1, 8])
def test_reference_fp32_head_dim_8(device, tq):
    """The reference's own kernel test (tests/kernels/test_paged_attention.py:46-70): fp32,
    block 16, 4 query / 2 KV heads, head_dim 8, one 32-token sequence written through
    the scatter, Tq 1 and 8; the same bar, atol = rtol = 1e-5."""
    print(f"reference fp32 D8 tq={tq}", flush=True)
    g = torch.Generator().manual_seed(1)
    block_size, n_q, n_kv, d, seq_len, n_blocks = 16, 4, 2, 8, 32, 4
    kv = torch.zeros((1, 2, n_blocks, block_size, n_kv, d), dtype=torch.float32, device=device)
    table = [0, 1]  # the block manager's first two blocks (block_manager.py:141-159)
    mapping = torch.tensor([table[i // block_size] * block_size + i % block_size for i in range(seq_len)],
                           dtype=torch.long, device=device)
    k = torch.randn(1, n_kv, seq_len, d, generator=g).to(device)
    v = torch.randn(1, n_kv, seq_len, d, generator=g).to(device)
    reshape_and_cache(k, v, kv, mapping, 0, block_size)
    q = torch.randn(1, n_q, tq, d, generator=g).to(device)
    tables = torch.tensor([table], dtype=torch.int32, device=device)
    lens = torch.tensor([seq_len], dtype=torch.int32, device=device)
    scale = d ** -0.5
    got = (paged_attention_decode if tq == 1 else paged_attention_prefill)(q, kv, tables, lens, 0, scale,
                                                                         block_size)
    assert got.shape == (1, tq, n_q, d) and got.dtype == torch.float32
    ref = ora.paged_attention(f64(q), f64(kv), np.array([table]), np.array([seq_len]), 0, scale, block_size)
    _assert_fp32_close(got, ref, f"reference fp32 D8 tq{tq}")


@pytest.mark.parametrize("dtype,head_dim", [(dt, d) for dt in (torch.bfloat16, torch.float16, torch.float32)
                                             for d in (80, 96, 112)] + [(torch.float32, 128)])
def test_decode_head_dims_and_fp32(device, dtype, head_dim):
    """Llama-style GQA (32 / 8 heads) decode over ragged lengths; head_dim 128 in fp32
    and the head_dims the MFMA tiles lack in every dtype."""
    print(f"general decode dtype={dtype} D={head_dim}", flush=True)
    ctx = [1, 15, 16, 17, 33, 300, 1000, 2049, 64, 777]
    b = workloads.build_batch(ctx, [1] * len(ctx), n_q=32, n_kv=8, head_dim=head_dim, block_size=16,
                              dtype=dtype, device="cpu", seed=head_dim, pool_factor=1.5)
    ref = _oracle_padded(b)
    out = paged_attention_decode(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                 b.context_lens.to(device), 0, b.scale, 16)
    torch.cuda.synchronize()
    _close(out, ref, f"decode {dtype} D{head_dim}")


@pytest.mark.parametrize("dtype,head_dim,block_size,n_q,n_kv", [
    (torch.float16, 64, 12, 8, 2),     # block size not a power of two
    (torch.bfloat16, 128, 1, 4, 4),    # one-token blocks
    (torch.float32, 64, 128, 14, 2),   # the reference's largest block (triton_paged.py:23)
    (torch.float16, 5, 16, 6, 3),      # 10-byte rows: element loads, no 16-byte alignment
    (torch.float32, 256, 32, 8, 1),    # fp32 at the largest head_dim, MQA
    (torch.bfloat16, 96, 48, 12, 12),  # MHA
])
def test_decode_block_sizes_and_unaligned_rows(device, dtype, head_dim, block_size, n_q, n_kv):
    print(f"general decode {dtype} D={head_dim} bs={block_size} {n_q}/{n_kv}", flush=True)
    ctx = [1, block_size, block_size + 1, 3 * block_size - 1, 250, 901, 40]
    b = workloads.build_batch(ctx, [1] * len(ctx), n_q=n_q, n_kv=n_kv, head_dim=head_dim, block_size=block_size,
                              dtype=dtype, device="cpu", seed=block_size, pool_factor=1.4)
    ref = _oracle_padded(b)
    out = paged_attention_decode(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                 b.context_lens.to(device), 0, b.scale, block_size)
    torch.cuda.synchronize()
    _close(out, ref, f"decode {dtype} D{head_dim} bs{block_size}")


@pytest.mark.parametrize("dtype,head_dim", [(torch.float32, 128), (torch.bfloat16, 80), (torch.float16, 112)])
def test_long_single_sequence_key_splits(device, dtype, head_dim):
    """One sequence, one KV head: the grid splits the keys (partials merged in split order)."""
    print(f"general key splits {dtype} D={head_dim}", flush=True)
    b = workloads.build_batch([6000, 37], [1, 1], n_q=2, n_kv=1, head_dim=head_dim, block_size=16, dtype=dtype,
                              device="cpu", seed=4, pool_factor=1.2)
    ref = _oracle_padded(b)
    out = paged_attention_decode(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                 b.context_lens.to(device), 0, b.scale, 16)
    torch.cuda.synchronize()
    _close(out, ref, f"key splits {dtype} D{head_dim}")
    again = paged_attention_decode(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                   b.context_lens.to(device), 0, b.scale, 16)
    assert torch.equal(out, again)  # the splits and the waves merge in a fixed order


@pytest.mark.parametrize("dtype,head_dim,tq", [(torch.float32, 64, 20), (torch.bfloat16, 96, 33),
                                               (torch.float16, 80, 7)])
def test_prefill_causal(device, dtype, head_dim, tq):
    """Padded prefill chunks (query j sees keys [0, seq_len - Tq + j]); a sequence with
    fewer keys than queries has rows with no visible key, which are zero."""
    print(f"general prefill {dtype} D={head_dim} tq={tq}", flush=True)
    ctx = [tq, tq + 5, 400, 1100, tq - 3]
    b = workloads.build_batch(ctx, [tq] * len(ctx), n_q=16, n_kv=4, head_dim=head_dim, block_size=16,
                              dtype=dtype, device="cpu", seed=tq, pool_factor=1.3)
    ref = _oracle_padded(b)
    out = paged_attention_prefill(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                  b.context_lens.to(device), 0, b.scale, 16)
    torch.cuda.synchronize()
    assert not f64(out[4, :3]).any()  # rows 0..2 of the short sequence see no key
    _close(out, ref, f"prefill {dtype} D{head_dim} tq{tq}")


@pytest.mark.parametrize("dtype,head_dim,block_size", [(torch.bfloat16, 96, 16), (torch.float32, 128, 16),
                                                       (torch.float16, 64, 24)])
def test_varlen_mixed_step(device, dtype, head_dim, block_size):
    """A packed step (decodes and prefill chunks in one token stream) on the general kernel."""
    print(f"general varlen {dtype} D={head_dim} bs={block_size}", flush=True)
    ctx = [300, 17, 90 + 64, 1500, 40, 2 + 100, 700]
    ql = [1, 1, 64, 1, 40, 100, 1]
    ctx[5] = 100  # a chunk that is the sequence's whole context
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=head_dim, block_size=block_size, dtype=dtype,
                              device="cpu", seed=head_dim + block_size, pool_factor=1.3)
    ref = _oracle_varlen(b)
    out = paged_attention_varlen(b.q.to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                 b.cu_seqlens.to(device), b.context_lens.to(device), 0, b.scale, block_size,
                                 b.max_query_len)
    torch.cuda.synchronize()
    _close(out, ref, f"varlen {dtype} D{head_dim} bs{block_size}")


def test_varlen_query_longer_than_max_query_len_is_zeroed_and_flagged(device, monkeypatch):
    """A broken max_query_len promise on the general kernel: the rows past the call's
    tiles are zero, the others exact, and the status word reports it."""
    monkeypatch.delenv("SLIPSTREAM_DEBUG", raising=False)
    b = workloads.build_batch([500, 200], [1, 60], n_q=8, n_kv=2, head_dim=80, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=2, pool_factor=1.3)
    ref = _oracle_varlen(b)
    attention_status(clear=True)
    mq = 10  # 10 * 4 = 40 rows per KV head: three 16-row tiles cover 48 of the 240
    out = paged_attention_varlen(b.q.to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                 b.cu_seqlens.to(device), b.context_lens.to(device), 0, b.scale, 16, mq)
    assert attention_status(clear=True) & SS_STATUS_QUERY_TOO_LONG
    assert attention_status(clear=True) == 0
    covered = 48 // 4  # query tokens whose every head's row is covered
    assert_attn_close(out[: 1 + covered], ref[: 1 + covered], "covered rows")
    assert not f64(out[1 + covered:]).any()


def test_table_holes_and_out_of_pool_entries(device):
    """Negative and out-of-pool table entries are masked (triton_paged.py:161-165)."""
    b = workloads.build_batch([200, 150, 64], [1, 1, 1], n_q=8, n_kv=2, head_dim=96, block_size=16,
                              dtype=torch.float32, device="cpu", seed=8, pool_factor=1.5)
    nb = b.kv_cache.shape[2]
    bt = b.block_tables.clone()
    bt[0, 3] = -1
    bt[1, 2] = nb + 7
    tables = [list(r) for r in bt.tolist()]
    tables_np = np.array([[x if 0 <= x < nb else -1 for x in r] for r in tables])
    ref = ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables_np, np.array(b.ctx_host), 0, b.scale, 16)
    out = paged_attention_decode(b.padded_q().to(device), b.kv_cache.to(device), bt.to(device),
                                 b.context_lens.to(device), 0, b.scale, 16)
    torch.cuda.synchronize()
    _assert_fp32_close(out, ref, "holes fp32")


@pytest.mark.parametrize("dtype,head_dim", [(torch.float32, 128), (torch.bfloat16, 80)])
def test_shared_prefix_entry_on_general_shapes(device, dtype, head_dim):
    """ss_paged_attention_shared_prefix on shapes the cascade does not take: the plain
    general decode inside the same entry point."""
    pb = 9
    ctx = [pb * 16 + s for s in (0, 1, 40, 333, 17, 5)]
    b = workloads.build_batch(ctx, [1] * len(ctx), n_q=28, n_kv=4, head_dim=head_dim, block_size=16,
                              dtype=dtype, device="cpu", seed=11, pool_factor=1.3, shared_prefix_blocks=pb)
    ref = _oracle_padded(b)
    out = paged_attention_shared_prefix(b.padded_q().to(device), b.kv_cache.to(device), b.block_tables.to(device),
                                        b.context_lens.to(device), 0, b.scale, 16, pb)
    torch.cuda.synchronize()
    _close(out, ref, f"shared prefix general {dtype} D{head_dim}")


def test_graph_replays_equal_eager(device):
    """A captured general decode replays to the eager result (split partials included)."""
    b = workloads.build_batch([3000, 9], [1, 1], n_q=4, n_kv=2, head_dim=80, block_size=16, dtype=torch.float32,
                              device=device, seed=6, pool_factor=1.2)
    args = (b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    first = paged_attention_decode(*args)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention_decode(*args)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
