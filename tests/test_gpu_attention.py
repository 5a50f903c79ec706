"""GPU parity of the HIP scatter and paged attention against the numpy oracle.

Every test builds seeded inputs (on the host when they are small, so the
oracle sees the identical bits), runs the HIP path through the C ABI, and
compares: the scatter bit for bit, attention within 2e-3 abs + 1e-2 rel.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from slipstream_amd import workloads
from slipstream_amd.kernels import (
    paged_attention_decode,
    paged_attention_prefill,
    paged_attention_varlen,
    reshape_and_cache,
)
from tests._helpers import assert_attn_close, bits, f64, gather_pool_f64, oracle_paged_rows, tables_array

pytestmark = pytest.mark.gpu


def _to(batch: workloads.PagedBatch, device) -> workloads.PagedBatch:
    for name in ("kv_cache", "block_tables", "context_lens", "cu_seqlens", "q", "k_new", "v_new",
                 "slot_mapping"):
        setattr(batch, name, getattr(batch, name).to(device))
    return batch


def _oracle_padded(batch: workloads.PagedBatch) -> np.ndarray:
    kv = f64(batch.kv_cache)
    tables = tables_array(batch.tables_host, batch.block_tables.shape[1])
    q = f64(batch.padded_q())
    return ora.paged_attention(q, kv, tables, np.array(batch.ctx_host), 0, batch.scale, batch.block_size)


# ---------------------------------------------------------------- scatter


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["flat", "bnhd"])
def test_scatter_bit_exact(device, dtype, layout):
    print(f"scatter dtype={dtype} layout={layout}", flush=True)
    b = workloads.build_batch([37, 5, 64, 17], [3, 5, 2, 1], n_q=8, n_kv=2, head_dim=64, block_size=16,
                              dtype=dtype, device="cpu", seed=3, num_blocks=24)
    kv_host = b.kv_cache.clone()
    _to(b, device)
    if layout == "flat":
        k, v = b.k_new, b.v_new
    else:  # [B, n_kv, T, D] needs equal query lengths: use 4 x 2 tokens of the packed stream
        k = b.k_new[:8].view(4, 2, 2, 64).transpose(1, 2)
        v = b.v_new[:8].view(4, 2, 2, 64).transpose(1, 2)
    n = k.shape[0] * (k.shape[2] if k.ndim == 4 else 1)
    slots = b.slot_mapping[:n].clone()
    reshape_and_cache(k, v, b.kv_cache, slots, 0, b.block_size)
    torch.cuda.synchronize()
    ref = kv_host.numpy() if dtype == torch.float32 else kv_host.view(torch.int16).numpy()
    kk = k.cpu().numpy() if dtype == torch.float32 else k.cpu().contiguous().view(torch.int16).numpy()
    vv = v.cpu().numpy() if dtype == torch.float32 else v.cpu().contiguous().view(torch.int16).numpy()
    ora.reshape_and_cache(kk, vv, ref, slots.cpu().numpy(), 0, b.block_size)
    got = b.kv_cache.cpu().numpy() if dtype == torch.float32 else bits(b.kv_cache)
    assert np.array_equal(got, ref)


def test_scatter_skips_negative_and_out_of_pool_slots(device):
    kv = torch.zeros((2, 2, 4, 8, 2, 64), dtype=torch.bfloat16, device=device)
    k = torch.randn(4, 2, 64, device=device).to(torch.bfloat16)
    v = torch.randn(4, 2, 64, device=device).to(torch.bfloat16)
    slots = torch.tensor([-1, 3, 4 * 8, 31], dtype=torch.int64, device=device)
    reshape_and_cache(k, v, kv, slots, 1, 8)
    torch.cuda.synchronize()
    ref = torch.zeros_like(kv)
    ref[1, 0, 0, 3], ref[1, 1, 0, 3] = k[1], v[1]
    ref[1, 0, 3, 7], ref[1, 1, 3, 7] = k[3], v[3]
    assert torch.equal(kv, ref)


def test_scatter_full_decode_step(device):
    """C2 shape: the 256 new tokens land in their slots; nothing else changes."""
    b = workloads.llama_decode(device=device, seed=1)
    before = b.kv_cache.clone()
    reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
    torch.cuda.synchronize()
    s = b.slot_mapping
    blk, off = s // 16, s % 16
    assert torch.equal(b.kv_cache[0, 0, blk, off], b.k_new)
    assert torch.equal(b.kv_cache[0, 1, blk, off], b.v_new)
    b.kv_cache[0, 0, blk, off] = before[0, 0, blk, off]
    b.kv_cache[0, 1, blk, off] = before[0, 1, blk, off]
    assert torch.equal(b.kv_cache, before)


# ---------------------------------------------------------------- decode


def test_decode_qwen05_config(device):
    """C1: fp16, 14/2 heads, D 64, 8 sequences, pool 512 blocks; scatter then decode."""
    b = workloads.qwen05_decode(device="cpu", seed=0)
    kv_host = b.kv_cache.clone()
    _to(b, device)
    reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert out.shape == (8, 1, 14, 64) and out.dtype == torch.float16
    kv = kv_host.float().numpy().astype(np.float64)
    kk, vv = f64(b.k_new), f64(b.v_new)
    ora.reshape_and_cache(kk, vv, kv, b.slot_mapping.cpu().numpy(), 0, 16)
    ref = ora.paged_attention(f64(b.padded_q()), kv, tables_array(b.tables_host, b.block_tables.shape[1]),
                              np.array(b.ctx_host), 0, b.scale, 16)
    assert_attn_close(out, ref, "qwen05 decode")


EDGE_LENS = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 257, 1000, 2049, 4000]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_decode_llama_shape_edge_lengths(device, dtype, block_size):
    print(f"decode llama-shape dtype={dtype} bs={block_size}", flush=True)
    b = workloads.build_batch(EDGE_LENS, [1] * len(EDGE_LENS), n_q=32, n_kv=8, head_dim=128,
                              block_size=block_size, dtype=dtype, device="cpu", seed=11)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale,
                                 block_size)
    assert_attn_close(out, ref, f"decode bs={block_size}")


@pytest.mark.parametrize("n_q,n_kv,tq", [(32, 8, 2), (32, 8, 4), (16, 8, 8), (14, 2, 2), (8, 8, 16)])
def test_decode_multi_query_rows_causal(device, n_q, n_kv, tq):
    """Tq > 1 through the decode tile (n_rep * Tq <= 16 rows): causal offsets per row."""
    lens = [tq, tq + 1, 40, 333, 1024]
    b = workloads.build_batch(lens, [tq] * len(lens), n_q=n_q, n_kv=n_kv, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=5)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, f"decode tq={tq}")


def test_decode_table_holes_and_zero_lengths(device):
    """Negative / out-of-pool table entries are masked; empty sequences give zeros."""
    b = workloads.build_batch([200, 64, 50, 0, 300], [1] * 5, n_q=32, n_kv=8, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=9, num_blocks=64)
    tables = [list(t) for t in b.tables_host]
    tables[0][3] = -1
    tables[2][1] = 10_000  # past the pool
    tables[4][0] = -7
    width = b.block_tables.shape[1]
    bt = torch.full((5, width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    b.block_tables = bt
    b.context_lens = torch.tensor([200, 64, 50, 0, 300], dtype=torch.int32)
    ref = ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables_array(tables, width),
                              np.array([200, 64, 50, 0, 300]), 0, b.scale, 16)
    _to(b, device)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, "holes")
    assert torch.count_nonzero(out[3]) == 0


@pytest.mark.parametrize("lens", [[3, 17, 40, 250, 511], [3, 17, 40, 250, 2000]])
def test_decode_ignores_stale_nan_slots(device, lens):
    """Slots past a sequence's length (the rest of its last block, and blocks its table
    lists past the length) hold NaN: the output must not see them. Short tables take the
    one-launch small-batch kernel (which requests the first pair before the length is
    known), the 2000-key table the split-K kernel."""
    print(f"decode stale NaN lens={lens}", flush=True)
    b = workloads.build_batch(lens, [1] * len(lens), n_q=14, n_kv=2, head_dim=64, block_size=16,
                              dtype=torch.float16, device="cpu", seed=21)
    width = b.block_tables.shape[1]
    kv = b.kv_cache
    used = set()
    for t, n in zip(b.tables_host, lens):
        for i, blk in enumerate(t):
            lo = i * 16
            if lo >= n:
                kv[0, :, blk] = float("nan")
            elif lo + 16 > n:
                kv[0, :, blk, n - lo:] = float("nan")
            used.add(blk)
    ref = _oracle_padded(b)
    # tables padded with real (NaN) blocks past each length, as a block manager may leave them
    bt = b.block_tables.clone()
    spare = [x for x in range(kv.shape[2]) if x not in used]
    for i, t in enumerate(b.tables_host):
        for c in range(len(t), width):
            bt[i, c] = spare[(i * width + c) % len(spare)]
    kv[0, :, spare] = float("nan")
    b.block_tables = bt
    _to(b, device)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert torch.isfinite(out).all()
    assert_attn_close(out, ref, f"stale NaN lens={lens}")


def test_decode_head_dim_64_and_256(device):
    for d in (64, 256):
        b = workloads.build_batch([5, 77, 600], [1, 1, 1], n_q=16, n_kv=4, head_dim=d, block_size=16,
                                  dtype=torch.bfloat16, device="cpu", seed=d)
        ref = _oracle_padded(b)
        _to(b, device)
        out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0,
                                     b.scale, 16)
        assert_attn_close(out, ref, f"D={d}")


def test_decode_full_llama_config_every_row(device):
    """C2 at full size (256 sequences, lognormal lengths, 1.2x pool): the scatter of the
    256 new tokens then split-K decode; every row against the float64 oracle."""
    b = workloads.llama_decode(device=device, seed=0)
    reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
    out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    torch.cuda.synchronize()
    q = f64(b.padded_q())
    ref = oracle_paged_rows(b.kv_cache, b.tables_host, b.ctx_host, list(q), b.scale, 16)
    assert_attn_close(out, np.stack(ref), "C2 every row")


def test_decode_against_the_reference_dtype_path(device):
    """Secondary check: the HIP decode against the reference's own dtype sequence
    (oracle.reference_path: bf16/fp16 GEMMs, fp32 softmax, rounded to the dtype;
    attention_ref.py:68-89, attention.py:64-88) at the C1 shape (fp16, 14/2 heads, D 64)
    and on 16 Llama-3-8B-shape sequences (bf16). The distance is within the sum of the
    two paths' bounds to the float64 oracle (HIP: 2e-3 + 1e-2|ref|; the reference's path:
    its dtype's rounding, pinned in tests/test_oracle_reference_path.py); both distances
    are recorded in the run's error summary."""
    from oracle import reference_path as rp
    from tests._helpers import record_error

    for name, b, tol in (
        ("C1 fp16", workloads.qwen05_decode(device="cpu", seed=0), (3e-3, 1.4e-2)),
        ("Llama bf16", workloads.build_batch([17, 300, 1000, 2500, 64, 129, 511, 4096, 33, 800, 1500, 90, 16, 3000,
                                               700, 250], [1] * 16, n_q=32, n_kv=8, head_dim=128, block_size=16,
                                              dtype=torch.bfloat16, device="cpu", seed=4), (8e-3, 3e-2)),
    ):
        tables = torch.full((b.batch, b.block_tables.shape[1]), -1, dtype=torch.int32)
        for i, t in enumerate(b.tables_host):
            tables[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        want = rp.paged_attention(b.padded_q(), b.kv_cache, tables, b.context_lens, 0, b.scale, b.block_size)
        exact = _oracle_padded(b)
        _to(b, device)
        out = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale,
                                     b.block_size)
        got = f64(out)
        a, _ = record_error(f"{name}: HIP vs reference dtype path", got, f64(want))
        record_error(f"{name}: reference dtype path vs float64", f64(want), exact)
        assert_attn_close(out, exact, f"{name}: HIP vs float64")
        np.testing.assert_allclose(got, f64(want), atol=tol[0], rtol=tol[1], err_msg=name)


def test_decode_is_invariant_to_block_permutation(device):
    """Relabelling physical blocks (and the tables with them) leaves outputs bit-identical."""
    b = workloads.build_batch([700, 33, 1500], [1, 1, 1], n_q=32, n_kv=8, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device=device, seed=21)
    out1 = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    nb = b.kv_cache.shape[2]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).to(device)
    kv2 = torch.empty_like(b.kv_cache)
    kv2[:, :, perm] = b.kv_cache
    bt = b.block_tables.long()
    bt2 = torch.where(bt >= 0, perm[bt.clamp_min(0)], bt).to(torch.int32)
    out2 = paged_attention_decode(b.padded_q(), kv2, bt2, b.context_lens, 0, b.scale, 16)
    assert torch.equal(out1, out2)


@pytest.mark.parametrize("tq", [1, 3])
def test_decode_cache_policies_agree(device, tq):
    """The page loads stream non-temporally when one layer's K+V pool exceeds 192 MiB and
    keep the default cache policy below that; the same batch in a small and in a 256 MiB
    pool gives bit-identical outputs (and matches the oracle)."""
    b = workloads.build_batch([3000, 700, 33, 1500, 16, 257], [tq] * 6, n_q=32, n_kv=8, head_dim=128,
                              block_size=16, dtype=torch.bfloat16, device=device, seed=23)
    nb = b.kv_cache.shape[2]
    big = torch.zeros((1, 2, 4096) + tuple(b.kv_cache.shape[3:]), dtype=b.kv_cache.dtype, device=device)
    big[:, :, :nb] = b.kv_cache
    assert big.numel() * big.element_size() > (192 << 20) > b.kv_cache.numel() * b.kv_cache.element_size()
    q = b.padded_q()
    out_small = paged_attention_decode(q, b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    out_big = paged_attention_decode(q, big, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert torch.equal(out_small, out_big)
    assert_attn_close(out_big, _oracle_padded(b), f"tq={tq}")


def test_decode_shared_prefix_equals_private_copies(device):
    """Prefix config (C4 shape, reduced batch): tables sharing 128 blocks == private copies."""
    b = workloads.prefix_share(device=device, seed=2, batch=16)
    out_shared = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0,
                                        b.scale, 16)
    # give every sequence a private copy of the prefix blocks
    nb = b.kv_cache.shape[2]
    shared = b.tables_host[0][: b.shared_blocks]
    extra = torch.cat([b.kv_cache[:, :, shared]] * b.batch, dim=2)
    kv2 = torch.cat([b.kv_cache, extra], dim=2)
    tables = []
    for i, t in enumerate(b.tables_host):
        fresh = list(range(nb + i * b.shared_blocks, nb + (i + 1) * b.shared_blocks))
        tables.append(fresh + t[b.shared_blocks :])
    bt2 = torch.tensor(tables_array(tables, b.block_tables.shape[1]), dtype=torch.int32, device=device)
    out_private = paged_attention_decode(b.padded_q(), kv2, bt2, b.context_lens, 0, b.scale, 16)
    assert torch.equal(out_shared, out_private)


# ---------------------------------------------------------------- prefill


@pytest.mark.parametrize("n_q,n_kv,tq,lens", [
    (32, 8, 8, [8, 9, 100, 700]),
    (32, 8, 33, [33, 64, 517]),
    (8, 8, 20, [20, 21, 300]),
    (32, 1, 1, [1, 50, 900]),          # MQA: 32 rows per KV head go to the prefill tile
    (28, 4, 64, [64, 1000]),
])
def test_prefill_padded(device, n_q, n_kv, tq, lens):
    print(f"prefill n_q={n_q} n_kv={n_kv} tq={tq}", flush=True)
    b = workloads.build_batch(lens, [tq] * len(lens), n_q=n_q, n_kv=n_kv, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=tq)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, f"prefill tq={tq}")


def test_prefill_fp16_head_dim_64(device):
    b = workloads.build_batch([96, 500], [96, 96], n_q=14, n_kv=2, head_dim=64, block_size=16,
                              dtype=torch.float16, device="cpu", seed=4)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, "prefill fp16 D64")


@pytest.mark.parametrize("block_size", [8, 32, 64])
def test_prefill_block_sizes(device, block_size):
    """Tiles of 64 keys cover several 16-key groups of one block (32, 64) or take the
    per-lane kernel (8); chunk lengths cut tiles and blocks at odd places."""
    print(f"prefill block_size={block_size}", flush=True)
    b = workloads.build_batch([77, 400, 1031], [77, 77, 77], n_q=32, n_kv=8, head_dim=128,
                              block_size=block_size, dtype=torch.bfloat16, device="cpu", seed=block_size)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale,
                                  block_size)
    assert_attn_close(out, ref, f"prefill bs={block_size}")


def test_prefill_table_holes(device):
    """Absent blocks (negative, past the pool) inside a chunk's prior context and inside
    the chunk itself are masked for every query row."""
    b = workloads.build_batch([300, 260], [100, 100], n_q=32, n_kv=8, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=31)
    tables = [list(t) for t in b.tables_host]
    tables[0][2] = -1          # keys 32..47: prior context
    tables[0][15] = 10_000     # keys 240..255: inside the chunk
    tables[1][0] = -3          # the first block
    width = b.block_tables.shape[1]
    bt = torch.full((2, width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    b.block_tables = bt
    ref = ora.paged_attention(f64(b.padded_q()), f64(b.kv_cache), tables_array(tables, width),
                              np.array(b.ctx_host), 0, b.scale, 16)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, "prefill holes")


@pytest.mark.parametrize("ctx,holes", [((700, 200), ()), ((520, 333), ((0, 3), (1, 2)))])
def test_prefill_every_key_weighted(device, ctx, holes):
    """K = 0 makes every visible key's weight 1/(visible keys); V one-hot on key // 8 then
    reads each 8-key bucket's share in one output column, so a key that is lost, zeroed or
    counted twice shows up in its own column. Covers the last (partial) tile of every
    chunk and, with holes, the block after an absent one in the same 16-key group."""
    b = workloads.build_batch(list(ctx), [8] * len(ctx), n_q=32, n_kv=8, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=sum(ctx))
    kv = b.kv_cache
    kv[0, 0].zero_()
    kv[0, 1].zero_()
    for s, c in enumerate(ctx):
        for p in range(c):
            kv[0, 1, b.tables_host[s][p // 16], p % 16, :, (p // 8) % 128] = 1.0
    tables = [list(t) for t in b.tables_host]
    for s, blk in holes:
        tables[s][blk] = -1
    width = b.block_tables.shape[1]
    bt = torch.full((len(ctx), width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    b.block_tables = bt
    ref = ora.paged_attention(f64(b.padded_q()), f64(kv), tables_array(tables, width), np.array(b.ctx_host), 0,
                              b.scale, 16)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, f"prefill bucket weights ctx={ctx} holes={holes}")


def test_prefill_head_dim_256(device):
    b = workloads.build_batch([40, 300], [40, 40], n_q=8, n_kv=2, head_dim=256, block_size=16,
                              dtype=torch.bfloat16, device="cpu", seed=256)
    ref = _oracle_padded(b)
    _to(b, device)
    out = paged_attention_prefill(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    assert_attn_close(out, ref, "prefill D256")


# ---------------------------------------------------------------- packed varlen


def _oracle_varlen(b: workloads.PagedBatch, kv: np.ndarray) -> np.ndarray:
    return ora.paged_attention_varlen(f64(b.q), kv, tables_array(b.tables_host, b.block_tables.shape[1]),
                                      f64(b.cu_seqlens).astype(np.int64), np.array(b.ctx_host), 0,
                                      b.scale, b.block_size)


def test_varlen_mixed_step_reduced(device):
    """C3 structure at reduced size: 24 decodes + 3 chunks of 96 with prior context, one stream."""
    ctx, ql = workloads.mixed_step_lengths(seed=7, n_prefill=3, chunk=96, n_decode=24)
    ctx = [min(c, 1200) if q == 1 else c for c, q in zip(ctx, ql)]
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device="cpu", seed=7)
    kv_host = b.kv_cache.clone()
    _to(b, device)
    reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
    out = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale,
                                 16, b.max_query_len)
    kv = kv_host.float().numpy().astype(np.float64)
    ora.reshape_and_cache(f64(b.k_new), f64(b.v_new), kv, b.slot_mapping.cpu().numpy(), 0, 16)
    assert_attn_close(out, _oracle_varlen(b, kv), "varlen mixed")


def test_varlen_many_prefill_items_and_empty_sequences(device):
    """The prefill work list at more items than resident workgroups (each persistent
    workgroup walks several snake rounds: 856 items for 256 workgroups): 24 prefill
    sequences with ragged query lengths (1-10 query tiles), decodes, short multi-token
    queries and zero-length sequences interleaved, GQA 4:1; every row
    against the oracle, and a repeat call is bit-identical (the order in which workgroups
    take items does not change any item's result)."""
    rng = np.random.default_rng(11)
    ql, ctx = [], []
    for i in range(54):
        kind = i % 9
        if kind in (0, 4):
            ql.append(0), ctx.append(int(rng.integers(1, 200)))  # empty sequence
        elif kind in (1, 5, 7):
            q = int(rng.integers(2, 300))
            ql.append(q), ctx.append(q + int(rng.integers(0, 400)))  # prefill, with or without prior
        elif kind == 2:
            ql.append(int(rng.integers(5, 17))), ctx.append(int(rng.integers(20, 300)))
        else:
            ql.append(1), ctx.append(int(rng.integers(1, 500)))  # decode
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device="cpu", seed=11)
    kv_host = b.kv_cache.float().numpy().astype(np.float64)
    _to(b, device)
    out = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale,
                                 16, b.max_query_len)
    again = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0,
                                   b.scale, 16, b.max_query_len)
    assert sum(1 for q in ql if q * 4 > 16) == 24
    assert torch.equal(out, again)
    assert_attn_close(out, _oracle_varlen(b, kv_host), "many prefill items")


def test_varlen_equals_padded_calls(device):
    """Packed step == the per-sequence padded calls concatenated."""
    ctx, ql = [300, 45, 700, 64], [1, 1, 64, 32]
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device=device, seed=8)
    out = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale,
                                 16, b.max_query_len)
    cu = [0, 1, 2, 66, 98]
    for i in range(4):
        qi = b.q[cu[i]:cu[i + 1]].unsqueeze(0).transpose(1, 2)
        oi = paged_attention_prefill(qi, b.kv_cache, b.block_tables[i:i + 1], b.context_lens[i:i + 1], 0,
                                     b.scale, 16)
        # same kernels, but the split-K partition (hence fp32 summation order) differs
        assert_attn_close(out[cu[i]:cu[i + 1]], f64(oi[0]), f"sequence {i}")


def test_varlen_full_mixed_step_every_row(device):
    """C3 at full size: 192 decodes + 4 x 512-token chunks, 2240 tokens; the scatter then
    attention; every row of every sequence against the float64 oracle."""
    b = workloads.mixed_step(device=device, seed=0)
    reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
    out = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale,
                                 16, b.max_query_len)
    torch.cuda.synchronize()
    cu = b.cu_seqlens.cpu().tolist()
    q = f64(b.q)
    queries = [q[cu[i]:cu[i + 1]].transpose(1, 0, 2) for i in range(b.batch)]
    ref = oracle_paged_rows(b.kv_cache, b.tables_host, b.ctx_host, queries, b.scale, 16)
    assert_attn_close(out, np.concatenate(ref, axis=0), "C3 every row")


def test_long_contexts_decode_and_prefill(device):
    """Lengths far past the bench's (C2 clips at 8192): one decode over 131072 keys (8192
    blocks, 4096 pairs, a table row of 8192 entries), one over 70001, a 1024-token chunk
    behind a 20000-token prior and two one-key sequences, in one packed call; every row
    against the float64 oracle."""
    print("long contexts: ctx [131072, 1, 70001, 21024, 5]", flush=True)
    ctx, ql = [131072, 1, 70001, 21024, 5], [1, 1, 1, 1024, 1]
    b = workloads.build_batch(ctx, ql, n_q=8, n_kv=2, head_dim=64, block_size=16, dtype=torch.bfloat16,
                              device=device, seed=21)
    assert b.block_tables.shape[1] == 8192
    out = paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale,
                                 16, b.max_query_len)
    torch.cuda.synchronize()
    cu = b.cu_seqlens.cpu().tolist()
    q = f64(b.q)
    queries = [q[cu[i]:cu[i + 1]].transpose(1, 0, 2) for i in range(b.batch)]
    ref = oracle_paged_rows(b.kv_cache, b.tables_host, b.ctx_host, queries, b.scale, 16)
    assert_attn_close(out, np.concatenate(ref, axis=0), "long contexts")


@pytest.mark.parametrize("max_q", [0, 1, 20, 40])
def test_varlen_query_longer_than_max_query_len_is_zeroed_and_flagged(device, max_q):
    """A packed sequence longer than max_query_len (a broken caller promise): the rows
    no kernel of the call covers are written as zeros -- never left as stale memory --
    and the device status word reports it; every covered row still matches the oracle.
    max_q 0/1: no prefill launch (4 decode rows per KV head), so the 40- and 3-token
    sequences are wholly zero; 20: the prefill covers 128 rows per KV head (tokens
    0-31 of the 40-token chunk); 40: the promise holds, status stays 0."""
    from slipstream_amd.kernels import attention_status

    ctx, ql = [90, 500, 140, 60], [1, 1, 40, 3]
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device="cpu", seed=21)
    ref = _oracle_varlen(b, f64(b.kv_cache))
    _to(b, device)
    attention_status(device)  # clear
    out = torch.full_like(b.q, float("nan"))
    paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale, 16,
                           max_q, out=out)
    flags = attention_status(device)
    got = f64(out)
    cu = [0, 1, 2, 42, 45]
    covered_tokens = {0: [1, 1, 0, 0], 1: [1, 1, 0, 0], 20: [1, 1, 32, 3], 40: [1, 1, 40, 3]}[max_q]
    for i in range(4):
        s0, s1 = cu[i], cu[i + 1]
        c = s0 + covered_tokens[i]
        if c > s0:
            assert_attn_close(out[s0:c], ref[s0:c], f"covered rows of sequence {i}")
        assert np.array_equal(got[c:s1], np.zeros_like(got[c:s1])), f"uncovered rows of sequence {i}"
    assert flags == (0 if max_q == 40 else 1), flags
    assert attention_status(device) == 0  # read-and-clear


def test_varlen_stream_past_total_tokens_is_clamped_and_flagged(device):
    """cu_seqlens running past the query tensor: every kernel clamps the sequences into
    [0, T) (no read or write outside q and out), the earlier sequences are unaffected
    and the status word reports the overrun."""
    from slipstream_amd.kernels import attention_status

    ctx, ql = [90, 500, 140, 60], [1, 1, 40, 3]
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device="cpu", seed=22)
    ref = _oracle_varlen(b, f64(b.kv_cache))
    _to(b, device)
    attention_status(device)
    q = b.q[:43].contiguous()  # the stream says 45 tokens
    out = paged_attention_varlen(q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0, b.scale, 16,
                                 b.max_query_len)
    flags = attention_status(device)
    assert flags == 2, flags
    assert_attn_close(out[:42], ref[:42], "sequences inside the stream")
    assert np.isfinite(f64(out[42])).all()


def test_varlen_packed_step_graph_replays(device):
    """The packed step (plan kernel writing the prefill work list into the workspace, the
    persistent prefill, then the decode and its merge) captured in a HIP graph after an
    eager warm-up: every replay equals the eager step, with eager steps in between."""
    ctx, ql = workloads.mixed_step_lengths(seed=9, n_prefill=2, chunk=80, n_decode=20)
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device=device, seed=9)

    def step():
        reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
        return paged_attention_varlen(b.q, b.kv_cache, b.block_tables, b.cu_seqlens, b.context_lens, 0,
                                      b.scale, 16, b.max_query_len)

    eager = step().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = step()
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        again = step()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
