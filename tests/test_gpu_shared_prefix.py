"""GPU parity of the shared-prefix decode (prefix pass, then the suffix decode whose merge
folds in the prefix parts by log-sum-exp weight) against the numpy oracle of
``paged_attention_ref`` (``attention_ref.py:68-89``).

The cascade reorders the softmax sum (prefix chunks and the suffix are normalised apart,
then mixed by ``2^(lse - max)``), so it matches the oracle to the attention tolerance, not
bit for bit. Batches whose query rows fit one decode tile, head_dim 256 and blocks under
16 tokens take the plain decode inside the same entry point, covered here too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from slipstream_amd import workloads
from slipstream_amd._ffi import SS_STATUS_PREFIX_SHORT
from slipstream_amd.kernels import attention_status, paged_attention_decode, paged_attention_shared_prefix
from tests._helpers import assert_attn_close, f64, oracle_paged_rows, tables_array

pytestmark = pytest.mark.gpu


def _oracle(b: workloads.PagedBatch, rows=None) -> np.ndarray:
    rows = list(range(b.batch)) if rows is None else rows
    kv = f64(b.kv_cache)
    tables = tables_array([b.tables_host[i] for i in rows], b.block_tables.shape[1])
    q = f64(b.padded_q()[rows])
    ctx = np.array([b.ctx_host[i] for i in rows])
    return ora.paged_attention(q, kv, tables, ctx, 0, b.scale, b.block_size)


def _run(b: workloads.PagedBatch, prefix_blocks: int) -> torch.Tensor:
    return paged_attention_shared_prefix(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale,
                                         b.block_size, prefix_blocks)


def test_c4_shape_reduced_batch(device):
    """C4 shape (28/4 heads, D 128, 2048-token prefix) at batch 32: 224 query rows per
    KV head, so the prefix pass runs."""
    b = workloads.prefix_share(device=device, seed=5, batch=32)
    out = _run(b, b.shared_blocks)
    assert out.shape == (32, 1, 28, 128) and out.dtype == torch.bfloat16
    assert_attn_close(out, _oracle(b), "c4 reduced")


def test_c4_full_config(device):
    """The full C4 batch (128 sequences): every row against the float64 oracle, and
    within tolerance of the plain decode."""
    b = workloads.prefix_share(device=device, seed=0)
    out = _run(b, b.shared_blocks)
    plain = paged_attention_decode(b.padded_q(), b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)
    torch.cuda.synchronize()
    ref = np.stack(oracle_paged_rows(b.kv_cache, b.tables_host, b.ctx_host, list(f64(b.padded_q())), b.scale, 16))
    assert_attn_close(out, ref, "C4 cascade every row")
    assert_attn_close(plain, ref, "C4 plain decode every row")
    torch.testing.assert_close(out.float(), plain.float(), atol=2e-3, rtol=1e-2)


def test_prefix_is_the_whole_table(device):
    """prefix_blocks == max_blocks: the suffix tables are empty (width 0), every sequence
    is exactly the shared prefix, and the suffix part is empty (log-sum-exp -inf)."""
    pb = 24
    b = workloads.build_batch([pb * 16] * 40, [1] * 40, n_q=28, n_kv=4, head_dim=128, block_size=16,
                              dtype=torch.bfloat16, device=device, seed=12, pool_factor=1.3,
                              shared_prefix_blocks=pb)
    assert b.block_tables.shape[1] == pb
    out = _run(b, pb)
    assert_attn_close(out, _oracle(b), "prefix == table")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n_q,n_kv,head_dim,block_size,prefix_blocks,batch", [
    (28, 4, 128, 16, 37, 24),   # prefix not a whole number of chunks
    (32, 8, 128, 16, 64, 40),   # GQA 4
    (8, 8, 64, 16, 20, 48),     # MHA, head_dim 64
    (16, 1, 128, 32, 9, 8),     # MQA, 32-token blocks
    (28, 4, 128, 16, 1, 20),    # one shared block
])
def test_shapes_and_empty_suffixes(device, dtype, n_q, n_kv, head_dim, block_size, prefix_blocks, batch):
    """Suffix lengths include 0 (the sequence is exactly the prefix), 1 and a block edge."""
    rng = np.random.default_rng(prefix_blocks + batch)
    p_tok = prefix_blocks * block_size
    suffix = [0, 1, block_size - 1, block_size, block_size + 1] + rng.integers(0, 600, batch - 5).tolist()
    ctx = [p_tok + s for s in suffix]
    b = workloads.build_batch(ctx, [1] * batch, n_q=n_q, n_kv=n_kv, head_dim=head_dim, block_size=block_size,
                              dtype=dtype, device=device, seed=batch, pool_factor=1.3,
                              shared_prefix_blocks=prefix_blocks)
    out = _run(b, prefix_blocks)
    assert_attn_close(out, _oracle(b), f"shared prefix {n_q}/{n_kv} D{head_dim} bs{block_size}")


@pytest.mark.parametrize("n_q,n_kv,head_dim,block_size,batch,prefix_blocks", [
    (28, 4, 128, 16, 2, 8),     # 14 rows per KV head: one decode tile, plain path
    (8, 8, 256, 16, 24, 8),     # head_dim 256: plain path
    (8, 8, 128, 8, 24, 16),     # 8-token blocks: plain path
    (28, 4, 128, 16, 24, 0),    # no shared prefix
    (32, 1, 128, 16, 6, 8),     # 32 query heads per KV head: the prefill kernel's plain path
])
def test_plain_path_cases(device, n_q, n_kv, head_dim, block_size, batch, prefix_blocks):
    rng = np.random.default_rng(batch)
    ctx = [prefix_blocks * block_size + int(s) for s in rng.integers(1, 300, batch)]
    b = workloads.build_batch(ctx, [1] * batch, n_q=n_q, n_kv=n_kv, head_dim=head_dim, block_size=block_size,
                              dtype=torch.bfloat16, device=device, seed=7, pool_factor=1.3,
                              shared_prefix_blocks=prefix_blocks)
    out = _run(b, prefix_blocks)
    assert_attn_close(out, _oracle(b), "plain path")


def test_repeat_calls_are_identical_and_graph_replays(device):
    """Deterministic: the prefix pass's item order does not change any result bit; a
    captured call replays to the eager result."""
    b = workloads.prefix_share(device=device, seed=9, batch=48)
    first = _run(b, b.shared_blocks)
    assert torch.equal(first, _run(b, b.shared_blocks))
    q = b.padded_q().clone()
    _run(b, b.shared_blocks)  # workspace size cached before capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention_shared_prefix(q, b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16,
                                            b.shared_blocks)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)


def test_rejects_bad_prefix(device):
    b = workloads.prefix_share(device=device, seed=1, batch=4)
    with pytest.raises(ValueError, match="prefix_blocks"):
        _run(b, b.block_tables.shape[1] + 1)
    with pytest.raises(ValueError, match="q must be"):
        paged_attention_shared_prefix(b.padded_q().expand(-1, -1, 2, -1), b.kv_cache, b.block_tables,
                                      b.context_lens, 0, b.scale, 16, 4)


def test_sequence_shorter_than_prefix_is_flagged(device, monkeypatch):
    """A sequence with fewer KV tokens than the shared prefix breaks the caller's promise:
    the call still writes defined values (that row's suffix counts as empty) and sets
    SS_STATUS_PREFIX_SHORT; the other rows keep their exact result, and a call that keeps
    the promise leaves the word clear."""
    monkeypatch.delenv("SLIPSTREAM_DEBUG", raising=False)
    b = workloads.prefix_share(device=device, seed=3, batch=32)
    attention_status(clear=True)
    _run(b, b.shared_blocks)
    assert attention_status(clear=True) == 0
    lens = b.context_lens.clone()
    lens[5] = b.shared_blocks * 16 - 7
    out = paged_attention_shared_prefix(b.padded_q(), b.kv_cache, b.block_tables, lens, 0, b.scale, 16,
                                        b.shared_blocks)
    assert attention_status(clear=True) & SS_STATUS_PREFIX_SHORT
    rows = [i for i in range(b.batch) if i != 5]
    assert_attn_close(out[rows], _oracle(b, rows), "rows that keep the promise")
    # the flagged row: its suffix counts as empty, so it is attention over the whole
    # shared prefix (the first shared_blocks entries of its own table)
    kv = f64(b.kv_cache)
    tables = tables_array([b.tables_host[5]], b.block_tables.shape[1])
    ref5 = ora.paged_attention(f64(b.padded_q()[5:6]), kv, tables, np.array([b.shared_blocks * 16]), 0, b.scale,
                               b.block_size)
    assert_attn_close(out[5:6], ref5, "flagged row = prefix only")


@pytest.mark.parametrize("n_kv", [8, 4])
def test_empty_suffixes_between_short_ones(device, n_kv):
    """Sequences with an empty suffix (seq_len == prefix tokens) sit between sequences of
    one or two 32-key pairs, with one long suffix so that every decode range holds
    several pairs: a range then finishes a run of short suffixes with empty ones inside
    it. Every row is checked against the oracle, and the result repeats bit for bit
    (no race between the range's merge block and an empty suffix's own block)."""
    rng = np.random.default_rng(40 + n_kv)
    prefix_blocks, batch = 20, 96
    p_tok = prefix_blocks * 16
    suffix = []
    for i in range(batch):
        suffix.append(0 if i % 2 else int(rng.integers(1, 65)))
    suffix[37] = 7000
    mk = lambda sfx, seed: workloads.build_batch(  # noqa: E731
        [p_tok + s for s in sfx], [1] * batch, n_q=4 * n_kv, n_kv=n_kv, head_dim=128, block_size=16,
        dtype=torch.bfloat16, device=device, seed=seed, pool_factor=1.3, shared_prefix_blocks=prefix_blocks)
    # a call of the same shape whose odd rows have suffixes first: the workspace (same
    # size, so the caching allocator hands the same block back) then holds finished-row
    # state for the rows that are empty in the call under test
    primed = mk([s if s else 40 for s in suffix], 90 + n_kv)
    _run(primed, prefix_blocks)
    b = mk(suffix, 3 + n_kv)
    out = _run(b, prefix_blocks)
    assert_attn_close(out, _oracle(b), f"empty suffixes between short ones, n_kv {n_kv}")
    for _ in range(3):
        assert torch.equal(out, _run(b, prefix_blocks))
