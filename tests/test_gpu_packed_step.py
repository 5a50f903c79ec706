"""A packed attention step of one layer (fused RoPE + scatter, then varlen attention) with
its metadata built on the device: equal to the composition of the separately tested
ops, and a decode step captured in a HIP graph replays as the sequences grow."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from slipstream_amd import workloads
from slipstream_amd.kernels import packed_attention, paged_attention_varlen, reshape_and_cache
from slipstream_amd.paged_cache import build_packed_step

pytestmark = pytest.mark.gpu


def _rope_torch(x, cos, sin):
    """apply_rotary_pos_emb's arithmetic (rope.py:33-35) with torch's own ops on the device."""
    d = x.shape[-1]
    c, s = cos[:, None], sin[:, None]
    return x * c + torch.cat((-x[..., d // 2:], x[..., : d // 2]), dim=-1) * s


def _tables_prior(b, device):
    ql = torch.tensor(b.query_lens, dtype=torch.int32, device=device)
    return ql, b.context_lens.to(torch.int32) - ql


def test_packed_attention_equals_rope_scatter_varlen(device):
    ctx, ql = workloads.mixed_step_lengths(seed=4, n_prefill=2, chunk=64, n_decode=12)
    b = workloads.build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=torch.bfloat16,
                              device=device, seed=4)
    t = b.q.shape[0]
    g = torch.Generator(device=device).manual_seed(4)
    cos = torch.randn(t, 128, generator=g, device=device).to(torch.bfloat16)
    sin = torch.randn(t, 128, generator=g, device=device).to(torch.bfloat16)
    qlens, prior = _tables_prior(b, device)
    step = build_packed_step(b.block_tables, prior, qlens, 16, t, b.max_query_len)
    kv_ref = b.kv_cache.clone()
    out = packed_attention(b.q, b.k_new, b.v_new, cos, sin, b.kv_cache, step, 0, b.scale, 16)
    reshape_and_cache(_rope_torch(b.k_new, cos, sin), b.v_new, kv_ref, b.slot_mapping, 0, 16)
    ref = paged_attention_varlen(_rope_torch(b.q, cos, sin), kv_ref, b.block_tables, b.cu_seqlens, b.context_lens,
                                 0, b.scale, 16, b.max_query_len)
    torch.cuda.synchronize()
    assert torch.equal(b.kv_cache, kv_ref)
    assert torch.equal(out, ref)
    # replay mode (PagedForward.write_kv = False): the cache is left alone
    before = b.kv_cache.clone()
    packed_attention(b.q, b.k_new, b.v_new, cos, sin, b.kv_cache, step, 0, b.scale, 16, write_kv=False)
    torch.cuda.synchronize()
    assert torch.equal(b.kv_cache, before)


def test_decode_step_graph_replays_as_sequences_grow(device):
    """Static buffers, one captured graph: metadata build, fused RoPE + scatter and the
    attention of a 16-sequence decode step. Between replays the host only writes new
    inputs and advances prior_lens on the device; each replay equals the eager step."""
    bsz, n_q, n_kv, d, bs, nb = 16, 32, 8, 128, 16, 512
    rng = np.random.default_rng(12)
    gen = torch.Generator(device=device).manual_seed(12)
    kv = (torch.randn(1, 2, nb, bs, n_kv, d, generator=gen, device=device) * 0.5).to(torch.bfloat16)
    tables = torch.from_numpy(rng.permutation(nb)[: bsz * 24].reshape(bsz, 24).astype(np.int32)).to(device)
    prior = torch.from_numpy(rng.integers(20, 300, bsz).astype(np.int32)).to(device)
    ones = torch.ones(bsz, dtype=torch.int32, device=device)
    q = torch.empty(bsz, n_q, d, dtype=torch.bfloat16, device=device)
    k = torch.empty(bsz, n_kv, d, dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    cos = torch.empty(bsz, d, dtype=torch.bfloat16, device=device)
    sin = torch.empty_like(cos)
    scale = d ** -0.5

    def fill(seed):
        g2 = torch.Generator(device=device).manual_seed(seed)
        for t in (q, k, v, cos, sin):
            t.copy_((torch.randn(t.shape, generator=g2, device=device) * 0.5).to(t.dtype))

    def step():
        meta = build_packed_step(tables, prior, ones, bs, bsz, 1)
        return packed_attention(q, k, v, cos, sin, kv, meta, 0, scale, bs)

    fill(0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kv_save = kv.clone()
        step()  # warm-up on the capture stream: the attention workspace is allocated here
        kv.copy_(kv_save)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = step()
    torch.cuda.synchronize()
    kv.copy_(kv_save)  # the capture itself does not run the kernels, but keep the state explicit
    for rep in range(4):
        fill(100 + rep)
        before = kv.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got, kv_graph = out.clone(), kv.clone()
        kv.copy_(before)
        want = step()  # eager, same inputs and cache state
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}: output"
        assert torch.equal(kv_graph, kv), f"replay {rep}: cache"
        prior.add_(1)  # the sequences grew by the token just written
