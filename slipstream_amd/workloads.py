"""Seeded synthetic workloads at the benchmark shapes (random data, no checkpoints).

Each builder returns the tensors one paged step consumes: the KV pool
``[1, 2, NB, bs, n_kv, D]`` filled with N(0,1)*0.5, block tables handing out
the pool's blocks in a seeded random permutation, the per-sequence context
lengths, the new tokens' K/V and their slot_mapping, and the queries.
Lengths are drawn with numpy's seeded ``default_rng``; tensor values with a
seeded torch generator on the target device (on the CPU when ``device`` is
CPU, so host-built inputs are identical on every machine).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class PagedBatch:
    kv_cache: torch.Tensor  # [1, 2, NB, bs, n_kv, D]
    block_tables: torch.Tensor  # [B, max_blocks] int32, -1 padded
    context_lens: torch.Tensor  # [B] int32, KV length after this step's tokens
    query_lens: list[int]  # new tokens per sequence
    cu_seqlens: torch.Tensor  # [B+1] int32
    q: torch.Tensor  # [T, n_q, D] packed queries
    k_new: torch.Tensor  # [T, n_kv, D]
    v_new: torch.Tensor  # [T, n_kv, D]
    slot_mapping: torch.Tensor  # [T] int64
    block_size: int
    n_q: int
    n_kv: int
    head_dim: int
    scale: float
    ctx_host: list[int] = field(default_factory=list)
    tables_host: list[list[int]] = field(default_factory=list)
    shared_blocks: int = 0  # leading table entries shared by every sequence (prefix config)

    @property
    def batch(self) -> int:
        return len(self.query_lens)

    @property
    def total_tokens(self) -> int:
        return int(sum(self.query_lens))

    @property
    def max_query_len(self) -> int:
        return max(self.query_lens) if self.query_lens else 0

    def padded_q(self) -> torch.Tensor:
        """``[B, n_q, Tq, D]`` view of the packed queries (all query_lens equal)."""
        tq = self.query_lens[0]
        return self.q.view(self.batch, tq, self.n_q, self.head_dim).transpose(1, 2)

    def padded_kv_new(self) -> tuple[torch.Tensor, torch.Tensor]:
        tq = self.query_lens[0]
        k = self.k_new.view(self.batch, tq, self.n_kv, self.head_dim).transpose(1, 2)
        v = self.v_new.view(self.batch, tq, self.n_kv, self.head_dim).transpose(1, 2)
        return k, v


def _randn(shape, gen: torch.Generator, dtype: torch.dtype, device: torch.device, std: float) -> torch.Tensor:
    out = torch.empty(shape, dtype=dtype, device=device)
    # chunked so a 2 GB pool never needs an fp32 copy of itself
    flat = out.view(-1)
    step = 1 << 26
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i : i + n] = (torch.randn(n, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)
    return out


def build_batch(
    context_lens: list[int],
    query_lens: list[int],
    *,
    n_q: int,
    n_kv: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
    device: torch.device | str,
    seed: int,
    num_blocks: int | None = None,
    pool_factor: float = 1.2,
    shared_prefix_blocks: int = 0,
    std: float = 0.5,
) -> PagedBatch:
    """One paged step over sequences with the given KV and query lengths.

    Sequence b's queries are its last ``query_lens[b]`` tokens (positions
    ``ctx - q .. ctx - 1``), whose slots are where the step's scatter writes.
    With ``shared_prefix_blocks = P`` every table starts with the same P pool
    blocks (a prefix-cache hit shares full blocks only, prefix_cache.py:50).
    """
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    bsz = len(context_lens)
    assert len(query_lens) == bsz
    need = [math.ceil(c / block_size) for c in context_lens]
    private = [max(0, n - shared_prefix_blocks) for n in need]
    total_need = shared_prefix_blocks + sum(private)
    nb = num_blocks if num_blocks is not None else max(1, math.ceil(pool_factor * total_need))
    if nb < total_need:
        raise ValueError(f"pool of {nb} blocks cannot hold {total_need}")
    perm = rng.permutation(nb).tolist()
    shared = perm[:shared_prefix_blocks]
    cursor = shared_prefix_blocks
    tables: list[list[int]] = []
    for b in range(bsz):
        t = shared[: min(shared_prefix_blocks, need[b])] + perm[cursor : cursor + private[b]]
        cursor += private[b]
        tables.append(t)
    max_blocks = max(1, max(len(t) for t in tables))
    bt = torch.full((bsz, max_blocks), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        if t:
            bt[b, : len(t)] = torch.tensor(t, dtype=torch.int32)

    slots: list[int] = []
    for b in range(bsz):
        for pos in range(context_lens[b] - query_lens[b], context_lens[b]):
            ok = 0 <= pos and pos // block_size < len(tables[b])
            slots.append(tables[b][pos // block_size] * block_size + pos % block_size if ok else -1)
    cu = [0]
    for ql in query_lens:
        cu.append(cu[-1] + ql)
    total = cu[-1]

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    kv = _randn((1, 2, nb, block_size, n_kv, head_dim), gen, dtype, device, std)
    q = _randn((total, n_q, head_dim), gen, dtype, device, std)
    k_new = _randn((total, n_kv, head_dim), gen, dtype, device, std)
    v_new = _randn((total, n_kv, head_dim), gen, dtype, device, std)
    return PagedBatch(
        kv_cache=kv,
        block_tables=bt.to(device),
        context_lens=torch.tensor(context_lens, dtype=torch.int32, device=device),
        query_lens=list(query_lens),
        cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device),
        q=q,
        k_new=k_new,
        v_new=v_new,
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        block_size=block_size,
        n_q=n_q,
        n_kv=n_kv,
        head_dim=head_dim,
        scale=head_dim**-0.5,
        ctx_host=list(context_lens),
        tables_host=tables,
        shared_blocks=shared_prefix_blocks,
    )


# ---- the BASELINE configurations -------------------------------------------------


def qwen05_decode(device="cpu", seed: int = 0, dtype=torch.float16) -> PagedBatch:
    """C1: Qwen2.5-0.5B shape decode, 8 sequences, ctx ~ U[32, 512], pool of 512 blocks."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(32, 513, size=8).tolist()
    return build_batch(ctx, [1] * 8, n_q=14, n_kv=2, head_dim=64, block_size=16, dtype=dtype,
                       device=device, seed=seed, num_blocks=512)


def llama_decode_lengths(seed: int = 0, batch: int = 256) -> list[int]:
    """C2 lengths: round(lognormal(ln 1024, 1.0)) clipped to [16, 8192]."""
    rng = np.random.default_rng(seed)
    x = np.rint(rng.lognormal(mean=math.log(1024.0), sigma=1.0, size=batch))
    return np.clip(x, 16, 8192).astype(int).tolist()


def llama_decode(device="cuda", seed: int = 0, dtype=torch.bfloat16, batch: int = 256) -> PagedBatch:
    """C2: Llama-3-8B shape ragged decode (32/8 heads, D 128, bs 16), pool 1.2x need."""
    ctx = llama_decode_lengths(seed, batch)
    return build_batch(ctx, [1] * batch, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=dtype,
                       device=device, seed=seed, pool_factor=1.2)


def mixed_step_lengths(seed: int = 0, n_prefill: int = 4, chunk: int = 512,
                       n_decode: int = 192) -> tuple[list[int], list[int]]:
    """C3 lengths: decodes first (the scheduler's order, scheduler.py:103-124), then chunks."""
    rng = np.random.default_rng(seed)
    dec = rng.integers(128, 4097, size=n_decode).tolist()
    prior = rng.integers(0, 4097, size=n_prefill).tolist()
    ctx = dec + [p + chunk for p in prior]
    ql = [1] * n_decode + [chunk] * n_prefill
    return ctx, ql


def mixed_step(device="cuda", seed: int = 0, dtype=torch.bfloat16, n_prefill: int = 4,
               chunk: int = 512, n_decode: int = 192) -> PagedBatch:
    """C3: 4 prefill chunks of 512 + 192 decodes packed into one 2240-token stream."""
    ctx, ql = mixed_step_lengths(seed, n_prefill, chunk, n_decode)
    return build_batch(ctx, ql, n_q=32, n_kv=8, head_dim=128, block_size=16, dtype=dtype,
                       device=device, seed=seed, pool_factor=1.2)


def prefix_share(device="cuda", seed: int = 0, dtype=torch.bfloat16, batch: int = 128,
                 prefix_tokens: int = 2048) -> PagedBatch:
    """C4: Qwen2.5-7B shape (28/4 heads), shared 2048-token prefix + private U[64,512] suffix."""
    rng = np.random.default_rng(seed)
    suffix = rng.integers(64, 513, size=batch).tolist()
    ctx = [prefix_tokens + s for s in suffix]
    return build_batch(ctx, [1] * batch, n_q=28, n_kv=4, head_dim=128, block_size=16, dtype=dtype,
                       device=device, seed=seed, pool_factor=1.2,
                       shared_prefix_blocks=prefix_tokens // 16)


def kv_bytes(batch: PagedBatch, unique: bool = False) -> int:
    """Algorithmic K+V bytes one attention pass reads (each page of each KV head once).

    ``unique``: count blocks shared by several tables once (prefix config).
    """
    elem = batch.kv_cache.element_size()
    per_token = 2 * batch.n_kv * batch.head_dim * elem
    if not unique or batch.shared_blocks == 0:
        return sum(batch.ctx_host) * per_token
    shared_tokens = batch.shared_blocks * batch.block_size
    return (shared_tokens + sum(c - shared_tokens for c in batch.ctx_host)) * per_token


# ---- W4A16 (C5) ----------------------------------------------------------------------


@dataclass
class W4A16Linear:
    """One int4 linear in the reference format (quant_ref.py:8-20) plus its activations."""

    x: torch.Tensor  # [M, K] bf16
    qweight: torch.Tensor  # [N, K/8] int32
    scales: torch.Tensor  # [N, K/g] fp16
    qzeros: torch.Tensor  # [N, K/g] int32
    group_size: int

    @property
    def m(self) -> int:
        return int(self.x.shape[0])

    @property
    def n(self) -> int:
        return int(self.qweight.shape[0])

    @property
    def k(self) -> int:
        return int(self.x.shape[1])

    def weight_bytes(self) -> int:
        return (self.qweight.numel() * 4 + self.scales.numel() * self.scales.element_size()
                + self.qzeros.numel() * 4)


def pack_int4_torch(q: torch.Tensor) -> torch.Tensor:
    """``[N, K]`` nibbles -> ``[N, K/8]`` int32, nibble n of word j = q[:, 8j+n] at bit 4n
    (quant_ref.py:45-60; packed in int64, the int32 keeps the 32-bit pattern)."""
    n, k = q.shape
    shifts = torch.arange(0, 32, 4, device=q.device, dtype=torch.int64)
    words = (q.to(torch.int64).view(n, k // 8, 8) << shifts).sum(dim=-1)
    return words.to(torch.int32)


def w4a16_linear(k: int, n: int, m: int, device="cuda", seed: int = 0, group_size: int = 128,
                 act: torch.dtype = torch.bfloat16, scale_dtype: torch.dtype = torch.float16) -> W4A16Linear:
    """C5 operands: q ~ U{0..15}, scales ~ U(0.005, 0.02) in fp16, zero points 8, x ~ N(0, 1)."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    q = torch.randint(0, 16, (n, k), generator=gen, device=device, dtype=torch.int32)
    qweight = pack_int4_torch(q)
    del q
    scales = torch.empty((n, k // group_size), device=device, dtype=torch.float32)
    scales.uniform_(0.005, 0.02, generator=gen)
    scales = scales.to(scale_dtype)
    qzeros = torch.full((n, k // group_size), 8, dtype=torch.int32, device=device)
    x = torch.randn((m, k), generator=gen, device=device, dtype=torch.float32).to(act)
    return W4A16Linear(x=x, qweight=qweight, scales=scales, qzeros=qzeros, group_size=group_size)

