"""numpy oracle of the paged KV scatter, gather and attention (test infrastructure).

Arrays only (no torch): K/V/Q values are float64 copies of the bf16/fp16
inputs (exact), the scatter works on the raw 16-bit patterns (bit exact).

Semantics chosen where the reference's two paths disagree (slipstream's
``attention_ref`` vs its Triton kernel), both followed by the HIP kernels:
  * negative slots are skipped (triton_paged.py:70-71), not written through
    Python negative indexing (attention_ref.py:36-39);
  * negative table entries inside the first ceil(len/bs) blocks are masked
    (triton_paged.py:161-165) rather than truncating the gather
    (attention_ref.py:50-51);
  * a query row with no visible key is zero (triton_paged.py:196-197) rather
    than raising (attention.py:44-45).
For tables without holes and 1 <= Tq <= seq_len these coincide with the
reference's gather + eager path.
"""

from __future__ import annotations

import numpy as np


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def reshape_and_cache(
    k: np.ndarray,
    v: np.ndarray,
    kv_cache: np.ndarray,
    slot_mapping: np.ndarray,
    layer_idx: int,
    block_size: int,
) -> None:
    """In place: ``kv_cache[layer, 0/1, slot // bs, slot % bs] = k/v[n]``.

    attention_ref.py:21-39 (index_put) with ``_flatten_kv`` (:8-18): ``k`` is
    ``[N, n_kv, D]`` or ``[B, n_kv, T, D]`` (token n = b*T + t). Works on any
    dtype, usually the uint16 bit patterns. Slots < 0 or past the pool are
    skipped; duplicate slots are last-writer-wins.
    """
    if k.shape != v.shape:
        raise ValueError(f"k/v shape mismatch {k.shape} vs {v.shape}")
    if k.ndim == 4:
        k = k.transpose(0, 2, 1, 3).reshape(-1, k.shape[1], k.shape[3])
        v = v.transpose(0, 2, 1, 3).reshape(-1, v.shape[1], v.shape[3])
    elif k.ndim != 3:
        raise ValueError(f"k must be [N,n_kv,D] or [B,n_kv,T,D], got {k.shape}")
    n_tok = k.shape[0]
    slots = np.asarray(slot_mapping).reshape(-1)
    if slots.size != n_tok:
        raise ValueError(f"slot_mapping {slots.size} != tokens {n_tok}")
    n_slots = kv_cache.shape[2] * block_size
    for n in range(n_tok):
        s = int(slots[n])
        if s < 0 or s >= n_slots:
            continue
        kv_cache[layer_idx, 0, s // block_size, s % block_size] = k[n]
        kv_cache[layer_idx, 1, s // block_size, s % block_size] = v[n]


def build_step_metadata(tables: list[list[int]], prior_lens, query_lens, block_size: int,
                        total_tokens: int | None = None):
    """Packed metadata of one step (paged_cache.py:71-109 with the packed description):
    ``cu_seqlens`` = [0] + cumsum(query_lens), ``context_lens`` = prior + query, and the
    slot of token j of sequence b at position p = prior[b] + j:
    ``tables[b][p // bs] * bs + p % bs`` (-1 past the table or on a negative entry).
    Negative lengths count as 0. With ``total_tokens`` the slot list has exactly that
    many entries: cut after it, or padded with -1 (one slot per new token,
    paged_cache.py:85-109; a padded entry names no token, so the scatter skips it)."""
    q = [max(int(v), 0) for v in query_lens]
    p0 = [max(int(v), 0) for v in prior_lens]
    cu = [0]
    for v in q:
        cu.append(cu[-1] + v)
    slots = []
    for b, table in enumerate(tables):
        for j in range(q[b]):
            pos = p0[b] + j
            bi = pos // block_size
            e = table[bi] if bi < len(table) else -1
            slots.append(e * block_size + pos % block_size if e >= 0 else -1)
    ctx = [a + b for a, b in zip(p0, q)]
    if total_tokens is not None:
        slots = (slots + [-1] * total_tokens)[:total_tokens]
    return np.array(cu, np.int32), np.array(ctx, np.int32), np.array(slots, np.int64)


def copy_blocks(kv_cache: np.ndarray, pairs) -> None:
    """In place: ``kv_cache[:, :, dst] = kv_cache[:, :, src]`` for each (src, dst), one
    pair after the other (attention_ref.py:92-94 iterates its dict in order). The swap
    copies of block_manager.py:196-200,220-225 are the same page copy between two arrays
    (``swap_blocks``). Any dtype; usually the raw 16-bit patterns (bit exact)."""
    for s, d in pairs:
        kv_cache[:, :, d] = kv_cache[:, :, s]


def swap_blocks(src_cache: np.ndarray, dst_cache: np.ndarray, pairs) -> None:
    """In place: ``dst_cache[:, :, dst] = src_cache[:, :, src]`` for each (src, dst)."""
    for s, d in pairs:
        dst_cache[:, :, d] = src_cache[:, :, s]


def gather_kv(
    kv_cache: np.ndarray, layer_idx: int, block_table: np.ndarray, seq_len: int, block_size: int
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Gather one sequence's keys: ``(K [S, n_kv, D], V [S, n_kv, D], valid [S])``.

    attention_ref.py:42-65 reshaped to token-major, over the first
    ``min(ceil(len/bs), len(table))`` table entries (triton_paged.py:138);
    ``valid[t]`` is False where the table entry is negative or past the pool.
    """
    seq_len = max(int(seq_len), 0)
    table = np.asarray(block_table).reshape(-1)
    n_blocks = min(cdiv(seq_len, block_size), table.size)
    s = min(seq_len, n_blocks * block_size)
    t = np.arange(s)
    phys = table[t // block_size].astype(np.int64) if s else np.zeros(0, np.int64)
    valid = (phys >= 0) & (phys < kv_cache.shape[2])
    safe = np.where(valid, phys, 0)
    k = kv_cache[layer_idx, 0, safe, t % block_size]
    v = kv_cache[layer_idx, 1, safe, t % block_size]
    return k, v, valid


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, valid: np.ndarray, seq_len: int,
           scale: float) -> np.ndarray:
    """One sequence: ``q`` ``[n_q, Tq, D]`` over gathered ``k``/``v`` ``[S, n_kv, D]``.

    eager_attention (attention.py:64-88): GQA head map h -> h // n_rep
    (repeat_kv, :20-29), query j at absolute index seq_len - Tq + j sees keys
    <= that index (packed_causal_mask, :32-51), softmax in float64. Returns
    ``[Tq, n_q, D]``; rows with no visible key are zero.
    """
    n_q, tq, d = q.shape
    n_kv = k.shape[1]
    n_rep = n_q // n_kv
    s = k.shape[0]
    out = np.zeros((tq, n_q, d), dtype=np.float64)
    if s == 0 or tq == 0:
        return out
    # query head h = g * n_rep + r reads KV head g (repeat_kv): the n_rep heads of a
    # group share one batched product with their KV head, [n_kv, n_rep * Tq, S]
    qg = q.astype(np.float64).reshape(n_kv, n_rep * tq, d)
    kg = np.ascontiguousarray(k.transpose(1, 0, 2), dtype=np.float64)  # [n_kv, S, D]
    vg = np.ascontiguousarray(v.transpose(1, 0, 2), dtype=np.float64)
    scores = np.matmul(qg, kg.transpose(0, 2, 1)).reshape(n_kv, n_rep, tq, s) * scale
    key_pos = np.arange(s)[None, :]
    query_abs = (seq_len - tq + np.arange(tq))[:, None]
    visible = (key_pos <= query_abs) & valid[None, :]  # [Tq, S]
    scores = np.where(visible, scores, -np.inf)
    m = scores.max(axis=-1, keepdims=True)
    any_vis = np.isfinite(m)
    p = np.where(visible, np.exp(scores - np.where(any_vis, m, 0.0)), 0.0)
    denom = p.sum(axis=-1, keepdims=True)
    w = np.where(denom > 0, p / np.where(denom > 0, denom, 1.0), 0.0)
    o = np.matmul(w.reshape(n_kv, n_rep * tq, s), vg)  # [n_kv, n_rep * Tq, D]
    return o.reshape(n_q, tq, d).transpose(1, 0, 2)


def paged_attention(
    q: np.ndarray,
    kv_cache: np.ndarray,
    block_tables: np.ndarray,
    seq_lens: np.ndarray,
    layer_idx: int,
    scale: float,
    block_size: int,
) -> np.ndarray:
    """``q`` ``[B, n_q, Tq, D]`` -> ``[B, Tq, n_q, D]`` (paged_attention_ref, attention_ref.py:68-89)."""
    b_, n_q, tq, d = q.shape
    out = np.zeros((b_, tq, n_q, d), dtype=np.float64)
    for b in range(b_):
        sl = max(int(seq_lens[b]), 0)
        k, v, valid = gather_kv(kv_cache, layer_idx, block_tables[b], sl, block_size)
        out[b] = attend(q[b], k, v, valid, sl, scale)
    return out


def paged_attention_varlen(
    q: np.ndarray,
    kv_cache: np.ndarray,
    block_tables: np.ndarray,
    cu_seqlens: np.ndarray,
    context_lens: np.ndarray,
    layer_idx: int,
    scale: float,
    block_size: int,
) -> np.ndarray:
    """Packed step ``q`` ``[T, n_q, D]`` -> ``[T, n_q, D]``: per-sequence calls concatenated.

    The reference has no packed entry; its engine runs each sequence's tokens as
    one ``[1, n_q, Tq, D]`` call (llm_engine.py:508-567), which is what this does.
    """
    out = np.zeros(q.shape, dtype=np.float64)
    cu = np.asarray(cu_seqlens).reshape(-1)
    for b in range(cu.size - 1):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        if s1 <= s0:
            continue
        sl = max(int(context_lens[b]), 0)
        k, v, valid = gather_kv(kv_cache, layer_idx, block_tables[b], sl, block_size)
        qb = q[s0:s1].transpose(1, 0, 2)  # [n_q, Tq, D]
        out[s0:s1] = attend(qb, k, v, valid, sl, scale)
    return out


def merge_partials(parts: list[tuple[np.ndarray, np.ndarray, np.ndarray]]) -> np.ndarray:
    """Combine split-K partials ``(m, l, acc)`` over disjoint key ranges.

    ``m`` row max, ``l = sum exp(s - m)``, ``acc = sum exp(s - m) v``: the
    log-sum-exp merge the decode kernel's second pass performs.
    """
    m = np.max(np.stack([p[0] for p in parts]), axis=0)
    lsum = sum(p[1] * np.exp(p[0] - m) for p in parts)
    acc = sum(p[2] * np.exp(p[0] - m)[..., None] for p in parts)
    return np.where(lsum[..., None] > 0, acc / np.where(lsum > 0, lsum, 1.0)[..., None], 0.0)


def partial_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float):
    """Unnormalised partial of one key range (no mask): ``(m, l, acc)`` per query row."""
    s = np.einsum("rd,sd->rs", q, k) * scale
    m = s.max(axis=-1)
    p = np.exp(s - m[:, None])
    return m, p.sum(axis=-1), p @ v
