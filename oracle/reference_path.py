"""The reference's own CPU path, restated in torch with its dtype sequence (test infrastructure).

This is what slipstream runs when its fast path is off or absent: a Python
loop over the batch, a gather of each sequence's pages into contiguous K/V,
``repeat_kv``, bf16/fp16 matmuls with a float32 softmax, and for W4A16 a full
dequantised weight then a dense matmul. ``bench.py`` times it on the host as
the CPU baseline, and the GPU tests report the HIP kernels' distance to it as
the dtype-faithful secondary check. Its own pins (tests/test_oracle_reference_path.py):
the scatter bit for bit against ``oracle.paged_attention.reshape_and_cache``; the
gather's copy, truncation and negative-index hole rule in closed form; attention in
float32 against the float64 oracle and torch's SDPA (1e-5), and in bf16/fp16 within
those dtypes' rounding bounds; W4A16 against the oracle's dequantise-then-matmul.
Where the reference and the HIP path's chosen semantics differ (holes in a table,
a query longer than its keys) this module keeps the reference's behaviour.
It restates (not imports) the reference:
  gather          slipstream/kernels/attention_ref.py:42-65
  eager attention slipstream/models/layers/attention.py:20-88
  paged loop      slipstream/kernels/attention_ref.py:68-89
  scatter         slipstream/kernels/attention_ref.py:21-39
  W4A16           slipstream/kernels/quant_ref.py:63-69,103-133
"""

from __future__ import annotations

import torch


def scatter(k: torch.Tensor, v: torch.Tensor, kv: torch.Tensor, slots: torch.Tensor, layer: int,
            block_size: int) -> None:
    """index_put of ``[N, n_kv, D]`` (or ``[B, n_kv, T, D]``, token b*T + t) rows at
    ``(slot // bs, slot % bs)``; a negative slot indexes from the end, as in the reference."""
    if k.shape != v.shape:
        raise ValueError(f"k/v shape mismatch {tuple(k.shape)} vs {tuple(v.shape)}")
    if k.ndim == 4:
        k = k.permute(0, 2, 1, 3).reshape(-1, k.shape[1], k.shape[3])
        v = v.permute(0, 2, 1, 3).reshape(-1, v.shape[1], v.shape[3])
    if slots.numel() != k.shape[0]:
        raise ValueError(f"slot_mapping {slots.numel()} != tokens {k.shape[0]}")
    if k.shape[0] == 0:
        return
    blk = torch.div(slots, block_size, rounding_mode="floor")
    off = slots % block_size
    kv[layer, 0, blk, off] = k
    kv[layer, 1, blk, off] = v


def gather(kv: torch.Tensor, layer: int, table: torch.Tensor, seq_len: int, block_size: int):
    """One sequence's pages -> contiguous ``[1, n_kv, S, D]`` K and V: the first
    ``min(ceil(seq_len / bs), #entries >= 0)`` table entries, so a short table truncates
    the keys and a -1 inside that range reads the pool's last block (Python indexing)."""
    valid = int((table >= 0).sum().item()) if table.numel() else 0
    n_blocks = min((seq_len + block_size - 1) // block_size, valid)
    n_kv, d = kv.shape[4], kv.shape[5]
    if n_blocks == 0:
        z = kv.new_zeros((1, n_kv, 0, d))
        return z, z.clone()
    ids = table[:n_blocks].long()
    k = kv[layer, 0, ids].reshape(n_blocks * block_size, n_kv, d)[:seq_len]
    v = kv[layer, 1, ids].reshape(n_blocks * block_size, n_kv, d)[:seq_len]
    return k.permute(1, 0, 2).unsqueeze(0).contiguous(), v.permute(1, 0, 2).unsqueeze(0).contiguous()


def eager(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """``[1, n_q, Tq, D]`` x ``[1, n_kv, S, D]`` -> ``[1, Tq, n_q, D]`` in q's dtype."""
    n_rep = q.shape[1] // k.shape[1]
    if n_rep > 1:
        b, h, s, d = k.shape
        k = k[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)
        v = v[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)
    tq, s = q.shape[2], k.shape[2]
    if tq > s:  # packed_causal_mask, attention.py:44-45
        raise ValueError(f"query_len {tq} > key_len {s}")
    scores = torch.matmul(q, k.transpose(2, 3)) * scale
    key_pos = torch.arange(s)
    q_abs = torch.arange(s - tq, s)
    allowed = key_pos.view(1, 1, 1, s) <= q_abs.view(1, 1, tq, 1)
    mask = torch.zeros((), dtype=scores.dtype).where(allowed, torch.tensor(float("-inf"), dtype=scores.dtype))
    w = torch.softmax(scores + mask, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w, v).transpose(1, 2).contiguous()


def paged_attention(q: torch.Tensor, kv: torch.Tensor, tables: torch.Tensor, seq_lens: torch.Tensor,
                    layer: int, scale: float, block_size: int) -> torch.Tensor:
    """``q`` ``[B, n_q, Tq, D]`` -> ``[B, Tq, n_q, D]``, one sequence at a time."""
    outs = []
    for i in range(q.shape[0]):
        sl = int(seq_lens[i].item())
        k, v = gather(kv, layer, tables[i], sl, block_size)
        outs.append(eager(q[i : i + 1], k, v, scale))
    return torch.cat(outs, dim=0)


def w4a16_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """Unpack (int64 nibbles) -> fp32 ``(q - z) * s`` -> scales.dtype -> x.dtype -> ``x @ W.T``."""
    out, n_groups = scales.shape
    k_in = n_groups * group_size
    p = qweight.to(torch.int64) & 0xFFFFFFFF
    shifts = (torch.arange(8, dtype=torch.int64) * 4).view(1, 1, 8)
    q = ((p.unsqueeze(-1) >> shifts) & 0xF).reshape(out, n_groups, group_size).float()
    w = (q - qzeros.reshape(out, n_groups, 1).float()) * scales.reshape(out, n_groups, 1).float()
    w = w.reshape(out, k_in).to(scales.dtype).to(x.dtype)
    return x @ w.t()
