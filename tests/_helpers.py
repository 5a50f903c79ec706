"""Conversions between device tensors and the numpy oracle."""

from __future__ import annotations

import numpy as np
import torch

# attention accumulates in fp32 -> 2e-3 abs / 1e-2 rel.
ATTN_ATOL = 2e-3
ATTN_RTOL = 1e-2


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns (bf16/fp16) for bit-exact comparisons."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


def assert_attn_close(got: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    g = f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    bound = ATTN_ATOL + ATTN_RTOL * np.abs(ref)
    bad = err > bound
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements out of tolerance; max abs err "
            f"{err.max():.3e}; first bad {idx.tolist()} got {g[tuple(idx[0])]:.5f} ref {ref[tuple(idx[0])]:.5f}"
        )


def gather_pool_f64(kv: torch.Tensor, tables: list[list[int]]):
    """Copy only the referenced blocks of a (possibly huge) pool to the host as float64.

    Returns (pool_subset [1, 2, nb_sub, bs, n_kv, D], remapped tables).
    """
    used = sorted({b for t in tables for b in t if b >= 0})
    idx = torch.tensor(used, dtype=torch.long, device=kv.device)
    sub = kv[:, :, idx]
    remap = {b: i for i, b in enumerate(used)}
    new_tables = [[remap.get(b, -1) if b >= 0 else -1 for b in t] for t in tables]
    return f64(sub), new_tables


def tables_array(tables: list[list[int]], width: int) -> np.ndarray:
    out = np.full((len(tables), max(width, 1)), -1, dtype=np.int64)
    for i, t in enumerate(tables):
        out[i, : len(t)] = t
    return out
