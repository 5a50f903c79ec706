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


# (test, check, max_abs, max_rel, elements) of every attention comparison of the run;
# conftest prints them in the terminal summary.
ERRORS: list[tuple[str, str, float, float, int]] = []


def error_stats(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    """max |got - ref|, and max |got - ref| / |ref| over the elements where the relative
    term of the bound is the larger one (|ref| >= ATTN_ATOL / ATTN_RTOL = 0.2); 0 when
    there are none."""
    err = np.abs(got - ref)
    big = np.abs(ref) >= ATTN_ATOL / ATTN_RTOL
    rel = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    return float(err.max()) if err.size else 0.0, rel


def record_error(what: str, got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    import os

    max_abs, max_rel = error_stats(got, ref)
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0].split("::")[-1]
    ERRORS.append((test, what, max_abs, max_rel, int(ref.size)))
    return max_abs, max_rel


def assert_attn_close(got: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    """Attention parity: |err| <= 2e-3 + 1e-2 |ref| per element;
    the max-abs and max-rel errors are recorded for the run's summary."""
    g = f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    record_error(what, g, ref)
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


def oracle_paged_rows(kv_cache: torch.Tensor, tables: list[list[int]], ctx: list[int],
                      queries: list[np.ndarray], scale: float, block_size: int, layer: int = 0,
                      workers: int | None = None) -> list[np.ndarray]:
    """Float64 oracle of every sequence of a (possibly full-size) batch: ``queries[i]`` is
    sequence i's ``[n_q, Tq, D]`` (float64), the result its ``[Tq, n_q, D]``. The
    referenced pages come to the host once, in their own dtype; each sequence's pages
    are widened to float64 and attended (``oracle.paged_attention.gather_kv`` /
    ``attend``) on a thread pool -- numpy's products and ufuncs release the GIL."""
    import concurrent.futures
    import os

    from oracle import paged_attention as ora

    used = sorted({b for t in tables for b in t if 0 <= b < kv_cache.shape[2]})
    idx = torch.tensor(used, dtype=torch.long, device=kv_cache.device)
    sub = kv_cache[layer : layer + 1, :, idx].cpu()  # [1, 2, n_used, bs, n_kv, D]
    remap = {b: i for i, b in enumerate(used)}

    def one(i: int) -> np.ndarray:
        t = [remap.get(b, -1) if b >= 0 else -1 for b in tables[i]]
        live = [x for x in t if x >= 0]
        pages = sub[:, :, torch.tensor(live, dtype=torch.long)].float().numpy().astype(np.float64)
        local, j = [], 0
        for x in t:  # this sequence's table over its own pages
            local.append(j if x >= 0 else -1)
            j += x >= 0
        k, v, valid = ora.gather_kv(pages, 0, np.array(local, dtype=np.int64), ctx[i], block_size)
        return ora.attend(queries[i], k, v, valid, ctx[i], scale)

    from threadpoolctl import threadpool_limits

    n = workers or min(16, len(os.sched_getaffinity(0)))
    torch_threads = torch.get_num_threads()
    torch.set_num_threads(1)  # one level of parallelism: the pool's
    try:
        with threadpool_limits(1), concurrent.futures.ThreadPoolExecutor(max_workers=n) as ex:
            return list(ex.map(one, range(len(tables))))
    finally:
        torch.set_num_threads(torch_threads)
