"""KV page copies (HIP, gfx950): copy-on-write inside a cache, swap with a pinned host cache.

Drop-in for ``copy_blocks_ref`` (``slipstream/kernels/attention_ref.py:92-94``), the
copy-on-write copy of ``slipstream/memory/block_manager.py:297-298``, and the page copies
of the block manager's swap (``block_manager.py:196-200`` out, ``:220-225`` in), which the
reference makes one page at a time through pageable host memory. Here a whole mapping is
one launch (``ss_copy_blocks``); a host cache must be pinned (``pin_memory=True``), and
is read or written by the kernel through its device mapping. Device tensors only for the
GPU side: there is no CPU or fallback path.
"""

from __future__ import annotations

import numpy as np
import torch

from slipstream_amd import _ffi


def _page_layout(cache: torch.Tensor, what: str) -> tuple[int, int, int, int, int]:
    """(planes, plane stride, block stride, blocks, page bytes) of a
    ``[L, 2, num_blocks, block_size, n_kv, D]`` cache whose pages are contiguous."""
    if cache.ndim != 6 or cache.shape[1] != 2:
        raise ValueError(f"{what} must be [num_layers, 2, num_blocks, block_size, n_kv, head_dim], "
                         f"got {tuple(cache.shape)}")
    n_layers, _, n_blocks, bs, n_kv, d = cache.shape
    if cache.stride(5) != 1 or cache.stride(4) != d or cache.stride(3) != n_kv * d:
        raise ValueError(f"{what}: each page [block_size, n_kv, head_dim] must be contiguous")
    if n_layers > 1 and cache.stride(0) != 2 * cache.stride(1):
        raise ValueError(f"{what}: the (layer, K/V) planes must be evenly spaced (stride(0) == 2 * stride(1))")
    es = cache.element_size()
    return 2 * n_layers, cache.stride(1) * es, cache.stride(2) * es, n_blocks, bs * n_kv * d * es


def ordered_batches(pairs: list[tuple[int, int]]) -> list[list[tuple[int, int]]]:
    """Split ``(src, dst)`` pairs, in order, into consecutive batches that may each run
    all at once with the result of running the pairs one by one: a pair starts a new
    batch when it reads a block the batch writes, or writes a block the batch reads or
    writes (``copy_blocks_ref`` copies in dict order)."""
    batches: list[list[tuple[int, int]]] = []
    cur: list[tuple[int, int]] = []
    srcs: set[int] = set()
    dsts: set[int] = set()
    for s, d in pairs:
        if s in dsts or d in srcs or d in dsts:
            batches.append(cur)
            cur, srcs, dsts = [], set(), set()
        cur.append((s, d))
        srcs.add(s)
        dsts.add(d)
    if cur:
        batches.append(cur)
    return batches


_HOST_PAIRS = None


def _host_pairs():
    """The host helper extension (``csrc/host_pairs.c``): ``pack(mapping, addr, cap, n_src,
    n_dst, check) -> (n, independent)`` writes a dict's (src, dst) pairs as int64 rows into
    a buffer, raising ValueError for an id outside its cache, and with ``check`` reports
    whether the pairs may all run at once -- the criterion of ``ordered_batches``: distinct
    destinations, none of them another pair's source (the block manager's copy-on-write
    targets are fresh free blocks)."""
    global _HOST_PAIRS
    if _HOST_PAIRS is None:
        import importlib.util

        from slipstream_amd import build

        path = build.host_ext_path()
        if not path.exists():
            raise _ffi.KernelError(f"{path.name} is not built: run `python -m slipstream_amd.build`")
        spec = importlib.util.spec_from_file_location("slipstream_amd._host_pairs", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _HOST_PAIRS = mod
    return _HOST_PAIRS


class _Uploader:
    """Per-device pinned staging and device buffers for the pair lists of dict calls,
    grown as needed and reused: a call waits for the previous call's copy out of the
    staging buffer (an event) before it overwrites it, so no pinned allocation and no
    full synchronisation happen per call."""

    def __init__(self) -> None:
        self.host: dict[int, torch.Tensor] = {}
        self.dev: dict[int, torch.Tensor] = {}
        self.done: dict[int, torch.cuda.Event] = {}

    @staticmethod
    def _index(device: torch.device) -> int:
        return device.index if device.index is not None else torch.cuda.current_device()

    def staging(self, n: int, device: torch.device) -> torch.Tensor:
        """The pinned int64 ``[cap, 2]`` staging buffer (cap >= n), free to overwrite."""
        idx = self._index(device)
        host = self.host.get(idx)
        if idx in self.done:
            self.done[idx].synchronize()  # the previous copy has left the staging buffer
        if host is None or host.shape[0] < n:
            cap = max(n, 1024)
            host = self.host[idx] = torch.empty((cap, 2), dtype=torch.int64, pin_memory=True)
            self.dev[idx] = torch.empty((cap, 2), dtype=torch.int64, device=device)
        return host

    def send(self, n: int, device: torch.device) -> torch.Tensor:
        """Copy the staging buffer's first n rows to the device buffer (stream-ordered)."""
        idx = self._index(device)
        host, dev = self.host[idx], self.dev[idx]
        dev[:n].copy_(host[:n], non_blocking=True)
        ev = self.done.get(idx)
        if ev is None:
            ev = self.done[idx] = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        return dev[:n]

    def upload(self, pairs: np.ndarray, device: torch.device) -> torch.Tensor:
        n = pairs.shape[0]
        self.staging(n, device)[:n].numpy()[...] = pairs
        return self.send(n, device)


_UPLOADER = _Uploader()


def _launch(dst: torch.Tensor, src: torch.Tensor, mapping, device: torch.device) -> None:
    planes, dps, dbs, dnb, page = _page_layout(dst, "destination cache")
    splanes, sps, sbs, snb, spage = _page_layout(src, "source cache")
    if (splanes, spage) != (planes, page) or src.dtype != dst.dtype or src.shape[3:] != dst.shape[3:]:
        raise ValueError(f"caches differ beyond num_blocks: {tuple(src.shape)} {src.dtype} vs "
                         f"{tuple(dst.shape)} {dst.dtype}")
    for t, what in ((dst, "destination"), (src, "source")):
        if t.device.type == "cpu" and not t.is_pinned():
            raise ValueError(f"{what} cache is pageable host memory: allocate it with pin_memory=True")
    lib = _ffi.lib()
    stream = _ffi.stream_ptr(device)

    def run(dev_pairs: torch.Tensor, n: int) -> None:
        status = lib.ss_copy_blocks(dst.data_ptr(), src.data_ptr(), planes, dps, dbs, dnb, sps, sbs, snb, page,
                                    dev_pairs.data_ptr(), n, stream)
        _ffi.check(status, "copy_blocks")

    if isinstance(mapping, torch.Tensor):
        if mapping.ndim != 2 or mapping.shape[1] != 2 or mapping.dtype != torch.int64 or mapping.device != device:
            raise ValueError(f"pairs must be an int64 [n, 2] tensor on {device}, got {tuple(mapping.shape)} "
                             f"{mapping.dtype} on {mapping.device}")
        if mapping.shape[0]:
            run(mapping.contiguous(), mapping.shape[0])
        return
    if not isinstance(mapping, dict):
        mapping = dict(mapping)
    # the pairs go straight into the pinned staging buffer, checked on the way; the common
    # case (fresh destinations) is one launch; pairs that depend on each other run in dict
    # order, batch by batch (only a copy inside one cache can depend)
    host = _UPLOADER.staging(len(mapping), device)
    n, indep = _host_pairs().pack(mapping, host.data_ptr(), host.shape[0], snb, dnb, src is dst)
    if indep:
        run(_UPLOADER.send(n, device), n)
        return
    pairs = host[:n].numpy().copy()
    for b in ordered_batches([tuple(r) for r in pairs.tolist()]):
        batch = np.asarray(b, dtype=np.int64).reshape(-1, 2)
        run(_UPLOADER.upload(batch, device), batch.shape[0])


def copy_blocks(kv_cache: torch.Tensor, src_to_dst) -> None:
    """``kv_cache[:, :, dst] <- kv_cache[:, :, src]`` for every (src, dst), in dict order
    (``attention_ref.py:92-94``). Block ids must lie in ``[0, num_blocks)``.

    ``src_to_dst`` may also be an int64 ``[n, 2]`` device tensor of (src, dst) rows,
    copied in one launch with no host work: its destinations must be distinct and not
    among its sources (as the block manager's copy-on-write targets, fresh free blocks,
    are); rows with an id outside the pool are skipped."""
    if not isinstance(src_to_dst, torch.Tensor) and not src_to_dst:
        return
    if kv_cache.device.type != "cuda":
        raise _ffi.KernelError(f"copy_blocks: slipstream_amd runs on HIP devices only; got {kv_cache.device}")
    _launch(kv_cache, kv_cache, src_to_dst, kv_cache.device)


def swap_blocks(src_cache: torch.Tensor, dst_cache: torch.Tensor, src_to_dst) -> None:
    """``dst_cache[:, :, dst] <- src_cache[:, :, src]`` for every (src, dst) between a device
    cache and a pinned host cache (either direction: swap out is device -> host,
    ``block_manager.py:196-200``; swap in host -> device, ``:220-225``), or between two
    device caches. ``src_to_dst`` is a dict or an int64 ``[n, 2]`` device tensor (as for
    ``copy_blocks``). Asynchronous on the device's current stream: synchronise before
    the host reads a swapped-out page."""
    if not isinstance(src_to_dst, torch.Tensor) and not src_to_dst:
        return
    devs = [t.device for t in (src_cache, dst_cache) if t.device.type == "cuda"]
    if not devs:
        raise _ffi.KernelError("swap_blocks: one of the caches must be on a HIP device")
    if len(devs) == 2 and devs[0] != devs[1]:
        raise ValueError(f"caches on different devices: {devs[0]} and {devs[1]}")
    _launch(dst_cache, src_cache, src_to_dst, devs[0])
