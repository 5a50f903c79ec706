"""GPU parity of the page copies (copy-on-write and swap) against the numpy oracle:
bit exact (``oracle.paged_attention.copy_blocks`` / ``swap_blocks``,
attention_ref.py:92-94, block_manager.py:196-200,220-225)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from slipstream_amd.kernels import copy_blocks, swap_blocks

pytestmark = pytest.mark.gpu


def _cache(shape, dtype, seed, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    view = {2: torch.int16, 4: torch.int32}[t.element_size()]
    return t.view(view).numpy().copy()


@pytest.mark.parametrize("shape,dtype", [
    ((3, 2, 40, 16, 8, 128), torch.bfloat16),   # Llama page (32 KB), three layers
    ((1, 2, 33, 5, 3, 24), torch.float16),      # 720-byte pages: 16-byte pieces, ragged last piece
    ((2, 2, 17, 3, 1, 6), torch.float16),       # 36-byte pages: 4-byte pieces
    ((1, 2, 9, 3, 1, 3), torch.float16),        # 18-byte pages: byte copies
    ((1, 2, 20, 16, 2, 64), torch.float32),
])
def test_copy_blocks_bit_exact(device, shape, dtype):
    print(f"copy_blocks {shape} {dtype}", flush=True)
    kv = _cache(shape, dtype, seed=shape[2])
    nb = shape[2]
    rng = np.random.default_rng(nb)
    srcs = rng.choice(nb, nb // 2, replace=False)
    free = [b for b in range(nb) if b not in set(srcs.tolist())]
    mapping = {int(s): int(d) for s, d in zip(srcs, rng.choice(free, len(srcs), replace=False))}
    ref = _bits(kv)
    ora.copy_blocks(ref, list(mapping.items()))
    kd = kv.to(device)
    copy_blocks(kd, mapping)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd), ref)


def test_copy_blocks_chains_follow_dict_order(device):
    """A destination that is also a later source, and a repeated destination: the
    result of copying one pair after the other (the wrapper splits the launches)."""
    kv = _cache((2, 2, 12, 16, 2, 32), torch.bfloat16, seed=3)
    mapping = {0: 1, 1: 2, 2: 3, 5: 5, 7: 4, 9: 8}
    pairs = list(mapping.items()) + [(6, 4)]  # dict keys are unique: the repeat goes through the pair list
    ref = _bits(kv)
    ora.copy_blocks(ref, pairs)
    kd = kv.to(device)
    copy_blocks(kd, mapping)
    copy_blocks(kd, {6: 4})
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd), ref)


def test_copy_blocks_rejects_bad_ids_and_layouts(device):
    kv = _cache((1, 2, 4, 16, 2, 32), torch.bfloat16, seed=1, device=device)
    with pytest.raises(ValueError):
        copy_blocks(kv, {0: 4})
    with pytest.raises(ValueError):
        copy_blocks(kv, {-1: 2})
    with pytest.raises(ValueError):
        copy_blocks(kv[:, :, :, :, :, :16], {0: 1})  # pages not contiguous
    copy_blocks(kv, {})  # empty mapping: nothing to do


def test_swap_out_and_in_round_trip(device):
    """Swap out to a pinned host cache and back into other blocks: bit exact."""
    shape = (2, 2, 24, 16, 8, 128)
    gpu = _cache(shape, torch.bfloat16, seed=11, device=device)
    host = torch.zeros((2, 2, 10, 16, 8, 128), dtype=torch.bfloat16).pin_memory()
    out_map = {3: 0, 17: 1, 8: 9, 23: 4}
    swap_blocks(gpu, host, out_map)
    torch.cuda.synchronize()
    ref_host = _bits(torch.zeros_like(host))
    ora.swap_blocks(_bits(gpu), ref_host, list(out_map.items()))
    assert np.array_equal(_bits(host), ref_host)
    back = torch.zeros_like(gpu)
    in_map = {0: 5, 1: 6, 9: 7, 4: 20}
    swap_blocks(host, back, in_map)
    torch.cuda.synchronize()
    ref_back = _bits(torch.zeros_like(gpu))
    ora.swap_blocks(ref_host, ref_back, list(in_map.items()))
    assert np.array_equal(_bits(back), ref_back)


def test_swap_needs_pinned_host_memory(device):
    gpu = _cache((1, 2, 4, 16, 2, 32), torch.bfloat16, seed=2, device=device)
    pageable = torch.zeros((1, 2, 4, 16, 2, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="pin_memory"):
        swap_blocks(gpu, pageable, {0: 0})


def test_copy_blocks_device_pairs_tensor(device):
    """Pairs already on the device: one launch, same bytes; rows with ids outside the pool
    are skipped."""
    kv = _cache((2, 2, 30, 16, 2, 64), torch.bfloat16, seed=21)
    pairs = [(4, 20), (11, 0), (29, 7), (3, 25)]
    ref = _bits(kv)
    ora.copy_blocks(ref, pairs)
    kd = kv.to(device)
    t = torch.tensor(pairs + [(40, 1), (2, -1)], dtype=torch.int64, device=device)
    copy_blocks(kd, t)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd), ref)
    with pytest.raises(ValueError):
        copy_blocks(kd, t.to(torch.int32))
