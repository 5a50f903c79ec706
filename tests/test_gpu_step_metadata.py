"""GPU parity of the on-device packed-step metadata builder against the numpy oracle
(``oracle.paged_attention.build_step_metadata``; paged_cache.py:71-109,
block_manager.py:141-159): exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora
from slipstream_amd import workloads
from slipstream_amd.paged_cache import build_packed_step

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,bs", [(1, 16), (37, 16), (300, 8), (5, 5)])
def test_build_step_metadata_equals_oracle(device, batch, bs):
    rng = np.random.default_rng(batch + bs)
    max_blocks = 40
    tables = []
    for _ in range(batch):
        n = int(rng.integers(0, max_blocks + 1))
        t = rng.integers(0, 5000, n).tolist()
        if n > 2 and rng.random() < 0.3:
            t[int(rng.integers(0, n))] = -1  # a hole
        tables.append(t)
    prior = rng.integers(-3, max_blocks * bs, batch)
    q = rng.integers(-2, 3 * bs, batch)
    q[rng.random(batch) < 0.2] = 0
    cu, ctx, slots = ora.build_step_metadata(tables, prior, q, bs)
    bt = torch.full((batch, max_blocks), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        if t:
            bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    step = build_packed_step(bt.to(device), torch.from_numpy(prior.astype(np.int32)).to(device),
                             torch.from_numpy(q.astype(np.int32)).to(device), bs, int(cu[-1]), int(max(q.max(), 0)))
    torch.cuda.synchronize()
    assert step.cu_seqlens.cpu().numpy().tolist() == cu.tolist()
    assert step.context_lens.cpu().numpy().tolist() == ctx.tolist()
    assert step.slot_mapping.cpu().numpy().tolist() == slots.tolist()


def test_device_metadata_equals_host_built_mixed_step(device):
    """The C3 mixed step: the device-built metadata equals what the host builds
    (workloads.build_batch follows build_paged_forward)."""
    b = workloads.mixed_step(device=device, seed=3)
    ql = torch.tensor(b.query_lens, dtype=torch.int32, device=device)
    prior = b.context_lens.to(torch.int32) - ql
    step = build_packed_step(b.block_tables, prior, ql, b.block_size, int(sum(b.query_lens)), b.max_query_len)
    torch.cuda.synchronize()
    assert torch.equal(step.cu_seqlens, b.cu_seqlens.to(torch.int32))
    assert torch.equal(step.context_lens, b.context_lens.to(torch.int32))
    assert torch.equal(step.slot_mapping, b.slot_mapping)


def test_slot_mapping_tail_past_the_step_is_minus_one(device):
    """A slot_mapping longer than the step's tokens: the tail is -1 on the device (it was
    stale memory, which the scatter would take for slots), through the C ABI on a buffer
    pre-filled with in-pool slots, and through build_packed_step."""
    from slipstream_amd import _ffi

    tables = [[7, 9], [4], [11, 12, 13]]
    prior, ql, bs, total = [3, 0, 20], [2, 5, 4], 16, 20
    cu, ctx, want = ora.build_step_metadata(tables, prior, ql, bs, total_tokens=total)
    assert want[11:].tolist() == [-1] * 9
    bt = torch.full((3, 3), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    bt = bt.to(device)
    pr = torch.tensor(prior, dtype=torch.int32, device=device)
    q = torch.tensor(ql, dtype=torch.int32, device=device)
    cu_d = torch.empty(4, dtype=torch.int32, device=device)
    ctx_d = torch.empty(3, dtype=torch.int32, device=device)
    slots = torch.full((total,), 5, dtype=torch.int64, device=device)
    st = _ffi.lib().ss_build_step_metadata(bt.data_ptr(), bt.stride(0), 3, pr.data_ptr(), q.data_ptr(), 3, bs,
                                           cu_d.data_ptr(), ctx_d.data_ptr(), slots.data_ptr(), total,
                                           _ffi.stream_ptr(device))
    _ffi.check(st, "build_step_metadata")
    torch.cuda.synchronize()
    assert slots.cpu().numpy().tolist() == want.tolist()
    assert cu_d.cpu().numpy().tolist() == cu.tolist() and ctx_d.cpu().numpy().tolist() == ctx.tolist()
    step = build_packed_step(bt, pr, q, bs, total, 5)
    torch.cuda.synchronize()
    assert step.slot_mapping.cpu().numpy().tolist() == want.tolist()
