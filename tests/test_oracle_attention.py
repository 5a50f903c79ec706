"""Pins of the numpy attention oracle (``oracle/paged_attention.py``) -- CPU only.

The reference holds no golden vectors for this path (only seeded tests), so each
oracle function is checked against something that does not re-evaluate its own
formula:
  * the reference's own round-trip test (tests/kernels/test_paged_attention.py:19-43)
    and mask test (tests/correctness/test_cache_and_sampler.py:204-214), restated;
  * torch's scaled_dot_product_attention (float64, explicit boolean mask, GQA by
    expansion) -- a library routine for the dense case;
  * a pure-Python scalar loop with ``math.exp`` on tiny inputs;
  * closed forms (uniform scores -> mean of V, a dominant key -> its V row) and
    invariants (block relabelling, shared prefix, split-K merge, packed == per-sequence);
  * the hand-derived known answers in tests/golden/known_answers.json.
Each check is chosen so that a plausible slip (swapped block/offset, wrong GQA
head map, off-by-one in the causal offset, a dropped scale) fails it.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged_attention as ora

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"


def _rng(seed):
    return np.random.default_rng(seed)


def _paged_from_dense(k, v, block_size, rng, extra_blocks=3):
    """Scatter dense [S, n_kv, D] K/V of one sequence into a pool through a random table."""
    s, n_kv, d = k.shape
    nb = -(-s // block_size)
    pool_blocks = nb + extra_blocks
    perm = rng.permutation(pool_blocks)
    table = perm[:nb]
    kv = rng.standard_normal((1, 2, pool_blocks, block_size, n_kv, d))  # garbage outside the sequence
    slots = np.array([table[t // block_size] * block_size + t % block_size for t in range(s)])
    ora.reshape_and_cache(k, v, kv, slots, 0, block_size)
    return kv, table


# ---------------------------------------------------------------- scatter / gather


@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("seq_len", [1, 17, 64])
def test_scatter_gather_roundtrip_exact(block_size, seq_len):
    """Restates tests/kernels/test_paged_attention.py:19-43: scatter then gather is the identity."""
    rng = _rng(seq_len * 100 + block_size)
    n_kv, d = 2, 8
    k = rng.standard_normal((seq_len, n_kv, d))
    v = rng.standard_normal((seq_len, n_kv, d))
    kv, table = _paged_from_dense(k, v, block_size, rng)
    kg, vg, valid = ora.gather_kv(kv, 0, np.concatenate([table, [-1] * 4]), seq_len, block_size)
    assert valid.all()
    assert np.array_equal(kg, k) and np.array_equal(vg, v)


def test_scatter_matches_flat_slot_indexing():
    """The pool viewed as [L, 2, NB*bs, n_kv, D] is indexed by the slot itself (paged_cache.py:31-32)."""
    rng = _rng(1)
    nb, bs, n_kv, d = 7, 4, 3, 5
    kv = np.zeros((2, 2, nb, bs, n_kv, d))
    k = rng.standard_normal((9, n_kv, d))
    v = rng.standard_normal((9, n_kv, d))
    slots = rng.permutation(nb * bs)[:9]
    ora.reshape_and_cache(k, v, kv, slots, 1, bs)
    flat = kv.reshape(2, 2, nb * bs, n_kv, d)
    assert np.array_equal(flat[1, 0, slots], k)
    assert np.array_equal(flat[1, 1, slots], v)
    assert not flat[0].any()  # other layer untouched
    untouched = np.setdiff1d(np.arange(nb * bs), slots)
    assert not flat[1, :, untouched].any()


def test_scatter_bnhd_input_is_token_major_b_then_t():
    """``[B, n_kv, T, D]`` is flattened as token n = b*T + t (_flatten_kv, attention_ref.py:8-18)."""
    rng = _rng(2)
    b, n_kv, t, d = 3, 2, 4, 6
    k = rng.standard_normal((b, n_kv, t, d))
    kv = np.zeros((1, 2, 8, 4, n_kv, d))
    slots = np.arange(b * t)[::-1].copy()
    ora.reshape_and_cache(k, k, kv, slots, 0, 4)
    flat = kv.reshape(1, 2, 32, n_kv, d)
    for bi in range(b):
        for ti in range(t):
            assert np.array_equal(flat[0, 0, slots[bi * t + ti]], k[bi, :, ti, :])


def test_scatter_skips_negative_and_out_of_pool_slots_and_checks_length():
    kv = np.zeros((1, 2, 2, 4, 1, 2))
    k = np.ones((3, 1, 2))
    ora.reshape_and_cache(k, k, kv, np.array([-1, 8, 5]), 0, 4)
    assert kv.sum() == 2 * 2  # only slot 5 written, K and V
    assert kv[0, 0, 1, 1].sum() == 2
    with pytest.raises(ValueError):
        ora.reshape_and_cache(k, k, kv, np.array([0, 1]), 0, 4)
    with pytest.raises(ValueError):
        ora.reshape_and_cache(k, k[:2], kv, np.array([0, 1, 2]), 0, 4)


def test_gather_masks_holes_and_truncates_to_table():
    kv = np.arange(1 * 2 * 4 * 2 * 1 * 1, dtype=np.float64).reshape(1, 2, 4, 2, 1, 1)
    k, v, valid = ora.gather_kv(kv, 0, np.array([2, -1, 9, 0]), 7, 2)
    assert k.shape == (7, 1, 1)
    assert valid.tolist() == [True, True, False, False, False, False, True]
    assert k[0, 0, 0] == kv[0, 0, 2, 0, 0, 0] and k[6, 0, 0] == kv[0, 0, 0, 0, 0, 0]
    k2, _, valid2 = ora.gather_kv(kv, 0, np.array([1]), 7, 2)  # table shorter than ceil(7/2)
    assert k2.shape[0] == 2 and valid2.all()


# ---------------------------------------------------------------- attention


def _sdpa(q, k, v, tq, seq_len, scale):
    """torch SDPA in float64: q [n_q, Tq, D], k/v [S, n_kv, D] -> [Tq, n_q, D]."""
    n_q = q.shape[0]
    n_kv = k.shape[1]
    kt = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(n_q // n_kv, dim=0)
    vt = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(n_q // n_kv, dim=0)
    qt = torch.from_numpy(q)
    key = torch.arange(k.shape[0])
    qabs = torch.arange(seq_len - tq, seq_len)
    mask = key[None, :] <= qabs[:, None]
    out = torch.nn.functional.scaled_dot_product_attention(qt[None], kt[None], vt[None], attn_mask=mask,
                                                           scale=scale)
    return out[0].permute(1, 0, 2).numpy()


@pytest.mark.parametrize("n_q,n_kv,tq,seq_len,bs", [
    (4, 2, 1, 32, 16), (4, 2, 8, 32, 16), (32, 8, 1, 100, 16), (14, 2, 5, 77, 8), (8, 1, 3, 40, 32),
    (6, 6, 6, 6, 4),
])
def test_paged_attention_equals_torch_sdpa(n_q, n_kv, tq, seq_len, bs):
    """Dense torch SDPA (library routine) on the un-paged K/V equals the paged oracle."""
    rng = _rng(n_q * 1000 + seq_len)
    d = 16
    k = rng.standard_normal((seq_len, n_kv, d))
    v = rng.standard_normal((seq_len, n_kv, d))
    q = rng.standard_normal((1, n_q, tq, d))
    kv, table = _paged_from_dense(k, v, bs, rng)
    scale = d**-0.5
    got = ora.paged_attention(q, kv, table[None], np.array([seq_len]), 0, scale, bs)
    ref = _sdpa(q[0], k, v, tq, seq_len, scale)
    np.testing.assert_allclose(got[0], ref, rtol=1e-12, atol=1e-12)


def test_attend_equals_scalar_loop():
    """Pure-Python loop with math.exp: GQA map h // n_rep and query j at seq_len - Tq + j."""
    rng = _rng(5)
    n_q, n_kv, tq, s, d = 4, 2, 3, 6, 3
    q = rng.standard_normal((n_q, tq, d))
    k = rng.standard_normal((s, n_kv, d))
    v = rng.standard_normal((s, n_kv, d))
    scale = 0.7
    got = ora.attend(q, k, v, np.ones(s, bool), s, scale)
    for h in range(n_q):
        g = h // (n_q // n_kv)
        for j in range(tq):
            last = s - tq + j
            sc = [scale * sum(q[h, j, x] * k[t, g, x] for x in range(d)) for t in range(last + 1)]
            mx = max(sc)
            w = [math.exp(c - mx) for c in sc]
            tot = sum(w)
            for x in range(d):
                ref = sum(w[t] * v[t, g, x] for t in range(last + 1)) / tot
                assert abs(got[j, h, x] - ref) < 1e-12


def test_uniform_scores_average_values_and_dominant_key_selects_row():
    """Closed forms: q = 0 gives the mean of visible V; a huge score picks that key's V."""
    rng = _rng(6)
    s, d = 20, 4
    k = rng.standard_normal((s, 1, d))
    v = rng.standard_normal((s, 1, d))
    out = ora.attend(np.zeros((1, 2, d)), k, v, np.ones(s, bool), s, 1.0)
    np.testing.assert_allclose(out[0, 0], v[: s - 1, 0].mean(axis=0), atol=1e-14)  # query s-2 sees 0..s-2
    np.testing.assert_allclose(out[1, 0], v[:, 0].mean(axis=0), atol=1e-14)
    kk = np.zeros((s, 1, d))
    kk[7, 0, 0] = 1.0
    q = np.zeros((1, 1, d))
    q[0, 0, 0] = 1.0
    out = ora.attend(q, kk, v, np.ones(s, bool), s, 1e4)
    np.testing.assert_allclose(out[0, 0], v[7, 0], atol=1e-12)


def test_decode_row_has_no_mask_and_empty_rows_are_zero():
    """Tq=1 sees every key (packed_causal_mask decode case); a row with no visible key is 0."""
    rng = _rng(7)
    k = rng.standard_normal((9, 1, 4))
    v = rng.standard_normal((9, 1, 4))
    q = rng.standard_normal((1, 1, 4))
    full = ora.attend(q, k, v, np.ones(9, bool), 9, 0.5)
    sc = 0.5 * (k[:, 0] @ q[0, 0])
    w = np.exp(sc - sc.max())
    np.testing.assert_allclose(full[0, 0], (w / w.sum()) @ v[:, 0], atol=1e-14)
    none = ora.attend(q, k, v, np.zeros(9, bool), 9, 0.5)
    assert not none.any()
    out = ora.paged_attention(q[None], np.zeros((1, 2, 2, 4, 1, 4)), np.array([[0, 1]]), np.array([0]), 0, 1.0, 4)
    assert out.shape == (1, 1, 1, 4) and not out.any()


def test_causal_mask_matches_reference_mask_test():
    """tests/correctness/test_cache_and_sampler.py:204-214: prefill 4x4 lower-triangular, decode 1x5 open."""
    # an indicator V exposes which keys each query row averages over (q = 0 -> uniform weights)
    s, tq = 4, 4
    v = np.eye(s)[:, None, :]
    out = ora.attend(np.zeros((1, tq, s)), np.zeros((s, 1, s)), v, np.ones(s, bool), s, 1.0)
    allowed = out[:, 0, :] > 0
    assert allowed.tolist() == np.tril(np.ones((4, 4), bool)).tolist()
    out = ora.attend(np.zeros((1, 1, 5)), np.zeros((5, 1, 5)), np.eye(5)[:, None, :], np.ones(5, bool), 5, 1.0)
    assert (out[0, 0] > 0).all()


def test_block_relabelling_invariance_and_shared_prefix():
    rng = _rng(8)
    bs, n_kv, d, s = 4, 2, 8, 23
    k = rng.standard_normal((s, n_kv, d))
    v = rng.standard_normal((s, n_kv, d))
    q = rng.standard_normal((1, 4, 2, d))
    kv, table = _paged_from_dense(k, v, bs, rng)
    base = ora.paged_attention(q, kv, table[None], np.array([s]), 0, 0.3, bs)
    perm = rng.permutation(kv.shape[2])
    kv2 = np.empty_like(kv)
    kv2[:, :, perm] = kv
    again = ora.paged_attention(q, kv2, perm[table][None], np.array([s]), 0, 0.3, bs)
    assert np.array_equal(base, again)
    # two sequences sharing the first 3 blocks == each with private copies
    nb = kv.shape[2]
    t2 = np.concatenate([table[:3], [nb]])
    kv3 = np.concatenate([kv, kv[:, :, table[3:4]]], axis=2)
    shared = ora.paged_attention(np.concatenate([q, q]), kv3, np.stack([table[:4], t2]), np.array([14, 14]), 0,
                                 0.3, bs)
    assert np.array_equal(shared[0], shared[1])


def test_split_k_merge_equals_single_pass():
    rng = _rng(9)
    q = rng.standard_normal((5, 16))
    k = rng.standard_normal((70, 16))
    v = rng.standard_normal((70, 16))
    parts = [ora.partial_attention(q, k[a:b], v[a:b], 0.25) for a, b in [(0, 13), (13, 40), (40, 70)]]
    merged = ora.merge_partials(parts)
    single = ora.attend(q[:, None, :], k[:, None, :], v[:, None, :], np.ones(70, bool), 70, 0.25)[0]
    # attend() treats the 5 rows as heads of one query token; shapes [5, 16] either way
    np.testing.assert_allclose(merged, single, atol=1e-13)


def test_varlen_equals_per_sequence_calls():
    rng = _rng(10)
    bs, n_q, n_kv, d = 8, 4, 2, 8
    ctx = [5, 30, 17]
    ql = [1, 6, 17]
    pool = rng.standard_normal((1, 2, 20, bs, n_kv, d))
    tables = np.full((3, 4), -1)
    perm = rng.permutation(20)
    c = 0
    for i, n in enumerate(ctx):
        nb = -(-n // bs)
        tables[i, :nb] = perm[c : c + nb]
        c += nb
    cu = np.concatenate([[0], np.cumsum(ql)])
    q = rng.standard_normal((cu[-1], n_q, d))
    got = ora.paged_attention_varlen(q, pool, tables, cu, np.array(ctx), 0, 0.4, bs)
    for i in range(3):
        qi = q[cu[i] : cu[i + 1]].transpose(1, 0, 2)[None]
        ref = ora.paged_attention(qi, pool, tables[i : i + 1], np.array([ctx[i]]), 0, 0.4, bs)
        assert np.array_equal(got[cu[i] : cu[i + 1]], ref[0])


def test_known_answers_attention():
    """Hand-derived vectors (tests/golden/known_answers.json), no oracle involved in making them."""
    gold = json.loads(GOLDEN.read_text())["attention"]
    for case in gold:
        kv = np.array(case["kv_cache"], dtype=np.float64)
        out = ora.paged_attention(np.array(case["q"], dtype=np.float64), kv, np.array(case["block_tables"]),
                                  np.array(case["seq_lens"]), 0, case["scale"], case["block_size"])
        np.testing.assert_allclose(out, np.array(case["expected"]), atol=1e-12, err_msg=case["name"])


# ---------------------------------------------------------------- page copies


def _pages(n_layers=2, nb=9, bs=4, n_kv=2, d=8, seed=0):
    return np.random.default_rng(seed).integers(0, 1 << 16, (n_layers, 2, nb, bs, n_kv, d)).astype(np.uint16)


def test_copy_blocks_closed_form_and_order():
    """attention_ref.py:92-94: page dst of every (layer, K/V) becomes page src; every other
    page is untouched; pairs apply in order, so a chain (0->1, 1->2) moves page 0 to 2."""
    kv = _pages()
    before = kv.copy()
    ora.copy_blocks(kv, [(3, 5), (0, 1), (1, 2), (7, 7)])
    assert np.array_equal(kv[:, :, 5], before[:, :, 3])
    assert np.array_equal(kv[:, :, 1], before[:, :, 0])
    assert np.array_equal(kv[:, :, 2], before[:, :, 0])  # sequential: 1 already holds page 0
    untouched = [b for b in range(kv.shape[2]) if b not in (1, 2, 5)]
    assert np.array_equal(kv[:, :, untouched], before[:, :, untouched])
    # repeated destination: the last pair wins
    kv2 = before.copy()
    ora.copy_blocks(kv2, [(3, 4), (6, 4)])
    assert np.array_equal(kv2[:, :, 4], before[:, :, 6])


def test_swap_round_trip_is_identity_on_the_pages():
    gpu = _pages(seed=1)
    cpu = np.zeros((2, 2, 5, 4, 2, 8), np.uint16)
    ora.swap_blocks(gpu, cpu, [(8, 0), (2, 3)])
    back = np.zeros_like(gpu)
    ora.swap_blocks(cpu, back, [(0, 1), (3, 6)])
    assert np.array_equal(back[:, :, 1], gpu[:, :, 8]) and np.array_equal(back[:, :, 6], gpu[:, :, 2])


def test_ordered_batches_reproduce_sequential_copies():
    """The wrapper's batching: running each batch all at once (reads before writes) gives
    the one-by-one result, on random pair lists full of chains and repeats."""
    from slipstream_amd.kernels.block_copy import ordered_batches

    rng = np.random.default_rng(5)
    for _ in range(200):
        pairs = [tuple(int(v) for v in rng.integers(0, 6, 2)) for _ in range(rng.integers(1, 9))]
        seq = _pages(n_layers=1, nb=6, bs=1, n_kv=1, d=2, seed=int(rng.integers(1 << 30)))
        par = seq.copy()
        ora.copy_blocks(seq, pairs)
        for batch in ordered_batches(pairs):
            snap = par.copy()
            for s, d in batch:
                par[:, :, d] = snap[:, :, s]
        assert np.array_equal(seq, par), pairs
        assert sum(len(b) for b in ordered_batches(pairs)) == len(pairs)


def test_independent_pairs_run_in_one_batch():
    """The dict path's packer (csrc/host_pairs.c): the pairs it writes are the dict's items
    in order, and it calls a mapping independent exactly when ordered_batches keeps the
    whole list as one batch (so one launch gives the one-by-one result; every other list
    goes through ordered_batches). Ids outside a cache raise the wrapper's ValueError."""
    from slipstream_amd.kernels.block_copy import _host_pairs, ordered_batches

    pack = _host_pairs().pack
    buf = np.zeros((16, 2), dtype=np.int64)
    addr = buf.ctypes.data
    rng = np.random.default_rng(6)
    for trial in range(600):
        nb = int(rng.integers(2, 12))
        d = {int(s): int(v) for s, v in rng.integers(0, nb, (int(rng.integers(1, 12)), 2))}  # distinct sources
        n, indep = pack(d, addr, buf.shape[0], nb, nb, True)
        assert n == len(d) and buf[:n].tolist() == [list(kv) for kv in d.items()], d
        assert bool(indep) == (len(ordered_batches(list(d.items()))) == 1), d
        assert pack(d, addr, buf.shape[0], nb, nb, False)[1] == 1  # no check: one launch (two caches)
    # numpy integers are ids too; an empty mapping packs nothing
    assert pack({np.int64(3): np.int32(4)}, addr, 16, 8, 8, True) == (1, 1) and buf[0].tolist() == [3, 4]
    assert pack({}, addr, 16, 8, 8, True) == (0, 1)
    with pytest.raises(ValueError, match="source block 9"):
        pack({1: 2, 9: 3}, addr, 16, 8, 8, True)
    with pytest.raises(ValueError, match="destination block -1"):
        pack({1: -1}, addr, 16, 8, 8, True)
    with pytest.raises(ValueError, match="destination block 8"):
        pack({1: 8}, addr, 16, 16, 8, False)  # destination cache of 8 blocks
    with pytest.raises(ValueError, match="pairs for a buffer"):
        pack({i: i + 20 for i in range(17)}, addr, 16, 64, 64, True)
    with pytest.raises(TypeError):
        pack({1.5: 2}, addr, 16, 8, 8, True)


# ---------------------------------------------------------------- rotary embedding


def test_rotate_half_known_answer():
    """test_layers_reference.py:36-42: [a, b, c, d] -> [-c, -d, a, b]."""
    from oracle import rope

    x = np.array([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]])
    assert np.array_equal(rope.rotate_half(x)[0], [-3.0, -4.0, 1.0, 2.0])


@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)])
def test_apply_rope_matches_torch_elementwise_rounding(dtype, tdt):
    """The reference formula evaluated by torch's CPU elementwise ops (the arithmetic the
    reference runs, rope.py:33-35), on random q and random cos/sin as the reference's
    own fused-kernel test uses (test_fused_kernels.py:37-46): bit identical."""
    from oracle import rope

    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 8, 64, generator=g).to(tdt)
    cos = torch.randn(2, 8, 64, generator=g).to(tdt)
    sin = torch.randn(2, 8, 64, generator=g).to(tdt)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    half = q.shape[-1] // 2
    want = q * c + torch.cat((-q[..., half:], q[..., :half]), dim=-1) * s
    got = rope.apply_rope(q.double().numpy(), c.double().numpy(), s.double().numpy(), dtype)
    assert np.array_equal(got, want.double().numpy())


def test_rope_is_a_rotation_in_exact_arithmetic():
    """With tables from angles (both halves equal) and no rounding: each (i, i + D/2)
    pair keeps its norm, and rotating by a then by b equals rotating by a + b."""
    from oracle import rope

    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 16))
    a, b = rng.uniform(-3, 3, (5, 8)), rng.uniform(-3, 3, (5, 8))
    def rot(v, ang):
        c, s = np.cos(np.concatenate((ang, ang), -1)), np.sin(np.concatenate((ang, ang), -1))
        return v * c + rope.rotate_half(v) * s
    y = rot(x, a)
    assert np.allclose(y[:, :8] ** 2 + y[:, 8:] ** 2, x[:, :8] ** 2 + x[:, 8:] ** 2)
    assert np.allclose(rot(rot(x, a), b), rot(x, a + b))


# ---------------------------------------------------------------- step metadata


class _MiniBlockManager:
    """block_manager.py:141-159,282-287 restated for the test: a token goes to the first
    not-full block of the table (a fresh block from the free list when none is)."""

    def __init__(self, n_blocks: int, block_size: int, seed: int):
        self.bs = block_size
        self.free = np.random.default_rng(seed).permutation(n_blocks).tolist()
        self.fill = [0] * n_blocks

    def append_slot(self, table: list[int]) -> tuple[int, int]:
        idx = next((i for i, b in enumerate(table) if self.fill[b] < self.bs), None)
        if idx is None:
            table.append(self.free.pop())
            idx = len(table) - 1
        bid = table[idx]
        off = self.fill[bid]
        self.fill[bid] += 1
        return bid, off


def test_step_metadata_matches_append_slot():
    """The slot rule of the device builder (table[p // bs] * bs + p % bs) equals the slots
    append_slot hands out, on random prefill + step sequences; cu_seqlens and
    context_lens are the packed description."""
    rng = np.random.default_rng(7)
    for trial in range(20):
        bs = int(rng.choice([1, 4, 16]))
        bm = _MiniBlockManager(4096, bs, seed=trial)
        batch = int(rng.integers(1, 12))
        tables = [[] for _ in range(batch)]
        prior = rng.integers(0, 70, batch).tolist()
        q = rng.integers(0, 20, batch).tolist()
        for b in range(batch):
            for _ in range(prior[b]):
                bm.append_slot(tables[b])
        want = []
        for b in range(batch):
            for _ in range(q[b]):
                bid, off = bm.append_slot(tables[b])
                want.append(bid * bs + off)
        cu, ctx, slots = ora.build_step_metadata(tables, prior, q, bs)
        assert slots.tolist() == want
        assert cu.tolist() == [0] + np.cumsum(q).tolist()
        assert ctx.tolist() == [a + b for a, b in zip(prior, q)]


def test_step_metadata_edges():
    """Positions past the table and negative entries give -1; negative lengths count as 0."""
    cu, ctx, slots = ora.build_step_metadata([[3, -1], [5]], [6, 0], [4, -2], 8)
    assert cu.tolist() == [0, 4, 4] and ctx.tolist() == [10, 0]
    assert slots.tolist() == [3 * 8 + 6, 3 * 8 + 7, -1, -1]  # positions 8, 9 sit on the hole
    _, _, past = ora.build_step_metadata([[2]], [3], [3], 4)
    assert past.tolist() == [2 * 4 + 3, -1, -1]  # positions 4, 5 are past the one-block table


def test_step_metadata_total_tokens_pads_and_cuts():
    """An explicit slot count: entries past the step's tokens are -1 (no token owns them,
    the scatter skips them), and a count below the step's tokens cuts the list."""
    _, _, slots = ora.build_step_metadata([[3], [5]], [0, 2], [2, 1], 4, total_tokens=6)
    assert slots.tolist() == [12, 13, 22, -1, -1, -1]
    _, _, cut = ora.build_step_metadata([[3], [5]], [0, 2], [2, 1], 4, total_tokens=2)
    assert cut.tolist() == [12, 13]
