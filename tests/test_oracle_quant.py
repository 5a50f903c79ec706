"""Pins of the numpy W4A16 oracle (``oracle/quant.py``) -- CPU only.

Checks restate the reference's own tests (tests/correctness/test_quant_w4a16.py:28-137),
the hand-derived words and dequantised values of tests/golden/known_answers.json,
torch's own casts for the rounding chain (quant_ref.py:112-116,132), and a
brute-force triple loop for the GEMM.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant
from oracle import reference_path as refp

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"
GROUP_SIZES = [32, 64, 128]


def test_pack_known_words_and_roundtrip():
    gold = json.loads(GOLDEN.read_text())["int4"]
    q = np.array(gold["nibbles"])
    packed = quant.pack_int4(q)
    assert packed.dtype == np.int32
    assert packed.tolist() == gold["packed"]
    assert np.array_equal(quant.unpack_int4(packed, 8), q)


def test_pack_unpack_roundtrip_exact():
    """test_quant_w4a16.py:28-35."""
    q = np.random.default_rng(0).integers(0, 16, (7, 128))
    packed = quant.pack_int4(q)
    assert packed.shape == (7, 16)
    assert np.array_equal(quant.unpack_int4(packed, 128), q)


def test_pack_bit_layout_against_independent_shift():
    """Nibble n of word j is q[8j+n] at bits 4n: read back with Python ints, not the oracle."""
    q = np.random.default_rng(1).integers(0, 16, (3, 24))
    packed = quant.pack_int4(q)
    for o in range(3):
        for j in range(3):
            w = int(packed[o, j]) & 0xFFFFFFFF
            for n in range(8):
                assert (w >> (4 * n)) & 0xF == q[o, 8 * j + n]


def test_dequant_known_answer():
    gold = json.loads(GOLDEN.read_text())["int4"]["dequant"]
    qw = quant.pack_int4(np.array(gold["q"]))
    w = quant.dequantize_w4a16(qw, np.array(gold["scale"]), np.array(gold["zero"]), gold["group_size"])
    assert w.tolist() == gold["expected"]


@pytest.mark.parametrize("group_size", GROUP_SIZES)
def test_dequant_error_bounded_by_scale(group_size):
    """test_quant_w4a16.py:45-65."""
    w = np.random.default_rng(1).standard_normal((16, 256)).astype(np.float32)
    qw, s, z = quant.quantize_w4a16(w, group_size)
    assert qw.shape == (16, 32) and s.shape == (16, 256 // group_size) and z.shape == s.shape
    assert z.min() >= 0 and z.max() <= 15
    w_hat = quant.dequantize_w4a16(qw, s, z, group_size)
    per = np.repeat(s, group_size, axis=1)
    assert np.all(np.abs(w - w_hat) <= per * (1 + 1e-4))


def test_quantize_is_idempotent_and_constant_group_exact():
    """test_quant_w4a16.py:68-75 and :120-125."""
    w = np.random.default_rng(2).standard_normal((8, 128)).astype(np.float32)
    qw1, s1, z1 = quant.quantize_w4a16(w, 32)
    w_hat = quant.dequantize_w4a16(qw1, s1, z1, 32).astype(np.float32)
    qw2, _, _ = quant.quantize_w4a16(w_hat, 32)
    assert np.array_equal(quant.unpack_int4(qw1, 128), quant.unpack_int4(qw2, 128))
    c = np.full((4, 64), 0.37, dtype=np.float32)
    qc, sc, zc = quant.quantize_w4a16(c, 32)
    np.testing.assert_allclose(quant.dequantize_w4a16(qc, sc, zc, 32), c, atol=1e-5, rtol=0)


def test_rejects_bad_arguments():
    """test_quant_w4a16.py:128-137."""
    with pytest.raises(ValueError):
        quant.quantize_w4a16(np.zeros((8, 100)), 32)
    with pytest.raises(ValueError):
        quant.quantize_w4a16(np.zeros((8, 96)), 12)
    with pytest.raises(ValueError):
        quant.quantize_w4a16(np.zeros(64), 32)
    with pytest.raises(ValueError):
        quant.pack_int4(np.zeros((8, 100), dtype=np.int64))


@pytest.mark.parametrize("group_size", GROUP_SIZES)
def test_gemm_equals_brute_force_loop(group_size):
    """x @ dequant(W).T (test_quant_w4a16.py:79-92) against explicit per-element sums."""
    rng = np.random.default_rng(3)
    n, k, m = 6, 256, 3
    q = rng.integers(0, 16, (n, k))
    s = rng.uniform(0.005, 0.02, (n, k // group_size))
    z = rng.integers(0, 16, (n, k // group_size))
    x = rng.standard_normal((m, k))
    y = quant.w4a16_gemm(x, quant.pack_int4(q), s, z, group_size)
    for i in range(m):
        for o in range(n):
            ref = sum(x[i, c] * (q[o, c] - z[o, c // group_size]) * s[o, c // group_size] for c in range(k))
            assert abs(y[i, o] - ref) < 1e-12


def test_gemm_keeps_batch_dims_and_accuracy_vs_full_precision():
    """test_quant_w4a16.py:95-117, on that test's own seeded torch inputs (4-bit noise on
    N(0,1) weights is ~0.10 relative, so the bar is data-dependent)."""
    torch.manual_seed(5)
    w = torch.randn(128, 512).numpy()
    x = torch.randn(16, 512).numpy().astype(np.float64)
    qw, s, z = quant.quantize_w4a16(w, 128)
    y = quant.w4a16_gemm(x.reshape(2, 8, 512), qw, s, z, 128)
    assert y.shape == (2, 8, 128)
    full = x @ w.T
    assert np.linalg.norm(y.reshape(16, 128) - full) / np.linalg.norm(full) < 0.1


def test_round_to_bf16_matches_torch_cast():
    v = np.concatenate([np.random.default_rng(6).standard_normal(10000).astype(np.float32) * 7,
                        np.array([1.00390625, 1.01171875, -3.0, 0.0, 65504.0], dtype=np.float32)])
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(quant.round_to_bf16(v), ref)


def test_faithful_dequant_matches_torch_chain_and_reference_path():
    """quant_ref.py:112-116,132: fp32 (q - z) * s -> fp16 -> bf16, computed here by torch casts."""
    rng = np.random.default_rng(7)
    n, k, g = 16, 256, 128
    q = rng.integers(0, 16, (n, k))
    s16 = rng.uniform(0.005, 0.02, (n, k // g)).astype(np.float16)
    z = np.full((n, k // g), 8, dtype=np.int32)
    qw = quant.pack_int4(q)
    ours = quant.dequantize_faithful(qw, s16, z, g, scale_dtype=np.float16, act_is_bf16=True)
    w32 = (torch.from_numpy(q).float().view(n, k // g, g) - torch.from_numpy(z).float()[..., None]) * \
        torch.from_numpy(s16).float()[..., None]
    ref = w32.view(n, k).to(torch.float16).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)
    x = torch.randn(4, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    y_ref = refp.w4a16_gemm(x, torch.from_numpy(qw), torch.from_numpy(s16), torch.from_numpy(z), g)
    assert y_ref.dtype == torch.bfloat16
    exact = quant.w4a16_gemm(x.float().numpy(), qw, s16.astype(np.float64), z, g)
    rel = np.linalg.norm(y_ref.float().numpy() - exact) / np.linalg.norm(exact)
    assert rel < 1e-2


def test_module_quantizer_equals_oracle_quantizer():
    """slipstream_amd.quantized.quantize_weight (the load-time format producer) restates
    quant_ref.py:72-100 with torch ops: identical to the pinned numpy oracle."""
    import torch

    from slipstream_amd.quantized import quantize_weight

    g = torch.Generator().manual_seed(2)
    for group in (32, 128):
        w = torch.randn(48, 512, generator=g) * 0.05
        w[3, :group] = 0.25  # a constant group: 0 joins its range
        qw, s, z = quantize_weight(w, group)
        rq, rs, rz = quant.quantize_w4a16(w.numpy(), group)
        assert np.array_equal(qw.numpy(), rq) and np.array_equal(z.numpy(), rz)
        assert np.array_equal(s.numpy(), rs.astype(np.float32))
