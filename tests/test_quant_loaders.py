"""AWQ / GPTQ checkpoint re-layout into the reference's W4A16 format -- CPU only.

The checkpoint words are built here by the packing loops the two formats publish (AutoAWQ's
``WQLinear_GEMM.from_linear``: nibble i of word j holds column 8j + [0,2,4,6,1,3,5,7][i];
AutoGPTQ's ``QuantLinear.pack``: qweight nibble i of word j is input row 8j+i, zero points
stored minus one and packed along the output columns), one Python int at a time, and the
converted tensors must dequantise (``oracle/quant.py``, ``quant_ref.py:103-116``) to the
weight the checkpoint describes. Hand-derived words pin the two nibble orders.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant
from slipstream_amd.quantized import W4A16Linear, W4A16MLP, awq_to_reference, gptq_to_reference

AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def _word(vals: list[int]) -> int:
    w = 0
    for i, v in enumerate(vals):
        w |= (int(v) & 0xF) << (4 * i)
    return w - (1 << 32) if w >= 1 << 31 else w  # int32 two's complement


def awq_pack(cols: np.ndarray) -> torch.Tensor:
    """[rows, out] nibbles -> AWQ words [rows, out/8]."""
    rows, out = cols.shape
    words = [[_word([cols[r, 8 * j + AWQ_ORDER[i]] for i in range(8)]) for j in range(out // 8)] for r in range(rows)]
    return torch.tensor(words, dtype=torch.int32)


def gptq_pack_weight(q_in_out: np.ndarray) -> torch.Tensor:
    """[in, out] nibbles -> GPTQ qweight [in/8, out]."""
    k, n = q_in_out.shape
    words = [[_word([q_in_out[8 * j + i, o] for i in range(8)]) for o in range(n)] for j in range(k // 8)]
    return torch.tensor(words, dtype=torch.int32)


def gptq_pack_zeros(z: np.ndarray, minus_one: bool) -> torch.Tensor:
    """[groups, out] zero points -> GPTQ qzeros [groups, out/8] (v1 stores z - 1)."""
    g, n = z.shape
    zz = z - 1 if minus_one else z
    words = [[_word([zz[r, 8 * j + i] for i in range(8)]) for j in range(n // 8)] for r in range(g)]
    return torch.tensor(words, dtype=torch.int32)


def _dense(qw: torch.Tensor, scales: torch.Tensor, qz: torch.Tensor, g: int) -> np.ndarray:
    return quant.dequantize_w4a16(qw.numpy(), scales.float().numpy(), qz.numpy(), g)


def _case(k: int, n: int, g: int, seed: int):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, (k, n))  # [in, out], checkpoint orientation
    z = rng.integers(0, 16, (k // g, n))
    s = torch.tensor(rng.uniform(0.005, 0.02, (k // g, n)), dtype=torch.float16)
    expect = (q.T - np.repeat(z.T, g, axis=1)) * np.repeat(s.float().numpy().T, g, axis=1)  # W[o, i]
    return q, z, s, expect


def test_known_words():
    # columns 0..7 hold 0..7: AWQ nibbles read 0,2,4,6,1,3,5,7 from low to high
    assert awq_pack(np.arange(8).reshape(1, 8)).item() & 0xFFFFFFFF == 0x75316420
    qw, s, z = awq_to_reference(torch.full((8, 1), 0x75316420, dtype=torch.int32),
                                torch.tensor([[0x75316420]], dtype=torch.int32),
                                torch.ones(1, 8, dtype=torch.float16), 8)
    # eight input rows, eight output rows: output o has q = o at every input, zero = o
    assert [v & 0xFFFFFFFF for v in qw[:, 0].tolist()] == [0x11111111 * o for o in range(8)]
    assert z[:, 0].tolist() == list(range(8))
    # GPTQ: input rows 0..7 of one column -> 0x76543210 in the reference's orientation too
    qg = gptq_pack_weight(np.arange(8).reshape(8, 1).repeat(8, axis=1))
    assert qg[0, 0].item() == 0x76543210
    ref, _, _ = gptq_to_reference(qg, gptq_pack_zeros(np.full((1, 8), 8), True), torch.ones(1, 8, dtype=torch.float16), 8)
    assert ref[:, 0].tolist() == [0x76543210] * 8


@pytest.mark.parametrize("k,n,g", [(64, 32, 32), (128, 24, 64), (256, 16, 128)])
def test_awq_dequantises_to_the_checkpoint_weight(k, n, g):
    q, z, s, expect = _case(k, n, g, seed=k + n)
    qw, sc, qz = awq_to_reference(awq_pack(q), awq_pack(z), s, g)
    assert qw.shape == (n, k // 8) and sc.shape == (n, k // g) and qz.shape == (n, k // g)
    assert sc.dtype == torch.float16 and qz.dtype == torch.int32
    np.testing.assert_array_equal(_dense(qw, sc, qz, g), expect.astype(np.float32))


@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2"])
@pytest.mark.parametrize("k,n,g", [(64, 32, 32), (256, 16, 128)])
def test_gptq_dequantises_to_the_checkpoint_weight(k, n, g, fmt):
    q, z, s, expect = _case(k, n, g, seed=3 * k + n)
    if fmt == "gptq":
        z = np.maximum(z, 1)  # v1 stores z - 1 in a nibble: a zero point of 0 is not storable as itself
    expect = (q.T - np.repeat(z.T, g, axis=1)) * np.repeat(s.float().numpy().T, g, axis=1)
    g_idx = torch.arange(k, dtype=torch.int32) // g
    qw, sc, qz = gptq_to_reference(gptq_pack_weight(q), gptq_pack_zeros(z, fmt == "gptq"), s, g, g_idx, fmt)
    np.testing.assert_array_equal(_dense(qw, sc, qz, g), expect.astype(np.float32))


def test_gptq_v1_zero_wraps_as_its_kernels_read_it():
    # a true zero point 0 is stored as nibble 15 (-1 masked); the v1 dequantisation adds one -> 16
    qz = gptq_pack_zeros(np.zeros((1, 8), dtype=np.int64), True)
    _, _, z = gptq_to_reference(torch.zeros(1, 8, dtype=torch.int32), qz, torch.ones(1, 8, dtype=torch.float16), 8)
    assert z.flatten().tolist() == [16] * 8


def test_rejections():
    s = torch.ones(2, 8, dtype=torch.float16)
    qw = torch.zeros(8, 8, dtype=torch.int32)  # gptq: in = 64, out = 8
    qz = torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="act-order"):
        gptq_to_reference(qw, qz, s, 32, torch.arange(64) % 2)
    with pytest.raises(ValueError, match="checkpoint_format"):
        gptq_to_reference(qw, qz, s, 32, checkpoint_format="exl2")
    with pytest.raises(ValueError, match="scales"):
        gptq_to_reference(qw, qz, torch.ones(3, 8, dtype=torch.float16), 32)
    with pytest.raises(ValueError, match="int32"):
        awq_to_reference(torch.zeros(64, 1, dtype=torch.int64), qz, s, 32)
    with pytest.raises(ValueError, match="group_size"):
        awq_to_reference(torch.zeros(64, 1, dtype=torch.int32), qz, s, 24)


def test_state_dict_loader_builds_modules():
    k, n, g = 128, 16, 64
    state = {}
    for name, (kk, nn_) in {"gate_proj": (k, n), "up_proj": (k, n), "down_proj": (n * 8, k)}.items():
        q, z, s, _ = _case(kk, nn_, g, seed=kk + nn_)
        state[f"model.layers.0.mlp.{name}.qweight"] = awq_pack(q)
        state[f"model.layers.0.mlp.{name}.qzeros"] = awq_pack(z)
        state[f"model.layers.0.mlp.{name}.scales"] = s
    mlp = W4A16MLP.from_state_dict(state, "model.layers.0.mlp", g)
    assert (mlp.gate_up_proj.in_features, mlp.gate_up_proj.out_features, mlp.intermediate) == (k, 2 * n, n)
    gate = W4A16Linear.from_state_dict(state, "model.layers.0.mlp.gate_proj", g)
    up = W4A16Linear.from_state_dict(state, "model.layers.0.mlp.up_proj", g)
    assert torch.equal(mlp.gate_up_proj.qweight, torch.cat([gate.qweight, up.qweight]))
    assert torch.equal(mlp.gate_up_proj.qzeros, torch.cat([gate.qzeros, up.qzeros]))
    assert torch.equal(mlp.gate_up_proj.scales, torch.cat([gate.scales, up.scales]))
    assert (mlp.down_proj.in_features, mlp.down_proj.out_features) == (n * 8, k)
    with pytest.raises(KeyError, match="qzeros"):
        W4A16Linear.from_state_dict({"x.qweight": state["model.layers.0.mlp.gate_proj.qweight"]}, "x", g)
