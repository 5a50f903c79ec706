"""GPU parity of the HIP W4A16 linear against the numpy oracle (oracle/quant.py).

Tolerance (north star): 1e-2 relative -- checked as a relative Frobenius error
below 1e-2 and elementwise |y - y_ref| <= 1e-2 |y_ref| + 2e-3 max|y_ref|. The
oracle uses the exact dequantised weight in float64. Shapes follow the
reference's own test (out 24, in 256, M 5, g 32/64/128,
tests/correctness/test_quant_w4a16.py:79-92) and the C5 Llama-3-8B layer
linears at M in {1, 16, 64, 256}; at full size every output column is checked
against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant
from slipstream_amd.kernels import w4a16_gemm
from slipstream_amd import workloads

pytestmark = pytest.mark.gpu

RTOL = 1e-2
ATOL_FRAC = 2e-3


def _assert_close(y: torch.Tensor, ref: np.ndarray, what: str) -> None:
    g = y.detach().float().cpu().numpy().astype(np.float64)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    rel = np.linalg.norm(g - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel < RTOL, f"{what}: relative error {rel:.3e}"
    atol = ATOL_FRAC * np.abs(ref).max()
    bad = np.abs(g - ref) > RTOL * np.abs(ref) + atol
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance, max err {np.abs(g - ref).max():.3e}"


def _host_case(n, k, m, g, seed, act=torch.bfloat16, sdt=torch.float16, zeros="eight", lead=None):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, (n, k))
    s = rng.uniform(0.005, 0.02, (n, k // g))
    z = np.full((n, k // g), 8) if zeros == "eight" else rng.integers(0, 16, (n, k // g))
    qw = quant.pack_int4(q)
    x = torch.from_numpy(rng.standard_normal((m, k))).to(act)
    if lead is not None:
        x = x.reshape(*lead, k)
    st = torch.from_numpy(s).to(sdt)
    s_exact = st.double().numpy()  # the scales the kernel sees, exactly
    ref = quant.w4a16_gemm(x.double().numpy(), qw, s_exact, z, g)
    return x, torch.from_numpy(qw), st, torch.from_numpy(z.astype(np.int32)), ref


@pytest.mark.parametrize("group_size", [32, 64, 128])
@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_reference_test_shape(device, group_size, act):
    """test_quant_w4a16.py:79-92 shape: out 24, in 256, M 5 (N not a multiple of the tile)."""
    x, qw, s, z, ref = _host_case(24, 256, 5, group_size, seed=group_size, act=act, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), group_size)
    assert y.shape == (5, 24) and y.dtype == act
    _assert_close(y, ref, f"g={group_size} {act}")


@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
def test_scale_dtypes_and_batch_dims(device, sdt):
    """test_quant_w4a16.py:95-102: leading dims kept, dtype of x kept."""
    x, qw, s, z, ref = _host_case(200, 512, 6, 128, seed=3, sdt=sdt, zeros="random", lead=(2, 3))
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), 128)
    assert y.shape == (2, 3, 200) and y.dtype == torch.bfloat16
    _assert_close(y, ref, f"scales {sdt}")


@pytest.mark.parametrize("m", [1, 3, 16, 17, 40, 64, 65, 130])
def test_m_sweep_tiles(device, m):
    """Every M tiling: activations in LDS (M <= 16 when they fit), 16/32/64-row tiles read
    from memory, several 64-row blocks above 64; 4 or 8 K slices per workgroup."""
    x, qw, s, z, ref = _host_case(320, 2048, m, 128, seed=m, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), 128)
    _assert_close(y, ref, f"m={m}")


@pytest.mark.parametrize("m,k,g", [(16, 4096, 128), (8, 8192, 128), (2, 4096, 32), (16, 2048, 64)])
def test_activation_paths(device, m, k, g):
    """M <= 16 with activations too large for LDS (64 weight rows per workgroup) and NARROW groups."""
    x, qw, s, z, ref = _host_case(192, k, m, g, seed=m + k + g, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), g)
    _assert_close(y, ref, f"m={m} k={k} g={g}")


@pytest.mark.parametrize("n,k,g,act,sdt", [
    (100, 1024, 128, torch.bfloat16, torch.float16),    # one wave; N not a multiple of 16
    (48, 2048, 32, torch.float16, torch.bfloat16),      # four groups per 128 keys
    (333, 4096, 64, torch.bfloat16, torch.float32),
    (17, 8192, 128, torch.float16, torch.float16),      # 8 waves of 1024 keys
    (64, 14336, 128, torch.bfloat16, torch.float16),    # 2048-key slices, 7 waves (the down projection)
    (40, 16384, 64, torch.float16, torch.bfloat16),     # the largest K the GEMV takes
])
def test_batch1_gemv(device, n, k, g, act, sdt):
    """M = 1: g = 128 takes the narrow MFMA kernel, g = 32 / 64 the bandwidth GEMV (one
    1024-key wave slice per wave up to K = 8192, 2048-key slices up to 16384): random zero
    points, every scale dtype, ragged N."""
    x, qw, s, z, ref = _host_case(n, k, 1, g, seed=n + k + g, act=act, sdt=sdt, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), g)
    assert y.shape == (1, n) and y.dtype == act
    _assert_close(y, ref, f"gemv n={n} k={k} g={g}")


@pytest.mark.parametrize("m,n,k,act,sdt", [
    (1, 100, 1024, torch.bfloat16, torch.float16),    # one wave; N not a multiple of 16
    (2, 333, 4096, torch.float16, torch.bfloat16),
    (3, 40, 8192, torch.bfloat16, torch.float32),     # 8 waves of 1024 keys; row 3 of the A tile is empty
    (4, 17, 14336, torch.float16, torch.float16),     # 7 waves of 2048 keys (the down projection)
    (4, 64, 16384, torch.bfloat16, torch.bfloat16),   # the largest K it takes
    (2, 4100, 2048, torch.bfloat16, torch.float16),   # many workgroups, a partial last one
])
def test_narrow_mfma_kernel(device, m, n, k, act, sdt):
    """1 <= M <= 4 with g = 128 takes the narrow kernel (dot products on MFMA, four-row
    weight loads, A rows = (piece, activation row)): random zero points, every scale and
    activation dtype, ragged N."""
    x, qw, s, z, ref = _host_case(n, k, m, 128, seed=n + k + m, act=act, sdt=sdt, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), 128)
    assert y.shape == (m, n) and y.dtype == act
    _assert_close(y, ref, f"narrow m={m} n={n} k={k}")


def test_narrow_strided_activation(device):
    """Three strided activation rows (views into a wider buffer) through the narrow kernel."""
    x, qw, s, z, ref = _host_case(96, 4096, 3, 128, seed=78, zeros="random")
    xd = torch.zeros((5, 8192), dtype=x.dtype, device=device)[1:4, 2048:6144]
    xd.copy_(x.to(device))
    y = w4a16_gemm(xd, qw.to(device), s.to(device), z.to(device), 128)
    _assert_close(y, ref, "narrow strided x")


def test_batch1_gemv_strided_activation(device):
    """A strided single activation row (a view into a wider buffer) through the GEMV (g = 64)."""
    x, qw, s, z, ref = _host_case(96, 4096, 1, 64, seed=77, zeros="random")
    xd = torch.zeros((3, 8192), dtype=x.dtype, device=device)[1:2, 1024:5120]
    xd.copy_(x.to(device))
    y = w4a16_gemm(xd, qw.to(device), s.to(device), z.to(device), 64)
    _assert_close(y, ref, "gemv strided x")


# (plans as the host computes them for 256 CUs: ranges x stages, weight tiles, M blocks)
@pytest.mark.parametrize("m,k,n,g,act,sdt", [
    (50, 3072, 12750, 128, torch.bfloat16, torch.float16),   # 32-row tiles, 2 M blocks, one range; 100 tiles: 4 padding ids
    (33, 3584, 2000, 896, torch.float16, torch.bfloat16),    # 7 ranges of 4 stages: groups of 7 stages straddle them
    (100, 4096, 1000, 256, torch.bfloat16, torch.float32),   # 32-row tiles (small grid), a partial fourth M block, 16 ranges
    (130, 1792, 700, 128, torch.bfloat16, torch.float16),    # 5 M blocks of one weight tile on one XCD; 42 pairs
    (24, 8192, 3000, 512, torch.float16, torch.float16),     # 32-row activation tiles
    (9, 8192, 700, 256, torch.bfloat16, torch.bfloat16),     # m <= 16, g 256 (the skinny kernel takes only g 128)
    (16, 1024, 24600, 256, torch.bfloat16, torch.float16),   # m <= 16 at N >= 24576, unsplit, 193 tiles
    (24, 2048, 3000, 128, torch.bfloat16, torch.float16),    # 32-row tiles, grid within the CUs: eight waves
    (32, 4096, 20480, 128, torch.bfloat16, torch.float16),   # 32-row tiles, 2 ranges, 320 workgroups: four waves
    (64, 2048, 8000, 128, torch.float16, torch.bfloat16),    # 32-row tiles, 2 ranges, grid within the CUs: eight waves
])
def test_tiled_split_k(device, m, k, n, g, act, sdt):
    """The tiled kernel (activations shared through LDS, K split over workgroups with
    fp32 partials added in range order): groups straddling ranges, ragged M and N, the
    XCD-grouped grid with padding ids, every scale dtype."""
    x, qw, s, z, ref = _host_case(n, k, m, g, seed=m + k + n, act=act, sdt=sdt, zeros="random")
    xd, qd, sd, zd = x.to(device), qw.to(device), s.to(device), z.to(device)
    y = w4a16_gemm(xd, qd, sd, zd, g)
    _assert_close(y, ref, f"tiled m={m} k={k} n={n} g={g}")
    assert torch.equal(y, w4a16_gemm(xd, qd, sd, zd, g))  # repeat: bit-identical


@pytest.mark.parametrize("m,n,act,sdt", [(48, 16512, torch.bfloat16, torch.float16),
                                         (24, 16384, torch.bfloat16, torch.float16),
                                         (130, 12352, torch.bfloat16, torch.float16),
                                         (40, 16400, torch.float16, torch.bfloat16)])
def test_tiled_two_ranges_finished_in_kernel(device, m, n, act, sdt):
    """Two K ranges (K 2048; N 16512 at m 48: 129 weight tiles, a 264-workgroup grid of
    four waves; N 16384 at m 24: 256 workgroups of eight; N 12352 at m 130: 97 tiles of 128
    rows, the last half full, in three 64-row blocks, the last of 2 rows; N 16400 at m 40:
    fp16 activations and bf16 scales, a last weight tile of 16 rows): the last range to
    arrive at a tile adds the other range's partials to its own (kept in registers),
    counted in arrival words behind the partials in the workspace,
    tagged per call. Correct on a workspace full of 0xFF bytes (no word carries the call's
    tag), bit-identical across repeats, and a captured graph (one tag for every replay)
    replays to the eager result with eager calls in between."""
    from slipstream_amd.kernels import quant_gemm
    print(f"w4a16 two-range tiled m={m} n={n} {act}", flush=True)
    x, qw, s, z, ref = _host_case(n, 2048, m, 128, seed=m + n, act=act, sdt=sdt, zeros="random")
    xd, qd, sd, zd = x.to(device), qw.to(device), s.to(device), z.to(device)
    y = w4a16_gemm(xd, qd, sd, zd, 128)
    assert y.dtype == act
    _assert_close(y, ref, f"two ranges m={m} n={n} {act}")
    torch.cuda.synchronize()
    for ws in quant_gemm._WORKSPACE.values():
        ws.fill_(0xFF)
    y1 = w4a16_gemm(xd, qd, sd, zd, 128)
    torch.cuda.synchronize()
    assert torch.equal(y1, y)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        w4a16_gemm(xd, qd, sd, zd, 128)
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        out = w4a16_gemm(xd, qd, sd, zd, 128)
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y), f"replay {rep}"
        again = w4a16_gemm(xd, qd, sd, zd, 128)  # eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(again, y)


# (plans as the host computes them for 256 CUs: 128-row activation blocks, 128- or
# 256-row weight tiles, ranges of a multiple of 4 stages and at least 16)
@pytest.mark.parametrize("m,k,n,act,sdt", [
    (300, 2048, 16000, torch.float16, torch.bfloat16),   # one range, 128-row weight tiles; 3 M blocks (the last of 44 rows)
    (256, 2048, 28600, torch.bfloat16, torch.float32),   # one range, 256-row weight tiles, the last of 184 rows
    (256, 4096, 8192, torch.bfloat16, torch.float16),    # two ranges of 16 stages, finished in the kernel
    (256, 8192, 6144, torch.bfloat16, torch.float32),    # three ranges (24, 24, 16 stages) and the reduce kernel
    (256, 4096, 8190, torch.bfloat16, torch.float16),    # two ranges, N % 4 != 0: partials and the reduce kernel
    (256, 2048, 16002, torch.bfloat16, torch.float16),   # one range, N % 4 != 0: element stores of the last chunk
])
def test_wide_kernel(device, m, k, n, act, sdt):
    """The wide kernel (m > 64, g = 128: weights dequantised once per wave with the scale
    inside the operand, 128 x 128 or 128 x 256 workgroup tiles, activations by DMA into
    LDS): ragged M and N, one, two and three K ranges, every scale dtype, random zero
    points. Within the tolerance of the float64 oracle and bit-identical across repeats."""
    print(f"w4a16 wide m={m} k={k} n={n} {act} {sdt}", flush=True)
    x, qw, s, z, ref = _host_case(n, k, m, 128, seed=m + k + n, act=act, sdt=sdt, zeros="random")
    xd, qd, sd, zd = x.to(device), qw.to(device), s.to(device), z.to(device)
    y = w4a16_gemm(xd, qd, sd, zd, 128)
    assert y.dtype == act
    _assert_close(y, ref, f"wide m={m} k={k} n={n}")
    assert torch.equal(y, w4a16_gemm(xd, qd, sd, zd, 128))
    xs = torch.zeros(m, k + 72, dtype=act, device=device)[:, 40:40 + k]  # rows 16-byte aligned, stride k + 72
    xs.copy_(xd)
    assert torch.equal(w4a16_gemm(xs, qd, sd, zd, 128), y)  # strided activations: the same result


def test_wide_kernel_two_ranges_graph_and_dirty_workspace(device):
    """The wide kernel's in-kernel finish of two K ranges (arrival words behind the
    partials, tagged per call): correct on a workspace full of 0xFF bytes and replayed
    from a captured graph (one tag for every replay) to the eager result, with eager
    calls in between."""
    from slipstream_amd.kernels import quant_gemm
    x, qw, s, z, ref = _host_case(8192, 4096, 256, 128, seed=77, zeros="random")
    xd, qd, sd, zd = x.to(device), qw.to(device), s.to(device), z.to(device)
    y = w4a16_gemm(xd, qd, sd, zd, 128)
    _assert_close(y, ref, "wide two ranges")
    torch.cuda.synchronize()
    for ws in quant_gemm._WORKSPACE.values():
        ws.fill_(0xFF)
    y1 = w4a16_gemm(xd, qd, sd, zd, 128)
    torch.cuda.synchronize()
    assert torch.equal(y1, y)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        w4a16_gemm(xd, qd, sd, zd, 128)
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        out = w4a16_gemm(xd, qd, sd, zd, 128)
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y), f"replay {rep}"
        again = w4a16_gemm(xd, qd, sd, zd, 128)
        torch.cuda.synchronize()
        assert torch.equal(again, y)


def test_tiled_uneven_ranges_from_the_table_cap(device):
    """K = 15360 at M = 40 over 258 weight tiles: one range per tile would need a 122 KB
    scale table, so the host splits K until a range's table fits 40 KB -- 4 ranges of 32,
    32, 32 and 24 stages (the only way ranges come out uneven). Every column against the
    float64 oracle."""
    k, n, m = 15360, 33000, 40
    lin = workloads.w4a16_linear(k, n, m, device=device, seed=5)
    y = w4a16_gemm(lin.x, lin.qweight, lin.scales, lin.qzeros, lin.group_size)
    torch.cuda.synchronize()
    _assert_close(y, _oracle_every_column(lin), "uneven ranges vs oracle, every column")
    assert torch.equal(y, w4a16_gemm(lin.x, lin.qweight, lin.scales, lin.qzeros, lin.group_size))


def test_tiled_without_workspace_takes_untiled_kernel(device):
    """Through the C-ABI with no workspace, a shape planned for the K split runs the
    untiled MFMA kernel instead: same answer within the tolerance."""
    import ctypes
    from slipstream_amd import _ffi

    m, k, n, g = 64, 8192, 2048, 128  # tiled with a K split (4096 x 4096 class shapes take the skinny kernel)
    x, qw, s, z, ref = _host_case(n, k, m, g, seed=64, zeros="random")
    xd, qd, sd, zd = x.to(device), qw.to(device), s.to(device), z.to(device)
    lib = _ffi.lib()
    need = ctypes.c_int64(0)
    assert lib.ss_w4a16_workspace_size(m, n, k, g, _ffi.SS_DTYPE_BF16, ctypes.byref(need)) == _ffi.SS_OK
    assert need.value > 0
    out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    st = lib.ss_w4a16_gemm(xd.data_ptr(), out.data_ptr(), qd.data_ptr(), sd.data_ptr(), zd.data_ptr(), m, n, k, g,
                           k, n, _ffi.SS_DTYPE_BF16, _ffi.SS_DTYPE_F16, None, 0, _ffi.stream_ptr(xd.device))
    assert st == _ffi.SS_OK, lib.ss_last_error()
    torch.cuda.synchronize()
    _assert_close(out, ref, "no workspace")
    _assert_close(w4a16_gemm(xd, qd, sd, zd, g), ref, "with workspace")


def test_large_scale_table_takes_scalar_kernel(device):
    """k/group_size too large for the LDS scale table: the scalar kernel, same answer."""
    x, qw, s, z, ref = _host_case(32, 20480, 2, 32, seed=5, zeros="random")
    y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), 32)
    _assert_close(y, ref, "k=20480 g=32")


def test_generic_path_fp32_activations_and_small_groups(device):
    """fp32 x and group sizes that are not multiples of 32 take the scalar kernel."""
    for act, g, k in [(torch.float32, 128, 256), (torch.bfloat16, 8, 96), (torch.float16, 24, 240),
                      (torch.bfloat16, 32, 96)]:
        x, qw, s, z, ref = _host_case(40, k, 7, g, seed=g + k, act=act, zeros="random")
        y = w4a16_gemm(x.to(device), qw.to(device), s.to(device), z.to(device), g)
        assert y.dtype == act
        _assert_close(y, ref, f"generic act={act} g={g} k={k}")


def test_non_contiguous_activations(device):
    x, qw, s, z, ref = _host_case(128, 512, 8, 128, seed=11)
    xd = torch.empty((8, 1024), dtype=x.dtype, device=device)[:, 256:768]
    xd.copy_(x.to(device))
    y = w4a16_gemm(xd, qw.to(device), s.to(device), z.to(device), 128)
    _assert_close(y, ref, "strided x")
    y2 = w4a16_gemm(x.to(device).t().contiguous().t(), qw.to(device), s.to(device), z.to(device), 128)
    _assert_close(y2, ref, "transposed x")


def test_deterministic_across_shapes_and_repeats(device):
    """K slices are added in wave order inside a workgroup: repeated calls are bit-identical,
    also when calls of other shapes run in between."""
    big = _host_case(6144, 4096, 1, 128, seed=21)     # activations staged in LDS, 4 K slices
    small = _host_case(512, 1024, 16, 64, seed=22)    # g=64: one fold per 32-key step
    dev = [tuple(t.to(device) if isinstance(t, torch.Tensor) else t for t in c[:4]) for c in (big, small)]
    y2 = w4a16_gemm(*dev[1], 64)
    y1 = w4a16_gemm(*dev[0], 128)
    y4 = w4a16_gemm(*dev[1], 64)
    y3 = w4a16_gemm(*dev[0], 128)
    torch.cuda.synchronize()
    assert torch.equal(y1, y3) and torch.equal(y2, y4)
    _assert_close(y1, big[4], "big")
    _assert_close(y2, small[4], "small")


def test_argument_errors(device):
    x = torch.zeros(2, 256, dtype=torch.bfloat16, device=device)
    qw = torch.zeros(8, 32, dtype=torch.int32, device=device)
    s = torch.ones(8, 2, dtype=torch.float16, device=device)
    z = torch.zeros(8, 2, dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        w4a16_gemm(x, qw, s, z, 12)
    with pytest.raises(ValueError):
        w4a16_gemm(x[:, :128], qw, s, z, 128)
    with pytest.raises(ValueError):
        w4a16_gemm(x, qw[:, :16], s, z, 128)
    assert w4a16_gemm(x[:0], qw, s, z, 128).shape == (0, 8)


def _oracle_every_column(lin) -> np.ndarray:
    """The float64 numpy oracle for every output column of a full-size linear, in column
    chunks (the dequantised float64 weight of a chunk stays near 64 MB)."""
    x = lin.x.double().cpu().numpy()
    qw, sc, zz = lin.qweight.cpu().numpy(), lin.scales.double().cpu().numpy(), lin.qzeros.cpu().numpy()
    m, n, k = x.shape[0], qw.shape[0], x.shape[1]
    ref = np.empty((m, n), dtype=np.float64)
    step = max(256, (1 << 23) // k)
    for c0 in range(0, n, step):
        c1 = min(n, c0 + step)
        ref[:, c0:c1] = quant.w4a16_gemm(x, qw[c0:c1], sc[c0:c1], zz[c0:c1], lin.group_size)
    return ref


C5_SHAPES = [(4096, 6144, "qkv"), (4096, 4096, "o"), (4096, 14336, "gate/up"), (14336, 4096, "down"),
             (4096, 28672, "gate_up stacked")]


@pytest.mark.parametrize("k,n,name", C5_SHAPES)
@pytest.mark.parametrize("m", [1, 16, 64, 256])
def test_c5_llama_layer_linears(device, k, n, name, m):
    """C5 at full size: int4 U[0,15], fp16 scales U(0.005,0.02), zeros 8, bf16 x ~ N(0,1)."""
    print(f"w4a16 C5 {name} k={k} n={n} m={m}", flush=True)
    lin = workloads.w4a16_linear(k, n, m, device=device, seed=k + n + m)
    y = w4a16_gemm(lin.x, lin.qweight, lin.scales, lin.qzeros, lin.group_size)
    torch.cuda.synchronize()
    _assert_close(y, _oracle_every_column(lin), f"C5 {name} m={m} vs oracle, every column")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("group", [32, 128])
def test_device_quantizer_equals_oracle_quantizer(device, dtype, group):
    """The load-time format producer (slipstream_amd.quantized.quantize_weight, a torch
    restatement of quant_ref.py:72-100) run on the device: qweight and qzeros identical to
    oracle.quant.quantize_w4a16 on the same weight, scales identical after the cast to the
    weight's dtype (the reference returns them in weight.dtype). The weight has a constant
    group (0 joins its range), an all-zero group and groups that hit both nibble ends."""
    from slipstream_amd.quantized import quantize_weight

    g = torch.Generator().manual_seed(group)
    w = (torch.randn(96, 1024, generator=g) * 0.05).to(dtype)
    w[3, :group] = 0.25
    w[5, group : 2 * group] = 0.0
    w[7, :group] = torch.linspace(-1.0, 1.0, group).to(dtype)
    qw, s, z = quantize_weight(w.to(device), group)
    rq, rs, rz = quant.quantize_w4a16(w.float().numpy(), group)
    assert qw.dtype == torch.int32 and z.dtype == torch.int32 and s.dtype == dtype
    assert np.array_equal(qw.cpu().numpy(), rq)
    assert np.array_equal(z.cpu().numpy(), rz)
    assert np.array_equal(s.cpu().float().numpy(), torch.from_numpy(rs).to(dtype).float().numpy())
    u = quant.unpack_int4(rq, 1024)
    assert u.min() == 0 and u.max() == 15
