"""GPU parity of the W8A8 path against the oracle (bit-exact).

Reference behaviour followed: src/w8a8.c (quantisers :688-855, GEMM
:955-1072 with the epilogue :654-686) and the fail-closed cases of
bench/kernel/test_w8a8.c:86-112, 150-170, 240-272.
"""
import errno as E

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (64, 1024), (17, 2816), (5, 4096)])
def test_quant_per_channel_bitexact(jt, orc, rows, cols):
    announce(f"quant_per_channel {rows}x{cols}")
    rng = np.random.default_rng(rows * 1000 + cols)
    X = (rng.standard_normal((rows, cols)) * rng.uniform(0.01, 10)).astype(np.float32)
    if rows > 2:
        X[1] = 0.0  # zero row -> scale 1, codes 0
    rc, Q, s = jt.w8a8_quant_per_channel(X)
    rc2, Q2, s2 = orc.quant_rows(X)
    assert rc == 0 and rc2 == 0
    assert np.array_equal(Q, Q2)
    assert np.array_equal(bits(s), bits(s2))


def test_quant_ties_round_half_away(jt, orc):
    announce("quant ties")
    # max|x| = 127 -> scale_d = 1, so x = k + 0.5 sits exactly on a tie
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 3.49999, -0.0],
                 np.float32)
    rc, q, s = jt.w8a8_quant_per_tensor(x)
    assert rc == 0 and s == np.float32(1.0)
    assert q.tolist() == [127, 3, -3, 1, -1, 127, -127, 3, 0]
    assert np.array_equal(q, orc.quant_tensor(x)[1])


@pytest.mark.parametrize("cols", [256, 1024, 2816, 4096, 4100])
def test_quant_rows_ties(jt, orc, cols):
    """Per-row codes on exact ties, at every register slot of a row: the
    kernel's single-precision guess must hand each tie to the exact path."""
    announce(f"quant rows ties cols={cols}")
    rng = np.random.default_rng(cols)
    X = (rng.standard_normal((9, cols)) * 20).astype(np.float32)
    X[:, 0] = 127.0                                   # scale_d = 1 on every row
    X[0, 1:] = rng.integers(-126, 126, cols - 1) + 0.5  # all ties
    X[1, 1:] = np.clip(X[1, 1:], -126, 126)
    X[1, rng.integers(1, cols, 40)] = -3.5            # a few scattered ties
    X[2, 1::64] = 7.5                                 # one lane, every slot
    X[3, 4 * 63 + 1::256] = -0.5                      # the last lane
    rc, Q, s = jt.w8a8_quant_per_channel(X)
    rc2, Q2, s2 = orc.quant_rows(X)
    assert rc == 0 and rc2 == 0
    assert np.array_equal(Q, Q2)
    assert np.array_equal(bits(s), bits(s2))
    assert Q[0, 1:].tolist() == [int(v + 0.5) if v > 0 else int(v - 0.5)
                                 for v in X[0, 1:].tolist()]


@pytest.mark.parametrize("cols", [100, 640, 2816])
def test_quant_tiny_rows_stay_in_row(jt, orc, cols):
    """Rows with max|x| below ~3.7e-37 make the fp32 reciprocal of the scale
    infinite, so every code of the row goes to the exact fp64 path. That
    path must rewrite only the row's own words: the tiny rows sit between
    normal rows, and the output has no slack after the last row."""
    announce(f"quant tiny rows cols={cols}")
    rng = np.random.default_rng(cols + 1)
    X = rng.standard_normal((6, cols)).astype(np.float32)
    X[1] *= np.float32(1e-38)
    X[3] = (rng.standard_normal(cols) * 1e-39).astype(np.float32)  # subnormal
    X[5] *= np.float32(3e-38)                                       # last row
    rc, Q, s = jt.w8a8_quant_per_channel(X)
    rc2, Q2, s2 = orc.quant_rows(X)
    assert rc == 0 and rc2 == 0
    assert np.array_equal(Q, Q2)
    assert np.array_equal(bits(s), bits(s2))


@pytest.mark.parametrize("n", [1, 255, 4096, 100003])
def test_quant_per_tensor_and_dequant(jt, orc, n):
    announce(f"quant_per_tensor n={n}")
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * 3
    rc, q, s = jt.w8a8_quant_per_tensor(x)
    rc2, q2, s2 = orc.quant_tensor(x)
    assert rc == rc2 == 0 and np.array_equal(q, q2) and bits(s) == bits(s2)
    rc, d = jt.w8a8_dequant_per_tensor(q, s)
    rc2, d2 = orc.dequant_rows(q.reshape(1, -1), np.array([s], np.float32))
    assert rc == rc2 == 0 and np.array_equal(bits(d), bits(d2.ravel()))
    rc, fq = jt.w8a8_fakequant_per_tensor(x)
    rc2, fq2 = orc.fakequant_rows(x.reshape(1, -1))
    assert rc == rc2 == 0 and np.array_equal(bits(fq), bits(fq2.ravel()))


def test_dequant_fakequant_per_channel(jt, orc):
    announce("dequant/fakequant per channel")
    rng = np.random.default_rng(5)
    X = rng.standard_normal((33, 130)).astype(np.float32)
    X[4] = 0
    _, Q, s = orc.quant_rows(X)
    rc, d = jt.w8a8_dequant_per_channel(Q, s)
    assert rc == 0 and np.array_equal(bits(d), bits(orc.dequant_rows(Q, s)[1]))
    rc, fq = jt.w8a8_fakequant_per_channel(X)
    assert rc == 0 and np.array_equal(bits(fq), bits(orc.fakequant_rows(X)[1]))


SHAPES = [(1, 8, 16), (4, 40, 72), (16, 130, 64), (17, 128, 128), (64, 1024, 1024),
          (200, 40, 72), (5, 2816, 1024), (33, 1024, 2816),
          # many tiles: the 128 x 256 tile configuration, ragged M, K padded
          (2100, 4096, 200)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_per_channel_bitexact(jt, orc, M, N, K):
    announce(f"gemm_per_channel {M}x{N}x{K}")
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    Aq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
    sB = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    sA = np.float32(0.0173)
    rc, C = jt.w8a8_gemm_per_channel(Aq, Bq, sA, sB)
    rc2, C2, _ = orc.w8a8_gemm(Aq, sA, Bq, sB)
    assert rc == rc2 == 0
    assert np.array_equal(bits(C), bits(C2))


@pytest.mark.parametrize("M,N,K", SHAPES[:5])
def test_gemm_per_tensor_bitexact(jt, orc, M, N, K):
    announce(f"gemm_per_tensor {M}x{N}x{K}")
    rng = np.random.default_rng(M + N + K)
    Aq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
    rc, C = jt.w8a8_gemm_per_tensor(Aq, Bq, 0.031, 0.0047)
    rc2, C2, _ = orc.w8a8_gemm(Aq, np.float32(0.031), Bq, np.float32(0.0047))
    assert rc == rc2 == 0 and np.array_equal(bits(C), bits(C2))


def test_gemm_matches_reference_library(jt, ref):
    announce("gemm vs reference build")
    rng = np.random.default_rng(11)
    for M, N, K in [(3, 40, 96), (20, 64, 128)]:
        Aq = rng.integers(-127, 128, (M, K), dtype=np.int8)
        Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
        sB = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
        rc, C = jt.w8a8_gemm_per_channel(Aq, Bq, 0.02, sB)
        rc2, C2 = ref.gemm_per_channel(Aq, Bq, 0.02, sB)
        assert rc == rc2 == 0 and np.array_equal(bits(C), bits(C2))


def test_device_gemm_per_row_scales_64x1024x1024(jt, orc, torch_cuda):
    """64x1024x1024 with per-row activation scales (device-resident API)."""
    torch = torch_cuda
    announce("device w8a8 gemm 64x1024x1024 per-row sA")
    rng = np.random.default_rng(2024)
    M, N, K = 64, 1024, 1024
    Aq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
    sA = rng.uniform(1e-3, 1e-2, M).astype(np.float32)
    sB = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    W = jt.W8A8(Bq_kn=torch.from_numpy(Bq).cuda(), sB=torch.from_numpy(sB).cuda())
    Bx, sx = W.export()
    assert np.array_equal(Bx, Bq) and np.array_equal(sx, sB)
    dA = torch.from_numpy(Aq).cuda()
    dsA = torch.from_numpy(sA).cuda()
    for m in (1, 4, 16, 64):
        out = torch.zeros((m, N), dtype=torch.float32, device="cuda")
        W.gemm(dA[:m].contiguous(), dsA[:m].contiguous(), out)
        assert jt.sync_errors() == 0
        rc, C2, _ = orc.w8a8_gemm(Aq[:m], sA[:m], Bq, sB)
        assert rc == 0 and np.array_equal(bits(out.cpu().numpy()), bits(C2))


def test_device_prepare_from_fp32(jt, orc, torch_cuda):
    torch = torch_cuda
    announce("device w8a8 prepare from fp32 + quant_rows")
    rng = np.random.default_rng(3)
    N, K, M = 256, 512, 40
    Wf = rng.standard_normal((N, K)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = jt.W8A8(W=torch.from_numpy(Wf).cuda())
    Bx, sx = W.export()
    _, Qw, sw = orc.quant_rows(Wf)
    assert np.array_equal(Bx, Qw.T) and np.array_equal(bits(sx), bits(sw))
    dX = torch.from_numpy(X).cuda()
    Xq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    sX = torch.zeros(M, dtype=torch.float32, device="cuda")
    jt.quant_rows(dX, Xq, sX)
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    W.gemm(Xq, sX, out)
    assert jt.sync_errors() == 0
    _, Qx, sxo = orc.quant_rows(X)
    assert np.array_equal(Xq.cpu().numpy(), Qx)
    rc, C2, _ = orc.w8a8_gemm(Qx, sxo, Qw.T.copy(), sw)
    assert np.array_equal(bits(out.cpu().numpy()), bits(C2))


@pytest.mark.parametrize("N,K", [(4096, 1024), (200, 100), (130, 64), (300, 4096)])
def test_device_projection_fp32_activations(jt, orc, torch_cuda, N, K):
    """The per-token INT8 projection (jt_hip_w8a8_gemm_f32): fp32 rows
    quantised inside the call, bit-identical to quant_rows + the GEMM, for
    the in-block quantiser (M <= 16) and the workspace path (M > 16); K not
    a multiple of 64 meets the zero-padded weight panels, K = 4096 the
    in-block quantiser's longest rows."""
    torch = torch_cuda
    announce(f"device w8a8 projection N={N} K={K}")
    rng = np.random.default_rng(N + K)
    Wf = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    W = jt.W8A8(W=torch.from_numpy(Wf).cuda())
    _, Qw, sw = orc.quant_rows(Wf)
    ws = None
    for M in (1, 2, 3, 4, 5, 16, 17, 64, 300):
        X = rng.standard_normal((M, K)).astype(np.float32)
        X[0, : K // 2] *= 50.0
        out = torch.full((M, N), np.nan, device="cuda")
        ws = W.gemm_f32(torch.from_numpy(X).cuda(), out, ws=ws)
        assert jt.sync_errors() == 0
        _, Qx, sx = orc.quant_rows(X)
        rc, C2, _ = orc.w8a8_gemm(Qx, sx, Qw.T.copy(), sw)
        assert rc == 0 and np.array_equal(bits(out.cpu().numpy()), bits(C2)), M


def test_fail_closed(jt):
    announce("w8a8 fail-closed cases")
    Aq = np.ones((4, 16), np.int8)
    Bq = np.ones((16, 8), np.int8)
    sB = np.full(8, 0.01, np.float32)
    keep = np.full((4, 8), 7.0, np.float32)
    # -128 code: rejected before any write (src/w8a8.c:979-999)
    bad = Aq.copy()
    bad[0, 0] = -128
    out = keep.copy()
    rc, _ = jt.w8a8_gemm_per_channel(bad, Bq, 0.5, sB, out=out)
    assert rc == 2 and jt.errno() == E.EINVAL and np.array_equal(out, keep)
    # sA = 0, NaN scales, NULL sB_col, M < 0, K > 4096 (src/w8a8.c:910-953)
    assert jt.w8a8_gemm_per_channel(Aq, Bq, 0.0, sB, out=out)[0] == 2
    nan_s = sB.copy()
    nan_s[3] = np.nan
    assert jt.w8a8_gemm_per_channel(Aq, Bq, 0.5, nan_s, out=out)[0] == 2
    assert jt.w8a8_gemm_per_channel(Aq, Bq, 0.5, None, out=out)[0] == 2
    assert jt.w8a8_gemm_per_tensor(Aq, Bq, 0.5, float("nan"), out=out)[0] == 2
    assert np.array_equal(out, keep)
    # computed overflow -> EINVAL return with errno ERANGE, output untouched
    big = np.full(8, 3e38, np.float32)
    A127 = np.full((4, 16), 127, np.int8)
    rc, _ = jt.w8a8_gemm_per_channel(A127, np.full((16, 8), 127, np.int8), 1e3, big, out=out)
    assert rc == 2 and jt.errno() == E.ERANGE and np.array_equal(out, keep)
    # M == 0 is a no-op (src/w8a8.c:959-971)
    lib = jt.lib()
    assert lib.jt_w8a8_gemm_per_channel(Aq, Bq, 0.5, sB.ctypes.data, out, 0, 8, 16) == 0
    assert lib.jt_w8a8_gemm_per_channel(Aq, Bq, 0.5, sB.ctypes.data, out, 0, 0, 16) == 2
    assert np.array_equal(out, keep)
    # non-finite input to the quantisers
    x = np.array([0.1, np.nan, 0.3], np.float32)
    assert jt.w8a8_quant_per_tensor(x)[0] == 2 and jt.errno() == E.EINVAL
    assert jt.w8a8_quant_per_channel(x.reshape(1, 3))[0] == 2
    q = np.array([-128, 1, 2, 3], np.int8)
    assert jt.w8a8_dequant_per_tensor(q, 0.01)[0] == 2
    assert jt.w8a8_dequant_per_tensor(q[1:], 0.0)[0] == 2
