"""GPU parity of Gated DeltaNet-2 (jt_gdn2_* and jt_hip_gdn2_*) against the
reference's outputs (golden vectors) and the oracle, bit for bit.

Reference behaviour followed: src/gdn2.c:129-862 (state helpers, L2 norm,
decode step, WY prefill chunk) and the tests of bench/kernel/gdn2.c. Every
operation is fp32 (fp64 only inside the norms) in the reference's order, so
results must match exactly.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import announce
from golden.gen import gdn2_boundary_inputs, gdn2_decode_inputs, gdn2_prefill_inputs

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_vectors.npz")
DEC = [(4, 8, 1), (5, 7, 2), (2, 3, 3), (8, 8, 4), (128, 128, 5)]
PF = [(16, 8, 8, 11), (16, 16, 16, 12), (32, 8, 16, 13), (32, 16, 8, 14), (32, 128, 128, 15)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same(a, b):
    return np.array_equal(bits(a), bits(b))


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def rand_step(rng, dk, dv, lo=0.0):
    S = (rng.standard_normal((dk, dv)) * 0.3).astype(np.float32)
    q, k, b = (rng.standard_normal(dk).astype(np.float32) for _ in range(3))
    a = rng.uniform(lo, 1.0, dk).astype(np.float32)
    v, w = (rng.standard_normal(dv).astype(np.float32) for _ in range(2))
    return S, q, k, v, b, w, a


def rand_chunk(rng, C_, dk, dv):
    Q, K, B = (rng.standard_normal((C_, dk)).astype(np.float32) for _ in range(3))
    A = rng.uniform(0.0, 1.0, (C_, dk)).astype(np.float32)
    A[0, : dk // 3] = 0.0
    A[1, : dk // 2] = 1.0
    V, W = (rng.standard_normal((C_, dv)).astype(np.float32) for _ in range(2))
    return Q, K, V, B, W, A


def test_gdn2_state_helpers(jt):
    L = jt.lib()
    n = C.c_size_t(0)
    assert L.jt_gdn2_state_bytes(4, 8, C.byref(n)) == 0 and n.value == 128
    assert L.jt_gdn2_state_bytes(0, 8, C.byref(n)) == jt.JT_ERR_INVAL
    assert L.jt_gdn2_state_bytes(2048, 8, C.byref(n)) == jt.JT_ERR_INVAL
    assert L.jt_gdn2_scratch_floats(4, 8, C.byref(n)) == 0 and n.value == 24
    p = C.c_void_p()
    assert L.jt_gdn2_state_alloc(C.byref(p), 4, 4) == 0 and p.value % 64 == 0
    assert L.jt_gdn2_state_alloc(None, 4, 4) == jt.JT_ERR_INVAL
    buf = (C.c_float * 16).from_address(p.value)
    assert all(x == 0.0 for x in buf)
    buf[0] = 1.0
    assert L.jt_gdn2_state_reset(p, 4, 4) == 0 and buf[0] == 0.0
    assert L.jt_gdn2_state_reset(None, 4, 4) == jt.JT_ERR_INVAL
    L.jt_gdn2_state_free(p)
    L.jt_gdn2_state_free(None)


def test_gdn2_l2norm(jt, orc):
    announce("gdn2 l2norm")
    rc, y = jt.gdn2_l2norm(np.array([3, 4, 0, 0], np.float32))
    assert rc == 0 and abs(y[0] - 0.6) < 1e-5 and abs(y[1] - 0.8) < 1e-5
    rc, y = jt.gdn2_l2norm(np.zeros(3, np.float32))
    assert rc == 0 and (y == 0).all()
    x = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    assert same(jt.gdn2_l2norm(x)[1], orc.gdn2_l2norm(x)[1])
    assert jt.gdn2_l2norm(x, eps=0.0)[0] == jt.JT_ERR_INVAL


@pytest.mark.parametrize("dk,dv,seed", DEC)
def test_gdn2_decode_golden(jt, gold, dk, dv, seed):
    announce(f"gdn2 decode golden {dk}x{dv} s{seed}")
    rc, S1, o = jt.gdn2_decode_step(*gdn2_decode_inputs(dk, dv, seed))
    assert rc == 0
    key = f"gdn2dec_{dk}x{dv}s{seed}"
    assert same(S1, gold[key + "_S"]) and same(o, gold[key + "_o"])


@pytest.mark.parametrize("dk,dv", [(1, 1), (7, 33), (128, 128), (130, 256), (1024, 8),
                                   (8, 1024), (256, 64), (64, 40), (128, 300), (64, 1024)])
def test_gdn2_decode_vs_oracle(jt, orc, dk, dv):
    announce(f"gdn2 decode {dk}x{dv}")
    rng = np.random.default_rng(dk * 7 + dv)
    st = rand_step(rng, dk, dv)
    st[6][: max(1, dk // 4)] = 0.0  # alpha = 0 rows forget everything
    rc, S1, o = jt.gdn2_decode_step(*st)
    rc2, S2, o2 = orc.gdn2_decode_step(*st)
    assert rc == 0 and rc2 == 0
    assert same(S1, S2) and same(o, o2)


def test_gdn2_decode_sequence(jt, orc):
    announce("gdn2 decode sequence")
    rng = np.random.default_rng(5)
    S = np.zeros((16, 24), np.float32)
    Sa = Sb = S
    for t in range(6):
        _, q, k, v, b, w, a = rand_step(rng, 16, 24, lo=0.5)
        if t == 3:
            q[:] = 0.0  # the zero-norm guard
        rc, Sa, oa = jt.gdn2_decode_step(Sa, q, k, v, b, w, a)
        rc2, Sb, ob = orc.gdn2_decode_step(Sb, q, k, v, b, w, a)
        assert rc == 0 and rc2 == 0 and same(Sa, Sb) and same(oa, ob)


def test_gdn2_decode_rejections(jt):
    announce("gdn2 decode rejections")
    S, q, k, v, b, w, a = gdn2_decode_inputs(4, 4, 7)
    for name, which, idx, val in (("q nan", 0, 0, np.nan), ("v inf", 2, 1, np.inf),
                                  ("alpha>1", 5, 2, 1.5), ("alpha<0", 5, 3, -0.1),
                                  ("alpha nan", 5, 0, np.nan), ("b inf", 3, 1, -np.inf),
                                  ("w nan", 4, 0, np.nan), ("k inf", 1, 2, np.inf)):
        args = [x.copy() for x in (q, k, v, b, w, a)]
        args[which][idx] = val
        rc, S1, o = jt.gdn2_decode_step(S, *args)
        assert rc == jt.JT_ERR_INVAL, name
        assert same(S1, S) and np.isnan(o).all(), name  # fail-closed
    # argument checks of the reference (bench/kernel/gdn2.c:342-395)
    L = jt.lib()
    st = jt._State(S)
    o = np.zeros(4, np.float32)
    f = [x.ctypes.data for x in (q, k, v, b, w, a)]
    scr = np.zeros(16, np.float32)
    assert L.jt_gdn2_decode_step(None, o.ctypes.data, *f, 4, 4, scr.ctypes.data, 16) == \
        jt.JT_ERR_INVAL
    assert L.jt_gdn2_decode_step(st.p, o.ctypes.data, *f, 0, 4, scr.ctypes.data, 16) == \
        jt.JT_ERR_INVAL
    assert L.jt_gdn2_decode_step(st.p, o.ctypes.data, *f, 4, 4, scr.ctypes.data, 15) == \
        jt.JT_ERR_INVAL
    raw = np.zeros(4 * 4 + 32, np.float32)
    mis = raw.ctypes.data + 4 if (raw.ctypes.data + 4) % 64 else raw.ctypes.data + 8
    assert L.jt_gdn2_decode_step(mis, o.ctypes.data, *f, 4, 4, scr.ctypes.data, 16) == \
        jt.JT_ERR_ALIGN


@pytest.mark.parametrize("C_,dk,dv,seed", PF)
def test_gdn2_prefill_golden(jt, gold, C_, dk, dv, seed):
    announce(f"gdn2 prefill golden C={C_} {dk}x{dv}")
    rc, S1, Out = jt.gdn2_prefill_chunk(*gdn2_prefill_inputs(C_, dk, dv, seed))
    assert rc == 0
    key = f"gdn2pf{C_}_{dk}x{dv}s{seed}"
    assert same(S1, gold[key + "_S"]) and same(Out, gold[key + "_Out"])


def test_gdn2_prefill_boundary_golden(jt, gold):
    announce("gdn2 prefill boundary golden")
    rc, S1, Out = jt.gdn2_prefill_chunk(*gdn2_boundary_inputs())
    assert rc == 0 and same(S1, gold["gdn2pfb_S"]) and same(Out, gold["gdn2pfb_Out"])


@pytest.mark.parametrize("C_,dk,dv", [(16, 1, 1), (16, 7, 33), (32, 128, 128), (32, 130, 70),
                                      (16, 1024, 16), (32, 64, 1024)])
def test_gdn2_prefill_vs_oracle(jt, orc, C_, dk, dv):
    announce(f"gdn2 prefill C={C_} {dk}x{dv}")
    rng = np.random.default_rng(C_ + dk + dv)
    S = (rng.standard_normal((dk, dv)) * 0.3).astype(np.float32)
    ch = rand_chunk(rng, C_, dk, dv)
    rc, S1, O1 = jt.gdn2_prefill_chunk(S, *ch)
    rc2, S2, O2 = orc.gdn2_prefill_chunk(S, *ch)
    assert rc == 0 and rc2 == 0 and same(S1, S2) and same(O1, O2)
    bad = [x.copy() for x in ch]
    bad[5][3, 0] = 2.0  # alpha > 1
    rc, S3, O3 = jt.gdn2_prefill_chunk(S, *bad)
    assert rc == jt.JT_ERR_INVAL and same(S3, S) and np.isnan(O3).all()


def _t(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def test_gdn2_decode_device_heads(jt, orc, torch_cuda):
    torch = torch_cuda
    H, dk, dv = 48, 128, 96
    announce(f"jt_hip_gdn2_decode H={H} {dk}x{dv}")
    rng = np.random.default_rng(9)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    q, k, b = (rng.standard_normal((H, dk)).astype(np.float32) for _ in range(3))
    a = rng.uniform(0, 1, (H, dk)).astype(np.float32)
    v, w = (rng.standard_normal((H, dv)).astype(np.float32) for _ in range(2))
    a[7, 5] = np.nan  # head 7 is rejected, the others run
    dS, dO = _t(torch, S), torch.full((H, dv), 42.0, device="cuda")
    rc = jt.gdn2_decode_device(dS, dO, *[_t(torch, x) for x in (q, k, v, b, w, a)])
    assert rc == 0
    assert jt.sync_errors() & jt.EF_NONFINITE_INPUT
    S1, O1 = dS.cpu().numpy(), dO.cpu().numpy()
    for h in range(H):
        if h == 7:
            assert same(S1[h], S[h]) and (O1[h] == 42.0).all()
            continue
        rc, Sh, oh = orc.gdn2_decode_step(S[h], q[h], k[h], v[h], b[h], w[h], a[h])
        assert rc == 0 and same(S1[h], Sh) and same(O1[h], oh), h


def test_gdn2_prefill_device_heads(jt, orc, torch_cuda):
    torch = torch_cuda
    H, T, C_, dk, dv = 6, 96, 32, 64, 80
    announce(f"jt_hip_gdn2_prefill H={H} T={T} C={C_}")
    rng = np.random.default_rng(10)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    Q, K, B = (rng.standard_normal((H, T, dk)).astype(np.float32) for _ in range(3))
    A = rng.uniform(0.3, 1, (H, T, dk)).astype(np.float32)
    V, W = (rng.standard_normal((H, T, dv)).astype(np.float32) for _ in range(2))
    V[4, 70, 3] = np.inf  # head 4 is rejected as a whole, before any chunk
    dS = _t(torch, S)
    dOut = torch.full((H, T, dv), 42.0, device="cuda")
    rc, _ = jt.gdn2_prefill_device(dS, dOut, *[_t(torch, x) for x in (Q, K, V, B, W, A)], C_)
    assert rc == 0
    assert jt.sync_errors() & jt.EF_NONFINITE_INPUT
    S1, O1 = dS.cpu().numpy(), dOut.cpu().numpy()
    for h in range(H):
        if h == 4:
            assert same(S1[h], S[h]) and (O1[h] == 42.0).all()
            continue
        Sh = S[h]
        for c0 in range(0, T, C_):
            sl = slice(c0, c0 + C_)
            rc, Sh, Oh = orc.gdn2_prefill_chunk(Sh, Q[h, sl], K[h, sl], V[h, sl], B[h, sl],
                                                W[h, sl], A[h, sl])
            assert rc == 0 and same(O1[h, sl], Oh), (h, c0)
        assert same(S1[h], Sh), h


@pytest.mark.parametrize("H,T,C_,dk,dv", [(3, 64, 16, 64, 48),     # 16-row chunks, 8-column blocks
                                          (4, 48, 16, 32, 1024),   # 16-row chunks, 16-column blocks
                                          (2, 64, 32, 32, 1024)])  # 32-row chunks, 8-column blocks
def test_gdn2_prefill_device_block_widths(jt, orc, torch_cuda, H, T, C_, dk, dv):
    """Every column-block width of the prefill's state kernel: blocks of
    128/C columns while the grid has fewer than 256 blocks of 256/C, then
    the wide blocks (4 heads x 1024 columns at C=16, 2 x 1024 at C=32),
    each head's state and outputs against the oracle's chunk chain."""
    torch = torch_cuda
    announce(f"jt_hip_gdn2_prefill H={H} T={T} C={C_} {dk}x{dv}")
    rng = np.random.default_rng(H * 100 + C_ + dv)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    Q, K, B = (rng.standard_normal((H, T, dk)).astype(np.float32) for _ in range(3))
    A = rng.uniform(0.5, 1, (H, T, dk)).astype(np.float32)
    V, W = (rng.standard_normal((H, T, dv)).astype(np.float32) for _ in range(2))
    dS = _t(torch, S)
    dOut = torch.empty((H, T, dv), device="cuda")
    rc, _ = jt.gdn2_prefill_device(dS, dOut, *[_t(torch, x) for x in (Q, K, V, B, W, A)], C_)
    assert rc == 0
    assert jt.sync_errors() == 0
    S1, O1 = dS.cpu().numpy(), dOut.cpu().numpy()
    for h in range(H):
        Sh = S[h]
        for c0 in range(0, T, C_):
            sl = slice(c0, c0 + C_)
            rc, Sh, Oh = orc.gdn2_prefill_chunk(Sh, Q[h, sl], K[h, sl], V[h, sl], B[h, sl],
                                                W[h, sl], A[h, sl])
            assert rc == 0 and same(O1[h, sl], Oh), (h, c0)
        assert same(S1[h], Sh), h


def test_gdn2_prefill_full_size(jt, orc, torch_cuda):
    """The prefill benchmark's shape: 8 heads x 4096 tokens of 128x128
    states in chunks of 32, every head's state and every output against the
    oracle's chunk chain, bit for bit."""
    torch = torch_cuda
    H, T, C_, dk, dv = 8, 4096, 32, 128, 128
    announce(f"jt_hip_gdn2_prefill full size H={H} T={T} C={C_}")
    rng = np.random.default_rng(13)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    Q, K, B = (rng.standard_normal((H, T, dk)).astype(np.float32) for _ in range(3))
    A = rng.uniform(0.9, 1, (H, T, dk)).astype(np.float32)
    V, W = (rng.standard_normal((H, T, dv)).astype(np.float32) for _ in range(2))
    dS = _t(torch, S)
    dOut = torch.empty((H, T, dv), device="cuda")
    rc, _ = jt.gdn2_prefill_device(dS, dOut, *[_t(torch, x) for x in (Q, K, V, B, W, A)], C_)
    assert rc == 0
    assert jt.sync_errors() == 0
    S1, O1 = dS.cpu().numpy(), dOut.cpu().numpy()
    for h in range(H):
        Sh = S[h]
        for c0 in range(0, T, C_):
            sl = slice(c0, c0 + C_)
            rc, Sh, Oh = orc.gdn2_prefill_chunk(Sh, Q[h, sl], K[h, sl], V[h, sl], B[h, sl],
                                                W[h, sl], A[h, sl])
            assert rc == 0 and same(O1[h, sl], Oh), (h, c0)
        assert same(S1[h], Sh), h


@pytest.mark.parametrize("H,dk,dv", [(512, 128, 128)])
def test_gdn2_decode_full_size(jt, orc, torch_cuda, H, dk, dv):
    """The decode benchmark's shape (8 heads x 64 sequences of 128x128
    states): every head against the oracle."""
    torch = torch_cuda
    announce(f"jt_hip_gdn2_decode full size H={H}")
    rng = np.random.default_rng(12)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    q, k, b = (rng.standard_normal((H, dk)).astype(np.float32) for _ in range(3))
    a = rng.uniform(0.9, 1, (H, dk)).astype(np.float32)
    v, w = (rng.standard_normal((H, dv)).astype(np.float32) for _ in range(2))
    dS, dO = _t(torch, S), torch.empty((H, dv), device="cuda")
    assert jt.gdn2_decode_device(dS, dO, *[_t(torch, x) for x in (q, k, v, b, w, a)]) == 0
    assert jt.sync_errors() == 0
    S1, O1 = dS.cpu().numpy(), dO.cpu().numpy()
    for h in range(H):
        rc, Sh, oh = orc.gdn2_decode_step(S[h], q[h], k[h], v[h], b[h], w[h], a[h])
        assert same(S1[h], Sh) and same(O1[h], oh), h


def test_error_words_are_per_stream(jt, orc, torch_cuda):
    """A rejected head on one stream sets that stream's error word only: a
    clean call on a second stream reads zero, and reading a word clears it."""
    torch = torch_cuda
    H, dk, dv = 4, 16, 16
    announce("error words per stream (jt_hip_gdn2_decode on two streams)")
    rng = np.random.default_rng(21)
    S = (rng.standard_normal((H, dk, dv)) * 0.3).astype(np.float32)
    q, k, b = (rng.standard_normal((H, dk)).astype(np.float32) for _ in range(3))
    a = rng.uniform(0, 1, (H, dk)).astype(np.float32)
    v, w = (rng.standard_normal((H, dv)).astype(np.float32) for _ in range(2))
    a_bad = a.copy()
    a_bad[1, 2] = np.nan
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    d1 = [_t(torch, x) for x in (S, q, k, v, b, w, a_bad)]
    d2 = [_t(torch, x) for x in (S, q, k, v, b, w, a)]
    o1, o2 = torch.empty(H, dv, device="cuda"), torch.empty(H, dv, device="cuda")
    torch.cuda.synchronize()
    assert jt.gdn2_decode_device(d1[0], o1, *d1[1:], stream=s1) == 0
    assert jt.gdn2_decode_device(d2[0], o2, *d2[1:], stream=s2) == 0
    assert jt.sync_errors(s2) == 0
    assert jt.sync_errors(s1) & jt.EF_NONFINITE_INPUT
    assert jt.sync_errors(s1) == 0
    assert jt.sync_errors() == 0
