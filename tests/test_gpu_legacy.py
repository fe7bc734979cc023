"""GPU parity of the remaining host-pointer ABI (the reference's own entry
points, run on the MI355X) against the oracle.

Reference behaviour followed: src/moe_gemm.c:17-170 (fp32 GEMM, transpose),
src/lowbit.c:31-267 (levels, col_to_idx, T-MAC GEMM), src/tmac.c:168-506
(LUT), src/routing.c:16-76 (top-k), src/moe_layer.c:895-978 (batch sort) and
:1616-1663 (batched layer in its fp32, W8A8 and low-bit modes).

Bit-exact except where the value passes through exp (softmax weights,
SwiGLU): there the reference's own tolerance applies (test_routing.c:35-37,
test_moe_layer.c:146-189).
"""
import errno

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("M,N,K", [(7, 19, 33), (64, 96, 128), (130, 70, 257)])
def test_gemm_mat_f32(jt, orc, M, N, K):
    announce(f"gemm_mat_f32 {M}x{N}x{K}")
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    rc, C = jt.gemm_mat_f32(A, B)
    assert rc == 0 and np.array_equal(bits(C), bits(orc.gemm_f32(A, B)))


def test_transpose_f32(jt):
    announce("transpose_f32")
    rng = np.random.default_rng(1)
    for r, c in [(1, 1), (3, 70), (129, 65)]:
        A = rng.standard_normal((r, c)).astype(np.float32)
        rc, T = jt.transpose_f32(A)
        assert rc == 0 and np.array_equal(T, A.T)


@pytest.mark.parametrize("b", [2, 4])
def test_lowbit_levels(jt, orc, b):
    announce(f"lowbit fakequant / col_to_idx bits={b}")
    rng = np.random.default_rng(b)
    w = rng.standard_normal(1000).astype(np.float32)
    rc, fq = jt.lowbit_fakequant(w, b)
    rc2, fq2 = orc.lowbit_fakequant(w, b)
    assert rc == rc2 == 0 and np.array_equal(bits(fq), bits(fq2))
    for k in (32, 64, 256):
        col = rng.standard_normal(k).astype(np.float32)
        rc, idx, ws = jt.lowbit_col_to_idx(col, b)
        rc2, idx2, ws2 = orc.col_to_idx(col, b)
        assert rc == rc2 == 0 and np.array_equal(idx, idx2) and ws == ws2


@pytest.mark.parametrize("b", [2, 4])
@pytest.mark.parametrize("me,h,k", [(1, 24, 64), (5, 40, 256), (3, 17, 100)])
def test_lowbit_gemm_lut(jt, orc, b, me, h, k):
    announce(f"lowbit_gemm_lut bits={b} {me}x{h}x{k}")
    rng = np.random.default_rng(b * 100 + me + h + k)
    X = rng.standard_normal((me, k)).astype(np.float32)
    W = rng.standard_normal((k, h)).astype(np.float32)
    rc, Y = jt.lowbit_gemm_lut(X, W, b)
    rc2, Y2 = orc.lowbit_gemm_lut(X, W, b)
    assert rc == rc2 == 0 and np.array_equal(bits(Y), bits(Y2))


def test_tmac(jt, orc):
    announce("tmac lut ctor + lookup")
    rng = np.random.default_rng(3)
    act = rng.standard_normal((4, 128)).astype(np.float32)
    rc, q, s, b = jt.tmac_lut_ctor(act)
    rc2, q2, s2, b2 = orc.tmac_lut_ctor(act)
    assert rc == rc2 == 0
    assert np.array_equal(q, q2) and np.array_equal(bits(s), bits(s2))
    assert np.array_equal(bits(b), bits(b2))
    col = rng.standard_normal(128).astype(np.float32)
    for bb in (2, 4):
        _, idx, ws = orc.col_to_idx(col, bb)
        for r in range(4):
            rc, o = jt.tmac_lookup_accum(q[r], idx, s[r], b[r], bb, ws)
            rc2, o2 = orc.tmac_lookup_accum(q2[r].ravel(), idx, s2[r], b2[r], bb, ws)
            assert rc == rc2 == 0 and bits(np.float32(o)) == bits(np.float32(o2))


def test_routing_topk(jt, orc):
    announce("routing_topk")
    rng = np.random.default_rng(4)
    cases = [rng.standard_normal(256).astype(np.float32),
             np.full(64, 1.0, np.float32),
             np.round(rng.standard_normal(300) * 2).astype(np.float32) / 2,
             np.array([2.0, 1.0, -np.inf, -np.inf], np.float32),
             # signed zeros compare equal: ties go to the lower index
             np.array([-0.0, 0.0, -0.0, 0.0, -1.0, 0.0, -0.0, 1e-45], np.float32),
             rng.standard_normal(4096).astype(np.float32)]
    for lg in cases:
        for k in (1, 2, min(8, lg.size)):
            rc, ids, w = jt.routing_topk(lg, k)
            rc2, ids2, w2 = orc.topk(lg, k)
            assert rc == rc2 == 0 and np.array_equal(ids, ids2)
            np.testing.assert_allclose(w, w2, rtol=1e-6, atol=0)
    # every selected logit -inf: the softmax has no finite maximum
    lg = np.full(6, -np.inf, np.float32)
    assert jt.routing_topk(lg, 2)[0] == orc.topk(lg, 2)[0]
    assert jt.routing_topk(np.array([1.0, np.nan], np.float32), 1)[0] == 2


# 800 pairs: one-block sort; 40000 pairs of 256 experts: two-launch sort;
# more than 1024 experts or more than 65536 pairs: five-launch sort
@pytest.mark.parametrize("T,k,E", [(200, 4, 16), (5000, 8, 256), (2000, 2, 1500),
                                   (9000, 8, 300)])
@pytest.mark.parametrize("cap", [1.0, 1.5])
def test_batch_sort(jt, orc, cap, T, k, E):
    announce(f"moe_batch_sort T={T} k={k} E={E} cap={cap}")
    rng = np.random.default_rng(5 + T + E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    ids = np.argsort(rng.random((T, E)) ** (1.0 / p[None, :]), axis=1)[:, ::-1][:, :k]
    rc, perm, off, drop, dropped = jt.moe_batch_sort(ids, T, k, E, cap)
    rc2, perm2, off2, drop2 = orc.batch_sort(ids, T, k, E, cap)
    assert rc == rc2 == 0
    assert np.array_equal(perm, perm2) and np.array_equal(off, off2)
    assert np.array_equal(drop, drop2) and dropped == int(drop2.sum())


@pytest.mark.parametrize("shape", [(12, 128, 64, 8, 2, 1), (512, 256, 128, 64, 8, 1),
                                   (100, 128, 96, 16, 4, 3)],
                         ids=["T12", "T512E64k8", "T100h96S3"])
@pytest.mark.parametrize("w8,lb", [(0, 0), (1, 0), (0, 1), (0, 2), (1, 1)])
def test_moe_fwd_batch_modes(jt, orc, w8, lb, shape):
    """The drop-in layer entry in all five flag modes, at a toy shape, at
    T=512, E=64, k=8 (4096 routed pairs, capacity 1.25 drops some), and
    with three shared experts and h = 96 (not a multiple of 64: the W8A8
    steps' padded panels)."""
    T, n, h, E, k, S = shape
    announce(f"moe_fwd_batch w8a8={w8} lowbit={lb} T={T} n={n} h={h} E={E} k={k}")
    rng = np.random.default_rng(10 + 3 * w8 + lb + T)
    X = rng.standard_normal((T, n)).astype(np.float32)
    W = [(rng.standard_normal(s) / 8).astype(np.float32)
         for s in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    lib = jt.lib()
    assert lib.jt_w8a8_set_enabled(w8) == 0 and lib.jt_lowbit_set_mode(lb) == 0
    try:
        r = jt.moe_fwd_batch(X, *W, k, 1.25)
        ru = jt.moe_fwd_batch(X, *W, k, 1.25, unchecked=True)
    finally:
        lib.jt_w8a8_set_enabled(0)
        lib.jt_lowbit_set_mode(0)
    o = orc.moe_fwd_batch(X, *W, k, 1.25, w8, lb)
    assert r["rc"] == o["rc"] == 0 and ru["rc"] == 0
    for key in ("ids", "perm", "off", "drop"):
        assert np.array_equal(r[key], o[key]), key
        assert np.array_equal(ru[key], o[key]), key
    np.testing.assert_allclose(r["w"], o["w"], rtol=1e-6, atol=0)
    tol = 1e-5 * float(np.abs(o["Y"]).max())
    np.testing.assert_allclose(r["Y"], o["Y"], rtol=1e-5, atol=tol)
    assert np.array_equal(bits(r["Y"]), bits(ru["Y"]))


@pytest.mark.parametrize("which", range(8))
def test_moe_fwd_batch_rejects_nonfinite(jt, which):
    """A non-finite value in any one of the eight inputs (X, the gate, the
    routed and the shared experts' matrices) fails the checked entry with
    EINVAL and writes no output (src/moe_layer.c:1074-1096); the next call
    with clean inputs succeeds."""
    import errno as E_
    T, n, h, E, k, S = 40, 64, 32, 8, 2, 1
    announce(f"moe_fwd_batch rejects a non-finite input {which}")
    rng = np.random.default_rng(700 + which)
    X = rng.standard_normal((T, n)).astype(np.float32)
    W = [(rng.standard_normal(s) / 8).astype(np.float32)
         for s in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    args = [X] + W
    bad = [a.copy() for a in args]
    flat = bad[which].reshape(-1)
    flat[rng.integers(flat.size)] = np.nan if which % 2 else np.inf
    r = jt.moe_fwd_batch(*bad, k, 1.25)
    assert r["rc"] == jt.JT_ERR_INVAL and jt.errno() == E_.EINVAL
    assert not r["Y"].any() and not r["w"].any() and not r["off"].any()
    assert jt.moe_fwd_batch(*args, k, 1.25)["rc"] == 0


def test_moe_fwd_batch_known_answer(jt):
    """bench/kernel/test_moe_layer.c:146-189 through the batched entry."""
    announce("moe_fwd_batch known answer")
    X = np.array([[1.0, 0.5]], np.float32)
    Wgate = np.array([1, 0, 0, 1, -1, 0], np.float32).reshape(3, 2)
    Wg = np.array([0.5, -0.5, 0.5, 1.0, 0, 0], np.float32).reshape(3, 1, 2)
    Wu = np.array([1.0, 0, 0.5, -0.5, 0, 0], np.float32).reshape(3, 1, 2)
    Wd = np.array([1.0, 2.0, -1.0, 0.5, 0, 0], np.float32).reshape(3, 1, 2)
    Ws = [np.array(v, np.float32).reshape(1, 1, 2) for v in ([0.5, 0.5], [1.0, -1.0],
                                                              [0.5, -0.5])]
    r = jt.moe_fwd_batch(X, Wgate, Wg, Wu, Wd, *Ws, 2, 1.5)
    assert r["rc"] == 0 and list(r["ids"][0]) == [0, 1]
    assert abs(r["Y"][0, 0] - 0.14582792210843093) < 1e-5
    assert abs(r["Y"][0, 1] - 0.08212054137232436) < 1e-5


def test_moe_fwd_batch_w8a8_row_limit(jt, orc):
    """With the W8A8 flag the shared experts are one W8A8 GEMM of M = T rows;
    above 4096 rows the reference fails closed with EINVAL (src/w8a8.c:926-929)
    and writes nothing, as the oracle does."""
    announce("moe_fwd_batch w8a8 T=4097")
    rng = np.random.default_rng(4097)
    T, n, h, E, k, S = 4097, 64, 64, 8, 2, 1
    X = rng.standard_normal((T, n)).astype(np.float32)
    W = [(rng.standard_normal(s) / 8).astype(np.float32)
         for s in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    lib = jt.lib()
    assert lib.jt_w8a8_set_enabled(1) == 0
    try:
        r = jt.moe_fwd_batch(X, *W, k, 1.5)
        err = jt.errno()
    finally:
        lib.jt_w8a8_set_enabled(0)
    o = orc.moe_fwd_batch(X, *W, k, 1.5, 1, 0)
    assert r["rc"] == o["rc"] == 2 and err == errno.EINVAL
    assert not r["Y"].any() and not r["ids"].any()
    # the rejection leaves no error bits behind for the stream's next call
    rc, ids, _ = jt.routing_topk(np.array([0.5, 2.0, 1.0], np.float32), 2)
    assert rc == 0 and list(ids) == [1, 2]


@pytest.mark.parametrize("n,k,mode", [(8192, 100, "normal"), (4097, 8, "normal"),
                                      (100, 65, "normal"), (10000, 50, "ties"),
                                      (5000, 300, "masked"), (70000, 200, "normal"),
                                      (4096, 64, "normal")])
def test_routing_topk_any_n_k(jt, orc, n, k, mode):
    """jt_routing_topk for any n and any k <= n (src/routing.c:16-76): the
    same ids as the reference's strict-> scan, including ties (lower index
    first), rows with fewer than k values above -inf (the remaining rounds
    keep index 0), and the softmax weights to the reference's tolerance."""
    announce(f"routing_topk n={n} k={k} {mode}")
    rng = np.random.default_rng(n + k)
    lg = rng.standard_normal(n).astype(np.float32)
    if mode == "ties":
        lg = np.round(lg * 2).astype(np.float32) / 2      # few distinct values
        lg[rng.integers(0, n, 30)] = -0.0
    if mode == "masked":
        lg[rng.permutation(n)[:n - 200]] = -np.inf        # 200 finite values < k
    rc, ids, w = jt.routing_topk(lg, k)
    rc2, ids2, w2 = orc.topk(lg, k)
    assert rc == rc2 == 0
    assert np.array_equal(ids, ids2)
    np.testing.assert_allclose(w, w2, rtol=1e-6, atol=1e-12)
    if mode == "masked":
        assert (ids[200:] == 0).all()


def test_routing_topk_large_rejects(jt, orc):
    """A +inf among the selected makes the softmax non-finite and a NaN
    anywhere is rejected: rc 2 (EINVAL) in both, beyond the wavefront kernel."""
    announce("routing_topk large rejects")
    lg = np.random.default_rng(1).standard_normal(6000).astype(np.float32)
    lg[4321] = np.inf
    assert jt.routing_topk(lg, 70)[0] == orc.topk(lg, 70)[0] == 2
    lg[4321] = np.nan
    assert jt.routing_topk(lg, 70)[0] == orc.topk(lg, 70)[0] == 2
