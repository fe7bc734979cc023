"""CPU checks that pin the oracle's Gated DeltaNet-2 (no GPU).

or_gdn2_l2norm / or_gdn2_decode_step / or_gdn2_prefill_chunk restate
src/gdn2.c:219-862. They are pinned by:
  * golden vectors of the reference build on the reference tests' own inputs
    (bench/kernel/gdn2.c:850-867): decode steps, prefill chunks of 16 and 32
    and the sequential decode of the same tokens, bit for bit;
  * the reference tests' float64 restatement of the recurrence
    S_t = (I - k (b*k)^T) D S_{t-1} + k (w*v)^T, o = S^T q at their tolerance
    2e-5 (a dropped decay, a swapped erase/write or a missing normalisation
    fails it), including the scalar-gate (KDA) special case and a three-step
    sequence carrying the state;
  * the chunk's algebraic identity: one WY chunk equals C sequential decode
    steps to 2e-5, including alpha in {0, 1} and zero q/k rows;
  * the L2-norm known answers and the rejections of the reference tests;
  * a live bit-for-bit comparison with oracle/_ref when it is built.
"""
import os

import numpy as np
import pytest

from golden.gen import (gdn2_boundary_inputs, gdn2_decode_inputs, gdn2_prefill_inputs, lpat)

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_vectors.npz")
DEC = [(4, 8, 1), (5, 7, 2), (2, 3, 3), (8, 8, 4), (128, 128, 5)]
PF = [(16, 8, 8, 11), (16, 16, 16, 12), (32, 8, 16, 13), (32, 16, 8, 14), (32, 128, 128, 15)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def ref_step64(S, q, k, v, b, w, a):
    """bench/kernel/gdn2.c:28-84 in float64 (the test's own reference)."""
    S = S.astype(np.float64).copy()
    def nrm(x):
        x = x.astype(np.float64)
        n = np.sqrt((x * x).sum())
        return np.zeros_like(x) if n < 1e-6 else x / n
    qn, kn = nrm(q), nrm(k)
    S *= a.astype(np.float64)[:, None]
    c = (b.astype(np.float64) * kn) @ S
    S -= np.outer(kn, c)
    S += np.outer(kn, w.astype(np.float64) * v.astype(np.float64))
    return S, qn @ S


@pytest.mark.parametrize("dk,dv,seed", DEC)
def test_gdn2_decode_golden(orc, gold, dk, dv, seed):
    S, q, k, v, b, w, a = gdn2_decode_inputs(dk, dv, seed)
    rc, S1, o = orc.gdn2_decode_step(S, q, k, v, b, w, a)
    assert rc == 0
    key = f"gdn2dec_{dk}x{dv}s{seed}"
    assert np.array_equal(bits(S1), bits(gold[key + "_S"]))
    assert np.array_equal(bits(o), bits(gold[key + "_o"]))
    rS, ro = ref_step64(S, q, k, v, b, w, a)  # the reference test's tolerance
    assert np.abs(S1 - rS).max() <= 2e-5 and np.abs(o - ro).max() <= 2e-5


def test_gdn2_decode_sequence_and_kda(orc):
    # three steps carrying the state (bench/kernel/gdn2.c:189-245)
    dk, dv = 4, 6
    S = np.zeros((dk, dv), np.float32)
    rS = np.zeros((dk, dv))
    f = np.float32
    for t in range(3):
        q = np.array([lpat(i, t, 100) + f(0.31) for i in range(dk)], f)
        k = np.array([lpat(i, t, 200) - f(0.17) for i in range(dk)], f)
        b, a = np.full(dk, 0.55, f), np.full(dk, 0.93, f)
        v = np.array([lpat(t, j, 300) + f(0.07) for j in range(dv)], f)
        w = np.full(dv, 0.65, f)
        rc, S, o = orc.gdn2_decode_step(S, q, k, v, b, w, a)
        assert rc == 0
        rS, ro = ref_step64(rS, q, k, v, b, w, a)
        assert np.abs(o - ro).max() <= 2e-5
    # scalar gates reduce GDN-2 to KDA (bench/kernel/gdn2.c:247-290)
    S = (0.1 * np.arange(1, 17, dtype=np.float32)).reshape(4, 4)
    q = np.array([0.5, -0.5, 0.25, 0.75], f)
    k = np.array([0.3, 0.8, -0.2, 0.1], f)
    v = np.array([1.0, -1.0, 0.5, 0.25], f)
    beta, gamma = np.full(4, 0.7, f), np.full(4, 0.9, f)
    rc, S1, o = orc.gdn2_decode_step(S, q, k, v, beta, beta, gamma)
    assert rc == 0
    rS, ro = ref_step64(S, q, k, v, beta, beta, gamma)
    assert np.abs(o - ro).max() <= 2e-5


@pytest.mark.parametrize("C,dk,dv,seed", PF)
def test_gdn2_prefill_golden_and_equivalence(orc, gold, C, dk, dv, seed):
    S, Q, K, V, B, W, A = gdn2_prefill_inputs(C, dk, dv, seed)
    key = f"gdn2pf{C}_{dk}x{dv}s{seed}"
    rc, S1, Out = orc.gdn2_prefill_chunk(S, Q, K, V, B, W, A)
    assert rc == 0
    assert np.array_equal(bits(S1), bits(gold[key + "_S"]))
    assert np.array_equal(bits(Out), bits(gold[key + "_Out"]))
    Ss = S
    for t in range(C):
        rc, Ss, o = orc.gdn2_decode_step(Ss, Q[t], K[t], V[t], B[t], W[t], A[t])
        assert rc == 0
        assert np.array_equal(bits(o), bits(gold[key + "_Oseq"][t]))
    assert np.array_equal(bits(Ss), bits(gold[key + "_Sseq"]))
    # the chunk is C decode steps up to fp32 rounding (bench/kernel/gdn2.c:590-605)
    assert np.abs(Out - gold[key + "_Oseq"]).max() <= 2e-5
    assert np.abs(S1 - Ss).max() <= 2e-5


def test_gdn2_prefill_boundary(orc, gold):
    S, Q, K, V, B, W, A = gdn2_boundary_inputs()
    rc, S1, Out = orc.gdn2_prefill_chunk(S, Q, K, V, B, W, A)
    assert rc == 0
    assert np.array_equal(bits(S1), bits(gold["gdn2pfb_S"]))
    assert np.array_equal(bits(Out), bits(gold["gdn2pfb_Out"]))
    assert np.abs(Out - gold["gdn2pfb_Oseq"]).max() <= 2e-5
    assert np.abs(S1 - gold["gdn2pfb_Sseq"]).max() <= 2e-5


def test_gdn2_l2norm_known(orc):
    rc, y = orc.gdn2_l2norm(np.array([3, 4, 0, 0], np.float32))
    assert rc == 0 and abs(y[0] - 0.6) < 1e-5 and abs(y[1] - 0.8) < 1e-5
    rc, y = orc.gdn2_l2norm(np.zeros(3, np.float32))
    assert rc == 0 and (y == 0).all()
    assert orc.gdn2_l2norm(np.ones(4, np.float32), eps=0.0)[0] == 2
    assert orc.gdn2_l2norm(np.ones(4, np.float32), eps=float("nan"))[0] == 2


def test_gdn2_rejections(orc):
    S, q, k, v, b, w, a = gdn2_decode_inputs(4, 4, 7)
    for name, arr, idx, val in (("q nan", q, 0, np.nan), ("v inf", v, 1, np.inf),
                                ("alpha>1", a, 2, 1.5), ("alpha<0", a, 3, -0.1),
                                ("alpha nan", a, 0, np.nan), ("b inf", b, 1, -np.inf)):
        x = arr.copy()
        x[idx] = val
        args = [x if arr is y else y for y in (q, k, v, b, w, a)]
        rc, S1, o = orc.gdn2_decode_step(S, *args)
        assert rc == 2, name
        assert np.array_equal(bits(S1), bits(S)), name  # state untouched
    for shape in ((0, 4), (4, 0), (1025, 4)):  # dims outside 1..1024
        assert orc.gdn2_decode_step(np.zeros(shape, np.float32), q, k, v, b, w, a)[0] == 2


def test_gdn2_vs_reference_build(orc, ref):
    rng = np.random.default_rng(11)
    for dk, dv in ((7, 33), (64, 256), (130, 10), (1024, 8)):
        S = (rng.standard_normal((dk, dv)) * 0.3).astype(np.float32)
        q, k, b = (rng.standard_normal(dk).astype(np.float32) for _ in range(3))
        a = rng.uniform(0.0, 1.0, dk).astype(np.float32)
        v, w = (rng.standard_normal(dv).astype(np.float32) for _ in range(2))
        x, y = orc.gdn2_decode_step(S, q, k, v, b, w, a), ref.gdn2_decode_step(S, q, k, v, b, w, a)
        assert x[0] == 0 and y[0] == 0
        assert np.array_equal(bits(x[1]), bits(y[1])) and np.array_equal(bits(x[2]), bits(y[2]))
        for C in (16, 32):
            Q, K, B = (rng.standard_normal((C, dk)).astype(np.float32) for _ in range(3))
            A = rng.uniform(0.0, 1.0, (C, dk)).astype(np.float32)
            V, W = (rng.standard_normal((C, dv)).astype(np.float32) for _ in range(2))
            x = orc.gdn2_prefill_chunk(S, Q, K, V, B, W, A)
            y = ref.gdn2_prefill_chunk(S, Q, K, V, B, W, A)
            assert x[0] == 0 and y[0] == 0
            assert np.array_equal(bits(x[1]), bits(y[1])) and np.array_equal(bits(x[2]), bits(y[2]))
