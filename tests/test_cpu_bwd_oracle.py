"""CPU checks that pin the oracle's batched MoE backward (no GPU).

or_moe_bwd_batch restates jt_moe_bwd_batch (src/moe_layer.c:1684-2502). It
is pinned by:
  * golden vectors of the reference's own functions on the inputs of the
    reference's backward tests (bench/kernel/test_moe_layer.c:1166-1206,
    1440-1488), forward caches included, and on a seeded case with drops;
  * the assertions those reference tests make (dLogits zero for dropped
    pairs, kept/dropped counts, a finite dX);
  * central differences of an independent float64 forward: a wrong sign, a
    swapped gate/up, a missing transpose or a dropped term in the backward
    moves the result far outside the tolerance;
  * a live bit-for-bit comparison with oracle/_ref when it is built;
  * the reference's rejections (fail-closed EINVAL cases).
"""
import os

import numpy as np
import pytest

from golden.gen import BWD_ARGS, bwd_args, bwd_case, capacity_sort, hpat

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_vectors.npz")
BWD_RND = (24, 42, 24, 6, 3, 2, 300, 1.0)  # tests/golden/make_golden.py
OUTS = ("dX", "dWgate", "dWg", "dWu", "dWd", "dWg_s", "dWu_s", "dWd_s", "dLogits")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def ref_case_args(gold, c):
    pre = f"bwdref{c}_"
    g = lambda k: gold[pre + k] if pre + k in gold.files else None
    return [g("dY"), g("X"), g("Wgate"), g("Wg"), g("Wu"), g("Wd"), g("Wg_s"), g("Wu_s"),
            g("Wd_s"), g("ids"), g("w"), g("Gsel"), g("Usel"), g("Ysel"), g("Gs"), g("Us"),
            g("perm"), g("off"), g("drop"), int(g("k"))]


def assert_same(out, want, names):
    for nm in names:
        assert np.array_equal(bits(out[nm]), bits(want[nm])), nm


@pytest.mark.parametrize("c", [0, 1])
def test_bwd_golden_reference_tests(orc, gold, c):
    args = ref_case_args(gold, c)
    o = orc.moe_bwd_batch(*args)
    assert o["rc"] == 0
    pre = f"bwdref{c}_out_"
    names = [nm for nm in OUTS if pre + nm in gold.files]
    assert_same(o, {nm: gold[pre + nm] for nm in names}, names)
    u = orc.moe_bwd_batch(*args, validate=0)
    assert_same(u, o, names)
    if c == 1:  # test_moe_layer.c:1480-1514
        drop, ids, k = gold["bwdref1_drop"], gold["bwdref1_ids"].ravel(), args[-1]
        assert int(gold["bwdref1_off"][-1]) == 13 and int(drop.sum()) == 3
        for q in np.nonzero(drop)[0]:
            assert o["dLogits"][q // k, ids[q]] == 0.0
        assert np.isfinite(o["dX"]).all()


def test_bwd_golden_seeded_case(orc, gold):
    c = bwd_case(*BWD_RND)
    assert c["drop"].any()  # the case exercises capacity drops
    o = orc.moe_bwd_batch(*bwd_args(c))
    assert o["rc"] == 0
    assert_same(o, {nm: gold["bwdrnd_" + nm] for nm in OUTS}, OUTS)


CASES = [(6, 4, 2, 4, 2, 1, 11, 1.25), (16, 32, 16, 8, 2, 1, 12, None),
         (24, 64, 32, 8, 4, 2, 13, 1.0), (40, 36, 20, 16, 3, 0, 14, 1.25),
         (9, 130, 64, 5, 5, 1, 15, None), (33, 17, 9, 7, 1, 3, 16, 1.0)]


@pytest.mark.parametrize("case", CASES)
def test_bwd_oracle_vs_reference_build(orc, ref, case):
    c = bwd_case(*case)
    for v in (1, 0):
        a = orc.moe_bwd_batch(*bwd_args(c), validate=v)
        b = ref.moe_bwd_batch(*bwd_args(c), validate=v)
        assert a["rc"] == 0 and b["rc"] == 0
        names = [nm for nm in OUTS if nm in b]
        assert_same(a, b, names)


# ------------------------------------------------------------ finite differences

def _forward64(P, ids, dY, k):
    """L = sum_t <dY_t, Y_t> of the layer in float64 with the routing ids
    fixed: w = softmax of the selected logits, routed experts
    Wd^T (silu(Wg x) * (Wu x)), plus the shared experts."""
    X, Wgate, Wg, Wu, Wd = P["X"], P["Wgate"], P["Wg"], P["Wu"], P["Wd"]
    lg = X @ Wgate.T + P["dlog"]
    T = X.shape[0]
    L = 0.0
    for t in range(T):
        sel = lg[t, ids[t]]
        e_ = np.exp(sel - sel.max())
        w = e_ / e_.sum()
        y = np.zeros(X.shape[1])
        for p in range(k):
            e = ids[t, p]
            g, u = Wg[e] @ X[t], Wu[e] @ X[t]
            y += w[p] * (Wd[e].T @ (g / (1 + np.exp(-g)) * u))
        for s in range(P["Wg_s"].shape[0]):
            g, u = P["Wg_s"][s] @ X[t], P["Wu_s"][s] @ X[t]
            y += P["Wd_s"][s].T @ (g / (1 + np.exp(-g)) * u)
        L += dY[t] @ y
    return L


def test_bwd_finite_differences(orc):
    T, n, h, E, k, S = 5, 6, 3, 4, 2, 1
    f32 = lambda a: np.asarray(a, np.float32)
    P = dict(X=hpat((T, n), 900), Wgate=hpat((E, n), 901, 1.0), Wg=hpat((E, h, n), 902, 0.6),
             Wu=hpat((E, h, n), 903, 0.6), Wd=hpat((E, h, n), 904, 0.6),
             Wg_s=hpat((S, h, n), 905, 0.6), Wu_s=hpat((S, h, n), 906, 0.6),
             Wd_s=hpat((S, h, n), 907, 0.6))
    dY = hpat((T, n), 908).astype(np.float64)
    P64 = {key: v.astype(np.float64) for key, v in P.items()}
    P64["dlog"] = np.zeros((T, E))
    lg = P64["X"] @ P64["Wgate"].T
    ids = np.argsort(-lg, axis=1, kind="stable")[:, :k]
    srt = -np.sort(-lg, axis=1)
    assert (srt[:, k - 1] - srt[:, k] > 1e-2).all()  # the selection is stable
    # caches of the float64 forward, as the forward would have stored them
    Gsel = np.zeros((T * k, h)); Usel = np.zeros((T * k, h)); Ysel = np.zeros((T * k, n))
    w = np.zeros((T, k))
    for t in range(T):
        sel = lg[t, ids[t]]
        e_ = np.exp(sel - sel.max())
        w[t] = e_ / e_.sum()
        for p in range(k):
            e = ids[t, p]
            g, u = P64["Wg"][e] @ P64["X"][t], P64["Wu"][e] @ P64["X"][t]
            Gsel[t * k + p], Usel[t * k + p] = g, u
            Ysel[t * k + p] = P64["Wd"][e].T @ (g / (1 + np.exp(-g)) * u)
    Gs = np.einsum("shn,tn->tsh", P64["Wg_s"], P64["X"])
    Us = np.einsum("shn,tn->tsh", P64["Wu_s"], P64["X"])
    perm, off, drop = capacity_sort(ids, E, None)
    o = orc.moe_bwd_batch(f32(dY), P["X"], P["Wgate"], P["Wg"], P["Wu"], P["Wd"], P["Wg_s"],
                          P["Wu_s"], P["Wd_s"], ids, f32(w), f32(Gsel), f32(Usel), f32(Ysel),
                          f32(Gs), f32(Us), perm, off, drop, k)
    assert o["rc"] == 0
    grads = dict(X="dX", Wgate="dWgate", Wg="dWg", Wu="dWu", Wd="dWd", Wg_s="dWg_s",
                 Wu_s="dWu_s", Wd_s="dWd_s", dlog="dLogits")
    for key, out in grads.items():
        fd = np.zeros_like(P64[key])
        for i in np.ndindex(fd.shape):
            Q = dict(P64)
            Q[key] = P64[key].copy()
            eps = 1e-5 * max(1.0, abs(Q[key][i]))
            Q[key][i] += eps
            lp = _forward64(Q, ids, dY, k)
            Q[key][i] -= 2 * eps
            lm = _forward64(Q, ids, dY, k)
            fd[i] = (lp - lm) / (2 * eps)
        got = o[out].astype(np.float64)
        tol = 2e-5 * np.abs(fd).max() + 1e-7
        assert np.abs(got - fd).max() <= tol, (key, np.abs(got - fd).max(), tol)


# ------------------------------------------------------------ rejections

def _mutations(c):
    """(name, mutated case) pairs the reference rejects with EINVAL when
    validating (src/moe_layer.c:1766-1880)."""
    def mut(**kw):
        d = dict(c)
        d.update(kw)
        return d
    ids = c["ids"].copy(); ids[1, 0] = 99
    w = c["w"].copy(); w[0, 0] = 1.5
    wn = c["w"].copy(); wn[0, 1] = np.nan
    drop = c["drop"].copy(); drop[0] = 2
    off = c["off"].copy(); off[2], off[3] = off[3], off[2] - 1
    perm = c["perm"].copy(); perm[1] = perm[0]
    X = c["X"].copy(); X[2, 3] = np.inf
    Gsel = c["Gsel"].copy(); Gsel[4, 1] = np.nan
    Wd = c["Wd"].copy(); Wd[0, 0, 0] = np.inf
    return [("ids", mut(ids=ids)), ("w>1", mut(w=w)), ("w nan", mut(w=wn)),
            ("drop", mut(drop=drop)), ("off", mut(off=off)), ("perm dup", mut(perm=perm)),
            ("X inf", mut(X=X)), ("Gsel nan", mut(Gsel=Gsel)), ("Wd inf", mut(Wd=Wd))]


def test_bwd_rejections(orc, request):
    c = bwd_case(12, 16, 8, 4, 2, 1, 40, None)
    ref = None
    try:
        ref = request.getfixturevalue("ref")
    except pytest.skip.Exception:
        pass
    for name, m in _mutations(c):
        o = orc.moe_bwd_batch(*bwd_args(m))
        assert o["rc"] == 2, name
        if ref is not None:
            assert ref.moe_bwd_batch(*bwd_args(m))["rc"] == 2, name
