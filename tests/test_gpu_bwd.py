"""GPU parity of the batched MoE backward (jt_moe_bwd_batch,
jt_moe_bwd_batch_unchecked, jt_hip_moe_bwd_batch) against the reference's
outputs (golden vectors) and the oracle.

Reference behaviour followed: src/moe_layer.c:1684-2502. Outputs that do
not pass through exp (dLogits, dWgate) must match to the bit. The others
go through the SwiGLU backward's sigmoid, whose fp64 exp may differ from
glibc's by an ulp; they must match to the bit in all but a tiny fraction of
elements and within 1e-6 of the array's largest magnitude everywhere (the
reference's own tolerance for these outputs is 1e-6,
bench/kernel/test_moe_layer.c:1384-1398).
"""
import errno
import os

import numpy as np
import pytest

from conftest import announce
from golden.gen import bwd_args, bwd_case

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_vectors.npz")
BWD_RND = (24, 42, 24, 6, 3, 2, 300, 1.0)
OUTS = ("dX", "dWgate", "dWg", "dWu", "dWd", "dWg_s", "dWu_s", "dWd_s", "dLogits")
EXACT = ("dWgate", "dLogits")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def check(out, want, names=OUTS, label=""):
    for nm in names:
        if nm not in want:
            continue
        a, b = np.asarray(out[nm], np.float32), np.asarray(want[nm], np.float32)
        assert a.shape == b.shape, (label, nm)
        if nm in EXACT:
            assert np.array_equal(bits(a), bits(b)), (label, nm)
            continue
        same = bits(a) == bits(b)
        scale = float(np.abs(b).max()) if b.size else 0.0
        err = float(np.abs(a.astype(np.float64) - b).max()) if b.size else 0.0
        assert err <= 1e-6 * scale + 1e-30, (label, nm, err, scale)
        assert same.mean() >= 0.999, (label, nm, int((~same).sum()), same.size)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def gold_args(gold, c):
    pre = f"bwdref{c}_"
    g = lambda k: gold[pre + k] if pre + k in gold.files else None
    return [g("dY"), g("X"), g("Wgate"), g("Wg"), g("Wu"), g("Wd"), g("Wg_s"), g("Wu_s"),
            g("Wd_s"), g("ids"), g("w"), g("Gsel"), g("Usel"), g("Ysel"), g("Gs"), g("Us"),
            g("perm"), g("off"), g("drop"), int(g("k"))]


@pytest.mark.parametrize("c", [0, 1])
def test_bwd_reference_tests_golden(jt, gold, c):
    announce(f"moe_bwd_batch golden case {c}")
    args = gold_args(gold, c)
    want = {nm: gold[f"bwdref{c}_out_{nm}"] for nm in OUTS
            if f"bwdref{c}_out_{nm}" in gold.files}
    for unchecked in (False, True):
        o = jt.moe_bwd_batch(*args, unchecked=unchecked)
        assert o["rc"] == 0
        check(o, want, label=f"case {c}")


def test_bwd_seeded_golden(jt, gold):
    announce("moe_bwd_batch seeded golden")
    o = jt.moe_bwd_batch(*bwd_args(bwd_case(*BWD_RND)))
    assert o["rc"] == 0
    check(o, {nm: gold["bwdrnd_" + nm] for nm in OUTS})


CASES = [(6, 4, 2, 4, 2, 1, 11, 1.25), (16, 32, 16, 8, 2, 1, 12, None),
         (24, 64, 32, 8, 4, 2, 13, 1.0), (40, 36, 20, 16, 3, 0, 14, 1.25),
         (9, 130, 64, 5, 5, 1, 15, None), (33, 17, 9, 7, 1, 3, 16, 1.0),
         (300, 130, 70, 12, 3, 2, 17, 1.0), (256, 256, 128, 16, 4, 1, 18, 1.25),
         (70, 96, 200, 64, 8, 1, 19, None), (1, 64, 64, 8, 2, 1, 20, None)]


@pytest.mark.parametrize("case", CASES)
def test_bwd_vs_oracle(jt, orc, case):
    announce(f"moe_bwd_batch vs oracle {case}")
    c = bwd_case(*case)
    want = orc.moe_bwd_batch(*bwd_args(c))
    assert want["rc"] == 0
    o = jt.moe_bwd_batch(*bwd_args(c))
    assert o["rc"] == 0
    check(o, want, label=str(case))
    u = jt.moe_bwd_batch(*bwd_args(c), unchecked=True)
    assert u["rc"] == 0
    for nm in OUTS:  # same kernels: the same bits, and deterministic
        if nm in o:
            assert np.array_equal(bits(u[nm]), bits(o[nm])), nm


def test_bwd_without_logits(jt, orc):
    announce("moe_bwd_batch dLogits NULL")
    c = bwd_case(20, 40, 24, 6, 2, 1, 31, 1.0)
    o = jt.moe_bwd_batch(*bwd_args(c), logits=False)
    assert o["rc"] == 0 and "dLogits" not in o
    check(o, orc.moe_bwd_batch(*bwd_args(c)), names=OUTS[:-1])


def _mutations(c):
    def mut(**kw):
        d = dict(c)
        d.update(kw)
        return d
    ids = c["ids"].copy(); ids[1, 0] = 99
    w = c["w"].copy(); w[0, 0] = 1.5
    drop = c["drop"].copy(); drop[0] = 2
    off = c["off"].copy(); off[2], off[3] = off[3], off[2] - 1
    perm = c["perm"].copy(); perm[1] = perm[0]
    perm_oob = c["perm"].copy(); perm_oob[0] = 10 ** 6
    off_big = c["off"].copy(); off_big[-1] += 1
    X = c["X"].copy(); X[2, 3] = np.inf
    Gsel = c["Gsel"].copy(); Gsel[4, 1] = np.nan
    Wd = c["Wd"].copy(); Wd[0, 0, 0] = np.inf
    checked = [("w>1", mut(w=w)), ("drop", mut(drop=drop)), ("X inf", mut(X=X)),
               ("Gsel nan", mut(Gsel=Gsel)), ("Wd inf", mut(Wd=Wd))]
    both = [("ids", mut(ids=ids)), ("off", mut(off=off)), ("perm dup", mut(perm=perm)),
            ("perm oob", mut(perm=perm_oob)), ("off[E] > T*k", mut(off=off_big))]
    return checked, both


def test_bwd_rejections_leave_outputs(jt):
    c = bwd_case(12, 16, 8, 4, 2, 1, 40, None)
    checked, both = _mutations(c)
    for unchecked, cases in ((False, checked + both), (True, both)):
        for name, m in cases:
            announce(f"moe_bwd_batch rejects {name} unchecked={unchecked}")
            o = jt.moe_bwd_batch(*bwd_args(m), unchecked=unchecked)
            assert o["rc"] == jt.JT_ERR_INVAL and jt.errno() == errno.EINVAL, name
            for nm in OUTS:  # fail-closed: nothing written
                if nm in o:
                    assert np.isnan(o[nm]).all(), (name, nm)
    # the unchecked form skips the finiteness scans (the reference's too)
    X = c["X"].copy()
    X[0, 0] = np.inf
    assert jt.moe_bwd_batch(*bwd_args(dict(c, X=X)))["rc"] == jt.JT_ERR_INVAL
    assert jt.moe_bwd_batch(*bwd_args(dict(c, X=X)), unchecked=True)["rc"] == 0


def test_bwd_after_device_forward(jt, orc):
    announce("moe_fwd_batch -> moe_bwd_batch on device caches")
    rng = np.random.default_rng(77)
    T, n, h, E, k, S = 48, 64, 32, 8, 2, 1
    X = rng.standard_normal((T, n)).astype(np.float32)
    Wgate = (rng.standard_normal((E, n)) / 8).astype(np.float32)
    W = [(rng.standard_normal((E, h, n)) / 8).astype(np.float32) for _ in range(3)]
    Ws = [(rng.standard_normal((S, h, n)) / 8).astype(np.float32) for _ in range(3)]
    f = jt.moe_fwd_batch(X, Wgate, *W, *Ws, k, 1.0, caches=True)
    assert f["rc"] == 0 and f["drop"].any()
    dY = rng.standard_normal((T, n)).astype(np.float32)
    args = [dY, X, Wgate, *W, *Ws, f["ids"], f["w"], f["Gsel"], f["Usel"], f["Ysel"],
            f["Gs"], f["Us"], f["perm"], f["off"], f["drop"], k]
    o = jt.moe_bwd_batch(*args)
    assert o["rc"] == 0
    check(o, orc.moe_bwd_batch(*args))


def _dev(torch, c):
    d = {}
    for key, v in c.items():
        if v is None or key == "k":
            d[key] = v
        elif v.dtype == np.uint8:
            d[key] = torch.from_numpy(np.ascontiguousarray(v)).cuda()
        elif v.dtype.kind in "iu":
            d[key] = torch.from_numpy(np.ascontiguousarray(v, np.int64)).cuda()
        else:
            d[key] = torch.from_numpy(np.ascontiguousarray(v, np.float32)).cuda()
    return d


def test_bwd_device_entry_matches_host_entry(jt, torch_cuda):
    torch = torch_cuda
    announce("jt_hip_moe_bwd_batch vs jt_moe_bwd_batch")
    c = bwd_case(200, 96, 64, 12, 4, 2, 50, 1.25)
    host = jt.moe_bwd_batch(*bwd_args(c))
    assert host["rc"] == 0
    d = _dev(torch, c)
    rc, out, ws = jt.moe_bwd_batch_device(*bwd_args(d))
    assert rc == 0 and jt.sync_errors() == 0
    for nm in OUTS:
        assert np.array_equal(bits(out[nm].cpu().numpy()), bits(host[nm])), nm
    # a second call reusing outputs and workspace, on a bad permutation
    d2 = dict(d)
    p = c["perm"].copy()
    p[3] = p[2]
    d2["perm"] = torch.from_numpy(p).cuda()
    rc, out, _ = jt.moe_bwd_batch_device(*bwd_args(d2), out=out, ws=ws)
    assert rc == 0 and jt.sync_errors() & jt.EF_BAD_ID


@pytest.mark.parametrize("shape", [(512, 64, 32, 8, 2, 1), (4096, 1024, 256, 64, 8, 1)])
def test_bwd_full_size_linearity(jt, torch_cuda, shape):
    """At the benchmark shapes: every output is linear in dY, and scaling
    by 2 is exact in binary floating point, so bwd(2 dY) must equal
    2 bwd(dY) to the bit; dLogits and dWgate rows are also checked against
    a float64 recomputation of a few tokens."""
    torch = torch_cuda
    T, n, h, E, k, S = shape
    announce(f"jt_hip_moe_bwd_batch linearity T={T} n={n} h={h} E={E} k={k} S={S}")
    c = bwd_case(T, n, h, E, k, S, 60, 1.25)
    d = _dev(torch, c)
    rc, o1, ws = jt.moe_bwd_batch_device(*bwd_args(d))
    assert rc == 0 and jt.sync_errors() == 0
    o1 = {nm: v.cpu().numpy() for nm, v in o1.items()}
    d2 = dict(d, dY=d["dY"] * 2)
    rc, o2, _ = jt.moe_bwd_batch_device(*bwd_args(d2), ws=ws)
    assert rc == 0 and jt.sync_errors() == 0
    for nm, v in o2.items():
        assert np.array_equal(bits(v.cpu().numpy()), bits(2 * o1[nm])), nm
    assert np.abs(o1["dWg"]).max() > 0 and np.isfinite(o1["dX"]).all()
    # dLogits of sampled tokens from the float64 restatement of
    # src/moe_layer.c:1985-2047 (lane-4 dots change only the last bits)
    ids, w, drop = c["ids"], c["w"].astype(np.float64), c["drop"].reshape(T, k)
    for t in (0, T // 2, T - 1):
        dw = np.array([0.0 if drop[t, p] else
                       c["Ysel"][t * k + p].astype(np.float64) @ c["dY"][t].astype(np.float64)
                       for p in range(k)])
        s = (w[t] * dw * (drop[t] == 0)).sum()
        for p in range(k):
            want = 0.0 if drop[t, p] else w[t, p] * (dw[p] - s)
            got = o1["dLogits"][t, ids[t, p]]
            assert abs(got - want) <= 1e-5 * (abs(want) + np.abs(w[t] * dw).max()), (t, p)
