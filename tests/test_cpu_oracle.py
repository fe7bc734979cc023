"""CPU checks that pin the oracle (no GPU).

Each oracle function is pinned by at least one of:
  * golden vectors written by the reference's own functions
    (tests/golden/ref_vectors.npz, made by tests/golden/make_golden.py from
    the reference sources compiled into oracle/_ref);
  * the known answers of the reference's tests
    (bench/kernel/test_routing.c, test_moe_layer.c, test_w8a8.c,
    test_lowbit.c);
  * closed forms and brute force that a plausible slip (dropped term, wrong
    sign, transposed operand, off-by-one index) would fail;
  * a live comparison with oracle/_ref when it has been built (skipped
    otherwise).
"""
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_vectors.npz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


# ---------------------------------------------------------------- golden

def test_golden_quant(orc, gold):
    rc, Q, s = orc.quant_rows(gold["quant_rows_X"])
    assert rc == 0
    assert np.array_equal(Q, gold["quant_rows_Q"])
    assert np.array_equal(bits(s), bits(gold["quant_rows_s"]))
    rc, q, s1 = orc.quant_tensor(gold["quant_tensor_x"])
    assert rc == 0 and np.array_equal(q, gold["quant_tensor_q"])
    assert bits(np.float32(s1)) == bits(gold["quant_tensor_s"])
    rc, F = orc.fakequant_rows(gold["quant_rows_X"])
    assert rc == 0 and np.array_equal(bits(F), bits(gold["fakequant_rows"]))
    rc, D = orc.dequant_rows(gold["quant_rows_Q"], gold["quant_rows_s"])
    assert rc == 0 and np.array_equal(bits(D), bits(gold["dequant_rows"]))


def test_golden_gemm(orc, gold):
    A, B = gold["gemm_pc_A"], gold["gemm_pc_B"]
    rc, C, acc = orc.w8a8_gemm(A, gold["gemm_pc_sA"], B, gold["gemm_pc_sB"])
    assert rc == 0 and np.array_equal(bits(C), bits(gold["gemm_pc_C"]))
    rc, C, _ = orc.w8a8_gemm(A, gold["gemm_pt_sA"], B, gold["gemm_pt_sB"])
    assert rc == 0 and np.array_equal(bits(C), bits(gold["gemm_pt_C"]))
    C = orc.gemm_f32(gold["gemm_f32_A"], gold["gemm_f32_B"])
    assert np.array_equal(bits(C), bits(gold["gemm_f32_C"]))


@pytest.mark.parametrize("b", [2, 4])
def test_golden_lowbit(orc, gold, b):
    rc, fq = orc.lowbit_fakequant(gold[f"fq{b}_w"], b)
    assert rc == 0 and np.array_equal(bits(fq), bits(gold[f"fq{b}_out"]))
    rc, idx, ws = orc.col_to_idx(gold[f"c2i{b}_col"], b)
    assert rc == 0 and np.array_equal(idx, gold[f"c2i{b}_idx"])
    assert bits(np.float32(ws)) == bits(gold[f"c2i{b}_ws"])
    rc, Y = orc.lowbit_gemm_lut(gold[f"lut{b}_X"], gold[f"lut{b}_W"], b)
    assert rc == 0 and np.array_equal(bits(Y), bits(gold[f"lut{b}_Y"]))


def test_golden_tmac(orc, gold):
    rc, ql, sc, bi = orc.tmac_lut_ctor(gold["tmac_act"])
    assert rc == 0
    assert np.array_equal(ql, gold["tmac_qlut"])
    assert np.array_equal(bits(sc), bits(gold["tmac_scales"]))
    assert np.array_equal(bits(bi), bits(gold["tmac_biases"]))
    outs = []
    for b in (2, 4):
        _, idx, ws = orc.col_to_idx(gold["tmac_col"], b)
        for r in range(3):
            rc, o = orc.tmac_lookup_accum(ql[r].ravel(), idx, sc[r], bi[r], b, ws)
            assert rc == 0
            outs.append(o)
    assert np.array_equal(bits(np.array(outs, np.float32)), bits(gold["tmac_out"]))


def test_golden_topk(orc, gold):
    L = gold["topk_logits"]
    for t in range(L.shape[0]):
        rc, ids, w = orc.topk(L[t], 8)
        assert rc == 0
        assert np.array_equal(ids, gold["topk_ids"][t])
        assert np.array_equal(bits(w), bits(gold["topk_w"][t]))


@pytest.mark.parametrize("tag,cap", [("c10", 1.0), ("c15", 1.5)])
def test_golden_sort(orc, gold, tag, cap):
    ids = gold["sort_ids"]
    rc, perm, off, drop = orc.batch_sort(ids, 64, 8, 32, cap)
    assert rc == 0
    assert np.array_equal(perm, gold[f"sort_{tag}_perm"])
    assert np.array_equal(off, gold[f"sort_{tag}_off"])
    assert np.array_equal(drop, gold[f"sort_{tag}_drop"])


@pytest.mark.parametrize("f,w8,lb", [(0, 0, 0), (1, 1, 0), (2, 0, 1)])
def test_golden_layer(orc, gold, f, w8, lb):
    g = {k[6:]: gold[k] for k in gold.files if k.startswith("layer_")}
    r = orc.moe_fwd_batch(g["X"], g["Wgate"], g["Wg"], g["Wu"], g["Wd"], g["Wgs"],
                          g["Wus"], g["Wds"], 2, 1.5, w8, lb)
    assert r["rc"] == 0
    assert np.array_equal(r["ids"], gold[f"layer{f}_ids"])
    assert np.array_equal(bits(r["w"]), bits(gold[f"layer{f}_w"]))
    assert np.array_equal(r["perm"], gold[f"layer{f}_perm"])
    assert np.array_equal(r["off"], gold[f"layer{f}_off"])
    assert np.array_equal(r["drop"], gold[f"layer{f}_drop"])
    assert np.array_equal(bits(r["Y"]), bits(gold[f"layer{f}_Y"]))


def test_golden_logits(orc, gold):
    X, W = gold["logits_X"], gold["logits_Wgate"]
    got = np.array([[orc.logit_lane4(X[t], W[e]) for e in range(W.shape[0])]
                    for t in range(X.shape[0])], np.float32)
    assert np.array_equal(bits(got), bits(gold["logits_out"]))
    Wa = gold["logits_adv_W"]
    ones = np.ones(Wa.shape[1], np.float32)
    adv = np.array([orc.logit_lane4(ones, Wa[e]) for e in range(Wa.shape[0])], np.float32)
    assert np.array_equal(bits(adv), bits(gold["logits_adv_out"]))
    # the sequential sum gives other values for these rows: the lane order is pinned
    seq = np.array([np.float32(sum(float(v) for v in Wa[e])) for e in range(Wa.shape[0])])
    assert not np.array_equal(seq, gold["logits_adv_out"])


# ------------------------------------------- the reference tests' answers

def test_known_topk(orc):
    """bench/kernel/test_routing.c:29-66, 152-188."""
    lg = [0.1, 2.0, 0.5, 3.0, 1.0]
    rc, ids, w = orc.topk(lg, 2)
    assert rc == 0 and list(ids) == [3, 1]
    assert abs(w[0] - 0.7310586) <= 1e-5 and abs(w[1] - 0.2689414) <= 1e-5
    rc, ids, w = orc.topk(lg, 1)
    assert list(ids) == [3] and abs(w[0] - 1.0) <= 1e-6
    rc, ids, w = orc.topk(lg, 5)
    assert list(ids) == [3, 1, 4, 2, 0] and abs(w.sum() - 1.0) <= 1e-6
    rc, ids, w = orc.topk([1.0, 1.0, 1.0], 2)
    assert list(ids) == [0, 1] and np.allclose(w, 0.5, atol=1e-6)
    rc, ids, _ = orc.topk([2.0, 1.0, -np.inf, -np.inf], 2)
    assert rc == 0 and list(ids) == [0, 1]
    assert orc.topk([1.0, np.nan, 0.5, 0.25], 2)[0] == 2
    assert orc.topk([np.inf, 1.0, 0.0], 2)[0] == 2
    rc, ids, w = orc.topk((np.arange(512) % 64).astype(np.float32), 8)
    assert ids[0] == 63 and ids[7] == 511 and abs(w[0] - 0.125) <= 1e-6
    rc, ids, w = orc.topk((np.arange(4096) % 256).astype(np.float32), 16)
    assert ids[0] == 255 and ids[15] == 4095 and abs(w.astype(np.float64).sum() - 1) < 1e-5


def test_known_sort(orc):
    """bench/kernel/test_moe_layer.c:668-728."""
    rc, perm, off, drop = orc.batch_sort([2, 0, 1, 2, 0, 1, 2, 1], 4, 2, 3, 1.0)
    assert rc == 0
    assert list(perm) == [1, 4, 2, 5, 7, 0, 3, 6] and list(off) == [0, 2, 5, 8]
    assert not drop.any()
    rc, perm, off, drop = orc.batch_sort([0, 0, 0, 0, 0, 1, 1, 1], 4, 2, 2, 1.0)
    assert list(perm) == [0, 1, 2, 3, 5, 6, 7] and list(off) == [0, 4, 7]
    assert list(drop) == [0, 0, 0, 0, 1, 0, 0, 0]


def test_known_layer_single_token(orc):
    """jt_moe_fwd known answer, bench/kernel/test_moe_layer.c:146-189, through
    the batched layer at T=1 (batch equals single within 1e-6, :836-855)."""
    X = np.array([[1.0, 0.5]], np.float32)
    Wgate = np.array([1, 0, 0, 1, -1, 0], np.float32).reshape(3, 2)
    Wg = np.array([0.5, -0.5, 0.5, 1.0, 0, 0], np.float32).reshape(3, 1, 2)
    Wu = np.array([1.0, 0, 0.5, -0.5, 0, 0], np.float32).reshape(3, 1, 2)
    Wd = np.array([1.0, 2.0, -1.0, 0.5, 0, 0], np.float32).reshape(3, 1, 2)
    Wgs = np.array([0.5, 0.5], np.float32).reshape(1, 1, 2)
    Wus = np.array([1.0, -1.0], np.float32).reshape(1, 1, 2)
    Wds = np.array([0.5, -0.5], np.float32).reshape(1, 1, 2)
    r = orc.moe_fwd_batch(X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, 2, 1.5)
    assert r["rc"] == 0 and list(r["ids"][0]) == [0, 1]
    assert abs(r["w"][0, 0] - 0.6224593312018546) < 1e-5
    assert abs(r["w"][0, 1] - 0.37754066879814546) < 1e-5
    assert abs(r["Y"][0, 0] - 0.14582792210843093) < 1e-5
    assert abs(r["Y"][0, 1] - 0.08212054137232436) < 1e-5


def test_known_quant_and_lowbit(orc):
    """test_w8a8.c:78-85 (zero row), test_lowbit.c:78-98 (odd grid), :215-221."""
    rc, q, s = orc.quant_tensor(np.zeros(4, np.float32))
    assert rc == 0 and s == 1.0 and not q.any()
    assert orc.quant_tensor(np.array([0.1, 0.2, np.nan, 0.4], np.float32))[0] == 2
    rng = np.random.default_rng(5)
    w = rng.standard_normal(4096).astype(np.float32)
    maxa = np.abs(w.astype(np.float64)).max()
    for b in (2, 4):
        nl = (1 << b) - 1
        rc, fq = orc.lowbit_fakequant(w, b)
        t = fq.astype(np.float64) / maxa * nl
        r = np.round(t)
        assert np.all(np.abs(t - r) < 1e-3)
        assert np.all(np.abs(r) <= nl) and np.all(r.astype(np.int64) % 2 != 0)
    # the test's smooth pattern lpat(i, 3, 7) * (1 + (i % 5) / 10), N = 256
    i = np.arange(256)
    wp = (((i * 31 + 3 * 17 + 7 * 13) % 11 - 5) / np.float32(5.0)).astype(np.float32)
    wp = (wp * (np.float32(1.0) + (i % 5).astype(np.float32) * np.float32(0.1))).astype(
        np.float32)
    mae2 = np.abs(wp.astype(np.float64) - orc.lowbit_fakequant(wp, 2)[1]).mean()
    mae4 = np.abs(wp.astype(np.float64) - orc.lowbit_fakequant(wp, 4)[1]).mean()
    assert mae4 < mae2 and mae4 < 0.10 and mae2 < 0.35
    rc, idx, ws = orc.col_to_idx(np.arange(1, 9, dtype=np.float32), 4)
    assert rc == 0 and ws == 8.0


# ------------------------------------------ closed forms and brute force

def _round_half_away(y):
    t = np.trunc(y)
    return np.where(np.abs(y - t) >= 0.5, t + np.sign(y), t)


def test_quant_closed_form(orc):
    rng = np.random.default_rng(7)
    X = (rng.standard_normal((50, 333)) * rng.uniform(1e-3, 1e3, (50, 1))).astype(np.float32)
    X[7] = 0
    rc, Q, s = orc.quant_rows(X)
    mx = np.abs(X.astype(np.float64)).max(axis=1)
    sd = mx / 127.0
    s_ref = np.where(mx == 0, 1.0, sd).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q_ref = np.clip(_round_half_away(X.astype(np.float64) / sd[:, None]), -127, 127)
    q_ref[mx == 0] = 0
    assert np.array_equal(bits(s), bits(s_ref))
    assert np.array_equal(Q, q_ref.astype(np.int8))
    # dequant / fakequant are (float)((double)q * scale)
    rc, D = orc.dequant_rows(Q, s)
    assert np.array_equal(bits(D), bits((Q * s[:, None].astype(np.float64)).astype(np.float32)))
    # fake-quant multiplies by the unrounded fp64 scale (src/w8a8.c:1074-1200)
    rc, F = orc.fakequant_rows(X)
    with np.errstate(invalid="ignore"):
        F_ref = (q_ref * sd[:, None]).astype(np.float32)
    F_ref[mx == 0] = 0
    assert np.array_equal(bits(F), bits(F_ref))


def test_gemm_closed_form(orc):
    rng = np.random.default_rng(8)
    M, N, K = 17, 29, 200
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    sA = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    sB = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    rc, C, acc = orc.w8a8_gemm(A, sA, B, sB)
    acc_ref = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(acc, acc_ref)
    C_ref = (acc_ref * (sA.astype(np.float64)[:, None] * sB.astype(np.float64)[None, :]))
    assert np.array_equal(bits(C), bits(C_ref.astype(np.float32)))
    # transposed operand or swapped scales must not pass
    assert not np.array_equal(acc, (A.astype(np.int64) @ B.astype(np.int64)[:, ::-1]))


def test_f16_conversion(orc):
    rng = np.random.default_rng(9)
    v = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 6, 4000),
                        [0.0, -0.0, 65504.0, 65520.0, 7e4, 2.0 ** -24, 2.0 ** -25,
                         3 * 2.0 ** -26, 6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16)
    for x, w in zip(v, want):
        h = orc.f64_to_f16(x)
        assert h == int(w.view(np.uint16)), x
        assert orc.lib.or_f16_to_f64(h) == float(w)


def test_lowbit_pack_closed_form(orc):
    rng = np.random.default_rng(10)
    N, K, G = 24, 256, 64
    W = rng.standard_normal((N, K)).astype(np.float32)
    for b in (2, 4):
        nl = (1 << b) - 1
        rc, codes, scales = orc.lowbit_pack_rows(W, b, G)
        assert rc == 0
        Wg = W.astype(np.float64).reshape(N, K // G, G)
        mx = np.abs(Wg).max(axis=2)
        li = np.floor(Wg / mx[:, :, None] * nl / 2 + nl / 2 + 0.5).clip(0, nl)
        assert np.array_equal(codes, li.reshape(N, K).astype(np.uint8))
        assert np.array_equal(scales, (mx / nl).astype(np.float16).view(np.uint16))
        # with one group spanning K the codes equal the reference's col_to_idx levels
        rc, c1, _ = orc.lowbit_pack_rows(W[:, :64], b, 64)
        for n in range(4):
            _, fq = orc.lowbit_fakequant(W[n, :64], b)
            m = np.abs(W[n, :64].astype(np.float64)).max()
            lv = np.round(fq.astype(np.float64) / m * nl)
            assert np.array_equal((lv + nl) / 2, c1[n].astype(np.float64))


def test_gemm_lowbit_group_brute_force(orc):
    """Power-of-two scales make every product and sum exact in fp32, so the
    brute-force integer sum is the answer to the bit."""
    rng = np.random.default_rng(11)
    M, N, K, G = 9, 20, 192, 64
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    sA = (2.0 ** rng.integers(-8, -2, M)).astype(np.float32)
    for b in (2, 4):
        nl = (1 << b) - 1
        codes = rng.integers(0, nl + 1, (N, K), dtype=np.uint8)
        e = rng.integers(-10, -4, (N, K // G))
        scales = (2.0 ** e).astype(np.float16).view(np.uint16)
        rc, out, acc = orc.gemm_lowbit_group(A, sA, codes, scales, b, G)
        assert rc == 0
        val = 2 * codes.astype(np.int64) - nl
        accr = np.einsum("mgk,ngk->mng", A.astype(np.int64).reshape(M, K // G, G),
                         val.reshape(N, K // G, G))
        assert np.array_equal(acc, accr)
        ref = (accr * (2.0 ** e)[None]).sum(axis=2) * sA.astype(np.float64)[:, None]
        assert np.array_equal(bits(out), bits(ref.astype(np.float32)))


def test_topk_brute_force(orc):
    rng = np.random.default_rng(12)
    for t in range(200):
        n = int(rng.integers(2, 300))
        k = int(rng.integers(1, min(n, 16) + 1))
        lg = np.round(rng.standard_normal(n) * 4) / 4  # many ties
        lg = lg.astype(np.float32)
        rc, ids, w = orc.topk(lg, k)
        order = sorted(range(n), key=lambda i: (-float(lg[i]), i))[:k]
        assert rc == 0 and list(ids) == order
        e = np.exp(lg[order].astype(np.float64) - float(lg[order[0]]))
        assert np.allclose(w, (e / e.sum()), rtol=2e-7, atol=1e-7)


def test_router_composition(orc, gold):
    """or_router = or_logit_lane4 per (token, expert) then or_topk per token,
    on the golden logit vectors (whose logits are pinned above) and on a
    tie-heavy case; a non-finite logit is an error."""
    X, W = gold["logits_X"], gold["logits_Wgate"]
    k = min(4, W.shape[0])
    rc, ids, w, lg = orc.router(X, W, k)
    assert rc == 0 and np.array_equal(bits(lg), bits(gold["logits_out"]))
    for t in range(X.shape[0]):
        rc2, ids2, w2 = orc.topk(gold["logits_out"][t], k)
        assert rc2 == 0 and np.array_equal(ids[t], ids2) and np.array_equal(bits(w[t]), bits(w2))
    rng = np.random.default_rng(14)
    Wt = np.round(rng.standard_normal((24, 8)) * 2).astype(np.float32)
    Wt[7] = Wt[3]
    Xt = np.round(rng.standard_normal((30, 8)) * 2).astype(np.float32)
    Xt[0] = 0.0
    rc, ids, w, lg = orc.router(Xt, Wt, 5)
    assert rc == 0
    for t in range(30):
        ref = (Xt[t].astype(np.float64) * Wt.astype(np.float64)).sum(axis=1)  # exact: small integers
        order = sorted(range(24), key=lambda e: (-ref[e], e))[:5]
        assert list(ids[t]) == order
    assert list(ids[0]) == [0, 1, 2, 3, 4]
    Xbad = Xt.copy()
    Xbad[3, 2] = np.inf
    assert orc.router(Xbad, Wt, 5)[0] != 0


def test_sort_invariants(orc):
    rng = np.random.default_rng(13)
    T, k, E = 300, 6, 40
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    for cap in (0.0, 1.0, 1.3):
        rc, perm, off, drop = orc.batch_sort(ids, T, k, E, cap)
        assert rc == 0
        flat = ids.ravel()
        assert off[0] == 0 and off[-1] == perm.size and np.all(np.diff(off) >= 0)
        for e in range(E):
            seg = perm[off[e]:off[e + 1]]
            assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)  # stable
        kept = np.zeros(T * k, bool)
        kept[perm] = True
        assert np.array_equal(~kept, drop.astype(bool))
        if cap <= 0:
            assert perm.size == T * k  # dropless
        else:
            c = math.ceil(cap * T * k / E)
            assert np.all(np.diff(off) <= c)


def test_silu_formula(orc):
    rng = np.random.default_rng(14)
    g = (rng.standard_normal(2000) * 6).astype(np.float32)
    u = rng.standard_normal(2000).astype(np.float32)
    for gi, ui in zip(g, u):
        rc, s = orc.silu_mul(gi, ui)
        gd = float(gi)
        ref = np.float32((gd * (1.0 / (1.0 + math.exp(-gd)))) * float(ui))
        assert rc == 0 and np.float32(s) == ref


def test_moe_q_composition(orc):
    """The prepared quantised layer equals the composition of its pinned
    parts: per-token int8 activations, group-64 low-bit GEMMs, fp64 SwiGLU,
    re-quantisation, fp64 combine in slot order, shared W8A8 experts."""
    rng = np.random.default_rng(15)
    T, n, h, E, k, S, hs = 10, 128, 64, 8, 3, 1, 96
    Wgate = (rng.standard_normal((E, n)) / 11).astype(np.float32)
    Wg = (rng.standard_normal((E, h, n)) / 11).astype(np.float32)
    Wu = (rng.standard_normal((E, h, n)) / 11).astype(np.float32)
    Wd = (rng.standard_normal((E, h, n)) / 8).astype(np.float32)
    Wgs = (rng.standard_normal((S, hs, n)) / 11).astype(np.float32)
    Wus = (rng.standard_normal((S, hs, n)) / 11).astype(np.float32)
    Wds = (rng.standard_normal((S, hs, n)) / 10).astype(np.float32)
    L = orc.moe_q(n, h, E, k, S, hs, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds)
    X = rng.standard_normal((T, n)).astype(np.float32)
    r = L.fwd(X)
    assert r["rc"] == 0
    # routing = reference top-k on the lane-ordered logits
    for t in range(T):
        lg = np.array([orc.logit_lane4(X[t], Wgate[e]) for e in range(E)], np.float32)
        _, ids, w = orc.topk(lg, k)
        assert np.array_equal(r["ids"][t], ids) and np.array_equal(bits(r["w"][t]), bits(w))
    _, Xq, sx = orc.quant_rows(X)
    Y = np.zeros((T, n), np.float64)
    for t in range(T):
        for p in range(k):
            e = int(r["ids"][t, p])
            gu, gus, dc, ds = L.routed_codes(e)
            _, g, _ = orc.gemm_lowbit_group(Xq[t:t + 1], sx[t:t + 1], gu[0], gus[0], 2)
            _, u, _ = orc.gemm_lowbit_group(Xq[t:t + 1], sx[t:t + 1], gu[1], gus[1], 2)
            s = np.array([[orc.silu_mul(a, b)[1] for a, b in zip(g[0], u[0])]], np.float32)
            _, sq, ss = orc.quant_rows(s)
            _, ye, _ = orc.gemm_lowbit_group(sq, ss, dc, ds, 4)
            Y[t] += float(r["w"][t, p]) * ye[0].astype(np.float64)
    for e in range(S):
        _, ys = orc.ffn_fwd(Wgs[e], Wus[e], Wds[e], X)
        Y += ys.astype(np.float64)
    assert np.array_equal(bits(r["Y"]), bits(Y.astype(np.float32)))


# ----------------------------------------- live comparison with the reference

def test_live_vs_reference(orc, ref):
    rng = np.random.default_rng(16)
    X = (rng.standard_normal((40, 515)) * 3).astype(np.float32)
    a, b = orc.quant_rows(X), ref.quant_rows(X)
    assert a[0] == b[0] == 0 and np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])
    A = rng.integers(-127, 128, (30, 300), dtype=np.int8)
    B = rng.integers(-127, 128, (300, 70), dtype=np.int8)
    sB = rng.uniform(1e-3, 1e-2, 70).astype(np.float32)
    _, C1, _ = orc.w8a8_gemm(A, 0.02, B, sB)
    _, C2 = ref.gemm_per_channel(A, B, 0.02, sB)
    assert np.array_equal(bits(C1), bits(C2))
    for b_ in (2, 4):
        Xl = rng.standard_normal((7, 128)).astype(np.float32)
        Wl = rng.standard_normal((128, 40)).astype(np.float32)
        assert np.array_equal(bits(orc.lowbit_gemm_lut(Xl, Wl, b_)[1]),
                              bits(ref.lowbit_gemm_lut(Xl, Wl, b_)[1]))
    T, n, h, E, k, S = 24, 128, 64, 16, 4, 2
    args = [rng.standard_normal((T, n)).astype(np.float32)] + [
        (rng.standard_normal(s) / 9).astype(np.float32)
        for s in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    for w8, lb in ((0, 0), (1, 0), (0, 1), (1, 1), (0, 2)):
        r1 = orc.moe_fwd_batch(*args, k, 1.25, w8, lb)
        r2 = ref.moe_fwd_batch(*args, k, 1.25, w8, lb)
        assert r1["rc"] == r2["rc"] == 0
        for key in ("ids", "perm", "off", "drop"):
            assert np.array_equal(r1[key], r2[key]), key
        assert np.array_equal(bits(r1["Y"]), bits(r2["Y"]))


# ------------------------------ the shared expert, rebuilt from pinned parts

def _np_quant_rows(X):
    """Closed form of the row quantiser (pinned by test_quant_closed_form and
    the golden quant_rows vectors): fp64 max|x|/127, round half away from
    zero, clamp +-127; a zero row gets scale 1 and codes 0."""
    X64 = np.asarray(X, np.float32).astype(np.float64)
    mx = np.abs(X64).max(axis=1)
    sd = np.where(mx == 0, 1.0, mx / 127.0)
    q = np.clip(_round_half_away(X64 / sd[:, None]), -127, 127)
    q[mx == 0] = 0
    return q.astype(np.int64), np.where(mx == 0, 1.0, mx / 127.0).astype(np.float32)


def _np_epilogue(acc, sa, sw):
    """W8A8 epilogue (float)((double)acc * ((double)sA * (double)sB))."""
    return (acc.astype(np.float64) * (np.float64(sa) * sw.astype(np.float64))).astype(np.float32)


def _np_silu_mul(g, u):
    """SwiGLU of the reference, fp64 with glibc exp (math.exp), one value at
    a time: (float)((g * (1 / (1 + exp(-g)))) * u)."""
    out = np.empty(g.shape, np.float32)
    for i, (gi, ui) in enumerate(zip(g.tolist(), u.tolist())):
        out[i] = np.float32((gi * (1.0 / (1.0 + math.exp(-gi)))) * ui)
    return out


def _np_ffn(Wg, Wu, Wd, X, swap_gu=False, wd_untransposed=False, wd_per_tensor=False):
    """One W8A8 SwiGLU expert from the pinned pieces: per-token codes of X,
    int8 gate/up rows of Wg/Wu [h][n] (one scale per hidden channel),
    integer dots, the W8A8 epilogue, SwiGLU, requantised hidden row, and the
    down projection with Wd [h][n] read as B[K = h][N = n] (output channel j
    is column j, quantised over its h values). The keyword switches plant
    the slips a restatement could make."""
    gq, gs = _np_quant_rows(Wg)
    uq, us = _np_quant_rows(Wu)
    if swap_gu:
        gq, gs, uq, us = uq, us, gq, gs
    Wdn = Wd if wd_untransposed else np.ascontiguousarray(Wd.T)   # [n][h]
    if wd_per_tensor:
        dq, ds1 = _np_quant_rows(Wdn.reshape(1, -1))
        dq, ds = dq.reshape(Wdn.shape), np.full(Wdn.shape[0], ds1[0], np.float32)
    else:
        dq, ds = _np_quant_rows(Wdn)
    xq, xs = _np_quant_rows(X)
    Y = np.zeros((X.shape[0], Wdn.shape[0]), np.float32)
    for t in range(X.shape[0]):
        g = _np_epilogue(gq @ xq[t], xs[t], gs)
        u = _np_epilogue(uq @ xq[t], xs[t], us)
        s = _np_silu_mul(g, u)
        sq, ss = _np_quant_rows(s[None, :])
        Y[t] = _np_epilogue(dq @ sq[0], ss[0], ds)
    return Y


def test_shared_expert_rebuilt_from_pinned_parts(orc):
    """or_ffn_fwd (the shared experts of the prepared layer) equals the
    composition of pinned pieces to the bit, and each planted slip (gate and
    up swapped, Wd not transposed, a per-tensor down scale) is caught."""
    n, h, T = 64, 64, 6   # square Wd, so an untransposed read still has the right shape
    rng = np.random.default_rng(31)
    Wg = (rng.standard_normal((h, n)) / 8).astype(np.float32)
    Wu = (rng.standard_normal((h, n)) / 8).astype(np.float32)
    Wd = (rng.standard_normal((h, n)) / 8).astype(np.float32)
    X = rng.standard_normal((T, n)).astype(np.float32)
    X[2] = 0.0
    rc, Y = orc.ffn_fwd(Wg, Wu, Wd, X)
    assert rc == 0
    assert np.array_equal(bits(Y), bits(_np_ffn(Wg, Wu, Wd, X)))
    for slip in ("swap_gu", "wd_untransposed", "wd_per_tensor"):
        assert not np.array_equal(bits(Y), bits(_np_ffn(Wg, Wu, Wd, X, **{slip: True}))), slip
    # a rectangular expert (h != n)
    n, h = 128, 96
    Wg = (rng.standard_normal((h, n)) / 11).astype(np.float32)
    Wu = (rng.standard_normal((h, n)) / 11).astype(np.float32)
    Wd = (rng.standard_normal((h, n)) / 10).astype(np.float32)
    X = rng.standard_normal((3, n)).astype(np.float32)
    rc, Y = orc.ffn_fwd(Wg, Wu, Wd, X)
    assert rc == 0 and np.array_equal(bits(Y), bits(_np_ffn(Wg, Wu, Wd, X)))


def test_shared_expert_vs_reference_w8a8_layer(orc, gold):
    """The reference's own layer in W8A8 mode, one token per call and with
    zero routed down weights, computes exactly the shared experts of the
    prepared layer (per-token activations; every down column has the same
    max|w|, so its per-tensor weight scale is the per-channel one). Its Y
    must equal the oracle's shared experts summed in fp64, bit for bit, and
    the numpy rebuild as well."""
    from golden.gen import shared_case
    X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds = shared_case()
    acc = np.zeros(X.shape, np.float64)
    acc_np = np.zeros(X.shape, np.float64)
    for s in range(Wgs.shape[0]):
        rc, ys = orc.ffn_fwd(Wgs[s], Wus[s], Wds[s], X)
        assert rc == 0
        acc += ys.astype(np.float64)
        acc_np += _np_ffn(Wgs[s], Wus[s], Wds[s], X).astype(np.float64)
    assert np.array_equal(bits(acc.astype(np.float32)), bits(gold["shared_Y"]))
    assert np.array_equal(bits(acc_np.astype(np.float32)), bits(gold["shared_Y"]))
    # the prepared oracle layer with the same weights (routed output 0)
    L = orc.moe_q(X.shape[1], Wg.shape[1], Wg.shape[0], 2, Wgs.shape[0], Wgs.shape[1],
                  Wgate, Wg, Wu, Wd, Wgs, Wus, Wds)
    r = L.fwd(X)
    assert r["rc"] == 0 and not r["Ye"].any()
    assert np.array_equal(bits(r["Y"]), bits(gold["shared_Y"]))


# ------------------------- accuracy of the prepared low-bit format (tolerance)

def _rel(a, b):
    """Mean |a - b| over mean |b| (bench/kernel/test_lowbit.c:130-157)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b).mean() / (np.abs(b).mean() + 1e-6)


def _group_gemm(orc, X, Wnk, b):
    _, Xq, sx = orc.quant_rows(X)
    _, codes, sc = orc.lowbit_pack_rows(Wnk, b)
    rc, Y, _ = orc.gemm_lowbit_group(Xq, sx, codes, sc, b)
    assert rc == 0
    return Y


def test_group64_accuracy_on_reference_inputs(orc, gold):
    """The reference's accuracy contract for its low-bit GEMM
    (bench/kernel/test_lowbit.c:112-157: INT4 rel < 0.10, INT2 rel < 0.45
    against the fp64 product) holds for the group-64 format that replaces it,
    on the reference test's own inputs."""
    from golden.gen import lpat_lut_inputs
    X, W = lpat_lut_inputs()                          # W [K][H]
    Yr = X.astype(np.float64) @ W.astype(np.float64)
    for b, thr in ((4, 0.10), (2, 0.45)):
        Y = _group_gemm(orc, X, np.ascontiguousarray(W.T), b)
        assert _rel(Y, Yr) < thr, (b, _rel(Y, Yr))
        # the reference's own T-MAC result on the same inputs meets it too
        assert _rel(gold[f"lpat_lut{b}"], Yr) < thr
        assert np.array_equal(bits(orc.lowbit_gemm_lut(X, W, b)[1]), bits(gold[f"lpat_lut{b}"]))


@pytest.mark.parametrize("dist", ["normal", "uniform", "laplace"])
def test_group64_no_worse_than_tmac(orc, dist):
    """At the layer's shapes the group-64 GEMM is at least as accurate as
    the reference's T-MAC GEMM it replaces (src/lowbit.c:158-267, per-column
    scale and an int8 LUT per 32 activations), both against fp64."""
    rng = np.random.default_rng(32)
    for (M, K, N) in ((64, 1024, 256), (64, 256, 1024)):
        X = rng.standard_normal((M, K)).astype(np.float32)
        W = {"normal": rng.standard_normal, "uniform": lambda s: rng.uniform(-1, 1, s),
             "laplace": lambda s: rng.laplace(size=s)}[dist]((N, K)).astype(np.float32)
        Yr = X.astype(np.float64) @ W.astype(np.float64).T
        for b in (2, 4):
            ours = _rel(_group_gemm(orc, X, W, b), Yr)
            tmac = _rel(orc.lowbit_gemm_lut(X, np.ascontiguousarray(W.T), b)[1], Yr)
            assert ours <= tmac * 1.01, (dist, M, K, N, b, ours, tmac)


def test_prepared_layer_vs_reference_fp32_layer(orc, gold):
    """The prepared quantised layer against the reference's fp32 layer
    (jt_moe_fwd_batch, flags off) on a routing without drops: the routing is
    identical, and the error of the routed expert outputs and of Y is below
    that of the reference's own true-LUT low-bit layer (flag mode 2, the
    scheme the group-64 path replaces) on the same inputs."""
    from golden.gen import accuracy_case
    args = accuracy_case(int(gold["acc_salt"]))
    X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds = args
    T, n = X.shape
    E, h = Wg.shape[:2]
    k, S = gold["acc0_ids"].shape[1], Wgs.shape[0]
    r = orc.moe_q(n, h, E, k, S, h, *args[1:]).fwd(X)
    assert r["rc"] == 0
    assert np.array_equal(r["ids"], gold["acc0_ids"])
    assert np.array_equal(bits(r["w"]), bits(gold["acc0_w"]))
    ye_ours, ye_lut = _rel(r["Ye"], gold["acc0_Ysel"]), _rel(gold["acc2_Ysel"], gold["acc0_Ysel"])
    y_ours, y_lut = _rel(r["Y"], gold["acc0_Y"]), _rel(gold["acc2_Y"], gold["acc0_Y"])
    print(f"rel error vs fp32 layer: Ye {ye_ours:.3f} (LUT {ye_lut:.3f}), "
          f"Y {y_ours:.3f} (LUT {y_lut:.3f})")
    assert ye_ours < ye_lut and y_ours < y_lut


def test_w8a8_layer_row_limit_vs_reference(orc, ref):
    """With the W8A8 flag on, the reference's layer runs its shared experts
    as one W8A8 GEMM of M = T rows and fails closed with EINVAL above
    JT_BWD_MAX_WIDE = 4096 rows (src/w8a8.c:926-929); so does the oracle."""
    rng = np.random.default_rng(33)
    T, n, h, E, k, S = 4097, 64, 64, 8, 2, 1
    args = [rng.standard_normal((T, n)).astype(np.float32)] + [
        (rng.standard_normal(s) / 8).astype(np.float32)
        for s in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    r1 = orc.moe_fwd_batch(*args, k, 1.5, 1, 0)
    r2 = ref.moe_fwd_batch(*args, k, 1.5, 1, 0)
    assert r1["rc"] == r2["rc"] == 2
    assert not r1["Y"].any() and not r2["Y"].any()
    # one row fewer passes in both
    r1 = orc.moe_fwd_batch(*(a[:4096] if i == 0 else a for i, a in enumerate(args)), k, 1.5, 1, 0)
    r2 = ref.moe_fwd_batch(*(a[:4096] if i == 0 else a for i, a in enumerate(args)), k, 1.5, 1, 0)
    assert r1["rc"] == r2["rc"] == 0
    assert np.array_equal(bits(r1["Y"]), bits(r2["Y"]))


def test_residual_add_closed_form(orc):
    """or_residual_add: (float)((double)x + (double)m), as the reference's
    training loop adds the residual after its layer
    (bench/kernel/train_tinystories.c:1147-1160). Rounding the fp64 sum once
    differs from the float sum x + m on inputs like these, and a non-finite
    sum is rejected."""
    rng = np.random.default_rng(34)
    X = (rng.standard_normal((7, 129)) * 1e3).astype(np.float32)
    Mo = (rng.standard_normal((7, 129)) * 1e-3).astype(np.float32)
    X[0, :4] = [1.0, 2.0 ** 24, -3.0, 3e38]
    Mo[0, :4] = [2.0 ** -24, 1.0, 3.0, 3e38]   # a tie to even, an exact 0, an overflow to inf
    rc, Y = orc.residual_add(X[1:], Mo[1:])
    assert rc == 0
    want = (X[1:].astype(np.float64) + Mo[1:].astype(np.float64)).astype(np.float32)
    assert np.array_equal(bits(Y), bits(want))
    rc, Y = orc.residual_add(X[0, :3], Mo[0, :3])
    assert rc == 0 and Y.tolist() == [1.0, 2.0 ** 24, 0.0]
    # 3e38 + 3e38 is finite in fp64 and overflows only when rounded to float
    rc, Y = orc.residual_add(X[0, 3:4], Mo[0, 3:4])
    assert rc == 0 and np.isinf(Y[0])
    inf = np.array([np.inf], np.float32)
    assert orc.residual_add(inf, np.zeros(1, np.float32))[0] == 2
