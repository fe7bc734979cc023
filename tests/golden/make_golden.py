#!/usr/bin/env python3
"""Write the golden vectors of tests/golden/ref_vectors.npz.

Expected outputs come from the reference's own hot-path functions,
compiled from the reference sources into oracle/_ref/libjtref.so by
``make -C oracle ref`` (src/w8a8.c, lowbit.c, tmac.c, routing.c,
moe_gemm.c, moe_layer.c, train_bwd.c with the reference's flags). Inputs
are seeded and synthetic. The fixture is data only: inputs and the
reference's outputs, no reference code.

    make -C oracle ref && python3 tests/golden/make_golden.py

Cases (key prefixes in the .npz):
  quant_rows_*   jt_w8a8_quant_per_channel, rows with exact ties, a zero row
  quant_tensor_* jt_w8a8_quant_per_tensor
  fakequant_rows / dequant_rows  jt_w8a8_fakequant_per_channel / dequant
  gemm_pc_* / gemm_pt_*  jt_w8a8_gemm_per_channel / _per_tensor
  gemm_f32_*     jt_gemm_mat_f32
  fq2_* / fq4_*  jt_lowbit_fakequant
  c2i2_* / c2i4_*  jt_lowbit_col_to_idx
  lut2_* / lut4_*  jt_lowbit_gemm_lut
  tmac_*         jt_tmac_lut_ctor + jt_tmac_lookup_accum
  topk_*         jt_routing_topk (random logits, exact ties, -inf masks)
  sort_*         jt_moe_batch_sort at cap 1.0 and 1.5 (drops)
  layer{f}_*     jt_moe_fwd_batch, f = 0 fp32, 1 W8A8 flag, 2 low-bit mode 1
  logits_*       jt_moe_fwd out_logits (gate logits, src/moe_layer.c:67-86), with
                 rows whose fp64 sum depends on the 4-lane summation order
  shared_*       jt_moe_fwd_batch with the W8A8 flag, one token per call, routed
                 down weights zero: Y is the shared experts' W8A8 SwiGLU output
                 (inputs from gen.shared_case)
  acc{0,2}_*     jt_moe_fwd_batch in fp32 (0) and true-LUT low-bit (2) modes on
                 gen.accuracy_case(acc_salt), a salt whose routing drops nothing
  lpat_lut{2,4}  jt_lowbit_gemm_lut on the reference test's own inputs
                 (bench/kernel/test_lowbit.c:112-157, gen.lpat_lut_inputs)
  bwdref{0,1}_*  jt_moe_fwd_batch (with its caches) then jt_moe_bwd_batch on the
                 reference backward tests' own inputs (gen.ref_bwd_inputs):
                 inputs, forward outputs and every backward output
  bwdrnd_*       jt_moe_bwd_batch outputs of gen.bwd_case(*BWD_RND) (drops, two
                 shared experts, n not a multiple of 4)
  gdn2dec_{dk}x{dv}s{seed}_{S,o}  jt_gdn2_decode_step on the reference test's
                 inputs (gen.gdn2_decode_inputs, bench/kernel/gdn2.c:850-860)
  gdn2pf{C}_{dk}x{dv}s{seed}_{S,Out,Sseq,Oseq}  jt_gdn2_prefill_chunk{C} and C
                 sequential jt_gdn2_decode_step calls on gen.gdn2_prefill_inputs;
                 gdn2pfb_* the same on gen.gdn2_boundary_inputs
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.pyoracle import RefLib  # noqa: E402
sys.path.insert(0, HERE)
from gen import (accuracy_case, bwd_args, bwd_case, gdn2_boundary_inputs,  # noqa: E402
                 gdn2_decode_inputs, gdn2_prefill_inputs, lpat_lut_inputs, ref_bwd_inputs,
                 shared_case)

OUT = os.path.join(HERE, "ref_vectors.npz")
# (T, n, h, E, k, S, salt, cap_factor) of the bwdrnd_* case
BWD_RND = (24, 42, 24, 6, 3, 2, 300, 1.0)


def main():
    R = RefLib()
    rng = np.random.default_rng(20261201)
    g = {}

    # ---- W8A8 quantisers ----
    X = rng.standard_normal((9, 77)).astype(np.float32)
    X[3] = 0.0
    # row 5: values that land exactly on .5 after division (max 127 -> scale 1)
    X[5] = np.float32(0.0)
    X[5, :6] = np.array([127.0, 0.5, -0.5, 2.5, -3.5, 126.5], np.float32)
    rc, Q, s = R.quant_rows(X)
    assert rc == 0
    g.update(quant_rows_X=X, quant_rows_Q=Q, quant_rows_s=s)
    F = np.zeros_like(X)
    assert R.lib.jt_w8a8_fakequant_per_channel(X, X.shape[0], X.shape[1], F) == 0
    D = np.zeros_like(X)
    assert R.lib.jt_w8a8_dequant_per_channel(Q, s, X.shape[0], X.shape[1], D) == 0
    g.update(fakequant_rows=F, dequant_rows=D)
    x = (rng.standard_normal(1001) * 3).astype(np.float32)
    rc, q, s1 = R.quant_tensor(x)
    assert rc == 0
    g.update(quant_tensor_x=x, quant_tensor_q=q, quant_tensor_s=np.float32(s1))

    # ---- W8A8 GEMMs ----
    M, N, K = 13, 40, 96
    Aq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
    sB = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    rc, C = R.gemm_per_channel(Aq, Bq, 0.0173, sB)
    assert rc == 0
    g.update(gemm_pc_A=Aq, gemm_pc_B=Bq, gemm_pc_sA=np.float32(0.0173), gemm_pc_sB=sB,
             gemm_pc_C=C)
    rc, C = R.gemm_per_tensor(Aq, Bq, 0.031, 0.0047)
    assert rc == 0
    g.update(gemm_pt_sA=np.float32(0.031), gemm_pt_sB=np.float32(0.0047), gemm_pt_C=C)
    A = rng.standard_normal((7, 33)).astype(np.float32)
    B = rng.standard_normal((33, 19)).astype(np.float32)
    rc, C = R.gemm_f32(A, B)
    assert rc == 0
    g.update(gemm_f32_A=A, gemm_f32_B=B, gemm_f32_C=C)

    # ---- low-bit levels ----
    w = rng.standard_normal(257).astype(np.float32)
    for bits in (2, 4):
        rc, fq = R.lowbit_fakequant(w, bits)
        assert rc == 0
        g[f"fq{bits}_w"], g[f"fq{bits}_out"] = w, fq
        col = rng.standard_normal(64).astype(np.float32)
        rc, idx, ws = R.col_to_idx(col, bits)
        assert rc == 0
        g[f"c2i{bits}_col"], g[f"c2i{bits}_idx"], g[f"c2i{bits}_ws"] = col, idx, np.float32(ws)
        Xl = rng.standard_normal((5, 64)).astype(np.float32)
        Wl = rng.standard_normal((64, 24)).astype(np.float32)
        rc, Y = R.lowbit_gemm_lut(Xl, Wl, bits)
        assert rc == 0
        g[f"lut{bits}_X"], g[f"lut{bits}_W"], g[f"lut{bits}_Y"] = Xl, Wl, Y

    # ---- T-MAC LUT ----
    act = rng.standard_normal((3, 64)).astype(np.float32)
    rc, ql, sc, bi = R.tmac_lut_ctor(act)
    assert rc == 0
    col = rng.standard_normal(64).astype(np.float32)
    outs = []
    for bits in (2, 4):
        rc, idx, ws = R.col_to_idx(col, bits)
        for r in range(3):
            rc, o = R.tmac_lookup_accum(ql[r].ravel(), idx, sc[r], bi[r], bits, ws)
            assert rc == 0
            outs.append(o)
    g.update(tmac_act=act, tmac_qlut=ql, tmac_scales=sc, tmac_biases=bi, tmac_col=col,
             tmac_out=np.array(outs, np.float32))

    # ---- routing top-k ----
    L = rng.standard_normal((8, 256)).astype(np.float32)
    L[1, 10:20] = 2.5  # exact ties
    L[2, :] = 1.0      # all equal
    L[3, 100:] = -np.inf  # masked
    ids = np.zeros((8, 8), np.int64)
    wts = np.zeros((8, 8), np.float32)
    for t in range(8):
        rc, ids[t], wts[t] = R.topk(L[t], 8)
        assert rc == 0
    g.update(topk_logits=L, topk_ids=ids, topk_w=wts)

    # ---- batch sort ----
    T, k, E = 64, 8, 32
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    sid = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)])
    g["sort_ids"] = sid.astype(np.int64)
    for tag, cap in (("c10", 1.0), ("c15", 1.5)):
        rc, perm, off, drop = R.batch_sort(sid, T, k, E, cap)
        assert rc == 0
        g[f"sort_{tag}_perm"], g[f"sort_{tag}_off"], g[f"sort_{tag}_drop"] = perm, off, drop

    # ---- legacy layer (small) ----
    T, n, h, E, k, S = 6, 64, 32, 8, 2, 1
    Xl = rng.standard_normal((T, n)).astype(np.float32)
    Wgate = (rng.standard_normal((E, n)) / 8).astype(np.float32)
    Wg = (rng.standard_normal((E, h, n)) / 8).astype(np.float32)
    Wu = (rng.standard_normal((E, h, n)) / 8).astype(np.float32)
    Wd = (rng.standard_normal((E, h, n)) / 6).astype(np.float32)
    Wgs = (rng.standard_normal((S, h, n)) / 8).astype(np.float32)
    Wus = (rng.standard_normal((S, h, n)) / 8).astype(np.float32)
    Wds = (rng.standard_normal((S, h, n)) / 6).astype(np.float32)
    g.update(layer_X=Xl, layer_Wgate=Wgate, layer_Wg=Wg, layer_Wu=Wu, layer_Wd=Wd,
             layer_Wgs=Wgs, layer_Wus=Wus, layer_Wds=Wds)
    for f, (w8, lb) in enumerate(((0, 0), (1, 0), (0, 1))):
        r = R.moe_fwd_batch(Xl, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, k, 1.5, w8, lb)
        assert r["rc"] == 0
        for key in ("Y", "ids", "w", "perm", "off", "drop"):
            g[f"layer{f}_{key}"] = r[key]

    # ---- gate logits (jt_moe_fwd's out_logits): random rows with an odd
    # tail, and rows whose fp64 sum depends on the 4-lane order ----
    n, E = 1027, 6
    Wg1 = (rng.standard_normal((E, 4, n)) / 30).astype(np.float32)
    WgateL = (rng.standard_normal((E, n)) / 30).astype(np.float32)
    lgs = []
    XL = rng.standard_normal((12, n)).astype(np.float32)
    for t in range(12):
        rc, _, _, _, lg = R.moe_fwd_single(XL[t], WgateL, Wg1, Wg1, Wg1, None, None, None, 2)
        assert rc == 0
        lgs.append(lg)
    g.update(logits_X=XL, logits_Wgate=WgateL, logits_out=np.array(lgs, np.float32))
    big = np.float32(2.0 ** 60)
    pat = np.array([big, 1, 1, 1, -big, 1, 1, 1, 1, -1, 1], np.float32)
    Wadv = np.stack([pat, pat[::-1].copy(), np.roll(pat, 1), np.roll(pat, 2)])
    Wa1 = np.zeros((4, 1, 11), np.float32)
    rc, _, _, _, lga = R.moe_fwd_single(np.ones(11, np.float32), Wadv, Wa1, Wa1, Wa1, None,
                                        None, None, 1)
    assert rc == 0
    g.update(logits_adv_W=Wadv, logits_adv_out=lga)

    # ---- shared experts through the reference's W8A8 layer, T = 1 per call
    # (per-tensor activations of one row = per-token), so the reference
    # computes the prepared layer's shared-expert formula ----
    X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds = shared_case()
    ys = []
    for t in range(X.shape[0]):
        r = R.moe_fwd_batch(X[t:t + 1], Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, 2, 1.0, 1, 0)
        assert r["rc"] == 0 and not r["drop"].any()
        assert not r["Ysel"].any()  # routed outputs are exactly zero
        ys.append(r["Y"][0])
    g["shared_Y"] = np.array(ys, np.float32)

    # ---- fp32 and true-LUT layers on a routing that drops nothing ----
    for salt in range(1000, 1100, 10):
        args = accuracy_case(salt)
        r0 = R.moe_fwd_batch(*args, 2, 1.5, 0, 0)
        assert r0["rc"] == 0
        if not r0["drop"].any():
            break
    else:
        raise RuntimeError("no salt without drops")
    r2 = R.moe_fwd_batch(*args, 2, 1.5, 0, 2)
    assert r2["rc"] == 0 and not r2["drop"].any()
    g["acc_salt"] = np.int64(salt)
    for key in ("Y", "Ysel", "ids", "w"):
        g[f"acc0_{key}"] = r0[key]
    g["acc2_Y"], g["acc2_Ysel"] = r2["Y"], r2["Ysel"]

    # ---- the reference low-bit test's own inputs ----
    Xp, Wp = lpat_lut_inputs()
    for bits in (2, 4):
        rc, Y = R.lowbit_gemm_lut(Xp, Wp, bits)
        assert rc == 0
        g[f"lpat_lut{bits}"] = Y

    # ---- batched backward ----
    for c in (0, 1):
        X, dY, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, k, cf = ref_bwd_inputs(c)
        f = R.moe_fwd_batch(X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, k, cf, caches=True)
        assert f["rc"] == 0
        if c == 1:  # the reference test's own expectation (test_moe_layer.c:1480-1486)
            assert f["off"][-1] == 13 and int(f["drop"].sum()) == 3
        b = R.moe_bwd_batch(dY, X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, f["ids"], f["w"],
                            f["Gsel"], f["Usel"], f["Ysel"], f.get("Gs"), f.get("Us"),
                            f["perm"], f["off"], f["drop"], k)
        assert b["rc"] == 0
        pre = f"bwdref{c}_"
        g.update({pre + "X": X, pre + "dY": dY, pre + "Wgate": Wgate, pre + "Wg": Wg,
                  pre + "Wu": Wu, pre + "Wd": Wd, pre + "k": np.int64(k)})
        if Wgs is not None:
            g.update({pre + "Wg_s": Wgs, pre + "Wu_s": Wus, pre + "Wd_s": Wds})
        for key in ("ids", "w", "Gsel", "Usel", "Ysel", "Gs", "Us", "perm", "off", "drop"):
            if key in f:
                g[pre + key] = f[key]
        for key, v in b.items():
            if key != "rc":
                g[pre + "out_" + key] = v
    c = bwd_case(*BWD_RND)
    b = R.moe_bwd_batch(*bwd_args(c))
    assert b["rc"] == 0
    for key, v in b.items():
        if key != "rc":
            g["bwdrnd_" + key] = v

    # ---- GDN-2 decode and prefill chunks (the reference tests' inputs) ----
    for dk, dv, seed in ((4, 8, 1), (5, 7, 2), (2, 3, 3), (8, 8, 4), (128, 128, 5)):
        S, q, k, v, b, w, a = gdn2_decode_inputs(dk, dv, seed)
        rc, S1, o = R.gdn2_decode_step(S, q, k, v, b, w, a)
        assert rc == 0
        g[f"gdn2dec_{dk}x{dv}s{seed}_S"], g[f"gdn2dec_{dk}x{dv}s{seed}_o"] = S1, o

    def prefill_case(key, S, Q, K, V, B, W, A):
        rc, S1, Out = R.gdn2_prefill_chunk(S, Q, K, V, B, W, A)
        assert rc == 0
        Ss, Os = S, []
        for t in range(Q.shape[0]):
            rc, Ss, o = R.gdn2_decode_step(Ss, Q[t], K[t], V[t], B[t], W[t], A[t])
            assert rc == 0
            Os.append(o)
        g.update({key + "_S": S1, key + "_Out": Out, key + "_Sseq": Ss,
                  key + "_Oseq": np.array(Os, np.float32)})
    for C, dk, dv, seed in ((16, 8, 8, 11), (16, 16, 16, 12), (32, 8, 16, 13), (32, 16, 8, 14),
                            (32, 128, 128, 15)):
        prefill_case(f"gdn2pf{C}_{dk}x{dv}s{seed}", *gdn2_prefill_inputs(C, dk, dv, seed))
    prefill_case("gdn2pfb", *gdn2_boundary_inputs())

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
