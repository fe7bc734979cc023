"""The stress prefill shape at full size: T=16384 tokens, d=2048, E=512
routed experts with f=512, top-8 under Zipf(1.1) routing, no shared experts.

131,072 (token, slot) pairs take the layer's large-sort path (five launches
plus the tile list) and the head expert gets about 14k rows. The sort is
compared with the oracle's dropless sort (src/moe_layer.c:895-978 without a
capacity) over every pair, bit for bit. Tokens are independent in the
dropless layer, so Y is checked on a token sample against an oracle layer
built from only the experts those tokens touch, with the ids renumbered.
"""
import numpy as np
import pytest

from conftest import announce, zipf_ids

pytestmark = pytest.mark.gpu


def test_stress_prefill_full_size(jt, orc, torch_cuda):
    torch = torch_cuda
    n, h, E, k, T = 2048, 512, 512, 8, 16384
    announce(f"stress prefill full size T={T} n={n} h={h} E={E} k={k}")
    rng = np.random.default_rng(16384)
    ids, w = zipf_ids(rng, T, k, E)
    g = torch.Generator(device="cuda").manual_seed(512)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")  # noqa: E731
    Wg, Wu, Wd = rn(E, h, n) / n ** 0.5, rn(E, h, n) / n ** 0.5, rn(E, h, n) / h ** 0.5
    X = rn(T, n)
    L = jt.MoE(n, h, E, k, 0, 0, T, None, Wg, Wu, Wd)
    Y = torch.empty(T, n, device="cuda")
    assert L.fwd_routed(X, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), Y) == 0
    assert jt.sync_errors() == 0
    Yh = Y.cpu().numpy()
    assert np.isfinite(Yh).all()

    # the sort over all pairs
    perm = L.read(jt.BUF_PERM, np.int32, (T * k,))
    off = L.read(jt.BUF_OFF, np.int32, (E + 1,))
    rc, operm, ooff, drop = orc.batch_sort(ids.astype(np.int64), T, k, E, 0.0)
    assert rc == 0 and not drop.any()
    assert np.array_equal(off, ooff) and np.array_equal(perm, operm)
    counts = np.diff(off)
    print(f"  head expert rows: {counts.max()}, experts with no rows: {(counts == 0).sum()}")

    # Y and the expert outputs on a token sample
    sample = np.sort(rng.choice(T, 48, replace=False))
    touched = np.unique(ids[sample])
    remap = np.full(E, -1, np.int32)
    remap[touched] = np.arange(touched.size, dtype=np.int32)
    sel = torch.from_numpy(touched.astype(np.int64)).cuda()
    sub = [a.index_select(0, sel).cpu().numpy() for a in (Wg, Wu, Wd)]
    Xs = X.cpu().numpy()[sample]
    OL = orc.moe_q(n, h, touched.size, k, 0, 0, None, *sub)
    o = OL.fwd(Xs, remap[ids[sample]], w[sample])
    assert o["rc"] == 0
    for e in (0, touched.size - 1):        # the prepared codes of two experts
        gu, gus, dc, ds = L.export_routed(int(touched[e]))
        ogu, ogus, odc, ods = OL.routed_codes(e)
        assert np.array_equal(gu, ogu) and np.array_equal(gus, ogus)
        assert np.array_equal(dc, odc) and np.array_equal(ds, ods)
    Ye = L.read(jt.BUF_YE, np.float32, (T * k, n))
    q = (sample[:, None] * k + np.arange(k)[None, :]).ravel()
    tol = 1e-5 * float(np.abs(o["Ye"]).max())
    np.testing.assert_allclose(Ye[q], o["Ye"], rtol=1e-5, atol=tol)
    assert np.array_equal(Ye[q].view(np.uint32), o["Ye"].view(np.uint32))
    # rows whose hidden codes equal the oracle's give the oracle's Ye bits
    Hq = L.read(jt.BUF_HQ, np.int8, (T * k, h))
    Hs = L.read(jt.BUF_HSCALE, np.float32, (T * k,))
    inv = np.empty(T * k, np.int64)
    inv[perm] = np.arange(T * k)
    oinv = np.empty(q.size, np.int64)
    oinv[o["perm"]] = np.arange(q.size)
    gq, gs = Hq[inv[q]], Hs[inv[q]]
    oq, os_ = o["Hq"][oinv], o["Hs"][oinv]
    same = np.all(gq == oq, axis=1) & (gs.view(np.uint32) == os_.view(np.uint32))
    print(f"  sampled hidden rows with other codes than the oracle's: {(~same).sum()} of {q.size}")
    assert (~same).sum() == 0
    assert np.array_equal(Ye[q][same].view(np.uint32), o["Ye"][same].view(np.uint32))
    tol = 1e-5 * float(np.abs(o["Y"]).max())
    np.testing.assert_allclose(Yh[sample], o["Y"], rtol=1e-5, atol=tol)
    assert np.array_equal(Yh[sample].view(np.uint32), o["Y"].view(np.uint32))
