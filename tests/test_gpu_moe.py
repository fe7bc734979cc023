"""GPU parity of the prepared quantised MoE layer (jt_hip_moe_*) and the
W8A8 SwiGLU expert (jt_hip_ffn_*) against the oracle.

Integer/index outputs (quantised codes, routing ids, sort permutation,
expert offsets) must be identical, and so must every fp32 output (routing
weights, hidden codes and scales, expert outputs, Y), bit for bit. The one
arithmetic the device does differently from the oracle is fp64 exp() (and
the SwiGLU's reciprocal), each within about an ulp of glibc's; a result can
differ only where an fp64 value lies within a few 1e-16 of a float rounding
boundary, and on every input drawn here none does. Each comparison first
asserts the reference tests' own tolerance (rtol 1e-5, atol 1e-5 * max|Y|),
so that a failure reports the size of a slip, then equality of the bits.
"""
import numpy as np
import pytest

from conftest import announce, zipf_ids

pytestmark = pytest.mark.gpu


def mk_weights(rng, n, h, E, S, hs, scale=1.0):
    f = np.float32
    Wgate = (rng.standard_normal((E, n)) / np.sqrt(n)).astype(f)
    Wg = (rng.standard_normal((E, h, n)) * scale / np.sqrt(n)).astype(f)
    Wu = (rng.standard_normal((E, h, n)) * scale / np.sqrt(n)).astype(f)
    Wd = (rng.standard_normal((E, h, n)) * scale / np.sqrt(h)).astype(f)
    if S:
        sh = [(rng.standard_normal((S, hs, n)) / np.sqrt(n)).astype(f),
              (rng.standard_normal((S, hs, n)) / np.sqrt(n)).astype(f),
              (rng.standard_normal((S, hs, n)) / np.sqrt(hs)).astype(f)]
    else:
        sh = [None, None, None]
    return Wgate, Wg, Wu, Wd, sh


def close(Y, Y2):
    """The reference's tolerance (a failure shows the size of a slip), then
    bit equality; returns the count of differing elements (zero)."""
    tol = 1e-5 * max(float(np.abs(Y2).max()), 1e-30)
    np.testing.assert_allclose(Y, Y2, rtol=1e-5, atol=tol)
    diff = int((Y.view(np.uint32) != Y2.view(np.uint32)).sum())
    assert diff == 0, f"{diff} of {Y.size} elements differ in their last bits"
    return diff


def same_weights(w, w2):
    np.testing.assert_allclose(w, w2, rtol=1e-6, atol=0)
    assert np.array_equal(w.view(np.uint32), w2.view(np.uint32)), "routing weights' bits"


def dev(torch, a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_layer(jt, torch, n, h, E, k, S, hs, T, W, X, ids=None, w=None):
    Wgate, Wg, Wu, Wd, sh = W
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate), dev(torch, Wg), dev(torch, Wu),
               dev(torch, Wd), dev(torch, sh[0]), dev(torch, sh[1]), dev(torch, sh[2]))
    dX = dev(torch, X)
    dY = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    if ids is None:
        rc = L.fwd(dX, dY)
    else:
        rc = L.fwd_routed(dX, dev(torch, ids), dev(torch, w), dY)
    assert rc == 0
    assert jt.sync_errors() == 0
    return L, dY.cpu().numpy()


def read_buf(torch, L, which, dtype, shape):
    return L.read(which, dtype, shape)


def check_hidden(jt, L, o, T, k, n, h):
    """The routed hidden rows' int8 codes and scales against the oracle's
    (sorted order): every row identical. Ye is compared on the rows first
    (the down projection is integer MFMA plus the oracle's group fold), so
    a row whose codes differed would be reported before its output."""
    Hq = L.read(jt.BUF_HQ, np.int8, (T * k, h))
    Hs = L.read(jt.BUF_HSCALE, np.float32, (T * k,))
    Ye = L.read(jt.BUF_YE, np.float32, (T * k, n))
    same = np.all(Hq == o["Hq"], axis=1) & (Hs.view(np.uint32) == o["Hs"].view(np.uint32))
    pairs = o["perm"][same]
    assert np.array_equal(Ye[pairs].view(np.uint32), o["Ye"][pairs].view(np.uint32))
    ndiff = int((~same).sum())
    print(f"  hidden rows with other codes than the oracle's: {ndiff} of {T * k}")
    assert ndiff == 0
    return ndiff


CASES = [
    # n, h, E, k, S, hs, T
    (128, 64, 8, 2, 2, 64, 37),
    # the shared experts' gate/ups as one GEMM (S >= 2, T > 64, whole
    # 256-channel tiles over the concatenated gate/up panels)
    (256, 128, 16, 4, 2, 128, 100),
    (128, 64, 8, 2, 4, 64, 130),
    (256, 128, 16, 4, 1, 192, 200),
    (128, 64, 32, 8, 0, 64, 16),
    (256, 64, 64, 8, 2, 128, 1),
    # 64-row tiles whose down projection quantises its own rows (f = 256,
    # 512, 1024 take the fused path)
    (256, 512, 8, 2, 1, 128, 300),
    (128, 1024, 4, 2, 0, 64, 200),
    (128, 256, 16, 4, 0, 64, 260),
    # down projection with its weights in registers (K = 256 and 512)
    (512, 256, 16, 4, 1, 128, 400),
    (256, 512, 16, 2, 0, 64, 333),
    # 16-row tiles with f = 256: one launch per tile for gate/up, SwiGLU,
    # row codes and down (n = 256, 512, 768, 1024)
    (256, 256, 64, 8, 1, 128, 16),
    (512, 256, 32, 4, 0, 64, 40),
    (768, 256, 16, 2, 1, 64, 100),
    (1024, 256, 256, 8, 2, 512, 16),
    # decode with concatenated shared experts: top-k, sort and shared gate/up
    # in one launch, routed FFN and shared down in another; E = 300 and 520
    # (not powers of two, up to 16 keys a lane), up to 256 pairs in the
    # ballot-ranked sort, 320 pairs in the scanning one (k = 20)
    (256, 256, 64, 8, 2, 128, 16),
    (512, 256, 300, 6, 2, 256, 7),
    (256, 256, 520, 16, 3, 128, 16),
    (256, 256, 40, 20, 2, 128, 16),
    # three to eight shared experts in the combine, with k <= 8 and k > 8
    (256, 128, 16, 4, 3, 64, 100),
    (128, 64, 32, 12, 8, 64, 50),
    (128, 64, 64, 16, 5, 128, 9),
]


@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}h{c[1]}E{c[2]}k{c[3]}S{c[4]}T{c[6]}"
                                              for c in CASES])
def test_layer_router_parity(jt, orc, torch_cuda, case):
    torch = torch_cuda
    n, h, E, k, S, hs, T = case
    announce(f"moe layer router {case}")
    rng = np.random.default_rng(sum(case))
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X)
    OL = orc.moe_q(n, h, E, k, S, hs, W[0], W[1], W[2], W[3], *W[4])
    o = OL.fwd(X)
    assert o["rc"] == 0
    ids = read_buf(torch, L, jt.BUF_IDS, np.int32, (T, k))
    wts = read_buf(torch, L, jt.BUF_WEIGHTS, np.float32, (T, k))
    perm = read_buf(torch, L, jt.BUF_PERM, np.int32, (T * k,))
    off = read_buf(torch, L, jt.BUF_OFF, np.int32, (E + 1,))
    assert np.array_equal(ids, o["ids"])
    same_weights(wts, o["w"])
    assert np.array_equal(off, o["off"]) and np.array_equal(perm, o["perm"])
    for e in (0, E - 1):
        gu, gus, dc, ds = L.export_routed(e)
        ogu, ogus, odc, ods = OL.routed_codes(e)
        assert np.array_equal(gu, ogu) and np.array_equal(gus, ogus)
        assert np.array_equal(dc, odc) and np.array_equal(ds, ods)
    check_hidden(jt, L, o, T, k, n, h)
    diff = close(Y, o["Y"])
    print(f"  last-bit differences in Y: {diff} of {Y.size}")


@pytest.mark.parametrize("T", [1, 4, 16, 130, 600])
def test_layer_zipf_routed_parity(jt, orc, torch_cuda, T):
    torch = torch_cuda
    n, h, E, k, S, hs = 256, 128, 64, 8, 1, 128
    announce(f"moe layer zipf-routed T={T}")
    rng = np.random.default_rng(100 + T)
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w = zipf_ids(rng, T, k, E)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X, ids, w)
    o = orc.moe_q(n, h, E, k, S, hs, None, W[1], W[2], W[3], *W[4]).fwd(X, ids, w)
    assert o["rc"] == 0
    Ye = read_buf(torch, L, jt.BUF_YE, np.float32, (T * k, n))
    close(Ye, o["Ye"])
    check_hidden(jt, L, o, T, k, n, h)
    close(Y, o["Y"])


@pytest.mark.parametrize("T", [1, 16, 33])
def test_layer_decode_fused_zipf(jt, orc, torch_cuda, T):
    """Decode widths (d=1024, E=256, f=256, k=8) under Zipf(1.1) routing: the
    popular experts get several 16-row tiles, including short ones."""
    torch = torch_cuda
    n, h, E, k, S, hs = 1024, 256, 256, 8, 0, 0
    announce(f"moe layer decode fused zipf T={T}")
    rng = np.random.default_rng(1600 + T)
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w = zipf_ids(rng, T, k, E)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X, ids, w)
    o = orc.moe_q(n, h, E, k, S, hs, None, W[1], W[2], W[3], *W[4]).fwd(X, ids, w)
    assert o["rc"] == 0
    Ye = read_buf(torch, L, jt.BUF_YE, np.float32, (T * k, n))
    diff = close(Ye, o["Ye"])
    print(f"  last-bit differences in Ye: {diff} of {Ye.size}")
    check_hidden(jt, L, o, T, k, n, h)
    close(Y, o["Y"])


@pytest.mark.parametrize("n,E,k,S,T", [(256, 64, 8, 0, 16), (512, 256, 8, 2, 16),
                                         (768, 40, 4, 1, 5), (1024, 64, 16, 0, 16),
                                         (256, 1000, 16, 0, 16), (256, 100, 2, 2, 1),
                                         (512, 8, 2, 0, 3)],
                         ids=["n256E64", "n512S2", "n768E40", "n1024Tk256", "n256E1000Tk256",
                              "n256T1S2", "n512E8"])
def test_layer_decode_routed_sort_in_gateup(jt, orc, torch_cuda, n, E, k, S, T):
    """Caller-routed decode with 16-row tiles of f = 256 and at most 256
    pairs: the token codes and the pair sort run inside the routed gate/up
    launch. The sort (offsets, permutation), the token codes and scales, the
    hidden codes, Ye and Y against the oracle, at every model width, with
    and without shared experts (which read the token codes), up to 256 pairs
    and 1024 experts, and with experts holding more than 16 pairs."""
    torch = torch_cuda
    h, hs = 256, 128
    announce(f"moe layer decode routed, sort in the gate/up launch: n={n} E={E} k={k} S={S} T={T}")
    rng = np.random.default_rng(7 * n + E + T)
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w = zipf_ids(rng, T, k, E)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X, ids, w)
    o = orc.moe_q(n, h, E, k, S, hs, None, W[1], W[2], W[3], *W[4]).fwd(X, ids, w)
    assert o["rc"] == 0
    perm = read_buf(torch, L, jt.BUF_PERM, np.int32, (T * k,))
    off = read_buf(torch, L, jt.BUF_OFF, np.int32, (E + 1,))
    assert np.array_equal(off, o["off"]) and np.array_equal(perm, o["perm"])
    Xq = read_buf(torch, L, jt.BUF_XQ, np.int8, (T, n))
    sx = read_buf(torch, L, jt.BUF_XSCALE, np.float32, (T,))
    _, oXq, osx = orc.quant_rows(X)
    assert np.array_equal(Xq, oXq) and np.array_equal(sx.view(np.uint32), osx.view(np.uint32))
    check_hidden(jt, L, o, T, k, n, h)
    Ye = read_buf(torch, L, jt.BUF_YE, np.float32, (T * k, n))
    close(Ye, o["Ye"])
    close(Y, o["Y"])


def test_layer_decode_routed_bad_id(jt, torch_cuda):
    """An expert id outside 0..E-1 among the caller's ids (the sort inside
    the routed gate/up launch) fails the call with the bad-id flag, and the
    next call with good ids succeeds."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 256, 256, 32, 4, 0, 64, 8
    announce("moe layer decode routed, bad expert id")
    rng = np.random.default_rng(99)
    W = mk_weights(rng, n, h, E, S, hs)
    Wgate, Wg, Wu, Wd, sh = W
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate), dev(torch, Wg), dev(torch, Wu),
               dev(torch, Wd), None, None, None)
    X = dev(torch, rng.standard_normal((T, n)).astype(np.float32))
    ids, w = zipf_ids(rng, T, k, E)
    bad = ids.copy()
    bad[3, 1] = E
    Y = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    rc = L.fwd_routed(X, dev(torch, bad), dev(torch, w), Y)
    assert rc == 0 and jt.sync_errors() & jt.EF_BAD_ID
    assert L.fwd_routed(X, dev(torch, ids), dev(torch, w), Y) == 0
    assert jt.sync_errors() == 0


@pytest.mark.parametrize("T", [16, 700])
def test_layer_stress_widths_zipf(jt, orc, torch_cuda, T):
    """The stress shape's widths (d=2048, f=512, k=8; 128 of its 512 experts
    to keep the oracle's weight preparation short) under Zipf(1.1) routing
    at a decode and a small prefill batch (16-row and 64-row tiles)."""
    torch = torch_cuda
    n, h, E, k, S, hs = 2048, 512, 128, 8, 0, 0
    announce(f"moe layer stress widths zipf T={T}")
    rng = np.random.default_rng(2048 + T)
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w = zipf_ids(rng, T, k, E)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X, ids, w)
    o = orc.moe_q(n, h, E, k, S, hs, None, W[1], W[2], W[3], *W[4]).fwd(X, ids, w)
    assert o["rc"] == 0
    check_hidden(jt, L, o, T, k, n, h)
    close(Y, o["Y"])


def _rel(a, b):
    """Mean |a - b| over mean |b| (bench/kernel/test_lowbit.c:130-157)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b).mean() / (np.abs(b).mean() + 1e-6)


def test_layer_vs_reference_fp32_layer(jt, torch_cuda):
    """The GPU layer against the reference's fp32 layer (golden vectors of
    jt_moe_fwd_batch with the flags off, on a routing without drops): the
    routing is the reference's, and the error of the routed expert outputs
    and of Y is below that of the reference's own true-LUT low-bit layer
    (flag mode 2, the scheme the group-64 weights replace)."""
    import os
    from golden.gen import accuracy_case
    torch = torch_cuda
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
    args = accuracy_case(int(gold["acc_salt"]))
    X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds = args
    T, n = X.shape
    E, h = Wg.shape[:2]
    k, S = gold["acc0_ids"].shape[1], Wgs.shape[0]
    announce(f"layer vs reference fp32 layer T={T} n={n} h={h} E={E} k={k} S={S}")
    L, Y = run_layer(jt, torch, n, h, E, k, S, h, T, (Wgate, Wg, Wu, Wd, [Wgs, Wus, Wds]), X)
    ids = L.read(jt.BUF_IDS, np.int32, (T, k))
    wts = L.read(jt.BUF_WEIGHTS, np.float32, (T, k))
    assert np.array_equal(ids, gold["acc0_ids"])
    same_weights(wts, gold["acc0_w"])
    Ye = L.read(jt.BUF_YE, np.float32, (T * k, n))
    ye_ours, ye_lut = _rel(Ye, gold["acc0_Ysel"]), _rel(gold["acc2_Ysel"], gold["acc0_Ysel"])
    y_ours, y_lut = _rel(Y, gold["acc0_Y"]), _rel(gold["acc2_Y"], gold["acc0_Y"])
    print(f"  rel error vs fp32 layer: Ye {ye_ours:.3f} (LUT {ye_lut:.3f}), "
          f"Y {y_ours:.3f} (LUT {y_lut:.3f})")
    assert ye_ours < ye_lut and y_ours < y_lut


def test_layer_full_size_token_sample(jt, orc, torch_cuda):
    """Full-layer prefill shape (T=4096, d=1024, E=256, f=256, k=8, two shared
    f=2816 experts). Tokens are independent in the dropless layer, so the
    oracle runs on a sample of 32 tokens and must match those rows."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 1024, 256, 256, 8, 2, 2816, 4096
    announce("moe layer full size, 32-token sample")
    rng = np.random.default_rng(4096)
    W = mk_weights(rng, n, h, E, S, hs)
    X = rng.standard_normal((T, n)).astype(np.float32)
    L, Y = run_layer(jt, torch, n, h, E, k, S, hs, T, W, X)
    off = read_buf(torch, L, jt.BUF_OFF, np.int32, (E + 1,))
    assert off[0] == 0 and off[-1] == T * k and np.all(np.diff(off) >= 0)
    sample = np.sort(rng.choice(T, 32, replace=False))
    o = orc.moe_q(n, h, E, k, S, hs, W[0], W[1], W[2], W[3], *W[4]).fwd(X[sample])
    assert o["rc"] == 0
    ids = read_buf(torch, L, jt.BUF_IDS, np.int32, (T, k))
    assert np.array_equal(ids[sample], o["ids"])
    close(Y[sample], o["Y"])


@pytest.mark.parametrize("M", [1, 4, 16, 17, 100])
def test_ffn_shared_expert_parity(jt, orc, torch_cuda, M):
    torch = torch_cuda
    n, h = 1024, 2816
    announce(f"ffn n={n} h={h} M={M}")
    rng = np.random.default_rng(M)
    Wg = (rng.standard_normal((h, n)) / 32).astype(np.float32)
    Wu = (rng.standard_normal((h, n)) / 32).astype(np.float32)
    Wd = (rng.standard_normal((h, n)) / 53).astype(np.float32)
    X = rng.standard_normal((M, n)).astype(np.float32)
    F = jt.FFN(dev(torch, Wg), dev(torch, Wu), dev(torch, Wd))
    dY = torch.zeros((M, n), dtype=torch.float32, device="cuda")
    F.fwd(dev(torch, X), dY)
    assert jt.sync_errors() == 0
    rc, Y2 = orc.ffn_fwd(Wg, Wu, Wd, X)
    assert rc == 0
    close(dY.cpu().numpy(), Y2)


def test_ffn_reserve_then_grow(jt, orc, torch_cuda):
    """jt_hip_ffn_reserve sizes the workspace ahead; forwards at and below
    the reserved rows, and one above it (which grows the workspace), all
    match the oracle."""
    torch = torch_cuda
    n, h = 256, 128
    announce(f"ffn reserve n={n} h={h}")
    rng = np.random.default_rng(77)
    Wg, Wu = ((rng.standard_normal((h, n)) / 16).astype(np.float32) for _ in range(2))
    Wd = (rng.standard_normal((h, n)) / 11).astype(np.float32)
    F = jt.FFN(dev(torch, Wg), dev(torch, Wu), dev(torch, Wd))
    F.reserve(64)
    for M in (64, 20, 150):
        X = rng.standard_normal((M, n)).astype(np.float32)
        dY = torch.zeros((M, n), dtype=torch.float32, device="cuda")
        F.fwd(dev(torch, X), dY)
        assert jt.sync_errors() == 0
        rc, Y2 = orc.ffn_fwd(Wg, Wu, Wd, X)
        assert rc == 0
        close(dY.cpu().numpy(), Y2)


@pytest.mark.parametrize("n,h,M", [(256, 128, 3), (768, 3072, 16), (4096, 64, 2)],
                         ids=["n256", "h3072", "n4096_fallback"])
def test_ffn_decode_widths(jt, orc, torch_cuda, n, h, M):
    """Decode-sized experts quantise their activation rows inside the GEMMs
    (K <= 3072 with SwiGLU, <= 4096 plain); wider rows fall back to the
    separate quantiser. Same codes either way, so the same outputs."""
    torch = torch_cuda
    announce(f"ffn decode n={n} h={h} M={M}")
    rng = np.random.default_rng(n + h + M)
    Wg = (rng.standard_normal((h, n)) / np.sqrt(n)).astype(np.float32)
    Wu = (rng.standard_normal((h, n)) / np.sqrt(n)).astype(np.float32)
    Wd = (rng.standard_normal((h, n)) / np.sqrt(h)).astype(np.float32)
    X = rng.standard_normal((M, n)).astype(np.float32)
    if M > 1:
        X[1] = 0.0                     # zero row: scale 1, codes 0
    F = jt.FFN(dev(torch, Wg), dev(torch, Wu), dev(torch, Wd))
    dY = torch.zeros((M, n), dtype=torch.float32, device="cuda")
    F.fwd(dev(torch, X), dY)
    assert jt.sync_errors() == 0
    rc, Y2 = orc.ffn_fwd(Wg, Wu, Wd, X)
    assert rc == 0
    close(dY.cpu().numpy(), Y2)


def test_ffn_decode_tiny_row(jt, orc, torch_cuda):
    """A decode activation row with max|x| ~ 1e-38 (its codes all take the
    exact path) between normal rows, at n = 128 where half the lanes of the
    in-GEMM quantiser are past the row."""
    torch = torch_cuda
    announce("ffn decode tiny row n=128 h=128")
    n, h, M = 128, 128, 3
    rng = np.random.default_rng(128)
    Wg = (rng.standard_normal((h, n)) / np.sqrt(n)).astype(np.float32)
    Wu = (rng.standard_normal((h, n)) / np.sqrt(n)).astype(np.float32)
    Wd = (rng.standard_normal((h, n)) / np.sqrt(h)).astype(np.float32)
    X = rng.standard_normal((M, n)).astype(np.float32)
    X[1] *= np.float32(1e-38)
    F = jt.FFN(dev(torch, Wg), dev(torch, Wu), dev(torch, Wd))
    dY = torch.zeros((M, n), dtype=torch.float32, device="cuda")
    F.fwd(dev(torch, X), dY)
    assert jt.sync_errors() == 0
    rc, Y2 = orc.ffn_fwd(Wg, Wu, Wd, X)
    assert rc == 0
    close(dY.cpu().numpy(), Y2)


def test_layer_ordered_with_torch_default_stream(jt, orc, torch_cuda):
    """A torch kernel writes X on torch's default stream, the layer runs with
    no stream given, and a torch op reads Y, with no synchronisation in
    between: the forward must be ordered after the producer and before the
    consumer."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 256, 128, 16, 4, 1, 128, 600
    announce("layer ordered with torch's default stream")
    rng = np.random.default_rng(77)
    W = mk_weights(rng, n, h, E, S, hs)
    Wgate, Wg, Wu, Wd, sh = W
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate), dev(torch, Wg), dev(torch, Wu),
               dev(torch, Wd), dev(torch, sh[0]), dev(torch, sh[1]), dev(torch, sh[2]))
    X0 = rng.standard_normal((T, n)).astype(np.float32)
    src = dev(torch, X0 * 0.5)
    torch.cuda.synchronize()
    dX = torch.empty((T, n), dtype=torch.float32, device="cuda")
    dY = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    big = torch.randn(4096, 4096, device="cuda")
    for _ in range(3):                      # keep the default stream busy
        big = big @ big / 64.0
    torch.mul(src, 2.0, out=dX)             # X = X0, written last on the default stream
    assert L.fwd(dX, dY) == 0
    Ysum = dY.double().sum(dim=1)           # consumer on the default stream
    got = Ysum.cpu().numpy()
    assert jt.sync_errors() == 0
    o = orc.moe_q(n, h, E, k, S, hs, Wgate, Wg, Wu, Wd, *sh).fwd(X0)
    assert o["rc"] == 0
    ref = o["Y"].astype(np.float64).sum(axis=1)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_ffn_decode_nonfinite_row(jt, torch_cuda):
    """A NaN in a decode activation row is reported (the reference's
    quantiser rejects non-finite input)."""
    torch = torch_cuda
    announce("ffn decode non-finite row")
    n, h = 256, 128
    rng = np.random.default_rng(7)
    W = [(rng.standard_normal((h, n)) / 16).astype(np.float32) for _ in range(3)]
    F = jt.FFN(*(dev(torch, w) for w in W))
    X = rng.standard_normal((4, n)).astype(np.float32)
    X[2, 5] = np.nan
    dY = torch.zeros((4, n), dtype=torch.float32, device="cuda")
    F.fwd(dev(torch, X), dY)
    assert jt.sync_errors() & 0x1  # JT_HIP_EF_NONFINITE_INPUT


@pytest.mark.parametrize("routed,T", [(False, 300), (True, 16), (False, 1)])
def test_layer_residual_fused(jt, orc, torch_cuda, routed, T):
    """jt_hip_moe_fwd_residual: Y = X + layer(X) with the training loop's two
    roundings (bench/kernel/train_tinystories.c:1147-1160) fused into the
    combine. Bit-exact against the layer's own output plus the oracle's
    residual add, also in place (Y = X), and to tolerance against the oracle
    layer."""
    torch = torch_cuda
    n, h, E, k, S, hs = 256, 128, 16, 4, 2, 128
    announce(f"layer residual routed={routed} T={T}")
    rng = np.random.default_rng(900 + T)
    W = mk_weights(rng, n, h, E, S, hs)
    Wgate, Wg, Wu, Wd, sh = W
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w = zipf_ids(rng, T, k, E) if routed else (None, None)
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate), dev(torch, Wg), dev(torch, Wu),
               dev(torch, Wd), dev(torch, sh[0]), dev(torch, sh[1]), dev(torch, sh[2]))
    dX = dev(torch, X)
    di, dw = dev(torch, ids), dev(torch, w)
    Y0 = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    rc = L.fwd_routed(dX, di, dw, Y0) if routed else L.fwd(dX, Y0)
    assert rc == 0
    Y1 = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    assert L.fwd_residual(dX, Y1, di, dw) == 0
    Xin = dev(torch, X)
    assert L.fwd_residual(Xin, Xin, di, dw) == 0        # in place
    assert jt.sync_errors() == 0
    m = Y0.cpu().numpy()
    rc, want = orc.residual_add(X, m)
    assert rc == 0
    assert np.array_equal(Y1.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(Xin.cpu().numpy().view(np.uint32), want.view(np.uint32))
    o = orc.moe_q(n, h, E, k, S, hs, None if routed else Wgate, Wg, Wu, Wd, *sh).fwd(X, ids, w)
    assert o["rc"] == 0
    close(Y1.cpu().numpy(), orc.residual_add(X, o["Y"])[1])


def test_layer_residual_nonfinite(jt, torch_cuda):
    """A sum that is not finite in fp64 is reported, as the training loop's
    EINVAL (an infinite input is already rejected by the quantiser)."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 128, 64, 8, 2, 0, 0, 4
    announce("layer residual non-finite")
    rng = np.random.default_rng(5)
    W = mk_weights(rng, n, h, E, S, hs)
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, W[0]), dev(torch, W[1]), dev(torch, W[2]),
               dev(torch, W[3]))
    X = rng.standard_normal((T, n)).astype(np.float32)
    X[2, 7] = np.inf
    Y = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    L.fwd_residual(dev(torch, X), Y)
    assert jt.sync_errors() != 0


def test_layer_decode_nonfinite_then_clean(jt, orc, torch_cuda):
    """Decode with concatenated shared experts (the launches that carry the
    shared experts' blocks and sort in the last top-k block): a NaN token is
    reported, and the next clean forward of the same layer matches the
    oracle, so a failed routing leaves the launch's block counter at zero."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 256, 256, 64, 8, 2, 128, 16
    announce("layer decode non-finite then clean")
    rng = np.random.default_rng(616)
    W = mk_weights(rng, n, h, E, S, hs)
    Wgate, Wg, Wu, Wd, sh = W
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate), dev(torch, Wg), dev(torch, Wu),
               dev(torch, Wd), dev(torch, sh[0]), dev(torch, sh[1]), dev(torch, sh[2]))
    Y = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    bad = rng.standard_normal((T, n)).astype(np.float32)
    bad[3, 17] = np.nan
    assert L.fwd(dev(torch, bad), Y) == 0
    assert jt.sync_errors() != 0
    X = rng.standard_normal((T, n)).astype(np.float32)
    for _ in range(2):
        assert L.fwd(dev(torch, X), Y) == 0
        assert jt.sync_errors() == 0
        o = orc.moe_q(n, h, E, k, S, hs, Wgate, Wg, Wu, Wd, *sh).fwd(X)
        assert o["rc"] == 0
        assert np.array_equal(L.read(jt.BUF_IDS, np.int32, (T, k)), o["ids"])
        assert np.array_equal(L.read(jt.BUF_PERM, np.int32, (T * k,)), o["perm"])
        close(Y.cpu().numpy(), o["Y"])


@pytest.mark.parametrize("router", [True, False])
def test_layer_save_load_roundtrip(jt, orc, torch_cuda, router):
    """jt_hip_moe_save / jt_hip_moe_load: the reloaded layer (no quantisation,
    no packing on load) gives the saved layer's outputs bit for bit, saves to
    the same bytes, and a corrupted, truncated or foreign buffer is refused."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 256, 128, 16, 4, 2, 192, 130
    announce(f"layer save/load router={router}")
    rng = np.random.default_rng(77 + router)
    W = mk_weights(rng, n, h, E, S, hs)
    Wgate, Wg, Wu, Wd, sh = W
    X = rng.standard_normal((T, n)).astype(np.float32)
    L = jt.MoE(n, h, E, k, S, hs, T, dev(torch, Wgate) if router else None, dev(torch, Wg),
               dev(torch, Wu), dev(torch, Wd), dev(torch, sh[0]), dev(torch, sh[1]),
               dev(torch, sh[2]))
    ids, w = (None, None) if router else zipf_ids(rng, T, k, E)
    dX = dev(torch, X)

    def fwd(layer):
        Y = torch.zeros((T, n), dtype=torch.float32, device="cuda")
        rc = layer.fwd(dX, Y) if router else layer.fwd_routed(dX, dev(torch, ids),
                                                              dev(torch, w), Y)
        assert rc == 0
        assert jt.sync_errors() == 0
        return Y.cpu().numpy()

    Y1 = fwd(L)
    blob = L.save()
    assert blob[:7] == b"JTMOEQ1" and len(blob) % 4096 == 0
    L2 = jt.MoE.load(blob, T + 50)
    Y2 = fwd(L2)
    assert np.array_equal(Y1.view(np.uint32), Y2.view(np.uint32))
    assert L2.save() == blob
    for e in (0, E - 1):
        assert all(np.array_equal(a, b) for a, b in zip(L.export_routed(e), L2.export_routed(e)))
    # the oracle layer agrees with the reloaded one as with the original
    o = orc.moe_q(n, h, E, k, S, hs, Wgate if router else None, Wg, Wu, Wd, *sh).fwd(X, ids, w)
    close(Y2, o["Y"])
    bad = bytearray(blob)
    bad[len(bad) // 2] ^= 0x40                  # one payload bit
    for b_, mt in ((bytes(bad), T), (blob[:-4096], T), (b"JTMOEQ2" + blob[7:], T),
                   (blob, 0)):
        with pytest.raises(ValueError, match="rc=2"):
            jt.MoE.load(b_, mt)
