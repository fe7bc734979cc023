"""GPU parity of the prepared layer's router against the oracle's router
(gate logits in the reference's lane order, src/moe_layer.c:67-86, then
top-k and softmax, src/routing.c:16-76).

Up to 16 tokens (d % 256 == 0) the layer evaluates the reference's fp64
sum for every expert in one launch. Otherwise, for E <= 256 and d % 64 == 0
it bounds every logit with int8 matrix products and evaluates the fp64 sum
only for the experts the bounds cannot rule out; other shapes take the fp64
router for every expert. Above 256 tokens with E % 16 == 0 and d in
{256, 512, 1024}, the codes, bounds and candidate selection run as one
launch of 16 tokens a block. All of them must give the reference's ids exactly (including ties, which
go to the lower expert index), the selected logits bit for bit, and the
softmax weights within rtol 1e-6 (device exp versus glibc's).
"""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def route(jt, torch, X, Wgate, k, h=64):
    T, n = X.shape
    E = Wgate.shape[0]
    rng = np.random.default_rng(0)
    f = np.float32
    Wg = (rng.standard_normal((E, h, n)) / np.sqrt(n)).astype(f)
    Wd = (rng.standard_normal((E, h, n)) / np.sqrt(h)).astype(f)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    L = jt.MoE(n, h, E, k, 0, 64, T, cu(Wgate), cu(Wg), cu(Wg), cu(Wd), None, None, None)
    dY = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    assert L.fwd(cu(X), dY) == 0
    assert jt.sync_errors() == 0
    ids = L.read(jt.BUF_IDS, np.int32, (T, k))
    w = L.read(jt.BUF_WEIGHTS, np.float32, (T, k))
    lg = L.read(jt.BUF_LOGITS, np.float32, (T, E))
    return ids, w, lg


def check(orc, X, Wgate, k, ids, w, lg):
    rc, oids, ow, olg = orc.router(X, Wgate, k)
    assert rc == 0
    bad = np.nonzero((ids != oids).any(axis=1))[0]
    assert bad.size == 0, f"tokens with other ids: {bad[:10]}"
    np.testing.assert_allclose(w, ow, rtol=1e-6, atol=0)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32)), "routing weights' bits"
    sel = np.take_along_axis(lg, ids.astype(np.int64), axis=1)
    osel = np.take_along_axis(olg, oids, axis=1)
    assert np.array_equal(bits(sel), bits(osel))


def test_router_full_size_every_token(jt, orc, torch_cuda):
    """Prefill router shape: 4096 tokens, d=1024, 256 experts, top-8."""
    T, n, E, k = 4096, 1024, 256, 8
    announce("router full size, every token")
    rng = np.random.default_rng(4097)
    Wgate = (rng.standard_normal((E, n)) / np.sqrt(n)).astype(np.float32)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w, lg = route(jt, torch_cuda, X, Wgate, k)
    check(orc, X, Wgate, k, ids, w, lg)


def adversarial(rng, T, n, E):
    f = np.float32
    W = (rng.standard_normal((E, n)) / np.sqrt(n)).astype(f)
    W[9] = W[5]            # exact ties between experts
    W[E - 1] = W[5]
    W[12] = W[11]
    W[12, 3] = np.nextafter(W[11, 3], f(np.inf))  # a one-ulp difference
    W[20] = W[21] * f(0.5)
    X = rng.standard_normal((T, n)).astype(f)
    X[0] = 0.0                                    # every logit 0: ids 0..k-1
    X[1] *= f(1e-3)
    X[2] *= f(1e3)
    X[3] = W[5] * f(4.0)                          # the tied experts lead
    X[4] = W[11]                                  # the near-tie leads
    X[5] = 0.0
    X[5, 7] = f(3.0)                              # one-hot: a column of W
    X[6] = np.round(X[6])                         # small integers
    X[7] = np.abs(X[7])
    X[8] = X[8] * f(2.0 ** -60)                   # tiny but normal
    X[9, ::2] = 0.0                               # half sparse
    X[10] = np.float32(1.0)                       # constant row
    X[11] = rng.integers(-126, 126, n) + f(0.5)   # int8 codes on exact ties
    X[11, 0] = f(127.0)
    return W, X


@pytest.mark.parametrize("E,k", [(64, 8), (256, 8), (32, 1), (40, 40), (320, 6)],
                         ids=["E64k8", "E256k8", "E32k1", "E40k40", "E320k6_fp64"])
def test_router_adversarial(jt, orc, torch_cuda, E, k):
    T, n = 96, 256
    announce(f"router adversarial E={E} k={k}")
    rng = np.random.default_rng(E * 100 + k)
    Wgate, X = adversarial(rng, T, n, E)
    ids, w, lg = route(jt, torch_cuda, X, Wgate, k)
    check(orc, X, Wgate, k, ids, w, lg)
    assert list(ids[0]) == list(range(k))


@pytest.mark.parametrize("E,k,n", [(64, 8, 256), (256, 8, 1024), (32, 1, 512), (48, 40, 256)],
                         ids=["E64k8d256", "E256k8d1024", "E32k1d512", "E48k40d256"])
def test_router_front_adversarial(jt, orc, torch_cuda, E, k, n):
    """More than 256 tokens with E % 16 == 0 take the one-launch front (codes,
    int8 bounds and candidates of 16 tokens a block against every expert);
    333 tokens leave a partial last block, and the adversarial rows (zero,
    tiny, tied, one-hot) sit in the first block."""
    T = 333
    announce(f"router front adversarial E={E} k={k} d={n}")
    rng = np.random.default_rng(E * 1000 + k * 10 + n)
    Wgate, X = adversarial(rng, T, n, E)
    ids, w, lg = route(jt, torch_cuda, X, Wgate, k)
    check(orc, X, Wgate, k, ids, w, lg)
    assert list(ids[0]) == list(range(k))


@pytest.mark.parametrize("n", [128, 384, 2048])
def test_router_widths(jt, orc, torch_cuda, n):
    T, E, k = 67, 128, 8
    announce(f"router width d={n}")
    rng = np.random.default_rng(n)
    Wgate = (rng.standard_normal((E, n)) / np.sqrt(n)).astype(np.float32)
    X = rng.standard_normal((T, n)).astype(np.float32)
    ids, w, lg = route(jt, torch_cuda, X, Wgate, k)
    check(orc, X, Wgate, k, ids, w, lg)


@pytest.mark.parametrize("T,n,E,k", [(16, 256, 64, 8), (11, 1024, 256, 8), (1, 512, 320, 6),
                                     (16, 1024, 40, 40)],
                         ids=["T16d256", "T11d1024", "T1E320", "T16k40"])
def test_router_decode_all_exact(jt, orc, torch_cuda, T, n, E, k):
    """Decode batches: every logit is exact, so all of BUF_LOGITS must equal
    the oracle's bit for bit, and the adversarial rows keep their ids."""
    announce(f"router decode T={T} d={n} E={E} k={k}")
    rng = np.random.default_rng(T * 1000 + E)
    Wgate, X = adversarial(rng, max(T, 16), n, E)
    X = X[:T]
    ids, w, lg = route(jt, torch_cuda, X, Wgate, k)
    check(orc, X, Wgate, k, ids, w, lg)
    rc, _, _, olg = orc.router(X, Wgate, k)
    assert np.array_equal(bits(lg), bits(olg))
