"""HIP graph capture of the prepared layer and the W8A8 expert.

Once its workspace is sized, a forward launches kernels only (no
allocation, no memset), so it can be captured into a HIP graph and
replayed. Each replay must redo all of the forward's device work: the test
replays several times with eager calls and host synchronisations in
between, on fresh inputs copied into the captured buffers, and checks every
replay bit for bit against the eager result on the same inputs.
"""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def _layer(jt, torch, n, h, E, k, S, hs, T, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")  # noqa: E731
    sh = (rn(S, hs, n) / n ** 0.5, rn(S, hs, n) / n ** 0.5, rn(S, hs, n) / hs ** 0.5) if S \
        else (None, None, None)
    return jt.MoE(n, h, E, k, S, hs, T, rn(E, n) / n ** 0.5, rn(E, h, n) / n ** 0.5,
                  rn(E, h, n) / n ** 0.5, rn(E, h, n) / h ** 0.5, *sh)


@pytest.mark.parametrize("T", [16, 300])
def test_layer_graph_replays(jt, torch_cuda, T):
    torch = torch_cuda
    n, h, E, k, S, hs = 512, 256, 64, 8, 2, 512
    announce(f"layer graph capture T={T}")
    L = _layer(jt, torch, n, h, E, k, S, hs, T, seed=T)
    stream = torch.cuda.Stream()
    X = torch.randn(T, n, device="cuda")
    Y = torch.empty(T, n, device="cuda")
    torch.cuda.synchronize()
    assert L.fwd(X, Y, stream) == 0  # first call: kernel attributes are set here
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        L.fwd(X, Y, stream)
    torch.cuda.synchronize()
    for rep in range(3):
        gen = torch.Generator(device="cuda").manual_seed(100 + rep)
        Xn = torch.randn(T, n, device="cuda", generator=gen)
        torch.cuda.synchronize()  # Xn is written on torch's stream
        assert L.fwd(Xn, Y, stream) == 0
        torch.cuda.synchronize()
        y_eager = Y.clone()
        Y.zero_()
        X.copy_(Xn)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, y_eager), f"replay {rep} differs from the eager forward"
    assert jt.sync_errors(stream) == 0 and jt.sync_errors() == 0


def test_ffn_graph_replays(jt, torch_cuda):
    torch = torch_cuda
    n, hs, M = 1024, 2816, 4
    announce("ffn graph capture M=4")
    g = torch.Generator(device="cuda").manual_seed(9)
    F = jt.FFN(torch.randn(hs, n, generator=g, device="cuda") / 32,
               torch.randn(hs, n, generator=g, device="cuda") / 32,
               torch.randn(hs, n, generator=g, device="cuda") / 53)
    stream = torch.cuda.Stream()
    X = torch.randn(M, n, device="cuda")
    Y = torch.empty(M, n, device="cuda")
    torch.cuda.synchronize()
    F.fwd(X, Y, stream)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        F.fwd(X, Y, stream)
    torch.cuda.synchronize()
    for rep in range(3):
        Xn = torch.randn(M, n, device="cuda")
        torch.cuda.synchronize()  # Xn is written on torch's stream
        F.fwd(Xn, Y, stream)
        torch.cuda.synchronize()
        y_eager = Y.clone()
        Y.zero_()
        X.copy_(Xn)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, y_eager), f"replay {rep} differs from the eager forward"
    assert jt.sync_errors(stream) == 0 and jt.sync_errors() == 0


def test_w8a8_gemm_graph_replays(jt, torch_cuda):
    """The W8A8 GEMM at 64 x 1024 x 1024 (the bench times it from a graph of
    back-to-back calls) replays bit for bit."""
    torch = torch_cuda
    M, N, K = 64, 1024, 1024
    announce("w8a8 gemm graph capture 64x1024x1024")
    g = torch.Generator(device="cuda").manual_seed(11)
    Bq = torch.randint(-127, 128, (K, N), generator=g, device="cuda", dtype=torch.int8)
    sB = torch.rand(N, generator=g, device="cuda") * 9e-3 + 1e-3
    W = jt.W8A8(Bq_kn=Bq, sB=sB)
    A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    sA = torch.rand(M, generator=g, device="cuda") * 9e-3 + 1e-3
    C = torch.empty(M, N, device="cuda")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    W.gemm(A, sA, C, stream)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        W.gemm(A, sA, C, stream)
    torch.cuda.synchronize()
    for rep in range(3):
        An = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        torch.cuda.synchronize()
        W.gemm(An, sA, C, stream)
        torch.cuda.synchronize()
        c_eager = C.clone()
        C.zero_()
        A.copy_(An)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, c_eager), f"replay {rep} differs from the eager call"
    assert jt.sync_errors(stream) == 0 and jt.sync_errors() == 0


def test_routed_decode_graph_replays(jt, torch_cuda):
    """The caller-routed decode (token codes and the pair sort inside the
    routed gate/up launch, shared experts after it) replays bit for bit."""
    torch = torch_cuda
    n, h, E, k, S, hs, T = 512, 256, 64, 8, 2, 512, 16
    announce("caller-routed decode graph capture T=16")
    L = _layer(jt, torch, n, h, E, k, S, hs, T, seed=77)
    rng = np.random.default_rng(77)
    ids = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
                           .astype(np.int32)).cuda()
    w = torch.from_numpy(rng.uniform(0, 1, (T, k)).astype(np.float32)).cuda()
    stream = torch.cuda.Stream()
    X = torch.randn(T, n, device="cuda")
    Y = torch.empty(T, n, device="cuda")
    torch.cuda.synchronize()
    assert L.fwd_routed(X, ids, w, Y, stream) == 0
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        L.fwd_routed(X, ids, w, Y, stream)
    torch.cuda.synchronize()
    for rep in range(3):
        gen = torch.Generator(device="cuda").manual_seed(200 + rep)
        Xn = torch.randn(T, n, device="cuda", generator=gen)
        torch.cuda.synchronize()
        assert L.fwd_routed(Xn, ids, w, Y, stream) == 0
        torch.cuda.synchronize()
        y_eager = Y.clone()
        Y.zero_()
        X.copy_(Xn)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, y_eager), f"replay {rep} differs from the eager forward"
    assert jt.sync_errors(stream) == 0 and jt.sync_errors() == 0
