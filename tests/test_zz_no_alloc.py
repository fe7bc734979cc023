"""jt_hip_ffn_fwd_noalloc: the W8A8 SwiGLU expert on the library's fixed
device scratch, against jt_hip_ffn_fwd (its own buffers) on the same inputs,
bit for bit, on two calls in a row with the second one smaller. The
library's own count of device allocations (jt_hip_alloc_count, every
hipMalloc of the library goes through it) must not move across the
no-allocation calls. The count is per process, so other processes on the
GPU cannot disturb it, unlike the device's free memory."""
import errno as E

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,h,Ts", [(1024, 2816, (16, 4)), (1024, 2816, (300, 17)),
                                    (1000, 2000, (200, 37)), (1000, 2000, (9, 1))],
                         ids=["decode", "prefill", "padded", "padded_decode"])
def test_noalloc_matches_ffn_fwd(jt, torch_cuda, n, h, Ts):
    torch = torch_cuda
    g = torch.Generator(device="cuda").manual_seed(n + h)
    Wg = torch.randn(h, n, generator=g, device="cuda") / n ** 0.5
    Wu = torch.randn(h, n, generator=g, device="cuda") / n ** 0.5
    Wd = torch.randn(h, n, generator=g, device="cuda") / h ** 0.5
    F = jt.FFN(Wg, Wu, Wd)
    stream = torch.cuda.Stream()
    for T in Ts:
        announce(f"ffn noalloc n={n} h={h} T={T}")
        X = torch.randn(T, n, generator=g, device="cuda")
        Y_ref = torch.empty(T, n, device="cuda")
        Y = torch.full((T, n), float("nan"), device="cuda")
        torch.cuda.synchronize()
        F.fwd(X, Y_ref, stream)
        torch.cuda.synchronize()
        n0 = jt.alloc_count()
        assert F.fwd_noalloc(X, Y, stream) == 0
        torch.cuda.synchronize()
        assert jt.alloc_count() == n0
        assert jt.sync_errors() == 0
        assert torch.equal(Y.view(torch.int32), Y_ref.view(torch.int32)), f"T={T} differs"


def test_noalloc_rejects_too_many_rows(jt, torch_cuda):
    torch = torch_cuda
    n, h, T = 1024, 2816, 1111          # 16 MiB holds the workspace of 1110 rows
    announce(f"ffn noalloc rejects T={T}")
    g = torch.Generator(device="cuda").manual_seed(5)
    F = jt.FFN(*(torch.randn(h, n, generator=g, device="cuda") / 32 for _ in range(3)))
    X = torch.randn(T, n, generator=g, device="cuda")
    Y = torch.zeros(T, n, device="cuda")
    torch.cuda.synchronize()
    n0 = jt.alloc_count()
    assert F.fwd_noalloc(X[:1110], Y[:1110]) == 0
    torch.cuda.synchronize()
    Y.zero_()
    torch.cuda.synchronize()
    assert F.fwd_noalloc(X, Y) == jt.JT_ERR_NOSUP and jt.errno() == E.E2BIG
    torch.cuda.synchronize()
    assert not Y.any()                  # nothing was enqueued
    assert jt.alloc_count() == n0
    assert jt.sync_errors() == 0
