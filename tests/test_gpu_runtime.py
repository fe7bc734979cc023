"""Runtime bookkeeping on the GPU: per-stream device error words and their
release (jt_hip_stream_forget), and the library's allocation count."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def _nan_rows(torch):
    X = torch.randn(4, 64, device="cuda")
    X[1, 3] = float("nan")  # a non-finite activation: the quantiser raises a bit
    return X, torch.empty(4, 64, dtype=torch.int8, device="cuda"), torch.empty(4, device="cuda")


def test_stream_forget_clears_and_frees_the_word(jt, torch_cuda):
    torch = torch_cuda
    announce("stream_forget")
    s = torch.cuda.Stream()
    X, Xq, sc = _nan_rows(torch)
    torch.cuda.synchronize()
    jt.quant_rows(X, Xq, sc, s)
    jt.stream_forget(s)  # waits for s, drops its unread bit, frees its slot
    s2 = torch.cuda.Stream()  # a new stream takes the freed slot
    jt.quant_rows(X[:1], Xq[:1], sc[:1], s2)  # a clean row
    assert jt.sync_errors(s2) == 0
    # s is new again for the library: its fresh word gets the next bit
    jt.quant_rows(X, Xq, sc, s)
    assert jt.sync_errors(s) & jt.EF_NONFINITE_INPUT
    assert jt.sync_errors(s) == 0
    jt.stream_forget(s)
    jt.stream_forget(s2)
    jt.stream_forget(s2)  # a stream the library no longer holds: no-op


def test_many_streams_keep_separate_words(jt, torch_cuda):
    """Past the table size, released slots are reused: 200 streams, each
    released after use, never see another stream's bits."""
    torch = torch_cuda
    announce("stream words x200")
    X, Xq, sc = _nan_rows(torch)
    torch.cuda.synchronize()
    for i in range(200):
        s = torch.cuda.Stream()
        bad = i % 3 == 0
        jt.quant_rows(X if bad else X[:1], Xq if bad else Xq[:1], sc if bad else sc[:1], s)
        f = jt.sync_errors(s)
        assert bool(f & jt.EF_NONFINITE_INPUT) == bad, i
        if i % 2 == 0:
            jt.quant_rows(X, Xq, sc, s)  # leave an unread bit behind
        jt.stream_forget(s)


def test_alloc_count_moves_with_allocations(jt, torch_cuda):
    torch = torch_cuda
    announce("alloc_count")
    n0 = jt.alloc_count()
    W = jt.W8A8(Bq_kn=torch.randint(-127, 128, (64, 32), dtype=torch.int8, device="cuda"),
                sB=torch.rand(32, device="cuda") + 0.5)
    assert jt.alloc_count() > n0
    del W
    assert np.isfinite(float(n0))
