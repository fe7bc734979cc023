"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (runs the HIP library); everything else runs on CPU.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an AMD MI355X GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle.pyoracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.pyoracle import RefLib, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (reference checkout absent at build time)")
    return RefLib()


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a gpu-marked test ran without a visible GPU")
    return torch


@pytest.fixture(scope="session")
def jt(torch_cuda):
    import jimotono_amd.api as api
    api.lib()
    assert api.lib().jt_hip_init(0) == 0
    return api


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(f"[case] {msg}", flush=True)


def zipf_ids(rng, T, k, E, s=1.1):
    """Per-token expert ids drawn from Zipf(s) over E experts without
    replacement, and weights U(0,1) normalised to sum 1 per token."""
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    ids = np.zeros((T, k), np.int32)
    for t in range(T):
        ids[t] = rng.choice(E, size=k, replace=False, p=p)
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    return ids, w.astype(np.float32)
