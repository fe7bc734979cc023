"""CPU checks of the boundary: the C-ABI library and its host-side logic.

No GPU is touched: the library is loaded, its exports are compared with the
prototypes of include/jimotono/*.h, argument validation that precedes any
device work is exercised, and the product's refusal to run without its HIP
library or without a GPU is checked.
"""
import ctypes as C
import errno as E
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "jimotono")
LIB = os.path.join(ROOT, "jimotono_amd", "libjimotono_hip.so")

_DECL = re.compile(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(jt_\w+)\s*\(", re.M)


def declared():
    names = set()
    for f in sorted(os.listdir(INC)):
        if not f.endswith(".h"):
            continue
        text = open(os.path.join(INC, f)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"#define[^\n]*", "", text)
        for m in _DECL.finditer(text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built: run `make -C jimotono_amd/csrc`")
    return C.CDLL(LIB, use_errno=True)


def test_headers_declare_the_path():
    names = declared()
    for must in ("jt_w8a8_gemm_per_channel", "jt_w8a8_quant_per_channel", "jt_routing_topk",
                 "jt_moe_batch_sort", "jt_moe_fwd_batch", "jt_lowbit_gemm_lut",
                 "jt_tmac_lut_ctor", "jt_gemm_mat_f32", "jt_hip_moe_fwd", "jt_hip_w8a8_gemm"):
        assert must in names
    assert len(names) >= 40


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_no_gpu_fails_loudly(lib):
    """Without a visible GPU the entry points report JT_ERR_IO with errno
    ENODEV (include/jimotono/common.h); there is no CPU fallback."""
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    lib.jt_hip_init.argtypes = [C.c_int]
    C.set_errno(0)
    assert lib.jt_hip_init(0) == 3 and C.get_errno() == E.ENODEV
    f32 = np.ones(4, np.float32)
    q = np.zeros(4, np.int8)
    s = np.zeros(1, np.float32)
    fn = lib.jt_w8a8_quant_per_tensor
    fn.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]
    assert fn(f32.ctypes.data, 4, q.ctypes.data, s.ctypes.data) == 3
    assert not q.any() and s[0] == 0  # outputs untouched


def test_validation_before_device_work(lib):
    """Fail-closed argument checks of the reference (src/w8a8.c:910-953,
    bench/kernel/test_w8a8.c:86-112) run before any device call."""
    g = lib.jt_w8a8_gemm_per_channel
    g.argtypes = [C.c_void_p, C.c_void_p, C.c_float, C.c_void_p, C.c_void_p, C.c_int,
                  C.c_int, C.c_int]
    A = np.ones((2, 4), np.int8)
    B = np.ones((4, 3), np.int8)
    sB = np.ones(3, np.float32)
    out = np.full((2, 3), 7.0, np.float32)
    p = lambda a: a.ctypes.data  # noqa: E731
    cases = [
        (None, p(B), 1.0, p(sB), p(out), 2, 3, 4),
        (p(A), p(B), 0.0, p(sB), p(out), 2, 3, 4),
        (p(A), p(B), float("nan"), p(sB), p(out), 2, 3, 4),
        (p(A), p(B), 1.0, p(sB), p(out), 2, 4097, 4),
        (p(A), p(B), 1.0, p(sB), p(out), -1, 3, 4),
        (p(A), p(B), 1.0, p(sB), p(out), 2, 3, 0),
        (p(A), p(B), 1.0, None, p(out), 2, 3, 4),
    ]
    for c in cases:
        C.set_errno(0)
        assert g(*c) == 2 and C.get_errno() == E.EINVAL, c
    assert np.all(out == 7.0)
    # M == 0 is a successful no-op (src/w8a8.c:959-971)
    assert g(p(A), p(B), 1.0, p(sB), p(out), 0, 3, 4) == 0
    t = lib.jt_routing_topk
    t.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]
    lg = np.zeros(2, np.float32)
    ids = np.zeros(2, np.uint64)
    w = np.zeros(2, np.float32)
    for args in [(None, 2, 1), (p(lg), 0, 1), (p(lg), 2, 0), (p(lg), 2, 3)]:
        assert t(args[0], args[1], args[2], p(ids), p(w)) == 2
    m = lib.jt_lowbit_set_mode
    m.argtypes = [C.c_int]
    assert m(3) == 2 and m(-1) == 2
    bf = lib.jt_lowbit_bits_for
    bf.argtypes = [C.c_int, C.POINTER(C.c_int)]
    b = C.c_int(0)
    assert bf(0, C.byref(b)) == 0 and b.value == 2
    assert bf(1, C.byref(b)) == 0 and b.value == 4


def test_api_refuses_without_library(monkeypatch, tmp_path):
    import jimotono_amd.api as api
    monkeypatch.setattr(api, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(api, "_LIB", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        api.lib()


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one MI355X" in r.stderr


def test_product_never_imports_the_oracle():
    """Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may
    use oracle/; the package and the C sources never do."""
    pkg = os.path.join(ROOT, "jimotono_amd")
    for dp, _, fs in os.walk(pkg):
        for f in fs:
            if f.endswith((".py", ".c", ".h", ".hip", "Makefile")):
                text = open(os.path.join(dp, f), errors="ignore").read()
                assert "oracle" not in text.replace("oracle/", "").lower() or f == "README", f


def test_tmac_size_functions(lib):
    """jt_tmac_qlut_bytes / jt_tmac_param_bytes (src/tmac.c:168-228): host
    arithmetic only, so they run without a GPU. Checked against the closed
    forms n*(k/4)*8 and n*(k/32)*4, the fail-closed cases (NULL, zero, k not
    a multiple of the group, size_t overflow -> ENOMEM) and, when it has been
    built, the reference's own functions on the same arguments."""
    fq, fp = lib.jt_tmac_qlut_bytes, lib.jt_tmac_param_bytes
    for f in (fq, fp):
        f.argtypes = [C.c_size_t, C.c_size_t, C.POINTER(C.c_size_t)]
    ref = None
    from oracle.pyoracle import REF_SO, ref_available
    if ref_available():
        ref = C.CDLL(REF_SO, use_errno=True)
        for name in ("jt_tmac_qlut_bytes", "jt_tmac_param_bytes"):
            getattr(ref, name).argtypes = [C.c_size_t, C.c_size_t, C.POINTER(C.c_size_t)]
    big = (1 << 64) - 1
    cases = [(1, 32), (3, 64), (7, 1024), (256, 4096), (0, 32), (4, 0), (4, 33), (4, 36),
             (big, 32), (big // 8 + 1, 32), (big // 64, 32)]
    for n, k in cases:
        for f, name, g, per in ((fq, "jt_tmac_qlut_bytes", 4, 8),
                                (fp, "jt_tmac_param_bytes", 32, 4)):
            out = C.c_size_t(12345)
            C.set_errno(0)
            rc = f(n, k, C.byref(out))
            er = C.get_errno()
            if n == 0 or k == 0 or k % g:
                assert rc == 2 and er == E.EINVAL and out.value == 0, (name, n, k)
            elif n * (k // g) * per > big:
                assert rc == 1 and er == E.ENOMEM and out.value == 0, (name, n, k)
            else:
                assert rc == 0 and out.value == n * (k // g) * per, (name, n, k)
            if ref is not None:
                o2 = C.c_size_t(12345)
                C.set_errno(0)
                rc2 = getattr(ref, name)(n, k, C.byref(o2))
                assert (rc2, C.get_errno(), o2.value) == (rc, er, out.value), (name, n, k)
    assert fq(4, 32, None) == 2 and fp(4, 32, None) == 2


def test_calibration_library_is_separate():
    """bench.py's issue-rate probes (libjimotono_calib.so) load without a GPU
    and export their two entries; the drop-in library and the package never
    refer to them."""
    cal = os.path.join(ROOT, "jimotono_amd", "libjimotono_calib.so")
    if not os.path.exists(cal):
        pytest.fail(f"{cal} not built: run `make -C jimotono_amd/csrc`")
    L = C.CDLL(cal)
    assert hasattr(L, "jt_calib_issue") and hasattr(L, "jt_calib_tile")
    assert not hasattr(C.CDLL(LIB), "jt_calib_issue")
    pkg = os.path.join(ROOT, "jimotono_amd")
    for dp, _, fs in os.walk(pkg):
        if os.path.basename(dp) == "calib":
            continue
        for f in fs:
            if f.endswith((".py", ".c", ".h", ".hip")):
                assert "calib" not in open(os.path.join(dp, f), errors="ignore").read(), f
