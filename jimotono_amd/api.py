"""ctypes wrappers over libjimotono_hip.so (the C ABI of include/jimotono/).

Host-pointer functions take and return numpy arrays and mirror the
reference's C names (``w8a8_gemm_per_channel`` -> ``jt_w8a8_gemm_per_channel``,
include/jimotono/w8a8.h:108-111 of the reference). Each returns ``(rc, ...)``
with the library's return code; ``errno()`` gives the errno of the last
call. Device-resident classes (``W8A8``, ``FFN``, ``MoE``) take torch
tensors on ``cuda`` for their device pointers.

Loading fails with an exception when the library has not been built:
there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import LIB_PATH

JT_OK, JT_ERR_NOMEM, JT_ERR_INVAL, JT_ERR_IO, JT_ERR_ALIGN, JT_ERR_NOSUP = range(6)
EF_NONFINITE_INPUT, EF_RANGE, EF_NONFINITE_MID, EF_BAD_ID = 1, 2, 4, 8

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_vp = C.c_void_p
_i, _sz, _fl = C.c_int, C.c_size_t, C.c_float

_LIB = None


class _Desc(C.Structure):
    _fields_ = [(f, C.c_int) for f in ("n", "h", "n_experts", "topk", "n_shared",
                                        "h_shared", "group", "max_tokens")]


# name -> argtypes (restype int unless noted)
_PROTOS = {
    "jt_w8a8_set_enabled": [_i],
    "jt_w8a8_get_enabled": [C.POINTER(_i)],
    "jt_w8a8_is_enabled": [],
    "jt_w8a8_quant_per_tensor": [_f32p, _sz, _i8p, _f32p],
    "jt_w8a8_dequant_per_tensor": [_i8p, _fl, _sz, _f32p],
    "jt_w8a8_quant_per_channel": [_f32p, _sz, _sz, _i8p, _f32p],
    "jt_w8a8_dequant_per_channel": [_i8p, _f32p, _sz, _sz, _f32p],
    "jt_w8a8_gemm_per_tensor": [_i8p, _i8p, _fl, _fl, _f32p, _i, _i, _i],
    "jt_w8a8_gemm_per_channel": [_i8p, _i8p, _fl, _vp, _f32p, _i, _i, _i],
    "jt_w8a8_fakequant_per_tensor": [_f32p, _sz, _f32p],
    "jt_w8a8_fakequant_per_channel": [_f32p, _sz, _sz, _f32p],
    "jt_gemm_mat_f32": [_f32p, _f32p, _f32p, _i, _i, _i],
    "jt_transpose_f32": [_f32p, _f32p, _i, _i],
    "jt_lowbit_set_mode": [_i],
    "jt_lowbit_get_mode": [],
    "jt_lowbit_bits_for": [_i, C.POINTER(_i)],
    "jt_lowbit_fakequant": [_f32p, _f32p, _sz, _i],
    "jt_lowbit_col_to_idx": [_f32p, _sz, _i, _u8p, _f32p],
    "jt_lowbit_gemm_lut": [_f32p, _f32p, _f32p, _i, _i, _i, _i],
    "jt_tmac_qlut_bytes": [_sz, _sz, C.POINTER(_sz)],
    "jt_tmac_param_bytes": [_sz, _sz, C.POINTER(_sz)],
    "jt_tmac_lut_ctor": [_f32p, _sz, _sz, _i8p, _f32p, _f32p],
    "jt_tmac_lookup_accum": [_i8p, _u8p, _f32p, _f32p, _sz, _sz, _i, _fl, _f32p],
    "jt_routing_topk": [_f32p, _sz, _sz, _u64p, _f32p],
    "jt_moe_batch_sort": [_u64p, _i, _i, _i, _fl, _u64p, _u64p, _u8p, _vp, _vp],
    "jt_moe_fwd_batch": [_vp] * 9 + [_i] * 6 + [_vp] * 7 + [_fl] + [_vp] * 5,
    "jt_moe_fwd_batch_unchecked": [_vp] * 9 + [_i] * 6 + [_vp] * 7 + [_fl] + [_vp] * 5,
    "jt_hip_init": [_i],
    "jt_hip_sync_errors": [_vp, C.POINTER(C.c_uint32)],
    "jt_hip_stream_forget": [_vp],
    "jt_hip_alloc_count": [C.POINTER(C.c_uint64)],
    "jt_hip_quant_rows": [_vp, _i, _i, _vp, _vp, _vp],
    "jt_hip_w8a8_prepare": [_vp, _i, _i, C.POINTER(_vp)],
    "jt_hip_w8a8_prepare_kn": [_vp, _vp, _i, _i, C.POINTER(_vp)],
    "jt_hip_w8a8_gemm": [_vp, _vp, _vp, _vp, _i, _vp],
    "jt_hip_w8a8_export": [_vp, _i8p, _f32p],
    "jt_hip_w8a8_free": ([_vp], None),
    "jt_hip_ffn_prepare": [_vp, _vp, _vp, _i, _i, C.POINTER(_vp)],
    "jt_hip_ffn_fwd": [_vp, _vp, _vp, _i, _vp],
    "jt_hip_ffn_fwd_noalloc": [_vp, _vp, _vp, _i, _vp],
    "jt_hip_ffn_reserve": [_vp, _i],
    "jt_hip_ffn_free": ([_vp], None),
    "jt_hip_moe_prepare": [C.POINTER(_Desc)] + [_vp] * 7 + [C.POINTER(_vp)],
    "jt_hip_moe_fwd": [_vp, _vp, _vp, _i, _vp],
    "jt_hip_moe_fwd_routed": [_vp, _vp, _vp, _vp, _vp, _i, _vp],
    "jt_hip_moe_fwd_residual": [_vp, _vp, _vp, _vp, _vp, _i, _vp],
    "jt_hip_moe_buffer": [_vp, _i, C.POINTER(_vp), C.POINTER(_sz)],
    "jt_hip_moe_export_routed": [_vp, _i, _u8p, _u16p, _u8p, _u16p],
    "jt_hip_moe_save": [_vp, _vp, _sz, C.POINTER(_sz)],
    "jt_hip_moe_load": [_vp, _sz, _i, C.POINTER(_vp)],
    "jt_hip_moe_set_profiling": [_vp, _i],
    "jt_hip_moe_stage_times": [_vp, C.POINTER(C.c_char_p), C.POINTER(C.c_double), _i,
                               C.POINTER(_i), C.POINTER(_i)],
    "jt_hip_moe_free": ([_vp], None),
    "jt_moe_bwd_batch": [_vp] * 28 + [_i] * 6,
    "jt_moe_bwd_batch_unchecked": [_vp] * 28 + [_i] * 6,
    "jt_hip_moe_bwd_batch_ws_bytes": ([_i] * 6, _sz),
    "jt_hip_moe_bwd_batch": [_vp] * 28 + [_i] * 7 + [_vp, _sz, _vp],
    "jt_gdn2_state_bytes": [_i, _i, C.POINTER(_sz)],
    "jt_gdn2_state_alloc": [C.POINTER(_vp), _i, _i],
    "jt_gdn2_state_free": ([_vp], None),
    "jt_gdn2_state_reset": [_vp, _i, _i],
    "jt_gdn2_scratch_floats": [_i, _i, C.POINTER(_sz)],
    "jt_gdn2_l2norm": [_vp, _vp, _i, _fl],
    "jt_gdn2_decode_step": [_vp] * 8 + [_i, _i, _vp, _sz],
    "jt_gdn2_prefill_chunk16": [_vp] * 8 + [_i, _i, _vp, _sz],
    "jt_gdn2_prefill_chunk32": [_vp] * 8 + [_i, _i, _vp, _sz],
    "jt_hip_gdn2_decode": [_vp] * 8 + [_i] * 3 + [_vp],
    "jt_hip_w8a8_gemm_f32_ws_bytes": ([_vp, _i], _sz),
    "jt_hip_w8a8_gemm_f32": [_vp, _vp, _vp, _i, _vp, _sz, _vp],
    "jt_hip_gdn2_prefill_ws_bytes": ([_i] * 4, _sz),
    "jt_hip_gdn2_prefill": [_vp] * 8 + [_i] * 5 + [_vp, _sz, _vp],
}


def lib() -> C.CDLL:
    """Load the HIP library (raises when it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C jimotono_amd/csrc` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH, use_errno=True)
        for name, spec in _PROTOS.items():
            fn = getattr(L, name)
            if isinstance(spec, tuple):
                fn.argtypes, fn.restype = spec
            else:
                fn.argtypes, fn.restype = spec, C.c_int
        _LIB = L
    return _LIB


def errno() -> int:
    return C.get_errno()


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------- host-pointer API (reference names) ----------------

def w8a8_quant_per_tensor(x):
    x = _c(x, np.float32).ravel()
    q = np.zeros(x.size, np.int8)
    s = np.zeros(1, np.float32)
    rc = lib().jt_w8a8_quant_per_tensor(x, x.size, q, s)
    return rc, q, s[0]


def w8a8_quant_per_channel(X):
    X = _c(X, np.float32)
    Q = np.zeros(X.shape, np.int8)
    s = np.zeros(X.shape[0], np.float32)
    rc = lib().jt_w8a8_quant_per_channel(X, X.shape[0], X.shape[1], Q, s)
    return rc, Q, s


def w8a8_dequant_per_tensor(q, scale):
    q = _c(q, np.int8).ravel()
    d = np.zeros(q.size, np.float32)
    rc = lib().jt_w8a8_dequant_per_tensor(q, float(scale), q.size, d)
    return rc, d


def w8a8_dequant_per_channel(Q, s):
    Q = _c(Q, np.int8)
    d = np.zeros(Q.shape, np.float32)
    rc = lib().jt_w8a8_dequant_per_channel(Q, _c(s, np.float32), Q.shape[0], Q.shape[1], d)
    return rc, d


def w8a8_fakequant_per_tensor(x):
    x = _c(x, np.float32).ravel()
    d = np.zeros_like(x)
    return lib().jt_w8a8_fakequant_per_tensor(x, x.size, d), d


def w8a8_fakequant_per_channel(X):
    X = _c(X, np.float32)
    d = np.zeros_like(X)
    return lib().jt_w8a8_fakequant_per_channel(X, X.shape[0], X.shape[1], d), d


def w8a8_gemm_per_tensor(Aq, Bq_kn, sA, sB, out=None):
    Aq, Bq = _c(Aq, np.int8), _c(Bq_kn, np.int8)
    M, K = Aq.shape
    N = Bq.shape[1]
    Cm = np.zeros((M, N), np.float32) if out is None else out
    rc = lib().jt_w8a8_gemm_per_tensor(Aq, Bq, float(sA), float(sB), Cm, M, N, K)
    return rc, Cm


def w8a8_gemm_per_channel(Aq, Bq_kn, sA, sB_col, out=None):
    Aq, Bq = _c(Aq, np.int8), _c(Bq_kn, np.int8)
    M, K = Aq.shape
    N = Bq.shape[1]
    Cm = np.zeros((M, N), np.float32) if out is None else out
    sB = None if sB_col is None else _c(sB_col, np.float32)
    rc = lib().jt_w8a8_gemm_per_channel(Aq, Bq, float(sA),
                                        None if sB is None else sB.ctypes.data, Cm, M, N, K)
    return rc, Cm


def gemm_mat_f32(A, B):
    A, B = _c(A, np.float32), _c(B, np.float32)
    out = np.zeros((A.shape[0], B.shape[1]), np.float32)
    return lib().jt_gemm_mat_f32(A, B, out, A.shape[0], B.shape[1], A.shape[1]), out


def transpose_f32(A):
    A = _c(A, np.float32)
    out = np.zeros((A.shape[1], A.shape[0]), np.float32)
    return lib().jt_transpose_f32(A, out, A.shape[0], A.shape[1]), out


def lowbit_fakequant(w, bits):
    w = _c(w, np.float32).ravel()
    out = np.zeros_like(w)
    return lib().jt_lowbit_fakequant(w, out, w.size, bits), out


def lowbit_col_to_idx(col, bits):
    col = _c(col, np.float32).ravel()
    idx = np.zeros(bits * (col.size // 4), np.uint8)
    ws = np.zeros(1, np.float32)
    rc = lib().jt_lowbit_col_to_idx(col, col.size, bits, idx, ws)
    return rc, idx, ws[0]


def lowbit_gemm_lut(X, W, bits):
    X, W = _c(X, np.float32), _c(W, np.float32)
    Y = np.zeros((X.shape[0], W.shape[1]), np.float32)
    return lib().jt_lowbit_gemm_lut(X, W, Y, X.shape[0], W.shape[1], X.shape[1], bits), Y


def tmac_lut_ctor(act):
    act = _c(act, np.float32)
    n, k = act.shape
    q = np.zeros((n, k // 4, 8), np.int8)
    s = np.zeros((n, k // 32), np.float32)
    b = np.zeros((n, k // 32), np.float32)
    return lib().jt_tmac_lut_ctor(act, n, k, q, s, b), q, s, b


def tmac_lookup_accum(qlut_row, idx, scales_row, biases_row, bits, w_scale):
    ng = qlut_row.size // 8
    out = np.zeros(1, np.float32)
    rc = lib().jt_tmac_lookup_accum(_c(qlut_row, np.int8).ravel(), _c(idx, np.uint8),
                                    _c(scales_row, np.float32), _c(biases_row, np.float32),
                                    ng, ng // 8, bits, w_scale, out)
    return rc, out[0]


def routing_topk(logits, k):
    logits = _c(logits, np.float32)
    ids = np.zeros(k, np.uint64)
    w = np.zeros(k, np.float32)
    rc = lib().jt_routing_topk(logits, logits.size, k, ids, w)
    return rc, ids.astype(np.int64), w


def moe_batch_sort(ids, T, k, E, cap_factor):
    ids = _c(ids, np.uint64).ravel()
    perm = np.zeros(T * k, np.uint64)
    off = np.zeros(E + 1, np.uint64)
    drop = np.zeros(T * k, np.uint8)
    kept, dropped = C.c_size_t(0), C.c_size_t(0)
    rc = lib().jt_moe_batch_sort(ids, T, k, E, cap_factor, perm, off, drop,
                                 C.addressof(kept), C.addressof(dropped))
    return rc, perm[: kept.value].astype(np.int64), off.astype(np.int64), drop, dropped.value


_BWD_OUT = ("dX", "dWgate", "dWg", "dWu", "dWd", "dWg_s", "dWu_s", "dWd_s", "dLogits")


def moe_bwd_batch(dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, w, Gsel, Usel, Ysel, Gs,
                  Us, perm, off, drop, k, unchecked=False, logits=True):
    """jt_moe_bwd_batch (or _unchecked) on numpy arrays: dY, X [T][n];
    W* [E][h][n] and [S][h][n] (Wg_s None for S = 0); ids, w [T][k];
    Gsel, Usel [T*k][h]; Ysel [T*k][n]; Gs, Us [T][S][h]; perm, off, drop
    as the forward returned them. Returns a dict of rc and the outputs
    (NaN-filled where the call wrote nothing)."""
    f = lambda a: _c(a, np.float32)
    dY, X, Wgate, Wg, Wu, Wd = map(f, (dY, X, Wgate, Wg, Wu, Wd))
    T, n = X.shape
    E, h = Wg.shape[0], Wg.shape[1]
    S = 0 if Wg_s is None else Wg_s.shape[0]
    ins = [dY, X, Wgate, Wg, Wu, Wd]
    ins += [None] * 3 if S == 0 else [f(Wg_s), f(Wu_s), f(Wd_s)]
    ins += [_c(ids, np.uint64), f(w), f(Gsel), f(Usel), f(Ysel)]
    ins += [None] * 2 if S == 0 else [f(Gs), f(Us)]
    pm = _c(perm, np.uint64)
    ins += [pm if pm.size else np.zeros(1, np.uint64), _c(off, np.uint64), _c(drop, np.uint8)]
    shapes = dict(dX=(T, n), dWgate=(E, n), dWg=(E, h, n), dWu=(E, h, n), dWd=(E, h, n))
    if S:
        shapes.update(dWg_s=(S, h, n), dWu_s=(S, h, n), dWd_s=(S, h, n))
    if logits:
        shapes["dLogits"] = (T, E)
    out = {nm: np.full(sh, np.nan, np.float32) for nm, sh in shapes.items()}
    ptr = lambda a: None if a is None else a.ctypes.data
    fn = lib().jt_moe_bwd_batch_unchecked if unchecked else lib().jt_moe_bwd_batch
    out["rc"] = fn(*[ptr(a) for a in ins], *[ptr(out.get(nm)) for nm in _BWD_OUT],
                   T, n, h, E, k, S)
    return out


def moe_bwd_batch_device(dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, w, Gsel, Usel,
                         Ysel, Gs, Us, perm, off, drop, k, validate=1, out=None, ws=None,
                         logits=True, stream=None):
    """jt_hip_moe_bwd_batch on torch tensors already on the GPU (ids, perm,
    off int64; drop uint8), asynchronous on `stream` (default: torch's
    current stream). `out` (dict of output tensors) and `ws` (uint8 tensor
    of jt_hip_moe_bwd_batch_ws_bytes) are allocated when not given.
    Returns (rc, out, ws); read the error bits with sync_errors()."""
    import torch
    T, n = X.shape
    E, h = Wg.shape[0], Wg.shape[1]
    S = 0 if Wg_s is None else Wg_s.shape[0]
    dev = X.device
    if out is None:
        out = dict(dX=torch.empty((T, n), device=dev), dWgate=torch.empty((E, n), device=dev),
                   dWg=torch.empty((E, h, n), device=dev), dWu=torch.empty((E, h, n), device=dev),
                   dWd=torch.empty((E, h, n), device=dev))
        if S:
            for nm in ("dWg_s", "dWu_s", "dWd_s"):
                out[nm] = torch.empty((S, h, n), device=dev)
        if logits:
            out["dLogits"] = torch.empty((T, E), device=dev)
    nb = lib().jt_hip_moe_bwd_batch_ws_bytes(T, n, h, E, k, S)
    if ws is None:
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    ptr = lambda a: None if a is None else a.data_ptr()
    ins = [dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, w, Gsel, Usel, Ysel, Gs, Us, perm,
           off, drop]
    st = _stream(stream)
    rc = lib().jt_hip_moe_bwd_batch(*[ptr(a) for a in ins],
                                    *[ptr(out.get(nm)) for nm in _BWD_OUT], T, n, h, E, k, S,
                                    int(validate), ptr(ws), ws.numel(), st)
    return rc, out, ws


# ---------------- Gated DeltaNet-2 (host pointers, reference names) ----------------

class _State:
    """A state from jt_gdn2_state_alloc (64-byte aligned host memory)."""

    def __init__(self, S):
        S = _c(S, np.float32)
        self.dk, self.dv = S.shape
        self.p = _vp()
        rc = lib().jt_gdn2_state_alloc(C.byref(self.p), self.dk, self.dv)
        if rc != JT_OK:
            raise RuntimeError(f"jt_gdn2_state_alloc rc={rc}")
        C.memmove(self.p, S.ctypes.data, S.nbytes)

    def read(self):
        a = np.empty((self.dk, self.dv), np.float32)
        C.memmove(a.ctypes.data, self.p, a.nbytes)
        return a

    def __del__(self):
        if getattr(self, "p", None):
            lib().jt_gdn2_state_free(self.p)


def gdn2_l2norm(x, eps=1e-6):
    x = _c(x, np.float32).ravel()
    y = np.full_like(x, np.nan)
    return lib().jt_gdn2_l2norm(x.ctypes.data, y.ctypes.data, x.size, eps), y


def gdn2_decode_step(S, q, k, v, b, w, alpha):
    """jt_gdn2_decode_step on a copy of S [dk][dv]; returns (rc, S', o)."""
    st = _State(S)
    f = lambda a: _c(a, np.float32).ravel()  # noqa: E731
    ins = [f(a) for a in (q, k, v, b, w, alpha)]
    o = np.full(st.dv, np.nan, np.float32)
    need = 2 * st.dk + 2 * st.dv
    scratch = np.zeros(need, np.float32)
    rc = lib().jt_gdn2_decode_step(st.p, o.ctypes.data, *[a.ctypes.data for a in ins],
                                   st.dk, st.dv, scratch.ctypes.data, need)
    return rc, st.read(), o


def gdn2_prefill_chunk(S, Q, K, V, B, W, A):
    """jt_gdn2_prefill_chunk16/32 (C = rows of Q) on a copy of S; returns
    (rc, S', Out)."""
    st = _State(S)
    Cn = Q.shape[0]
    f = lambda a: _c(a, np.float32)  # noqa: E731
    ins = [f(a) for a in (Q, K, V, B, W, A)]
    Out = np.full((Cn, st.dv), np.nan, np.float32)
    need = 4 * Cn * st.dk + 2 * Cn * st.dv + Cn * Cn + st.dk
    scratch = np.zeros(need, np.float32)
    fn = lib().jt_gdn2_prefill_chunk16 if Cn == 16 else lib().jt_gdn2_prefill_chunk32
    rc = fn(st.p, Out.ctypes.data, *[a.ctypes.data for a in ins], st.dk, st.dv,
            scratch.ctypes.data, need)
    return rc, st.read(), Out


def gdn2_decode_device(S, O, q, k, v, b, w, alpha, stream=None):
    """jt_hip_gdn2_decode on torch tensors: S [H][dk][dv] in place,
    O [H][dv], q/k/b/alpha [H][dk], v/w [H][dv]. Returns rc."""
    H, dk, dv = S.shape
    return lib().jt_hip_gdn2_decode(*[t.data_ptr() for t in (S, O, q, k, v, b, w, alpha)], H,
                                    dk, dv, _stream(stream))


def gdn2_prefill_device(S, Out, Q, K, V, B, W, A, C_, ws=None, stream=None):
    """jt_hip_gdn2_prefill on torch tensors: S [H][dk][dv] in place,
    Q/K/B/A [H][T][dk], V/W/Out [H][T][dv], chunks of C_ (16 or 32).
    Returns (rc, ws)."""
    import torch
    H, dk, dv = S.shape
    T = Q.shape[1]
    nb = lib().jt_hip_gdn2_prefill_ws_bytes(H, T, C_, dk)
    if ws is None or ws.numel() < nb:
        ws = torch.empty(nb, dtype=torch.uint8, device=S.device)
    rc = lib().jt_hip_gdn2_prefill(*[t.data_ptr() for t in (S, Out, Q, K, V, B, W, A)], H, T,
                                   C_, dk, dv, ws.data_ptr(), ws.numel(), _stream(stream))
    return rc, ws


def moe_fwd_batch(X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, k, cap_factor, unchecked=False,
                  caches=False):
    """jt_moe_fwd_batch with the process flags as currently set; caches=True
    also returns the backward's caches Gsel, Usel [T*k][h] and Gs, Us
    [T][S][h]."""
    X = _c(X, np.float32)
    T, n = X.shape
    E, h = Wg.shape[0], Wg.shape[1]
    S = 0 if Wg_s is None else Wg_s.shape[0]
    keep = [X, _c(Wgate, np.float32), _c(Wg, np.float32), _c(Wu, np.float32),
            _c(Wd, np.float32)]
    sh = [None, None, None] if S == 0 else [_c(a, np.float32) for a in (Wg_s, Wu_s, Wd_s)]
    Y = np.zeros((T, n), np.float32)
    ids = np.zeros((T, k), np.uint64)
    w = np.zeros((T, k), np.float32)
    perm = np.zeros(T * k, np.uint64)
    off = np.zeros(E + 1, np.uint64)
    drop = np.zeros(T * k, np.uint8)
    Ysel = np.zeros((T * k, n), np.float32)
    kept, dropped = C.c_size_t(0), C.c_size_t(0)
    cache = {}
    if caches:
        cache = dict(Gsel=np.zeros((T * k, h), np.float32), Usel=np.zeros((T * k, h), np.float32))
        if S:
            cache.update(Gs=np.zeros((T, S, h), np.float32), Us=np.zeros((T, S, h), np.float32))
    cp = lambda nm: cache[nm].ctypes.data if nm in cache else None
    fn = lib().jt_moe_fwd_batch_unchecked if unchecked else lib().jt_moe_fwd_batch
    p = [a.ctypes.data for a in keep] + [None if a is None else a.ctypes.data for a in sh]
    rc = fn(*p[:5], *p[5:], Y.ctypes.data, T, n, h, E, k, S, ids.ctypes.data, w.ctypes.data,
            cp("Gsel"), cp("Usel"), Ysel.ctypes.data, cp("Gs"), cp("Us"), cap_factor,
            perm.ctypes.data, off.ctypes.data, drop.ctypes.data, C.addressof(kept),
            C.addressof(dropped))
    return dict(rc=rc, Y=Y, ids=ids.astype(np.int64), w=w,
                perm=perm[: kept.value].astype(np.int64), off=off.astype(np.int64),
                drop=drop, Ysel=Ysel, **cache)


# ---------------- device-resident API ----------------

def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream):
    """HIP stream handle for a call: torch's current stream when None (its
    default stream is the HIP null stream, handle 0, which the library takes
    as the null stream too), so the call is ordered with the caller's torch
    work on that stream."""
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _check(rc, what):
    if rc != JT_OK:
        raise RuntimeError(f"{what} failed: rc={rc} errno={errno()}")


_HIP = None


def d2h(out: np.ndarray, dptr: int) -> None:
    """Synchronous device-to-host copy of out.nbytes bytes (HIP runtime)."""
    global _HIP
    if _HIP is None:
        lib()
        _HIP = C.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.argtypes = [_vp, _vp, _sz, _i]
        _HIP.hipDeviceSynchronize.argtypes = []
    _check(_HIP.hipDeviceSynchronize(), "hipDeviceSynchronize")
    _check(_HIP.hipMemcpy(out.ctypes.data, dptr, out.nbytes, 2), "hipMemcpy")


def sync_errors(stream=None) -> int:
    f = C.c_uint32(0)
    _check(lib().jt_hip_sync_errors(_stream(stream), C.byref(f)), "jt_hip_sync_errors")
    return f.value


def stream_forget(stream) -> None:
    """Release the device error word of `stream` (call before the stream is
    destroyed; HIP may reuse its handle for a later stream)."""
    _check(lib().jt_hip_stream_forget(_stream(stream)), "jt_hip_stream_forget")


def alloc_count() -> int:
    """Device allocations the library has made so far in this process."""
    v = C.c_uint64(0)
    _check(lib().jt_hip_alloc_count(C.byref(v)), "jt_hip_alloc_count")
    return v.value


def quant_rows(X, Xq, scale, stream=None):
    _check(lib().jt_hip_quant_rows(_ptr(X), X.shape[0], X.shape[1], _ptr(Xq), _ptr(scale),
                                   _stream(stream)), "jt_hip_quant_rows")


class W8A8:
    """Prepared W8A8 weights W [N][K] (fp32 cuda tensor, quantised on the GPU)."""

    def __init__(self, W=None, Bq_kn=None, sB=None):
        h = C.c_void_p()
        if W is not None:
            self.N, self.K = W.shape
            _check(lib().jt_hip_w8a8_prepare(_ptr(W), self.N, self.K, C.byref(h)),
                   "jt_hip_w8a8_prepare")
        else:
            self.K, self.N = Bq_kn.shape
            _check(lib().jt_hip_w8a8_prepare_kn(_ptr(Bq_kn), _ptr(sB), self.N, self.K,
                                                C.byref(h)), "jt_hip_w8a8_prepare_kn")
        self.h = h

    def gemm(self, Aq, sA, out, stream=None):
        _check(lib().jt_hip_w8a8_gemm(self.h, _ptr(Aq), _ptr(sA), _ptr(out), Aq.shape[0],
                                      _stream(stream)), "jt_hip_w8a8_gemm")

    def gemm_f32(self, X, out, ws=None, stream=None):
        """out [M][N] = the per-token INT8 projection of fp32 X [M][K]
        (jt_hip_w8a8_gemm_f32); returns the workspace it used (M > 16)."""
        import torch
        M = X.shape[0]
        nb = lib().jt_hip_w8a8_gemm_f32_ws_bytes(self.h, M)
        if nb and (ws is None or ws.numel() < nb):
            ws = torch.empty(nb, dtype=torch.uint8, device=X.device)
        _check(lib().jt_hip_w8a8_gemm_f32(self.h, _ptr(X), _ptr(out), M,
                                          _ptr(ws) if nb else None, nb, _stream(stream)),
               "jt_hip_w8a8_gemm_f32")
        return ws

    def export(self):
        Bq = np.zeros((self.K, self.N), np.int8)
        sB = np.zeros(self.N, np.float32)
        _check(lib().jt_hip_w8a8_export(self.h, Bq, sB), "jt_hip_w8a8_export")
        return Bq, sB

    def __del__(self):
        if getattr(self, "h", None) and _LIB is not None:
            _LIB.jt_hip_w8a8_free(self.h)
            self.h = None


class FFN:
    """One W8A8 SwiGLU expert (the shared-expert block)."""

    def __init__(self, Wg, Wu, Wd):
        self.h_, self.n = Wg.shape
        h = C.c_void_p()
        _check(lib().jt_hip_ffn_prepare(_ptr(Wg), _ptr(Wu), _ptr(Wd), self.n, self.h_,
                                        C.byref(h)), "jt_hip_ffn_prepare")
        self.h = h

    def fwd(self, X, Y, stream=None):
        _check(lib().jt_hip_ffn_fwd(self.h, _ptr(X), _ptr(Y), X.shape[0], _stream(stream)),
               "jt_hip_ffn_fwd")

    def reserve(self, T):
        """jt_hip_ffn_reserve: size the own workspace for T rows now."""
        _check(lib().jt_hip_ffn_reserve(self.h, T), "jt_hip_ffn_reserve")

    def fwd_noalloc(self, X, Y, stream=None):
        """jt_hip_ffn_fwd_noalloc: the same forward on the library's fixed
        device scratch; returns the return code (JT_ERR_NOSUP when T is too
        large for the scratch)."""
        return lib().jt_hip_ffn_fwd_noalloc(self.h, _ptr(X), _ptr(Y), X.shape[0],
                                            _stream(stream))

    def __del__(self):
        if getattr(self, "h", None) and _LIB is not None:
            _LIB.jt_hip_ffn_free(self.h)
            self.h = None


(BUF_IDS, BUF_WEIGHTS, BUF_PERM, BUF_OFF, BUF_XQ, BUF_XSCALE, BUF_YE, BUF_YS, BUF_LOGITS,
 BUF_HQ, BUF_HSCALE) = range(11)


class MoE:
    """Prepared quantised MoE layer (jt_hip_moe)."""

    def __init__(self, n, h, E, k, S, hs, max_tokens, Wgate, Wg, Wu, Wd, Wg_s=None,
                 Wu_s=None, Wd_s=None, group=64, _handle=None):
        self.desc = _Desc(n, h, E, k, S, hs, group, max_tokens)
        self.n, self.h, self.E, self.k, self.S, self.hs = n, h, E, k, S, hs
        if _handle is not None:
            self.h_ = _handle
            return
        hd = C.c_void_p()
        _check(lib().jt_hip_moe_prepare(C.byref(self.desc), _ptr(Wgate), _ptr(Wg), _ptr(Wu),
                                        _ptr(Wd), _ptr(Wg_s), _ptr(Wu_s), _ptr(Wd_s),
                                        C.byref(hd)), "jt_hip_moe_prepare")
        self.h_ = hd

    def save(self) -> bytes:
        """The layer serialised by jt_hip_moe_save."""
        nb = C.c_size_t()
        _check(lib().jt_hip_moe_save(self.h_, None, 0, C.byref(nb)), "jt_hip_moe_save")
        buf = C.create_string_buffer(nb.value)
        _check(lib().jt_hip_moe_save(self.h_, buf, nb.value, C.byref(nb)), "jt_hip_moe_save")
        return buf.raw

    @classmethod
    def load(cls, data: bytes, max_tokens: int):
        """A layer rebuilt from save()'s bytes by jt_hip_moe_load (raises on a
        bad buffer; rc and errno as the C function)."""
        hd = C.c_void_p()
        rc = lib().jt_hip_moe_load(data, len(data), max_tokens, C.byref(hd))
        if rc != JT_OK:
            raise ValueError(f"jt_hip_moe_load rc={rc} errno={errno()}")
        f = np.frombuffer(data[16:44], np.int32)
        return cls(int(f[0]), int(f[1]), int(f[2]), int(f[3]), int(f[4]), int(f[5]),
                   max_tokens, None, None, None, None, group=int(f[6]), _handle=hd)

    def fwd(self, X, Y, stream=None):
        return lib().jt_hip_moe_fwd(self.h_, _ptr(X), _ptr(Y), X.shape[0], _stream(stream))

    def fwd_routed(self, X, ids, w, Y, stream=None):
        return lib().jt_hip_moe_fwd_routed(self.h_, _ptr(X), _ptr(ids), _ptr(w), _ptr(Y),
                                           X.shape[0], _stream(stream))

    def fwd_residual(self, X, Y, ids=None, w=None, stream=None):
        """Y = X + layer(X) with the reference's two roundings (Y may be X)."""
        return lib().jt_hip_moe_fwd_residual(self.h_, _ptr(X), _ptr(ids), _ptr(w), _ptr(Y),
                                             X.shape[0], _stream(stream))

    def buffer(self, which):
        p, nb = C.c_void_p(), C.c_size_t()
        _check(lib().jt_hip_moe_buffer(self.h_, which, C.byref(p), C.byref(nb)),
               "jt_hip_moe_buffer")
        return p.value, nb.value

    def read(self, which, dtype, shape):
        """Copy one of the layer's device buffers to a numpy array."""
        p, nb = self.buffer(which)
        out = np.empty(shape, dtype)
        if out.nbytes != nb:
            raise ValueError(f"buffer {which} holds {nb} bytes, asked for {out.nbytes}")
        d2h(out, p)
        return out

    def export_routed(self, e):
        n, h = self.n, self.h
        gu = np.zeros((2, h, n), np.uint8)
        gus = np.zeros((2, h, n // 64), np.uint16)
        dc = np.zeros((n, h), np.uint8)
        ds = np.zeros((n, h // 64), np.uint16)
        _check(lib().jt_hip_moe_export_routed(self.h_, e, gu, gus, dc, ds),
               "jt_hip_moe_export_routed")
        return gu, gus, dc, ds

    def set_profiling(self, on):
        _check(lib().jt_hip_moe_set_profiling(self.h_, 1 if on else 0), "set_profiling")

    def stage_times(self):
        names = (C.c_char_p * 32)()
        ms = (C.c_double * 32)()
        n, cnt = C.c_int(), C.c_int()
        _check(lib().jt_hip_moe_stage_times(self.h_, names, ms, 32, C.byref(n), C.byref(cnt)),
               "stage_times")
        return {names[i].decode(): ms[i] for i in range(n.value)}, cnt.value

    def __del__(self):
        if getattr(self, "h_", None) and _LIB is not None:
            _LIB.jt_hip_moe_free(self.h_)
            self.h_ = None
