"""ctypes bindings of the CPU checkers (TEST INFRASTRUCTURE ONLY).

Two libraries are wrapped:

* ``Oracle``  -- oracle/liboracle.so, the C11 restatement (jt_oracle.c);
* ``RefLib``  -- oracle/_ref/libjtref.so, the reference's own hot-path
  translation units compiled from the reference sources by
  ``make -C oracle ref`` (absent when the reference checkout is not present
  at build time; callers must then skip).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libjtref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class _OrMoeQ(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n", "h", "E", "k", "S", "hs", "group")] + [
        ("Wgate", C.c_void_p),
        ("gu_codes", C.c_void_p),
        ("gu_scales", C.c_void_p),
        ("d_codes", C.c_void_p),
        ("d_scales", C.c_void_p),
        ("sgu_q", C.c_void_p),
        ("sgu_s", C.c_void_p),
        ("sd_q", C.c_void_p),
        ("sd_s", C.c_void_p),
    ]


def bwd_batch_call(fn, idx_dtype, dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, w,
                   Gsel, Usel, Ysel, Gs, Us, perm, off, drop, k, extra=(), logits=True):
    """Call a jt_moe_bwd_batch-shaped function (the reference's, the
    oracle's or the device library's host-pointer entry). Shapes: dY, X
    [T][n]; W* [E][h][n] / [S][h][n]; ids, w [T][k]; Gsel, Usel [T*k][h];
    Ysel [T*k][n]; Gs, Us [T][S][h]; perm [kept]; off [E+1]; drop [T*k].
    Returns a dict of rc and the outputs."""
    f32 = lambda a: _c(a, np.float32)
    dY, X, Wgate, Wg, Wu, Wd = map(f32, (dY, X, Wgate, Wg, Wu, Wd))
    T, n = X.shape
    E, h = Wg.shape[0], Wg.shape[1]
    S = 0 if Wg_s is None else Wg_s.shape[0]
    ins = [dY, X, Wgate, Wg, Wu, Wd]
    ins += [None, None, None] if S == 0 else [f32(Wg_s), f32(Wu_s), f32(Wd_s)]
    ins += [_c(ids, idx_dtype), f32(w), f32(Gsel), f32(Usel), f32(Ysel)]
    ins += [None, None] if S == 0 else [f32(Gs), f32(Us)]
    permc = _c(perm, idx_dtype)
    if permc.size == 0:
        permc = np.zeros(1, idx_dtype)
    ins += [permc, _c(off, idx_dtype), _c(drop, np.uint8)]
    out = dict(dX=np.full((T, n), np.nan, np.float32),
               dWgate=np.full((E, n), np.nan, np.float32),
               dWg=np.full((E, h, n), np.nan, np.float32),
               dWu=np.full((E, h, n), np.nan, np.float32),
               dWd=np.full((E, h, n), np.nan, np.float32))
    if S:
        for nm in ("dWg_s", "dWu_s", "dWd_s"):
            out[nm] = np.full((S, h, n), np.nan, np.float32)
    if logits:
        out["dLogits"] = np.full((T, E), np.nan, np.float32)
    outs = [out["dX"], out["dWgate"], out["dWg"], out["dWu"], out["dWd"],
            out.get("dWg_s"), out.get("dWu_s"), out.get("dWd_s"), out.get("dLogits")]
    ptr = lambda a: None if a is None else a.ctypes.data
    rc = fn(*[ptr(a) for a in ins + outs], T, n, h, E, k, S, *extra)
    out["rc"] = rc
    return out


class Oracle:
    """The C restatement. Every method returns numpy arrays (or raises)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.or_quant_row.argtypes = [_f32p, C.c_size_t, _i8p, _f32p]
        L.or_quant_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i8p, _f32p]
        L.or_dequant_rows.argtypes = [_i8p, _f32p, C.c_size_t, C.c_size_t, _f32p]
        L.or_fakequant_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p]
        L.or_w8a8_gemm.argtypes = [_i8p, _f32p, C.c_int, _i8p, _f32p, C.c_int,
                                   _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int]
        L.or_gemm_f32.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.or_gemm_f32.restype = None
        L.or_lowbit_code.argtypes = [C.c_double, C.c_double, C.c_int]
        L.or_lowbit_fakequant.argtypes = [_f32p, _f32p, C.c_size_t, C.c_int]
        L.or_lowbit_col_to_idx.argtypes = [_f32p, C.c_size_t, C.c_int, _u8p, _f32p]
        L.or_f64_to_f16.argtypes = [C.c_double]
        L.or_f64_to_f16.restype = C.c_uint16
        L.or_f16_to_f64.argtypes = [C.c_uint16]
        L.or_f16_to_f64.restype = C.c_double
        L.or_lowbit_pack_rows.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                          _u8p, _u16p]
        L.or_gemm_lowbit_group.argtypes = [_i8p, _f32p, _u8p, _u16p, C.c_int, C.c_int,
                                           _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int]
        L.or_tmac_lut_ctor.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i8p, _f32p, _f32p]
        L.or_tmac_lookup_accum.argtypes = [_i8p, _u8p, _f32p, _f32p, C.c_size_t,
                                           C.c_size_t, C.c_int, C.c_float, _f32p]
        L.or_lowbit_gemm_lut.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int,
                                         C.c_int]
        L.or_logit_lane4.argtypes = [_f32p, _f32p, C.c_int]
        L.or_logit_lane4.restype = C.c_double
        L.or_topk.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i64p, _f32p]
        L.or_router.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, _i64p,
                                _f32p, _f32p]
        L.or_batch_sort.argtypes = [_i64p, C.c_int, C.c_int, C.c_int, C.c_float, _i64p,
                                    _i64p, _u8p, C.c_void_p]
        L.or_silu_mul.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_float)]
        L.or_moe_fwd_batch.argtypes = [_f32p] * 9 + [C.c_int] * 6 + [
            _i64p, _f32p, C.c_float, _i64p, _i64p, _u8p, C.POINTER(C.c_int64),
            C.c_int, C.c_int, C.c_void_p]
        L.or_moe_q_prepare.argtypes = [C.POINTER(_OrMoeQ)] + [C.c_int] * 7 + [C.c_void_p] * 7
        L.or_moe_q_free.argtypes = [C.POINTER(_OrMoeQ)]
        L.or_moe_q_free.restype = None
        L.or_moe_q_fwd.argtypes = [C.POINTER(_OrMoeQ), _f32p, C.c_int, C.c_void_p,
                                   C.c_void_p, _f32p] + [C.c_void_p] * 8
        L.or_ffn_fwd.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, _f32p, C.c_int,
                                 _f32p]
        L.or_residual_add.argtypes = [_f32p, _f32p, _f32p, C.c_size_t]
        L.or_moe_bwd_batch.argtypes = [C.c_void_p] * 28 + [C.c_int] * 7
        L.or_gdn2_l2norm.argtypes = [_f32p, _f32p, C.c_int, C.c_float]
        L.or_gdn2_decode_step.argtypes = [_f32p] * 8 + [C.c_int] * 2
        L.or_gdn2_prefill_chunk.argtypes = [_f32p] * 8 + [C.c_int] * 3

    # ---- W8A8 ----
    def quant_rows(self, X):
        X = _c(X, np.float32)
        rows, cols = X.shape
        Q = np.zeros((rows, cols), np.int8)
        s = np.zeros(rows, np.float32)
        rc = self.lib.or_quant_rows(X, rows, cols, Q, s)
        return rc, Q, s

    def quant_tensor(self, x):
        x = _c(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        s = np.zeros(1, np.float32)
        rc = self.lib.or_quant_row(x, x.size, q, s)
        return rc, q, s[0]

    def fakequant_rows(self, X):
        X = _c(X, np.float32)
        out = np.zeros_like(X)
        rc = self.lib.or_fakequant_rows(X, X.shape[0], X.shape[1], out)
        return rc, out

    def dequant_rows(self, Q, s):
        Q = _c(Q, np.int8)
        out = np.zeros(Q.shape, np.float32)
        rc = self.lib.or_dequant_rows(Q, _c(s, np.float32), Q.shape[0], Q.shape[1], out)
        return rc, out

    def w8a8_gemm(self, Aq, sA, Bq_kn, sB):
        """Aq [M][K], sA [M] or scalar, Bq_kn [K][N], sB [N] or scalar."""
        Aq = _c(Aq, np.int8)
        Bq = _c(Bq_kn, np.int8)
        M, K = Aq.shape
        N = Bq.shape[1]
        sA = np.atleast_1d(_c(sA, np.float32))
        sB = np.atleast_1d(_c(sB, np.float32))
        Cm = np.zeros((M, N), np.float32)
        acc = np.zeros((M, N), np.int32)
        rc = self.lib.or_w8a8_gemm(Aq, sA, int(sA.size > 1), Bq, sB, int(sB.size > 1),
                                   Cm, acc.ctypes.data, M, N, K)
        return rc, Cm, acc

    def gemm_f32(self, A, B):
        A = _c(A, np.float32)
        B = _c(B, np.float32)
        out = np.zeros((A.shape[0], B.shape[1]), np.float32)
        self.lib.or_gemm_f32(A, B, out, A.shape[0], B.shape[1], A.shape[1])
        return out

    # ---- low-bit ----
    def f64_to_f16(self, x):
        return self.lib.or_f64_to_f16(float(x))

    def lowbit_pack_rows(self, W, bits, group=64):
        W = _c(W, np.float32)
        N, K = W.shape
        codes = np.zeros((N, K), np.uint8)
        scales = np.zeros((N, K // group), np.uint16)
        rc = self.lib.or_lowbit_pack_rows(W, N, K, bits, group, codes, scales)
        return rc, codes, scales

    def gemm_lowbit_group(self, Aq, sA, codes, scales, bits, group=64):
        Aq = _c(Aq, np.int8)
        M, K = Aq.shape
        N = codes.shape[0]
        out = np.zeros((M, N), np.float32)
        acc = np.zeros((M, N, K // group), np.int32)
        rc = self.lib.or_gemm_lowbit_group(Aq, _c(sA, np.float32), _c(codes, np.uint8),
                                           _c(scales, np.uint16), bits, group, out,
                                           acc.ctypes.data, M, N, K)
        return rc, out, acc

    def lowbit_fakequant(self, w, bits):
        w = _c(w, np.float32).ravel()
        out = np.zeros_like(w)
        rc = self.lib.or_lowbit_fakequant(w, out, w.size, bits)
        return rc, out

    def col_to_idx(self, col, bits):
        col = _c(col, np.float32).ravel()
        idx = np.zeros(bits * (col.size // 4), np.uint8)
        ws = np.zeros(1, np.float32)
        rc = self.lib.or_lowbit_col_to_idx(col, col.size, bits, idx, ws)
        return rc, idx, ws[0]

    def tmac_lut_ctor(self, act):
        act = _c(act, np.float32)
        n, k = act.shape
        q = np.zeros((n, k // 4, 8), np.int8)
        s = np.zeros((n, k // 32), np.float32)
        b = np.zeros((n, k // 32), np.float32)
        rc = self.lib.or_tmac_lut_ctor(act, n, k, q, s, b)
        return rc, q, s, b

    def tmac_lookup_accum(self, qlut_row, idx, scales_row, biases_row, bits, w_scale):
        ng = qlut_row.size // 8
        out = np.zeros(1, np.float32)
        rc = self.lib.or_tmac_lookup_accum(_c(qlut_row, np.int8), _c(idx, np.uint8),
                                           _c(scales_row, np.float32),
                                           _c(biases_row, np.float32), ng, ng // 8, bits,
                                           w_scale, out)
        return rc, out[0]

    def lowbit_gemm_lut(self, X, W, bits):
        X = _c(X, np.float32)
        W = _c(W, np.float32)
        me, k = X.shape
        h = W.shape[1]
        Y = np.zeros((me, h), np.float32)
        rc = self.lib.or_lowbit_gemm_lut(X, W, Y, me, h, k, bits)
        return rc, Y

    # ---- routing ----
    def logit_lane4(self, x, w):
        return self.lib.or_logit_lane4(_c(x, np.float32), _c(w, np.float32), len(x))

    def topk(self, logits, k):
        logits = _c(logits, np.float32)
        ids = np.zeros(k, np.int64)
        w = np.zeros(k, np.float32)
        rc = self.lib.or_topk(logits, logits.size, k, ids, w)
        return rc, ids, w

    def router(self, X, Wgate, k):
        X = _c(X, np.float32)
        Wgate = _c(Wgate, np.float32)
        T, n = X.shape
        E = Wgate.shape[0]
        ids = np.zeros((T, k), np.int64)
        w = np.zeros((T, k), np.float32)
        logits = np.zeros((T, E), np.float32)
        rc = self.lib.or_router(X, Wgate, T, E, n, k, ids, w, logits)
        return rc, ids, w, logits

    def batch_sort(self, ids, T, k, E, cap_factor):
        ids = _c(ids, np.int64).ravel()
        perm = np.full(T * k, -1, np.int64)
        off = np.zeros(E + 1, np.int64)
        drop = np.zeros(T * k, np.uint8)
        kept = C.c_int64(0)
        rc = self.lib.or_batch_sort(ids, T, k, E, cap_factor, perm, off, drop,
                                    C.addressof(kept))
        return rc, perm[: kept.value], off, drop

    def silu_mul(self, g, u):
        s = C.c_float(0)
        rc = self.lib.or_silu_mul(float(g), float(u), C.byref(s))
        return rc, s.value

    # ---- layers ----
    def moe_fwd_batch(self, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, k, cap_factor,
                      w8a8_on=0, lowbit_mode=0):
        X = _c(X, np.float32)
        T, n = X.shape
        E, h = Wg.shape[0], Wg.shape[1]
        S = 0 if Wg_s is None else Wg_s.shape[0]
        z = np.zeros(1, np.float32)
        Y = np.zeros((T, n), np.float32)
        ids = np.zeros((T, k), np.int64)
        w = np.zeros((T, k), np.float32)
        perm = np.zeros(T * k, np.int64)
        off = np.zeros(E + 1, np.int64)
        drop = np.zeros(T * k, np.uint8)
        kept = C.c_int64(0)
        Ysel = np.zeros((T * k, n), np.float32)
        rc = self.lib.or_moe_fwd_batch(
            X, _c(Wgate, np.float32), _c(Wg, np.float32), _c(Wu, np.float32),
            _c(Wd, np.float32), z if S == 0 else _c(Wg_s, np.float32),
            z if S == 0 else _c(Wu_s, np.float32), z if S == 0 else _c(Wd_s, np.float32),
            Y, T, n, h, E, k, S, ids, w, cap_factor, perm, off, drop, C.byref(kept),
            w8a8_on, lowbit_mode, Ysel.ctypes.data)
        return dict(rc=rc, Y=Y, ids=ids, w=w, perm=perm[: kept.value], off=off,
                    drop=drop, Ysel=Ysel)

    def ffn_fwd(self, Wg, Wu, Wd, X):
        X = _c(X, np.float32)
        T, n = X.shape
        h = Wg.shape[0]
        Y = np.zeros((T, n), np.float32)
        rc = self.lib.or_ffn_fwd(_c(Wg, np.float32), _c(Wu, np.float32), _c(Wd, np.float32),
                                 n, h, X, T, Y)
        return rc, Y

    def residual_add(self, X, Mo):
        X = _c(X, np.float32)
        Y = np.zeros_like(X)
        rc = self.lib.or_residual_add(X.ravel(), _c(Mo, np.float32).ravel(), Y.reshape(-1),
                                      X.size)
        return rc, Y

    def gdn2_l2norm(self, x, eps=1e-6):
        x = _c(x, np.float32).ravel()
        y = np.full_like(x, np.nan)
        return self.lib.or_gdn2_l2norm(x, y, x.size, eps), y

    def gdn2_decode_step(self, S, q, k, v, b, w, alpha):
        """One step on a copy of S; returns rc, S', o."""
        S = np.array(S, np.float32, order="C", copy=True)
        dk, dv = S.shape
        o = np.full(dv, np.nan, np.float32)
        f = lambda a: _c(a, np.float32).ravel()  # noqa: E731
        rc = self.lib.or_gdn2_decode_step(S, o, f(q), f(k), f(v), f(b), f(w), f(alpha), dk, dv)
        return rc, S, o

    def gdn2_prefill_chunk(self, S, Q, K, V, B, W, A):
        """One chunk (C = rows of Q) on a copy of S; returns rc, S', Out."""
        S = np.array(S, np.float32, order="C", copy=True)
        dk, dv = S.shape
        C_ = Q.shape[0]
        Out = np.full((C_, dv), np.nan, np.float32)
        f = lambda a: _c(a, np.float32)  # noqa: E731
        rc = self.lib.or_gdn2_prefill_chunk(S, Out, f(Q), f(K), f(V), f(B), f(W), f(A), dk, dv,
                                            C_)
        return rc, S, Out

    def moe_bwd_batch(self, *args, validate=1, **kw):
        """or_moe_bwd_batch; arguments as bwd_batch_call."""
        return bwd_batch_call(self.lib.or_moe_bwd_batch, np.int64, *args,
                              extra=(validate,), **kw)

    def moe_q(self, n, h, E, k, S, hs, Wgate, Wg, Wu, Wd, Wg_s=None, Wu_s=None,
              Wd_s=None, group=64):
        return OracleMoeQ(self, n, h, E, k, S, hs, group, Wgate, Wg, Wu, Wd, Wg_s, Wu_s,
                          Wd_s)


class OracleMoeQ:
    """Prepared quantised layer of the oracle (mirror of jt_hip_moe)."""

    def __init__(self, orc, n, h, E, k, S, hs, group, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s):
        self.o = orc
        self.keep = [None if a is None else _c(a, np.float32)
                     for a in (Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s)]
        ptr = [None if a is None else a.ctypes.data for a in self.keep]
        self.st = _OrMoeQ()
        rc = orc.lib.or_moe_q_prepare(C.byref(self.st), n, h, E, k, S, hs, group, *ptr)
        if rc != 0:
            raise ValueError(f"or_moe_q_prepare rc={rc}")
        self.n, self.h, self.E, self.k, self.S, self.hs, self.group = n, h, E, k, S, hs, group

    def __del__(self):
        try:
            self.o.lib.or_moe_q_free(C.byref(self.st))
        except Exception:
            pass

    def routed_codes(self, e):
        n, h, g = self.n, self.h, self.group
        nh = n * h
        gu = np.ctypeslib.as_array(C.cast(self.st.gu_codes, C.POINTER(C.c_uint8)),
                                   (self.E * 2 * nh,))[e * 2 * nh:(e + 1) * 2 * nh]
        gus = np.ctypeslib.as_array(C.cast(self.st.gu_scales, C.POINTER(C.c_uint16)),
                                    (self.E * 2 * nh // g,))[e * 2 * nh // g:(e + 1) * 2 * nh // g]
        dc = np.ctypeslib.as_array(C.cast(self.st.d_codes, C.POINTER(C.c_uint8)),
                                   (self.E * nh,))[e * nh:(e + 1) * nh]
        ds = np.ctypeslib.as_array(C.cast(self.st.d_scales, C.POINTER(C.c_uint16)),
                                   (self.E * nh // g,))[e * nh // g:(e + 1) * nh // g]
        return (gu.reshape(2, h, n).copy(), gus.reshape(2, h, n // g).copy(),
                dc.reshape(n, h).copy(), ds.reshape(n, h // g).copy())

    def fwd(self, X, ids=None, w=None):
        X = _c(X, np.float32)
        T = X.shape[0]
        k, E, n, S = self.k, self.E, self.n, self.S
        Y = np.zeros((T, n), np.float32)
        ids_o = np.zeros((T, k), np.int32)
        w_o = np.zeros((T, k), np.float32)
        perm = np.zeros(T * k, np.int32)
        off = np.zeros(E + 1, np.int32)
        Ye = np.zeros((T * k, n), np.float32)
        Ys = np.zeros((max(S, 1), T, n), np.float32)
        Hq = np.zeros((T * k, self.h), np.int8)
        Hs = np.zeros(T * k, np.float32)
        ids_in = None if ids is None else _c(ids, np.int32)
        w_in = None if w is None else _c(w, np.float32)
        rc = self.o.lib.or_moe_q_fwd(
            C.byref(self.st), X, T, None if ids_in is None else ids_in.ctypes.data,
            None if w_in is None else w_in.ctypes.data, Y, ids_o.ctypes.data,
            w_o.ctypes.data, perm.ctypes.data, off.ctypes.data, Ye.ctypes.data,
            Ys.ctypes.data, Hq.ctypes.data, Hs.ctypes.data)
        # Hq/Hs: the routed hidden rows' int8 codes and scales in sorted order
        return dict(rc=rc, Y=Y, ids=ids_o, w=w_o, perm=perm, off=off, Ye=Ye, Ys=Ys[:S],
                    Hq=Hq, Hs=Hs)


class RefLib:
    """The reference's own hot-path functions (oracle/_ref/libjtref.so)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.jt_w8a8_quant_per_tensor.argtypes = [_f32p, C.c_size_t, _i8p, _f32p]
        L.jt_w8a8_quant_per_channel.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i8p, _f32p]
        L.jt_w8a8_dequant_per_channel.argtypes = [_i8p, _f32p, C.c_size_t, C.c_size_t,
                                                  _f32p]
        L.jt_w8a8_dequant_per_tensor.argtypes = [_i8p, C.c_float, C.c_size_t, _f32p]
        L.jt_w8a8_fakequant_per_tensor.argtypes = [_f32p, C.c_size_t, _f32p]
        L.jt_w8a8_fakequant_per_channel.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p]
        L.jt_w8a8_gemm_per_channel.argtypes = [_i8p, _i8p, C.c_float, _f32p, _f32p,
                                               C.c_int, C.c_int, C.c_int]
        L.jt_w8a8_gemm_per_tensor.argtypes = [_i8p, _i8p, C.c_float, C.c_float, _f32p,
                                              C.c_int, C.c_int, C.c_int]
        L.jt_w8a8_set_enabled.argtypes = [C.c_int]
        L.jt_gemm_mat_f32.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.jt_transpose_f32.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        L.jt_lowbit_set_mode.argtypes = [C.c_int]
        L.jt_lowbit_fakequant.argtypes = [_f32p, _f32p, C.c_size_t, C.c_int]
        L.jt_lowbit_col_to_idx.argtypes = [_f32p, C.c_size_t, C.c_int, _u8p, _f32p]
        L.jt_lowbit_gemm_lut.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int,
                                         C.c_int]
        L.jt_tmac_lut_ctor.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i8p, _f32p, _f32p]
        L.jt_tmac_lookup_accum.argtypes = [_i8p, _u8p, _f32p, _f32p, C.c_size_t,
                                           C.c_size_t, C.c_int, C.c_float, _f32p]
        L.jt_routing_topk.argtypes = [_f32p, C.c_size_t, C.c_size_t, _u64p, _f32p]
        L.jt_moe_batch_sort.argtypes = [_u64p, C.c_int, C.c_int, C.c_int, C.c_float, _u64p,
                                        _u64p, _u8p, C.c_void_p, C.c_void_p]
        L.jt_moe_fwd_batch.argtypes = [_f32p] * 9 + [C.c_int] * 6 + [
            _u64p, _f32p] + [C.c_void_p] * 5 + [C.c_float, _u64p, _u64p, _u8p,
                                                C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.jt_moe_fwd.argtypes = [_f32p] * 9 + [C.c_int] * 5 + [_u64p, _f32p, _f32p] + [
            C.c_void_p] * 5
        for fn in (L.jt_moe_bwd_batch, L.jt_moe_bwd_batch_unchecked):
            fn.argtypes = [C.c_void_p] * 28 + [C.c_int] * 6
        L.jt_gdn2_l2norm.argtypes = [_f32p, _f32p, C.c_int, C.c_float]
        L.jt_gdn2_state_alloc.argtypes = [C.POINTER(C.c_void_p), C.c_int, C.c_int]
        L.jt_gdn2_state_free.argtypes = [C.c_void_p]
        L.jt_gdn2_state_free.restype = None
        L.jt_gdn2_decode_step.argtypes = [C.c_void_p] + [_f32p] * 7 + [C.c_int] * 2 + [
            _f32p, C.c_size_t]
        for fn in (L.jt_gdn2_prefill_chunk16, L.jt_gdn2_prefill_chunk32):
            fn.argtypes = [C.c_void_p] + [_f32p] * 7 + [C.c_int] * 2 + [_f32p, C.c_size_t]

    def quant_rows(self, X):
        X = _c(X, np.float32)
        Q = np.zeros(X.shape, np.int8)
        s = np.zeros(X.shape[0], np.float32)
        rc = self.lib.jt_w8a8_quant_per_channel(X, X.shape[0], X.shape[1], Q, s)
        return rc, Q, s

    def quant_tensor(self, x):
        x = _c(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        s = np.zeros(1, np.float32)
        rc = self.lib.jt_w8a8_quant_per_tensor(x, x.size, q, s)
        return rc, q, s[0]

    def gemm_per_channel(self, Aq, Bq_kn, sA, sB):
        Aq = _c(Aq, np.int8)
        Bq = _c(Bq_kn, np.int8)
        M, K = Aq.shape
        N = Bq.shape[1]
        out = np.zeros((M, N), np.float32)
        rc = self.lib.jt_w8a8_gemm_per_channel(Aq, Bq, float(sA), _c(sB, np.float32), out,
                                               M, N, K)
        return rc, out

    def gemm_per_tensor(self, Aq, Bq_kn, sA, sB):
        Aq = _c(Aq, np.int8)
        Bq = _c(Bq_kn, np.int8)
        M, K = Aq.shape
        N = Bq.shape[1]
        out = np.zeros((M, N), np.float32)
        rc = self.lib.jt_w8a8_gemm_per_tensor(Aq, Bq, float(sA), float(sB), out, M, N, K)
        return rc, out

    def gemm_f32(self, A, B):
        A = _c(A, np.float32)
        B = _c(B, np.float32)
        out = np.zeros((A.shape[0], B.shape[1]), np.float32)
        rc = self.lib.jt_gemm_mat_f32(A, B, out, A.shape[0], B.shape[1], A.shape[1])
        return rc, out

    def lowbit_fakequant(self, w, bits):
        w = _c(w, np.float32).ravel()
        out = np.zeros_like(w)
        rc = self.lib.jt_lowbit_fakequant(w, out, w.size, bits)
        return rc, out

    def col_to_idx(self, col, bits):
        col = _c(col, np.float32).ravel()
        idx = np.zeros(bits * (col.size // 4), np.uint8)
        ws = np.zeros(1, np.float32)
        rc = self.lib.jt_lowbit_col_to_idx(col, col.size, bits, idx, ws)
        return rc, idx, ws[0]

    def lowbit_gemm_lut(self, X, W, bits):
        X = _c(X, np.float32)
        W = _c(W, np.float32)
        Y = np.zeros((X.shape[0], W.shape[1]), np.float32)
        rc = self.lib.jt_lowbit_gemm_lut(X, W, Y, X.shape[0], W.shape[1], X.shape[1], bits)
        return rc, Y

    def tmac_lut_ctor(self, act):
        act = _c(act, np.float32)
        n, k = act.shape
        q = np.zeros((n, k // 4, 8), np.int8)
        s = np.zeros((n, k // 32), np.float32)
        b = np.zeros((n, k // 32), np.float32)
        rc = self.lib.jt_tmac_lut_ctor(act, n, k, q, s, b)
        return rc, q, s, b

    def tmac_lookup_accum(self, qlut_row, idx, scales_row, biases_row, bits, w_scale):
        ng = qlut_row.size // 8
        out = np.zeros(1, np.float32)
        rc = self.lib.jt_tmac_lookup_accum(_c(qlut_row, np.int8), _c(idx, np.uint8),
                                           _c(scales_row, np.float32),
                                           _c(biases_row, np.float32), ng, ng // 8, bits,
                                           w_scale, out)
        return rc, out[0]

    def topk(self, logits, k):
        logits = _c(logits, np.float32)
        ids = np.zeros(k, np.uint64)
        w = np.zeros(k, np.float32)
        rc = self.lib.jt_routing_topk(logits, logits.size, k, ids, w)
        return rc, ids.astype(np.int64), w

    def batch_sort(self, ids, T, k, E, cap_factor):
        ids = _c(ids, np.uint64).ravel()
        perm = np.zeros(T * k, np.uint64)
        off = np.zeros(E + 1, np.uint64)
        drop = np.zeros(T * k, np.uint8)
        kept = C.c_size_t(0)
        rc = self.lib.jt_moe_batch_sort(ids, T, k, E, cap_factor, perm, off, drop,
                                        C.addressof(kept), None)
        return rc, perm[: kept.value].astype(np.int64), off.astype(np.int64), drop

    def moe_fwd_batch(self, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, k, cap_factor,
                      w8a8_on=0, lowbit_mode=0, caches=False):
        X = _c(X, np.float32)
        T, n = X.shape
        E, h = Wg.shape[0], Wg.shape[1]
        S = 0 if Wg_s is None else Wg_s.shape[0]
        z = np.zeros(1, np.float32)
        Y = np.zeros((T, n), np.float32)
        cache = {}
        if caches:
            cache = dict(Gsel=np.zeros((T * k, h), np.float32),
                         Usel=np.zeros((T * k, h), np.float32))
            if S:
                cache.update(Gs=np.zeros((T, S, h), np.float32), Us=np.zeros((T, S, h), np.float32))
        cp = lambda nm: cache[nm].ctypes.data if nm in cache else None
        ids = np.zeros((T, k), np.uint64)
        w = np.zeros((T, k), np.float32)
        perm = np.zeros(T * k, np.uint64)
        off = np.zeros(E + 1, np.uint64)
        drop = np.zeros(T * k, np.uint8)
        kept = C.c_size_t(0)
        dropped = C.c_size_t(0)
        Ysel = np.zeros((T * k, n), np.float32)
        self.lib.jt_w8a8_set_enabled(w8a8_on)
        self.lib.jt_lowbit_set_mode(lowbit_mode)
        try:
            rc = self.lib.jt_moe_fwd_batch(
                X, _c(Wgate, np.float32), _c(Wg, np.float32), _c(Wu, np.float32),
                _c(Wd, np.float32), z if S == 0 else _c(Wg_s, np.float32),
                z if S == 0 else _c(Wu_s, np.float32),
                z if S == 0 else _c(Wd_s, np.float32), Y, T, n, h, E, k, S, ids, w,
                cp("Gsel"), cp("Usel"), Ysel.ctypes.data, cp("Gs"), cp("Us"), cap_factor,
                perm, off, drop, C.byref(kept), C.byref(dropped))
        finally:
            self.lib.jt_w8a8_set_enabled(0)
            self.lib.jt_lowbit_set_mode(0)
        return dict(rc=rc, Y=Y, ids=ids.astype(np.int64), w=w,
                    perm=perm[: kept.value].astype(np.int64), off=off.astype(np.int64),
                    drop=drop, Ysel=Ysel, **cache)


    def gdn2_l2norm(self, x, eps=1e-6):
        x = _c(x, np.float32).ravel()
        y = np.full_like(x, np.nan)
        return self.lib.jt_gdn2_l2norm(x, y, x.size, eps), y

    def _gdn2_state(self, S):
        """S copied into a state of the reference's own allocator (64-byte
        aligned, as jt_gdn2_decode_step requires)."""
        dk, dv = S.shape
        p = C.c_void_p()
        assert self.lib.jt_gdn2_state_alloc(C.byref(p), dk, dv) == 0
        C.memmove(p, _c(S, np.float32).ctypes.data, S.size * 4)
        return p

    def _gdn2_take(self, p, dk, dv):
        out = np.ctypeslib.as_array((C.c_float * (dk * dv)).from_address(p.value)).copy()
        self.lib.jt_gdn2_state_free(p)
        return out.reshape(dk, dv)

    def gdn2_decode_step(self, S, q, k, v, b, w, alpha):
        dk, dv = S.shape
        p = self._gdn2_state(S)
        o = np.full(dv, np.nan, np.float32)
        need = 2 * dk + 2 * dv
        scratch = np.zeros(need, np.float32)
        f = lambda a: _c(a, np.float32).ravel()  # noqa: E731
        rc = self.lib.jt_gdn2_decode_step(p, o, f(q), f(k), f(v), f(b), f(w), f(alpha), dk, dv,
                                          scratch, need)
        return rc, self._gdn2_take(p, dk, dv), o

    def gdn2_prefill_chunk(self, S, Q, K, V, B, W, A):
        dk, dv = S.shape
        C_ = Q.shape[0]
        p = self._gdn2_state(S)
        Out = np.full((C_, dv), np.nan, np.float32)
        need = 4 * C_ * dk + 2 * C_ * dv + C_ * C_ + dk
        scratch = np.zeros(need, np.float32)
        fn = self.lib.jt_gdn2_prefill_chunk16 if C_ == 16 else self.lib.jt_gdn2_prefill_chunk32
        f = lambda a: _c(a, np.float32)  # noqa: E731
        rc = fn(p, Out, f(Q), f(K), f(V), f(B), f(W), f(A), dk, dv, scratch, need)
        return rc, self._gdn2_take(p, dk, dv), Out

    def moe_bwd_batch(self, *args, validate=1, **kw):
        """jt_moe_bwd_batch / _unchecked; arguments as bwd_batch_call."""
        fn = self.lib.jt_moe_bwd_batch if validate else self.lib.jt_moe_bwd_batch_unchecked
        return bwd_batch_call(fn, np.uint64, *args, **kw)

    def moe_fwd_single(self, x, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, k):
        """jt_moe_fwd for one token; returns rc, Y, ids, weights, logits."""
        x = _c(x, np.float32).ravel()
        n = x.size
        E, h = Wg.shape[0], Wg.shape[1]
        S = 0 if Wg_s is None else Wg_s.shape[0]
        z = np.zeros(1, np.float32)
        Y = np.zeros(n, np.float32)
        ids = np.zeros(k, np.uint64)
        w = np.zeros(k, np.float32)
        lg = np.zeros(E, np.float32)
        rc = self.lib.jt_moe_fwd(
            x, _c(Wgate, np.float32), _c(Wg, np.float32), _c(Wu, np.float32),
            _c(Wd, np.float32), z if S == 0 else _c(Wg_s, np.float32),
            z if S == 0 else _c(Wu_s, np.float32), z if S == 0 else _c(Wd_s, np.float32),
            Y, n, h, E, k, S, ids, w, lg, None, None, None, None, None)
        return rc, Y, ids.astype(np.int64), w, lg


def ref_available() -> bool:
    return os.path.exists(REF_SO)
