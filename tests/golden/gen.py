"""Deterministic synthetic inputs shared by make_golden.py and the tests.

hpat() draws from a hash of the element index (the splitmix64 finaliser), so
the same (shape, salt) gives the same float32 array on any machine and any
numpy version, and a fixture only has to store the reference's outputs.
The sum of four hashed uniforms, centred and scaled, is an Irwin-Hall(4)
variable: mean 0, standard deviation 1, range (-2*sqrt(3), 2*sqrt(3)).
"""
import numpy as np

_M1 = np.uint64(0x9E3779B97F4A7C15)
_M2 = np.uint64(0xBF58476D1CE4E5B9)
_M3 = np.uint64(0x94D049BB133111EB)


def _mix(x):
    x = x ^ (x >> np.uint64(30))
    x = x * _M2
    x = x ^ (x >> np.uint64(27))
    x = x * _M3
    return x ^ (x >> np.uint64(31))


def hpat(shape, salt, scale=1.0):
    """float32 array of `shape`, approximately N(0, scale^2), from `salt`."""
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.uint64)
    acc = np.zeros(n, np.float64)
    with np.errstate(over="ignore"):
        for r in range(4):
            key = np.uint64((salt * 4 + r + 1) & 0xFFFFFFFFFFFFFFFF)
            x = _mix(i * _M1 + key * _M2)
            acc += (x >> np.uint64(11)).astype(np.float64) / 2.0 ** 53
    v = (acc - 2.0) * np.sqrt(3.0) * float(scale)
    return v.astype(np.float32).reshape(shape)


def lpat(a, b, salt):
    """The pattern of the reference's low-bit test inputs
    (bench/kernel/test_lowbit.c:32-35): (a*31 + b*17 + salt*13) % 11,
    mapped to {-1, -0.8, ..., 1} in float32."""
    v = (a * 31 + b * 17 + salt * 13) % 11
    return np.float32(np.float32(v - 5) / np.float32(5.0))


def lpat_lut_inputs():
    """X [4][64] and W [64][8] of test_lowbit.c:112-125 (W = lpat * 0.5)."""
    M, H, K = 4, 8, 64
    X = np.array([lpat(i, 1, 11) for i in range(M * K)], np.float32).reshape(M, K)
    W = np.array([np.float32(lpat(i, 2, 13) * np.float32(0.5)) for i in range(K * H)],
                 np.float32).reshape(K, H)
    return X, W


def shared_case(n=128, h=128, E=4, S=2, T=5):
    """Inputs of the shared-expert golden case. The routed down weights are
    zero, so the reference layer's routed outputs are exactly 0 and Y is the
    fp64 sum of the shared experts. Every output column of each shared down
    matrix has the same max|w| (row 0 holds +-c, the rest is clipped below c),
    so the reference's per-tensor down quantisation equals a per-output-
    channel one code for code."""
    X = hpat((T, n), 101)
    Wgate = hpat((E, n), 102, 1 / np.sqrt(n))
    Wg = hpat((E, h, n), 103, 1 / np.sqrt(n))
    Wu = hpat((E, h, n), 104, 1 / np.sqrt(n))
    Wd = np.zeros((E, h, n), np.float32)
    Wgs = hpat((S, h, n), 105, 1 / np.sqrt(n))
    Wus = hpat((S, h, n), 106, 1 / np.sqrt(n))
    c = np.float32(3.0 / np.sqrt(h))
    Wds = np.clip(hpat((S, h, n), 107, 1 / np.sqrt(h)), -0.9 * c, 0.9 * c).astype(np.float32)
    sign = np.where(hpat((S, n), 108) >= 0, c, -c).astype(np.float32)
    Wds[:, 0, :] = sign
    return X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds


def accuracy_case(salt, T=32, n=128, h=64, E=8, S=1):
    """Inputs of the prepared-layer accuracy case (reference fp32 and
    true-LUT layers against the group-64 layer)."""
    X = hpat((T, n), salt)
    Wgate = hpat((E, n), salt + 1, 1 / np.sqrt(n))
    Wg = hpat((E, h, n), salt + 2, 1 / np.sqrt(n))
    Wu = hpat((E, h, n), salt + 3, 1 / np.sqrt(n))
    Wd = hpat((E, h, n), salt + 4, 1 / np.sqrt(h))
    Wgs = hpat((S, h, n), salt + 5, 1 / np.sqrt(n))
    Wus = hpat((S, h, n), salt + 6, 1 / np.sqrt(n))
    Wds = hpat((S, h, n), salt + 7, 1 / np.sqrt(h))
    return X, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds


def capacity_sort(ids, E, cap_factor):
    """The reference's capacity sort (src/moe_layer.c:895-978) of ids [T][k]:
    stable by expert, the first cap = ceil(cap_factor*T*k/E) pairs of each
    expert (in flattened index order) kept. cap_factor None: dropless.
    Returns perm [kept], off [E+1], drop [T*k] (uint8)."""
    flat = np.asarray(ids, np.int64).ravel()
    Tk = flat.size
    cap = Tk if cap_factor is None else int(np.ceil(np.float64(np.float32(cap_factor)) * Tk / E))
    drop = np.ones(Tk, np.uint8)
    perm, off = [], [0]
    for e in range(E):
        qs = np.nonzero(flat == e)[0][:cap]
        drop[qs] = 0
        perm.append(qs)
        off.append(off[-1] + qs.size)
    return (np.concatenate(perm).astype(np.int64), np.array(off, np.int64), drop)


def bwd_case(T, n, h, E, k, S, salt, cap_factor=None):
    """Inputs of a batched-backward case: distinct expert ids per token (a
    hashed shuffle), weights in (0, 1], caches and weights ~ N(0, .), the
    permutation of the capacity sort. The caches need not come from a
    forward: the backward reads them as given."""
    dY = hpat((T, n), salt)
    X = hpat((T, n), salt + 1)
    Wgate = hpat((E, n), salt + 2, 1 / np.sqrt(n))
    Wg = hpat((E, h, n), salt + 3, 1 / np.sqrt(n))
    Wu = hpat((E, h, n), salt + 4, 1 / np.sqrt(n))
    Wd = hpat((E, h, n), salt + 5, 1 / np.sqrt(h))
    keys = hpat((T, E), salt + 6)
    ids = np.argsort(keys, axis=1, kind="stable")[:, :k].astype(np.int64)
    w = (np.abs(hpat((T, k), salt + 7)) / 3.5 + 0.01).clip(0, 1).astype(np.float32)
    Gsel = hpat((T * k, h), salt + 8, 2.0)
    Usel = hpat((T * k, h), salt + 9)
    Ysel = hpat((T * k, n), salt + 10)
    perm, off, drop = capacity_sort(ids, E, cap_factor)
    Ysel[drop.astype(bool)] = 0.0
    if S:
        Wgs = hpat((S, h, n), salt + 11, 1 / np.sqrt(n))
        Wus = hpat((S, h, n), salt + 12, 1 / np.sqrt(n))
        Wds = hpat((S, h, n), salt + 13, 1 / np.sqrt(h))
        Gs = hpat((T, S, h), salt + 14, 2.0)
        Us = hpat((T, S, h), salt + 15)
    else:
        Wgs = Wus = Wds = Gs = Us = None
    return dict(dY=dY, X=X, Wgate=Wgate, Wg=Wg, Wu=Wu, Wd=Wd, Wg_s=Wgs, Wu_s=Wus,
                Wd_s=Wds, ids=ids, w=w, Gsel=Gsel, Usel=Usel, Ysel=Ysel, Gs=Gs, Us=Us,
                perm=perm, off=off, drop=drop, k=k)


BWD_ARGS = ("dY", "X", "Wgate", "Wg", "Wu", "Wd", "Wg_s", "Wu_s", "Wd_s", "ids", "w",
            "Gsel", "Usel", "Ysel", "Gs", "Us", "perm", "off", "drop", "k")


def bwd_args(c):
    """The case's arguments in jt_moe_bwd_batch order."""
    return [c[a] for a in BWD_ARGS]


def ref_bwd_inputs(case):
    """The inputs of the reference's batched-backward tests
    (bench/kernel/test_moe_layer.c:1166-1206 for case 0, the shape of
    test_bwd_batch_gate_bitmatch / test_bwd_batch_equiv; :1440-1488 for
    case 1, test_bwd_batch_drop), built with the tests' own float32
    arithmetic. Returns (X, dY, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, k,
    cap_factor); the forward (jt_moe_fwd_batch) then gives the caches."""
    f = np.float32
    if case == 0:
        T, n, h, E, k, S = 6, 4, 2, 4, 2, 1
        X = np.array([f(0.4) * lpat(i, 0, 51) + f(0.2) for i in range(T * n)], f).reshape(T, n)
        dY = np.array([f(0.5) * lpat(i, 1, 71) + f(0.15) for i in range(T * n)], f).reshape(T, n)
        Wgate = np.array([f(0.3) * lpat(e, j, 52) for e in range(E) for j in range(n)],
                         f).reshape(E, n)
        W = [np.array([f(0.3) * lpat(i, r, salt) for i in range(E * h * n)], f).reshape(E, h, n)
             for r, salt in ((0, 53), (1, 54), (2, 55))]
        Ws = [np.array([f(0.3) * lpat(i, r, salt) for i in range(S * h * n)], f).reshape(S, h, n)
              for r, salt in ((0, 56), (1, 57), (2, 58))]
        return (X, dY, Wgate, *W, *Ws, k, 1.25)
    T, n, h, E, k = 8, 2, 1, 4, 2
    X = np.zeros((T, n), f)
    dY = np.zeros((T, n), f)
    for t in range(T):
        X[t] = (1.0, f(0.125) * f(t))
        dY[t] = (0.5, -0.25)
    Wgate = np.array([2.0, 0.0, 1.2, -1.5, 0.0, 1.5, -5.0, 0.0], f).reshape(E, n)
    W = [np.array([f(0.3) * lpat(i, r, salt) for i in range(E * h * n)], f).reshape(E, h, n)
         for r, salt in ((0, 59), (1, 60), (2, 61))]
    return (X, dY, Wgate, *W, None, None, None, k, 1.25)


def gdn2_decode_inputs(dk, dv, seed):
    """The inputs of the reference's GDN-2 decode test
    (bench/kernel/gdn2.c:95-157, test_numeric_case): S0, q, k, v, b, w,
    alpha in the test's float32 arithmetic."""
    f = np.float32
    q = np.array([lpat(i, 0, seed) + f(0.37) for i in range(dk)], f)
    k = np.array([lpat(i, 1, seed + 1) - f(0.23) for i in range(dk)], f)
    b = np.array([f(0.5) + f(0.1) * lpat(i, 2, seed) for i in range(dk)], f)
    a = np.array([f(0.9) + f(0.05) * lpat(i, 3, seed) for i in range(dk)], f)
    v = np.array([lpat(0, j, seed + 2) + f(0.11) for j in range(dv)], f)
    w = np.array([f(0.6) + f(0.1) * lpat(1, j, seed) for j in range(dv)], f)
    S = np.array([[f(0.25) * lpat(i, j, seed + 3) for j in range(dv)] for i in range(dk)], f)
    return S, q, k, v, b, w, a


def gdn2_prefill_inputs(C, dk, dv, seed):
    """The inputs of the reference's prefill equivalence test
    (bench/kernel/gdn2.c:522-580): S0, Q, K, V, B, W, A."""
    f = np.float32
    Q = np.array([[lpat(t, i, seed) + f(0.37) for i in range(dk)] for t in range(C)], f)
    K = np.array([[lpat(t, i, seed + 1) - f(0.23) for i in range(dk)] for t in range(C)], f)
    B = np.array([[f(0.5) + f(0.1) * lpat(t, i, seed + 2) for i in range(dk)] for t in range(C)], f)
    A = np.array([[f(0.9) + f(0.05) * lpat(t, i, seed + 3) for i in range(dk)] for t in range(C)],
                 f)
    V = np.array([[lpat(t, j, seed + 4) + f(0.11) for j in range(dv)] for t in range(C)], f)
    W = np.array([[f(0.6) + f(0.1) * lpat(t, j, seed + 5) for j in range(dv)] for t in range(C)], f)
    S = np.array([f(0.25) * lpat(i, 0, seed + 6) for i in range(dk * dv)], f).reshape(dk, dv)
    return S, Q, K, V, B, W, A


def gdn2_boundary_inputs():
    """The reference's prefill boundary test (bench/kernel/gdn2.c:623-668):
    alpha in {0, 1, 0.9}, a zero q row and a zero k row; C=16, dk=dv=8."""
    f = np.float32
    C, dk, dv = 16, 8, 8
    Q = np.array([[lpat(t, i, 21) + f(0.37) for i in range(dk)] for t in range(C)], f)
    K = np.array([[lpat(t, i, 22) - f(0.23) for i in range(dk)] for t in range(C)], f)
    B = np.full((C, dk), 0.5, f)
    A = np.array([[0.0 if t % 3 == 0 else (1.0 if t % 3 == 1 else 0.9) for _ in range(dk)]
                  for t in range(C)], f)
    V = np.array([[lpat(t, j, 23) + f(0.11) for j in range(dv)] for t in range(C)], f)
    W = np.full((C, dv), 0.6, f)
    Q[3] = 0.0
    K[5] = 0.0
    S = np.array([f(0.25) * lpat(i, 0, 24) for i in range(dk * dv)], f).reshape(dk, dv)
    return S, Q, K, V, B, W, A
