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
