"""CPU baselines of the benchmark shapes (TEST INFRASTRUCTURE ONLY).

bench.py's cpu_baseline leg times the reference's own CPU path here, on one
pinned host core, beside the GPU numbers. Nothing here is the product:
oracle/_ref is built from the reference sources (make -C oracle ref) and
only loaded by this module, the tests and smoke().

Method (the reference's, bench/common/bench_common.h:24-45): each case runs
as repeated trials on a monotonic clock until a time budget is spent; the
median and the median absolute deviation of the trials are reported.

Builds timed: the reference's default (libjtref.so: -mavx2 on the W8A8 and
layer sources, the AVX2-emulated int8 dot) and, where the host supports it,
its VNNI form (-DJIMOTONO_NATIVE=ON selects the VNNI dot of src/w8a8.c:9-34
through -march=native; libjtref_avx512vnni.so / libjtref_avxvnni.so are the
same sources with those ISA flags given explicitly). Both give bit-identical
int32 accumulators.
"""
from __future__ import annotations

import ctypes
import os
import time

import numpy as np

from .pyoracle import REF_SO, RefLib, ref_available

HERE = os.path.dirname(os.path.abspath(__file__))


def host_info():
    model = "unknown"
    flags = set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        pass
    return model, flags


def vnni_lib():
    """(name, path) of the VNNI build this host can run, or None."""
    _, flags = host_info()
    for flag, name in (("avx512_vnni", "libjtref_avx512vnni.so"),
                       ("avx_vnni", "libjtref_avxvnni.so")):
        path = os.path.join(HERE, "_ref", name)
        if flag in flags and os.path.exists(path):
            if name.startswith("libjtref_avx512") and "avx512bw" not in flags:
                continue
            return name, path
    return None


class pinned:
    """Run the body on one host core (the first one this process may use)."""

    def __enter__(self):
        self.prev = os.sched_getaffinity(0)
        self.core = min(self.prev)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *a):
        os.sched_setaffinity(0, self.prev)


def trials(fn, seconds, min_trials=3, max_trials=200):
    """Median and MAD (seconds) of repeated calls of fn, within a budget."""
    ts = []
    t_end = time.perf_counter() + seconds
    while len(ts) < min_trials or (time.perf_counter() < t_end and len(ts) < max_trials):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    a = np.array(ts)
    med = float(np.median(a))
    return med, float(np.median(np.abs(a - med))), len(ts)


def _swiglu(G, U):
    """The reference SwiGLU in fp64 (src/moe_layer.c:139-156), vectorised."""
    g = G.astype(np.float64)
    return ((g * (1.0 / (1.0 + np.exp(-g)))) * U.astype(np.float64)).astype(np.float32)


def w8a8_gemm_rows(R, seconds, M=64, N=1024, K=1024, seed=5):
    """W8A8 GEMM M x N x K with per-row activation scales: one
    jt_w8a8_gemm_per_channel call per row (its sA is one float per call)."""
    rng = np.random.default_rng(seed)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (K, N), dtype=np.int8)
    sA = rng.uniform(1e-3, 1e-2, M).astype(np.float32)
    sB = rng.uniform(1e-3, 1e-2, N).astype(np.float32)

    def run():
        for m in range(M):
            R.gemm_per_channel(A[m:m + 1], B, float(sA[m]), sB)
    med, mad, nt = trials(run, seconds)
    med1, _, _ = trials(lambda: R.gemm_per_channel(A, B, float(sA[0]), sB), seconds / 4)
    return {"us_per_gemm": med * 1e6, "mad_us": mad * 1e6, "trials": nt,
            "gops": 2.0 * M * N * K / med / 1e9,
            "us_one_call_per_tensor_scale": med1 * 1e6}


def shared_expert(R, M, seconds, n=1024, hs=2816, seed=6):
    """One shared W8A8 SwiGLU expert on M token rows: per-token int8 rows,
    gate and up per row (jt_w8a8_gemm_per_channel), fp64 SwiGLU, per-row
    requantisation, down per row. Weights quantised once beforehand."""
    rng = np.random.default_rng(seed)
    Wg = (rng.standard_normal((hs, n)) / 32).astype(np.float32)
    Wu = (rng.standard_normal((hs, n)) / 32).astype(np.float32)
    Wd = (rng.standard_normal((hs, n)) / 53).astype(np.float32)
    X = rng.standard_normal((M, n)).astype(np.float32)
    _, qg, sg = R.quant_rows(Wg)
    _, qu, su = R.quant_rows(Wu)
    _, qd, sd = R.quant_rows(np.ascontiguousarray(Wd.T))
    Bg, Bu, Bd = (np.ascontiguousarray(q.T) for q in (qg, qu, qd))

    def run():
        _, Xq, sx = R.quant_rows(X)
        S = np.zeros((M, hs), np.float32)
        for t in range(M):
            _, G = R.gemm_per_channel(Xq[t:t + 1], Bg, float(sx[t]), sg)
            _, U = R.gemm_per_channel(Xq[t:t + 1], Bu, float(sx[t]), su)
            S[t] = _swiglu(G, U)[0]
        _, Sq, ss = R.quant_rows(S)
        for t in range(M):
            R.gemm_per_channel(Sq[t:t + 1], Bd, float(ss[t]), sd)
    med, mad, nt = trials(run, seconds)
    wbytes = 3 * hs * n + 4 * (2 * hs + n)
    return {"us_per_expert": med * 1e6, "mad_us": mad * 1e6, "trials": nt,
            "gbps": (wbytes + 8 * M * n) / med / 1e9}


def routed_experts(R, ids, X, W, bits_gu=2, bits_d=4):
    """The routed experts of tokens X with ids [T][k] on the dropless
    permutation: per touched expert, jt_lowbit_gemm_lut for gate and up
    (INT2) and down (INT4), the reference's T-MAC driver
    (src/moe_layer.c:1301-1396). W maps expert -> (WgT [n][h], WuT [n][h],
    Wd [h][n]), the layouts the reference hands to jt_lowbit_gemm_lut."""
    for e in np.unique(ids):
        rows = np.nonzero((ids == e).any(axis=1))[0]
        Xe = np.ascontiguousarray(X[rows])
        WgT, WuT, Wd = W[int(e)]
        _, G = R.lowbit_gemm_lut(Xe, WgT, bits_gu)
        _, U = R.lowbit_gemm_lut(Xe, WuT, bits_gu)
        R.lowbit_gemm_lut(_swiglu(G, U), Wd, bits_d)


def routed_layer(R, seconds, T, n, h, E, k, seed, max_tokens=None):
    """Routed-expert layer under Zipf(1.1) routing at T tokens (the routed
    decode at T=16; the stress shape on a token sample when max_tokens < T). Expert
    weights are random and generated only for the experts the sampled
    tokens touch. Returns tokens/s and the per-layer time of the sample."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    tok = T if max_tokens is None else min(T, max_tokens)
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(tok)])
    X = rng.standard_normal((tok, n)).astype(np.float32)
    W = {}
    for e in np.unique(ids):
        W[int(e)] = (np.ascontiguousarray((rng.standard_normal((n, h)) / np.sqrt(n)).astype(np.float32)),
                     np.ascontiguousarray((rng.standard_normal((n, h)) / np.sqrt(n)).astype(np.float32)),
                     np.ascontiguousarray((rng.standard_normal((h, n)) / np.sqrt(h)).astype(np.float32)))
    med, mad, nt = trials(lambda: routed_experts(R, ids, X, W), seconds, min_trials=1)
    return {"tokens": tok, "touched_experts": len(W), "ms_per_sample": med * 1e3,
            "mad_ms": mad * 1e3, "trials": nt, "tokens_per_s": tok / med}


def bwd_inputs(R, T, n, h, E, k, S, seed):
    """Synthetic inputs of the batched backward: distinct ids per token,
    weights in (0, 1], caches ~ N(0, 1) and the reference's capacity sort at
    cap 1.25 (jt_moe_batch_sort)."""
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)  # noqa: E731
    ids = np.argsort(rng.random((T, E)), axis=1)[:, :k].astype(np.int64)
    rc, perm, off, drop = R.batch_sort(ids, T, k, E, 1.25)
    assert rc == 0
    Ysel = f(T * k, n)
    Ysel[drop.astype(bool)] = 0.0
    return [f(T, n), f(T, n), f(E, n) / n ** 0.5, f(E, h, n) / n ** 0.5, f(E, h, n) / n ** 0.5,
            f(E, h, n) / h ** 0.5, f(S, h, n) / n ** 0.5, f(S, h, n) / n ** 0.5,
            f(S, h, n) / h ** 0.5, ids, rng.uniform(0.01, 1.0, (T, k)).astype(np.float32),
            f(T * k, h), f(T * k, h), Ysel, f(T, S, h), f(T, S, h), perm, off, drop, k]


def bwd_batch(R, seconds, T, n, h, E, k, S, max_tokens=None, seed=3):
    """jt_moe_bwd_batch of the reference on T tokens (a sample of max_tokens
    when smaller); its work is linear in the tokens (every GEMM has the
    kept rows or T as one dimension), so tokens/s carries over."""
    tok = T if max_tokens is None else min(T, max_tokens)
    args = bwd_inputs(R, tok, n, h, E, k, S, seed)
    med, mad, nt = trials(lambda: R.moe_bwd_batch(*args), seconds, min_trials=1)
    return {"tokens": tok, "ms_per_sample": med * 1e3, "mad_ms": mad * 1e3, "trials": nt,
            "tokens_per_s": tok / med}


def gdn2_decode(R, seconds, H=512, dk=128, dv=128, sample=64, seed=7):
    """jt_gdn2_decode_step of the reference on `sample` of the H heads (one
    call per head, states 64-byte aligned); the heads are independent, so
    the time scales to H."""
    rng = np.random.default_rng(seed)
    L = R.lib
    states = []
    for _ in range(sample):
        p = ctypes.c_void_p()
        assert L.jt_gdn2_state_alloc(ctypes.byref(p), dk, dv) == 0
        S = (rng.standard_normal(dk * dv) * 0.3).astype(np.float32)
        ctypes.memmove(p, S.ctypes.data, S.nbytes)
        states.append(p)
    vec = lambda n, lo=None: (rng.uniform(lo, 1.0, n) if lo is not None  # noqa: E731
                              else rng.standard_normal(n)).astype(np.float32)
    q, k, b, a = vec(dk), vec(dk), vec(dk, 0.0), vec(dk, 0.9)
    v, w, o = vec(dv), vec(dv, 0.0), np.zeros(dv, np.float32)
    scratch = np.zeros(2 * dk + 2 * dv, np.float32)

    def run():
        for p in states:
            L.jt_gdn2_decode_step(p, o, q, k, v, b, w, a, dk, dv, scratch, scratch.size)
    med, mad, nt = trials(run, seconds)
    for p in states:
        L.jt_gdn2_state_free(p)
    return {"heads_timed": sample, "us_per_head": med / sample * 1e6,
            "us_per_step_all_heads": med / sample * H * 1e6, "trials": nt,
            "gbps": H * 2 * dk * dv * 4 / (med / sample * H) / 1e9}


def gdn2_prefill(R, seconds, T=4096, C=32, dk=128, dv=128, H=8, chunks=8, seed=8):
    """jt_gdn2_prefill_chunk32 of the reference on `chunks` consecutive
    chunks of one head; chunks cost the same, so tokens/s carries to T and
    H heads."""
    rng = np.random.default_rng(seed)
    L = R.lib
    p = ctypes.c_void_p()
    assert L.jt_gdn2_state_alloc(ctypes.byref(p), dk, dv) == 0
    f = lambda *sh: rng.standard_normal(sh).astype(np.float32)  # noqa: E731
    Q, K = f(chunks, C, dk), f(chunks, C, dk)
    B = rng.uniform(0, 1, (chunks, C, dk)).astype(np.float32)
    A = rng.uniform(0.9, 1, (chunks, C, dk)).astype(np.float32)
    V, W = f(chunks, C, dv), rng.uniform(0, 1, (chunks, C, dv)).astype(np.float32)
    Out = np.zeros((C, dv), np.float32)
    need = 4 * C * dk + 2 * C * dv + C * C + dk
    scratch = np.zeros(need, np.float32)

    def run():
        for c in range(chunks):
            L.jt_gdn2_prefill_chunk32(p, Out, Q[c], K[c], V[c], B[c], W[c], A[c], dk, dv,
                                      scratch, need)
    med, mad, nt = trials(run, seconds, min_trials=1)
    L.jt_gdn2_state_free(p)
    per_tok = med / (chunks * C)
    return {"chunks_timed": chunks, "ms_per_chunk": med / chunks * 1e3, "trials": nt,
            "tokens_per_s_one_head": 1.0 / per_tok, "tokens_per_s": 1.0 / per_tok / H}


def attn_proj(R, seconds, M, N=3072, K=1024, sample=16, seed=9):
    """The INT8 projection of M fp32 rows: per row jt_w8a8_quant_per_channel
    and jt_w8a8_gemm_per_channel (its sA is one float per call), weights
    quantised once; `sample` rows timed when M is larger."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) / 32).astype(np.float32)
    _, qw, sw = R.quant_rows(W)
    Bq = np.ascontiguousarray(qw.T)
    m = min(M, sample)
    X = rng.standard_normal((m, K)).astype(np.float32)

    def run():
        _, Xq, sx = R.quant_rows(X)
        for r in range(m):
            R.gemm_per_channel(Xq[r:r + 1], Bq, float(sx[r]), sw)
    med, mad, nt = trials(run, seconds)
    return {"rows_timed": m, "us_per_call": med / m * M * 1e6, "trials": nt}


DROPIN_MODES = {"fp32": (0, 0), "w8a8": (1, 0), "lowbit_fakequant": (0, 1),
                "lowbit_lut": (0, 2), "w8a8_and_lowbit_fakequant": (1, 1)}


def dropin_layer(R, seconds, T=512, n=64, h=32, E=8, k=2, S=1, seed=512):
    """The reference's jt_moe_fwd_batch at its trainer's shape
    (bench/kernel/train_tinystories.c:78-81) in each flag mode, the inputs of
    bench.py's drop-in sub-benchmark."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((T, n)).astype(np.float32)
    W = [(rng.standard_normal(sh) / np.sqrt(sh[-1])).astype(np.float32)
         for sh in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    out = {}
    for name, (w8, lb) in DROPIN_MODES.items():
        med, mad, nt = trials(lambda: R.moe_fwd_batch(X, *W, k, 1.5, w8, lb), seconds / 5)
        out[name] = {"ms_per_call": med * 1e3, "mad_ms": mad * 1e3, "trials": nt,
                     "tokens_per_s": T / med}
    return {"modes": out}


def decode_and_stress(seconds):
    """The W8A8 GEMM 64x1024x1024, the shared-expert decode at 1, 4 and 16
    rows, the routed decode at 16 tokens, a token sample of the E=512
    stress shape, the batched backward (training shape; a token sample of
    the layer shape), the GDN-2 decode step and prefill and the INT8
    attention projection, on one pinned core, for the default reference build
    and (for the W8A8 shapes) its VNNI form when the host can run one."""
    if not ref_available():
        return {"error": "oracle/_ref not built"}
    model, _ = host_info()
    out = {"host_cpu": model, "cores": 1, "kind": "reference"}
    builds = [("default (-mavx2, AVX2-emulated int8 dot)", REF_SO)]
    v = vnni_lib()
    if v is not None:
        builds.append((f"VNNI ({v[0]})", v[1]))
    else:
        out["vnni"] = "host has no AVX512-VNNI or AVX-VNNI: VNNI build not timed"
    with pinned() as pn:
        out["core"] = pn.core
        for bi, (name, path) in enumerate(builds):
            R = RefLib(path)
            res = {"w8a8_gemm_64x1024x1024": w8a8_gemm_rows(R, seconds)}
            for m in (1, 4, 16):
                res[f"shared_decode_M{m}"] = shared_expert(R, m, seconds)
            if bi == 0:  # the T-MAC path has no VNNI form
                res["routed_decode_T16"] = routed_layer(R, seconds, 16, 1024, 256, 256, 8, 16)
                res["stress_prefill_E512_sample"] = routed_layer(R, 2 * seconds, 16384, 2048,
                                                                 512, 512, 8, 17, max_tokens=4)
                res["moe_bwd_T512_train"] = bwd_batch(R, seconds, 512, 64, 32, 8, 2, 1)
                res["moe_bwd_T4096_layer"] = bwd_batch(R, seconds, 4096, 1024, 256, 64, 8, 1,
                                                       max_tokens=512)
                res["dropin_moe_fwd_batch_T512_train"] = dropin_layer(R, seconds)
                res["gdn2_decode_H512"] = gdn2_decode(R, seconds)
                res["gdn2_prefill_T4096_H8"] = gdn2_prefill(R, seconds)
            for m in (1, 16, 4096):
                res[f"attn_proj_int8_M{m}"] = attn_proj(R, seconds, m)
            out[name] = res
    return out
