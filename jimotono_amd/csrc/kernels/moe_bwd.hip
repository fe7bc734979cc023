// Kernels of the batched MoE backward on the forward's permutation
// (the reference's jt_moe_bwd_batch, src/moe_layer.c:1684-2502), gfx950.
//
// Index checks (every call, both the checked and the unchecked form):
//  k_bwd_check_q    : ids / weights / drop per pair, kept count, dWgate keys
//  k_bwd_check_off  : off[] from 0, monotone, <= T*k, off[E] == kept count
//  k_bwd_check_perm : perm[0..kept) an exact enumeration of the kept pairs
// A failed check raises EF_BAD_ID and clamps what later kernels index with,
// so every access stays in bounds; the result is then not used.
//
// Gate path (steps 1-4 of the reference):
//  k_bwd_dots   : dw[q] = fp64 dot(Ysel[q], dY[t]) in the reference's
//                 lane-4 order (src/moe_layer.c:67-86, 1985-2010)
//  k_bwd_token  : softmax Jacobian per token (:2011-2047), dLogits, the
//                 gate-path dX terms (:2048-2081) and the token's perm rows
//  k_bwd_dwgate : dWgate[e][j] in token/slot order (:2082-2103) over the
//                 stable expert sort of the kept pairs
// Expert path (steps 5-6): three bit-exact fp32 GEMM forms (per output, a
// k-ascending sequence of rounded multiplies and rounded adds, as
// src/moe_gemm.c:47-89) on 64x64 tiles:
//  k_bwd_gemm<AT, BT, EPI> with EPI_DSWIGLU (dY Wd^T -> SwiGLU backward
//  -> Dg, Du, S), EPI_DUAL ((float)((double)Dg Wg + (double)Du Wu)) and
//  EPI_STORE (D^T X weight gradients).
//  k_bwd_dx     : dX = (float)(gate + routed rows in perm order + shared)
//                 in fp64 (:2236-2245, 2354-2363, 2411-2429)
#include "jt_dev.h"
#include "jt_launch.h"

namespace {

constexpr int BM = 64, BN = 64, BK = 16, TM = 4, TN = 4, PAD = 4;
constexpr int EPI_STORE = 0, EPI_DUAL = 1, EPI_DSWIGLU = 2;

// One GEMM family: C_g(r, c) = sum_k A_g(r, k) B_g(k, c) for groups g.
//  A_g = A + g*sAg + kbase*sAk (kbase = koff[g] when koff, else 0);
//  AT: A_g(r, k) = A_g[k*lda + r], else A_g[r*lda + k]; B alike with BT:
//  B_g(k, c) = B_g[c*ldb + k], else B_g[k*ldb + c].
//  Rows: a tile list {g, row0, rows} (ragged M, rows are global) or
//  blockIdx.x*BM within M with g = blockIdx.z.
struct GemmP {
    const float *A, *B, *A2, *B2;
    int lda, ldb;
    int64_t sAg, sBg, sAk, sBk;
    float *C, *C2, *C3;
    int ldc;
    int64_t sCg;
    const float *G, *U;     // EPI_DSWIGLU inputs: row q of G_g = G + g*sGg + q*ldg
    const int32_t *rowq;    // q of each output row (NULL: q = row)
    int ldg;
    int64_t sGg;
    int M, N, K;
    const int32_t *koff;    // per-group K ranges (ragged K)
    const int4 *tiles;      // ragged M
    const int32_t *ntiles;
    uint32_t *err;
};

// SwiGLU backward of one element (src/moe_layer.c:1680-1682, 2204-2233) in
// fp64: sig = 1/(1+exp(-g)) with a correctly rounded division, exp within
// about an ulp of glibc's; false when acc or a result is not finite.
__device__ __forceinline__ bool dswiglu(float g, float u, float dot, float *dg, float *du,
                                        float *sv) {
    const double gi = (double)g, ui = (double)u, acc = (double)dot;
    const double sig = 1.0 / (1.0 + exp_tang(-gi));
    const double silu = gi * sig;
    const double dsilu = sig * (1.0 + gi * (1.0 - sig));
    const double gd = acc * ui * dsilu, ud = acc * silu, s = silu * ui;
    *dg = (float)gd;
    *du = (float)ud;
    *sv = (float)s;
    return isfinite(acc) && isfinite(gd) && isfinite(ud) && isfinite(s);
}

template <bool T_>
__device__ __forceinline__ void load_a(float (*As)[BM + PAD], const float *Ag, int lda, int rb,
                                       int rc, int k0, int K, int tid) {
#pragma unroll
    for (int it = 0; it < BM * BK / 256; it++) {
        const int idx = tid + 256 * it;
        int r, kk;
        if (T_) {
            kk = idx / BM, r = idx % BM;
        } else {
            r = idx / BK, kk = idx % BK;
        }
        float v = 0.0f;
        if (r < rc && k0 + kk < K)
            v = T_ ? Ag[(int64_t)(k0 + kk) * lda + rb + r] : Ag[(int64_t)(rb + r) * lda + k0 + kk];
        As[kk][r] = v;
    }
}

template <bool T_>
__device__ __forceinline__ void load_b(float (*Bs)[BN + PAD], const float *Bg, int ldb, int cb,
                                       int cc, int k0, int K, int tid) {
#pragma unroll
    for (int it = 0; it < BN * BK / 256; it++) {
        const int idx = tid + 256 * it;
        int c, kk;
        if (T_) {
            c = idx / BK, kk = idx % BK;
        } else {
            kk = idx / BN, c = idx % BN;
        }
        float v = 0.0f;
        if (c < cc && k0 + kk < K)
            v = T_ ? Bg[(int64_t)(cb + c) * ldb + k0 + kk] : Bg[(int64_t)(k0 + kk) * ldb + cb + c];
        Bs[kk][c] = v;
    }
}

__device__ __forceinline__ void fma_step(float (&acc)[TM][TN], const float *as, const float *bs) {
    const float4 a = *(const float4 *)as, b = *(const float4 *)bs;
    const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __fadd_rn(acc[i][j], __fmul_rn(av[i], bv[j]));
}

template <bool AT, bool BT, int EPI>
__global__ __launch_bounds__(256) void k_bwd_gemm(GemmP p) {
    constexpr int NP = EPI == EPI_DUAL ? 2 : 1;
    __shared__ __attribute__((aligned(16))) float As[NP][BK][BM + PAD];
    __shared__ __attribute__((aligned(16))) float Bs[NP][BK][BN + PAD];
    const int tid = threadIdx.x;
    int g, rb, rc;
    if (p.tiles) {
        if ((int)blockIdx.x >= *p.ntiles) return;
        const int4 tl = p.tiles[blockIdx.x];
        g = tl.x, rb = tl.y, rc = tl.z;
    } else {
        g = blockIdx.z, rb = blockIdx.x * BM;
        rc = min(BM, p.M - rb);
    }
    const int cb = blockIdx.y * BN, cc = min(BN, p.N - cb);
    int K = p.K;
    int64_t kb = 0;
    if (p.koff) {
        kb = p.koff[g];
        K = p.koff[g + 1] - p.koff[g];
    }
    const float *Ag = p.A + g * p.sAg + kb * p.sAk, *Bg = p.B + g * p.sBg + kb * p.sBk;
    const float *Ag2 = nullptr, *Bg2 = nullptr;
    if (EPI == EPI_DUAL) {
        Ag2 = p.A2 + g * p.sAg + kb * p.sAk;
        Bg2 = p.B2 + g * p.sBg + kb * p.sBk;
    }
    const int ty = tid / (BN / TN), tx = tid % (BN / TN);
    float acc[TM][TN], acc2[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = acc2[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BK) {
        load_a<AT>(As[0], Ag, p.lda, rb, rc, k0, K, tid);
        load_b<BT>(Bs[0], Bg, p.ldb, cb, cc, k0, K, tid);
        if (EPI == EPI_DUAL) {
            load_a<AT>(As[NP - 1], Ag2, p.lda, rb, rc, k0, K, tid);
            load_b<BT>(Bs[NP - 1], Bg2, p.ldb, cb, cc, k0, K, tid);
        }
        __syncthreads();
        const int kend = min(BK, K - k0);
        if (kend == BK) {
#pragma unroll
            for (int kk = 0; kk < BK; kk++) {
                fma_step(acc, &As[0][kk][ty * TM], &Bs[0][kk][tx * TN]);
                if (EPI == EPI_DUAL) fma_step(acc2, &As[NP - 1][kk][ty * TM], &Bs[NP - 1][kk][tx * TN]);
            }
        } else {
            for (int kk = 0; kk < kend; kk++) {
                fma_step(acc, &As[0][kk][ty * TM], &Bs[0][kk][tx * TN]);
                if (EPI == EPI_DUAL) fma_step(acc2, &As[NP - 1][kk][ty * TM], &Bs[NP - 1][kk][tx * TN]);
            }
        }
        __syncthreads();
    }
    bool bad = false;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int r = ty * TM + i;
        if (r >= rc) continue;
        const int64_t row = rb + r;
        float *crow = p.C + g * p.sCg + row * p.ldc;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int c = tx * TN + j;
            if (c >= cc) continue;
            const int col = cb + c;
            if (EPI == EPI_STORE) {
                crow[col] = acc[i][j];
            } else if (EPI == EPI_DUAL) {
                crow[col] = (float)((double)acc[i][j] + (double)acc2[i][j]);
            } else {
                const int64_t q = p.rowq ? p.rowq[row] : row;
                const int64_t at = g * p.sGg + q * p.ldg + col;
                float dg, du, sv;
                bad |= !dswiglu(p.G[at], p.U[at], acc[i][j], &dg, &du, &sv);
                const int64_t o = g * p.sCg + row * p.ldc + col;
                p.C[o] = dg;
                p.C2[o] = du;
                p.C3[o] = sv;
            }
        }
    }
    if (bad) raise_err(p.err, EF_NONFINITE_MID);
}

template <bool AT, bool BT, int EPI>
int launch_gemm(const GemmP &p, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((k_bwd_gemm<AT, BT, EPI>), grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

__device__ __forceinline__ int block_sum_256(int v, int *red) {
    v = wave_sum_i(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// ctrl[0] = number of kept pairs (drop == 0), ctrl[1] = kept as used (off[E]
// when the checks pass, else 0); ctrl must be zero before.
__global__ __launch_bounds__(256) void k_bwd_check_q(const uint64_t *__restrict__ ids,
                                                     const float *__restrict__ w,
                                                     const uint8_t *__restrict__ drop, int Tk,
                                                     int E, int validate,
                                                     int32_t *__restrict__ key,
                                                     int32_t *__restrict__ inv,
                                                     uint32_t *__restrict__ seen,
                                                     uint32_t *ctrl, uint32_t *err) {
    __shared__ int red[4];
    const int q = blockIdx.x * 256 + threadIdx.x;
    int kept = 0;
    if (q < Tk) {
        const uint8_t d = drop[q];
        const uint64_t id = ids[q];
        bool bad;
        if (validate) {
            const float wv = w[q];
            bad = id >= (uint64_t)E || !(wv >= 0.0f && wv <= 1.0f) || d > 1;
        } else {
            bad = d == 0 && id >= (uint64_t)E;
        }
        if (bad) raise_err(err, EF_BAD_ID);
        key[q] = (d != 0 || id >= (uint64_t)E) ? E : (int)id;
        inv[q] = -1;
        seen[q] = 0;
        kept = d == 0;
    }
    kept = block_sum_256(kept, red);
    if (threadIdx.x == 0 && kept) atomicAdd(ctrl, (uint32_t)kept);
}

__global__ __launch_bounds__(1024) void k_bwd_check_off(const uint64_t *__restrict__ off, int E,
                                                        int Tk, int32_t *__restrict__ off32,
                                                        uint32_t *ctrl, uint32_t *err) {
    bool bad = false;
    for (int e = threadIdx.x; e <= E; e += 1024) {
        const uint64_t v = off[e];
        bad |= v > (uint64_t)Tk || (e == 0 && v != 0) || (e > 0 && off[e - 1] > v);
    }
    bad = __syncthreads_or(bad);
    const uint64_t kept = off[E];
    bad = bad || kept != (uint64_t)ctrl[0];
    for (int e = threadIdx.x; e <= E; e += 1024) off32[e] = bad ? 0 : (int)off[e];
    if (threadIdx.x == 0) {
        ctrl[1] = bad ? 0u : (uint32_t)kept;
        if (bad) raise_err(err, EF_BAD_ID);
    }
}

__global__ __launch_bounds__(256) void k_bwd_check_perm(const uint64_t *__restrict__ perm,
                                                        const uint8_t *__restrict__ drop,
                                                        int Tk, const uint32_t *ctrl,
                                                        uint32_t *__restrict__ seen,
                                                        int32_t *__restrict__ inv,
                                                        uint32_t *err) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= (int)ctrl[1]) return;
    const uint64_t q = perm[i];
    if (q >= (uint64_t)Tk || drop[q] != 0 || atomicAdd(&seen[q], 1u) != 0) {
        raise_err(err, EF_BAD_ID);
        return;
    }
    inv[q] = i;
}

// Row i of the kept rows in perm order: Xp[i] = X[t], dYp[i] =
// (float)((double)w*(double)dY[t]) (src/moe_layer.c:2164-2194), rowq[i] = q.
__global__ __launch_bounds__(256) void k_bwd_gather(const uint64_t *__restrict__ perm,
                                                    const float *__restrict__ X,
                                                    const float *__restrict__ dY,
                                                    const float *__restrict__ w, int Tk, int k,
                                                    int n, const uint32_t *ctrl,
                                                    float *__restrict__ Xp,
                                                    float *__restrict__ dYp,
                                                    int32_t *__restrict__ rowq) {
    const int i = blockIdx.x;
    if (i >= (int)ctrl[1]) return;
    const uint64_t q0 = perm[i];
    const int q = q0 < (uint64_t)Tk ? (int)q0 : 0;
    const int64_t t = q / k;
    const double wv = (double)w[q];
    if (threadIdx.x == 0) rowq[i] = q;
    for (int j = threadIdx.x; j < n; j += 256) {
        Xp[(int64_t)i * n + j] = X[t * n + j];
        dYp[(int64_t)i * n + j] = (float)(wv * (double)dY[t * n + j]);
    }
}

// dw[q] for every pair, 0 for dropped ones.
__global__ __launch_bounds__(256) void k_bwd_dots(const float *__restrict__ Ysel,
                                                  const float *__restrict__ dY,
                                                  const uint8_t *__restrict__ drop, int Tk,
                                                  int k, int n, double *__restrict__ dw,
                                                  uint32_t *err) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= Tk) return;
    if (drop[q]) {
        dw[q] = 0.0;
        return;
    }
    const float *y = Ysel + (int64_t)q * n, *d = dY + (int64_t)(q / k) * n;
    double l0 = 0.0, l1 = 0.0, l2 = 0.0, l3 = 0.0;
    const int n4 = n & ~3;
    int j = 0;
    if ((n & 3) == 0) {
        for (; j < n4; j += 4) {
            const float4 a = *(const float4 *)(y + j), b = *(const float4 *)(d + j);
            l0 = l0 + (double)a.x * (double)b.x;
            l1 = l1 + (double)a.y * (double)b.y;
            l2 = l2 + (double)a.z * (double)b.z;
            l3 = l3 + (double)a.w * (double)b.w;
        }
    } else {
        for (; j < n4; j += 4) {
            l0 = l0 + (double)y[j] * (double)d[j];
            l1 = l1 + (double)y[j + 1] * (double)d[j + 1];
            l2 = l2 + (double)y[j + 2] * (double)d[j + 2];
            l3 = l3 + (double)y[j + 3] * (double)d[j + 3];
        }
    }
    double s = (l0 + l1) + (l2 + l3);
    for (; j < n; j++) s = s + (double)y[j] * (double)d[j];
    if (!isfinite(s)) raise_err(err, EF_NONFINITE_MID);
    dw[q] = s;
}

// Per token: s = sum_kept (double)w*dw in slot order; dlog[q] =
// (double)w*(dw - s); dLogits[t][id] = (float)dlog; the first two kept slots
// ordered by expert id for the gate-path dX; the token's perm rows in
// ascending order (= experts ascending, then the expert's row order).
__global__ __launch_bounds__(256) void k_bwd_token(
    const uint64_t *__restrict__ ids, const float *__restrict__ w,
    const uint8_t *__restrict__ drop, const double *__restrict__ dw,
    const int32_t *__restrict__ inv, int T, int k, int E, double *__restrict__ dlog,
    float *__restrict__ dLogits, int32_t *__restrict__ gate_e, double *__restrict__ gate_dl,
    int32_t *__restrict__ gate_n, int32_t *__restrict__ tokpos, int32_t *__restrict__ tokcnt,
    uint32_t *err) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    const int64_t q0 = (int64_t)t * k;
    double s = 0.0;
    for (int p = 0; p < k; p++)
        if (!drop[q0 + p]) s = s + (double)w[q0 + p] * dw[q0 + p];
    bool bad = !isfinite(s);
    int es[2] = {0, 0}, nk = 0, c = 0;
    double dl[2] = {0.0, 0.0};
    int32_t *pos = tokpos + q0;
    for (int p = 0; p < k; p++) {
        const int64_t q = q0 + p;
        if (drop[q]) {
            dlog[q] = 0.0;
            continue;
        }
        const uint64_t id0 = ids[q];
        const int id = id0 < (uint64_t)E ? (int)id0 : 0;
        if (id0 >= (uint64_t)E) raise_err(err, EF_BAD_ID);
        const double v = (double)w[q] * (dw[q] - s);
        bad |= !isfinite(v);
        dlog[q] = v;
        if (dLogits) dLogits[(int64_t)t * E + id] = (float)v;
        if (nk < 2) {
            es[nk] = id;
            dl[nk] = v;
            nk++;
        }
        const int i = inv[q];
        if (i >= 0) {  // insertion into the ascending list
            int at = c++;
            while (at > 0 && pos[at - 1] > i) {
                pos[at] = pos[at - 1];
                at--;
            }
            pos[at] = i;
        }
    }
    if (bad) raise_err(err, EF_NONFINITE_MID);
    if (nk == 2 && es[0] > es[1]) {
        const int te = es[0];
        const double td = dl[0];
        es[0] = es[1], dl[0] = dl[1];
        es[1] = te, dl[1] = td;
    }
    gate_e[2 * t] = es[0];
    gate_e[2 * t + 1] = es[1];
    gate_dl[2 * t] = dl[0];
    gate_dl[2 * t + 1] = dl[1];
    gate_n[t] = nk;
    tokcnt[t] = c;
}

// dWgate[e][j] = float sum over the kept pairs of expert e in flattened
// index order of (float)(dlog*(double)X[t][j]); 0 for experts without one.
__global__ __launch_bounds__(256) void k_bwd_dwgate(const int32_t *__restrict__ off2,
                                                    const int32_t *__restrict__ perm2,
                                                    const double *__restrict__ dlog,
                                                    const float *__restrict__ X, int k, int n,
                                                    float *__restrict__ dWgate) {
    const int e = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (j >= n) return;
    float rg = 0.0f;
    const int i1 = off2[e + 1];
    for (int i = off2[e]; i < i1; i++) {
        const int q = perm2[i];
        rg = rg + (float)(dlog[q] * (double)X[(int64_t)(q / k) * n + j]);
    }
    dWgate[(int64_t)e * n + j] = rg;
}

// dX[t][j] = (float)(0 + gate term + routed rows in ascending perm order +
// shared experts in index order), all in fp64.
__global__ __launch_bounds__(256) void k_bwd_dx(
    const float *__restrict__ Wgate, const int32_t *__restrict__ gate_e,
    const double *__restrict__ gate_dl, const int32_t *__restrict__ gate_n,
    const int32_t *__restrict__ tokpos, const int32_t *__restrict__ tokcnt,
    const float *__restrict__ Dxe, const float *__restrict__ SDxe, int S, int T, int k, int n,
    float *__restrict__ dX, uint32_t *err) {
    const int t = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (j >= n) return;
    double acc = 0.0;
    const int nk = gate_n[t];
    for (int a = 0; a < nk; a++)
        acc = acc + gate_dl[2 * t + a] * (double)Wgate[(int64_t)gate_e[2 * t + a] * n + j];
    double dx = 0.0;
    dx = dx + acc;
    const int c = tokcnt[t];
    for (int u = 0; u < c; u++) dx = dx + (double)Dxe[(int64_t)tokpos[(int64_t)t * k + u] * n + j];
    for (int s = 0; s < S; s++) dx = dx + (double)SDxe[((int64_t)s * T + t) * n + j];
    if (!isfinite(dx)) raise_err(err, EF_NONFINITE_MID);
    dX[(int64_t)t * n + j] = (float)dx;
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

// Workspace carve-up (256-byte aligned pieces); returns the total bytes.
extern "C" size_t jtk_bwd_ws_layout(int T, int n, int h, int E, int k, int S, jtk_bwd_ws *w,
                                    char *base) {
    const int64_t Tk = (int64_t)T * k;
    const int64_t NB = (Tk + 255) / 256;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        char *p = base ? base + at : nullptr;
        at += (bytes + 255) / 256 * 256;
        return (void *)p;
    };
    jtk_bwd_ws v;
    v.ctrl = (uint32_t *)take(64);
    v.key = (int32_t *)take(Tk * 4);
    v.inv = (int32_t *)take(Tk * 4);
    v.seen = (uint32_t *)take(Tk * 4);
    v.rowq = (int32_t *)take(Tk * 4);
    v.rank = (int32_t *)take(Tk * 4);
    v.cnt = (int32_t *)take(NB * (E + 1) * 4);
    v.tot = (int32_t *)take(((size_t)E + 1) * 4);
    v.off2 = (int32_t *)take(((size_t)E + 2) * 4);
    v.perm2 = (int32_t *)take(Tk * 4);
    v.off32 = (int32_t *)take(((size_t)E + 1) * 4);
    v.tiles = (int32_t *)take((Tk / BM + E + 1) * 16);
    v.ntiles = (int32_t *)take(4);
    v.dw = (double *)take(Tk * 8);
    v.dlog = (double *)take(Tk * 8);
    v.gate_e = (int32_t *)take((size_t)T * 8);
    v.gate_dl = (double *)take((size_t)T * 16);
    v.gate_n = (int32_t *)take((size_t)T * 4);
    v.tokpos = (int32_t *)take(Tk * 4);
    v.tokcnt = (int32_t *)take((size_t)T * 4);
    v.Xp = (float *)take(Tk * n * 4);
    v.dYp = (float *)take(Tk * n * 4);
    v.Dg = (float *)take(Tk * h * 4);
    v.Du = (float *)take(Tk * h * 4);
    v.Ss = (float *)take(Tk * h * 4);
    v.Dxe = (float *)take(Tk * n * 4);
    v.SDg = (float *)take((int64_t)S * T * h * 4);
    v.SDu = (float *)take((int64_t)S * T * h * 4);
    v.SSs = (float *)take((int64_t)S * T * h * 4);
    v.SDxe = (float *)take((int64_t)S * T * n * 4);
    if (w) *w = v;
    return at;
}

extern "C" int jtk_bwd_batch(const jtk_bwd_io *io, int T, int n, int h, int E, int k, int S,
                             int validate, const jtk_bwd_ws *w, uint32_t *err, hipStream_t s) {
    const int Tk = T * k;
    const int64_t nh = (int64_t)n * h;
    int le = 0;
    // index checks
    le |= jtk_zero_u32(w->ctrl, 16, s);
    hipLaunchKernelGGL(k_bwd_check_q, dim3(cdiv(Tk, 256)), dim3(256), 0, s, io->ids,
                       io->weights, io->drop, Tk, E, validate, w->key, w->inv, w->seen, w->ctrl,
                       err);
    hipLaunchKernelGGL(k_bwd_check_off, dim3(1), dim3(1024), 0, s, io->off, E, Tk, w->off32,
                       w->ctrl, err);
    hipLaunchKernelGGL(k_bwd_check_perm, dim3(cdiv(Tk, 256)), dim3(256), 0, s, io->perm,
                       io->drop, Tk, w->ctrl, w->seen, w->inv, err);
    le |= (int)hipGetLastError();
    if (validate) {  // src/moe_layer.c:1766-1800
        const int64_t Tn = (int64_t)T * n;
        le |= jtk_check_finite(io->dY, Tn, err, s);
        le |= jtk_check_finite(io->X, Tn, err, s);
        le |= jtk_check_finite(io->Wgate, (int64_t)E * n, err, s);
        le |= jtk_check_finite(io->Wg, E * nh, err, s);
        le |= jtk_check_finite(io->Wu, E * nh, err, s);
        le |= jtk_check_finite(io->Wd, E * nh, err, s);
        le |= jtk_check_finite(io->weights, Tk, err, s);
        le |= jtk_check_finite(io->Gsel, (int64_t)Tk * h, err, s);
        le |= jtk_check_finite(io->Usel, (int64_t)Tk * h, err, s);
        le |= jtk_check_finite(io->Ysel, (int64_t)Tk * n, err, s);
        if (S) {
            le |= jtk_check_finite(io->Wg_s, S * nh, err, s);
            le |= jtk_check_finite(io->Wu_s, S * nh, err, s);
            le |= jtk_check_finite(io->Wd_s, S * nh, err, s);
            le |= jtk_check_finite(io->Gs, (int64_t)T * S * h, err, s);
            le |= jtk_check_finite(io->Us, (int64_t)T * S * h, err, s);
        }
    }
    // gate path
    if (io->dLogits) le |= jtk_zero_u32((uint32_t *)io->dLogits, (int64_t)T * E, s);
    hipLaunchKernelGGL(k_bwd_dots, dim3(cdiv(Tk, 256)), dim3(256), 0, s, io->Ysel, io->dY,
                       io->drop, Tk, k, n, w->dw, err);
    hipLaunchKernelGGL(k_bwd_token, dim3(cdiv(T, 256)), dim3(256), 0, s, io->ids, io->weights,
                       io->drop, w->dw, w->inv, T, k, E, w->dlog, io->dLogits, w->gate_e,
                       w->gate_dl, w->gate_n, w->tokpos, w->tokcnt, err);
    le |= (int)hipGetLastError();
    le |= jtk_sort(w->key, Tk, E + 1, (int64_t)Tk, w->rank, w->cnt, w->tot, w->off2, nullptr,
                   w->perm2, nullptr, nullptr, err, s);
    hipLaunchKernelGGL(k_bwd_dwgate, dim3((unsigned)E, cdiv(n, 256)), dim3(256), 0, s, w->off2,
                       w->perm2, w->dlog, io->X, k, n, io->dWgate);
    // routed experts on the perm rows
    hipLaunchKernelGGL(k_bwd_gather, dim3((unsigned)Tk), dim3(256), 0, s, io->perm, io->X,
                       io->dY, io->weights, Tk, k, n, w->ctrl, w->Xp, w->dYp, w->rowq);
    le |= (int)hipGetLastError();
    le |= jtk_make_tiles(w->off32, E, BM, w->tiles, w->ntiles, s);
    const unsigned mt = (unsigned)(Tk / BM + E);
    GemmP p{};
    p.err = err;
    p.tiles = (const int4 *)w->tiles;
    p.ntiles = w->ntiles;
    // Dg, Du, S = SwiGLU backward of (dYp Wd_e^T)
    p.A = w->dYp, p.lda = n;
    p.B = io->Wd, p.ldb = n, p.sBg = nh;
    p.C = w->Dg, p.C2 = w->Du, p.C3 = w->Ss, p.ldc = h;
    p.G = io->Gsel, p.U = io->Usel, p.rowq = w->rowq, p.ldg = h;
    p.N = h, p.K = n;
    le |= launch_gemm<false, true, EPI_DSWIGLU>(p, dim3(mt, cdiv(h, BN)), s);
    // Dxe = (float)((double)(Dg Wg_e) + (double)(Du Wu_e))
    p = GemmP{};
    p.err = err;
    p.tiles = (const int4 *)w->tiles;
    p.ntiles = w->ntiles;
    p.A = w->Dg, p.A2 = w->Du, p.lda = h;
    p.B = io->Wg, p.B2 = io->Wu, p.ldb = n, p.sBg = nh;
    p.C = w->Dxe, p.ldc = n;
    p.N = n, p.K = h;
    le |= launch_gemm<false, false, EPI_DUAL>(p, dim3(mt, cdiv(n, BN)), s);
    // dWg_e = Dg^T Xp, dWu_e = Du^T Xp, dWd_e = S^T dYp over the expert's rows
    const float *dA[3] = {w->Dg, w->Du, w->Ss}, *dB[3] = {w->Xp, w->Xp, w->dYp};
    float *dC[3] = {io->dWg, io->dWu, io->dWd};
    for (int m = 0; m < 3; m++) {
        p = GemmP{};
        p.err = err;
        p.koff = w->off32;
        p.A = dA[m], p.lda = h, p.sAk = h;
        p.B = dB[m], p.ldb = n, p.sBk = n;
        p.C = dC[m], p.ldc = n, p.sCg = nh;
        p.M = h, p.N = n;
        le |= launch_gemm<true, false, EPI_STORE>(p, dim3(cdiv(h, BM), cdiv(n, BN), E), s);
    }
    // shared experts on all tokens, dY unweighted
    if (S) {
        p = GemmP{};
        p.err = err;
        p.A = io->dY, p.lda = n;
        p.B = io->Wd_s, p.ldb = n, p.sBg = nh;
        p.C = w->SDg, p.C2 = w->SDu, p.C3 = w->SSs, p.ldc = h, p.sCg = (int64_t)T * h;
        p.G = io->Gs, p.U = io->Us, p.ldg = S * h, p.sGg = h;
        p.M = T, p.N = h, p.K = n;
        le |= launch_gemm<false, true, EPI_DSWIGLU>(p, dim3(cdiv(T, BM), cdiv(h, BN), S), s);
        p = GemmP{};
        p.err = err;
        p.A = w->SDg, p.A2 = w->SDu, p.lda = h, p.sAg = (int64_t)T * h;
        p.B = io->Wg_s, p.B2 = io->Wu_s, p.ldb = n, p.sBg = nh;
        p.C = w->SDxe, p.ldc = n, p.sCg = (int64_t)T * n;
        p.M = T, p.N = n, p.K = h;
        le |= launch_gemm<false, false, EPI_DUAL>(p, dim3(cdiv(T, BM), cdiv(n, BN), S), s);
        const float *sA[3] = {w->SDg, w->SDu, w->SSs}, *sB[3] = {io->X, io->X, io->dY};
        float *sC[3] = {io->dWg_s, io->dWu_s, io->dWd_s};
        for (int m = 0; m < 3; m++) {
            p = GemmP{};
            p.err = err;
            p.A = sA[m], p.lda = h, p.sAg = (int64_t)T * h;
            p.B = sB[m], p.ldb = n;
            p.C = sC[m], p.ldc = n, p.sCg = nh;
            p.M = h, p.N = n, p.K = T;
            le |= launch_gemm<true, false, EPI_STORE>(p, dim3(cdiv(h, BM), cdiv(n, BN), S), s);
        }
    }
    hipLaunchKernelGGL(k_bwd_dx, dim3((unsigned)T, cdiv(n, 256)), dim3(256), 0, s, io->Wgate,
                       w->gate_e, w->gate_dl, w->gate_n, w->tokpos, w->tokcnt, w->Dxe, w->SDxe,
                       S, T, k, n, io->dX, err);
    le |= (int)hipGetLastError();
    return le;
}

extern "C" int jtk_preload_bwd(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_bwd_dx));
}
