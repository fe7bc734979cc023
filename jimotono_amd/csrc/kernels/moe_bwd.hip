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

constexpr int EPI_STORE = 0, EPI_DUAL = 1, EPI_DSWIGLU = 2;
constexpr int MODE_ROWS = 0, MODE_WGRAD = 1;
constexpr int PAD = 4;

// Operands of one side of a launch (side 0: shared experts, side 1: routed).
// A GEMM computes C(r, c) = sum over k ascending of A(r, k) B(k, c) with
//  A_g = A[m] + g*sAg + kb*sAk, B_g = B[m] + g*sBg + kb*sBk,
//  AT: A_g(r, k) = A_g[k*lda + r], else A_g[r*lda + k];
//  BT: B_g(k, c) = B_g[c*ldb + k], else B_g[k*ldb + c];
// m selects one of three matrices (weight gradients), or A[1]/B[1] are the
// second product of EPI_DUAL; g is the expert (group), kb the first row of
// its K range (koff, ragged K) or 0.
struct Side {
    const float *A[3], *B[3];
    float *C[3];  // EPI_DSWIGLU: Dg, Du, S
    int lda, ldb, ldc;
    int64_t sAg, sBg, sCg, sAk, sBk;
    const float *G, *U;     // EPI_DSWIGLU: row q of G_g = G + g*sGg + q*ldg
    const int32_t *rowq;    // q of each output row (NULL: q = row)
    int ldg;
    int64_t sGg;
    int M, K;               // dense rows and fixed K
    const int32_t *koff;    // ragged K: rows koff[g] .. koff[g+1]
    const int4 *tiles;      // ragged M: {g, first row, rows}
    const int32_t *ntiles;
};
// MODE_ROWS: blockIdx.x < nsh are side 0's dense row tiles (mt_sh per
// group), the rest side 1's tile list; blockIdx.y the column tile.
// MODE_WGRAD: blockIdx.z < nsh is side 0, then side 1, z = 3*g + m;
// blockIdx.x / blockIdx.y the row / column tiles.
struct GemmP {
    Side sd[2];
    int nsh, mt_sh, N;
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

// A (R x BK) chunk of an operand: NL elements per thread, loaded into
// registers (next chunk, while the current one is computed) and stored to
// LDS as [k][r]. KMAJ: memory is contiguous along r (k-major), else along k.
template <int R, int BK, bool KMAJ>
struct Chunk {
    static constexpr int NL = R * BK / 256;
    float v[NL];
    __device__ __forceinline__ void load(const float *P, int ld, int b, int cnt, int k0, int K,
                                         int tid) {
#pragma unroll
        for (int it = 0; it < NL; it++) {
            const int idx = tid + 256 * it;
            const int r = KMAJ ? idx % R : idx / BK, kk = KMAJ ? idx / R : idx % BK;
            v[it] = (r < cnt && k0 + kk < K)
                        ? (KMAJ ? P[(int64_t)(k0 + kk) * ld + b + r] : P[(int64_t)(b + r) * ld + k0 + kk])
                        : 0.0f;
        }
    }
    __device__ __forceinline__ void store(float (*S)[R + PAD], int tid) const {
#pragma unroll
        for (int it = 0; it < NL; it++) {
            const int idx = tid + 256 * it;
            const int r = KMAJ ? idx % R : idx / BK, kk = KMAJ ? idx / R : idx % BK;
            S[kk][r] = v[it];
        }
    }
};

// acc[i][j] += a[i] * b[j]: one rounded multiply, one rounded add
template <int TM, int TN>
__device__ __forceinline__ void mul_add(float (&acc)[TM][TN], const float *as, const float *bs) {
    float av[TM], bv[TN];
#pragma unroll
    for (int i = 0; i < TM; i += 4) *(float4 *)&av[i] = *(const float4 *)(as + i);
#pragma unroll
    for (int j = 0; j < TN; j += 4) *(float4 *)&bv[j] = *(const float4 *)(bs + j);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __fadd_rn(acc[i][j], __fmul_rn(av[i], bv[j]));
}

template <bool AT, bool BT, int EPI, int MODE, int TM, int TN>
__global__ __launch_bounds__(256) void k_bwd_gemm(GemmP p) {
    constexpr int BM = 16 * TM, BN = 16 * TN, BK = 2048 / (BM > BN ? BM : BN);
    constexpr int NP = EPI == EPI_DUAL ? 2 : 1;
    __shared__ __attribute__((aligned(16))) float As[NP][BK][BM + PAD];
    __shared__ __attribute__((aligned(16))) float Bs[NP][BK][BN + PAD];
    const int tid = threadIdx.x;
    int side, g, m = 0, rb, rc;
    if (MODE == MODE_ROWS) {
        const int bx = blockIdx.x;
        if (bx < p.nsh) {
            side = 0, g = bx / p.mt_sh, rb = (bx % p.mt_sh) * BM;
            rc = min(BM, p.sd[0].M - rb);
        } else {
            side = 1;
            if (bx - p.nsh >= *p.sd[1].ntiles) return;
            const int4 tl = p.sd[1].tiles[bx - p.nsh];
            g = tl.x, rb = tl.y, rc = tl.z;
        }
    } else {
        int z = blockIdx.z;
        side = z < p.nsh ? 0 : 1;
        z -= side ? p.nsh : 0;
        g = z / 3, m = z % 3;
        rb = blockIdx.x * BM;
        rc = min(BM, p.sd[side].M - rb);
    }
    const Side &S = p.sd[side];
    const int cb = blockIdx.y * BN, cc = min(BN, p.N - cb);
    int K = S.K;
    int64_t kb = 0;
    if (MODE == MODE_WGRAD && S.koff) {
        kb = S.koff[g];
        K = S.koff[g + 1] - S.koff[g];
    }
    const float *Ag = S.A[m] + g * S.sAg + kb * S.sAk, *Bg = S.B[m] + g * S.sBg + kb * S.sBk;
    const float *Ag2 = Ag, *Bg2 = Bg;
    if (EPI == EPI_DUAL) {
        Ag2 = S.A[1] + g * S.sAg + kb * S.sAk;
        Bg2 = S.B[1] + g * S.sBg + kb * S.sBk;
    }
    const int ty = tid / 16, tx = tid % 16;
    float acc[TM][TN], acc2[EPI == EPI_DUAL ? TM : 1][EPI == EPI_DUAL ? TN : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = 0.0f;
    if constexpr (EPI == EPI_DUAL) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc2[i][j] = 0.0f;
    }
    Chunk<BM, BK, AT> ca, ca2;
    Chunk<BN, BK, !BT> cbk, cb2;
    if (K > 0) {
        ca.load(Ag, S.lda, rb, rc, 0, K, tid);
        cbk.load(Bg, S.ldb, cb, cc, 0, K, tid);
        if (EPI == EPI_DUAL) {
            ca2.load(Ag2, S.lda, rb, rc, 0, K, tid);
            cb2.load(Bg2, S.ldb, cb, cc, 0, K, tid);
        }
    }
    for (int k0 = 0; k0 < K; k0 += BK) {
        ca.store(As[0], tid);
        cbk.store(Bs[0], tid);
        if (EPI == EPI_DUAL) {
            ca2.store(As[NP - 1], tid);
            cb2.store(Bs[NP - 1], tid);
        }
        __syncthreads();
        if (k0 + BK < K) {  // the next chunk's loads overlap this chunk's products
            ca.load(Ag, S.lda, rb, rc, k0 + BK, K, tid);
            cbk.load(Bg, S.ldb, cb, cc, k0 + BK, K, tid);
            if (EPI == EPI_DUAL) {
                ca2.load(Ag2, S.lda, rb, rc, k0 + BK, K, tid);
                cb2.load(Bg2, S.ldb, cb, cc, k0 + BK, K, tid);
            }
        }
        const int kend = min(BK, K - k0);
        if (kend == BK) {
#pragma unroll 8
            for (int kk = 0; kk < BK; kk++) {
                mul_add<TM, TN>(acc, &As[0][kk][ty * TM], &Bs[0][kk][tx * TN]);
                if constexpr (EPI == EPI_DUAL)
                    mul_add<TM, TN>(acc2, &As[NP - 1][kk][ty * TM], &Bs[NP - 1][kk][tx * TN]);
            }
        } else {
            for (int kk = 0; kk < kend; kk++) {
                mul_add<TM, TN>(acc, &As[0][kk][ty * TM], &Bs[0][kk][tx * TN]);
                if constexpr (EPI == EPI_DUAL)
                    mul_add<TM, TN>(acc2, &As[NP - 1][kk][ty * TM], &Bs[NP - 1][kk][tx * TN]);
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
        const int64_t o = g * S.sCg + row * S.ldc;
        const int64_t q = (EPI == EPI_DSWIGLU && S.rowq) ? S.rowq[row] : row;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int c = tx * TN + j;
            if (c >= cc) continue;
            const int col = cb + c;
            if constexpr (EPI == EPI_STORE) {
                S.C[m][o + col] = acc[i][j];
            } else if constexpr (EPI == EPI_DUAL) {
                S.C[0][o + col] = (float)((double)acc[i][j] + (double)acc2[i][j]);
            } else {
                const int64_t at = g * S.sGg + q * S.ldg + col;
                float dg, du, sv;
                bad |= !dswiglu(S.G[at], S.U[at], acc[i][j], &dg, &du, &sv);
                S.C[0][o + col] = dg;
                S.C[1][o + col] = du;
                S.C[2][o + col] = sv;
            }
        }
    }
    if (bad) raise_err(p.err, EF_NONFINITE_MID);
}

template <bool AT, bool BT, int EPI, int MODE, int TM, int TN>
int launch_gemm(const GemmP &p, dim3 grid, hipStream_t s) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
    hipLaunchKernelGGL((k_bwd_gemm<AT, BT, EPI, MODE, TM, TN>), grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

// Finiteness of up to 16 arrays in one launch (blockIdx.y = array).
struct FinList {
    const float *p[16];
    int64_t n[16];
};
__global__ __launch_bounds__(256) void k_bwd_finite(FinList L, uint32_t *err) {
    const float *x = L.p[blockIdx.y];
    const int64_t n = L.n[blockIdx.y];
    int bad = 0;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * 256;
    if (((uintptr_t)x & 15) == 0) {  // float4 body
        const float4 *x4 = (const float4 *)x;
        for (; i < n / 4; i += step) {
            const float4 v = x4[i];
            bad |= !isfinite(v.x) || !isfinite(v.y) || !isfinite(v.z) || !isfinite(v.w);
        }
        for (i = n / 4 * 4 + blockIdx.x * 256 + threadIdx.x; i < n; i += step)
            bad |= !isfinite(x[i]);
    } else {
        for (; i < n; i += step) bad |= !isfinite(x[i]);
    }
    bad = wave_or_i(bad);
    if (bad && (threadIdx.x & 63) == 0) raise_err(err, EF_NONFINITE_INPUT);
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
// The pairs are read 16 at a time ahead of the (ordered) sums.
__global__ __launch_bounds__(256) void k_bwd_dwgate(const int32_t *__restrict__ off2,
                                                    const int32_t *__restrict__ perm2,
                                                    const double *__restrict__ dlog,
                                                    const float *__restrict__ X, int k, int n,
                                                    float *__restrict__ dWgate) {
    const int e = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (j >= n) return;
    float rg = 0.0f;
    const int i0 = off2[e], i1 = off2[e + 1];
    int i = i0;
    for (; i + 16 <= i1; i += 16) {
        float x[16];
        double dl[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int q = perm2[i + u];
            dl[u] = dlog[q];
            x[u] = X[(int64_t)(q / k) * n + j];
        }
#pragma unroll
        for (int u = 0; u < 16; u++) rg = rg + (float)(dl[u] * (double)x[u]);
    }
    for (; i < i1; i++) {
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

// Tile shapes (threads hold TM x TN outputs; blocks 16 TM x 16 TN). The row
// GEMMs share one routed tile list, so they share TM.
constexpr int TM_ROWS = 4, TN_DOT = 4, TN_DX = 4, TM_WG = 4, TN_WG = 4;
constexpr int BM_ROWS = 16 * TM_ROWS;

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
    v.tiles = (int32_t *)take((Tk / BM_ROWS + E + 1) * 16);
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
        FinList L{};
        int c = 0;
        auto add = [&](const float *x, int64_t cnt) {
            L.p[c] = x;
            L.n[c++] = cnt;
        };
        add(io->dY, (int64_t)T * n);
        add(io->X, (int64_t)T * n);
        add(io->Wgate, (int64_t)E * n);
        add(io->Wg, E * nh);
        add(io->Wu, E * nh);
        add(io->Wd, E * nh);
        add(io->weights, Tk);
        add(io->Gsel, (int64_t)Tk * h);
        add(io->Usel, (int64_t)Tk * h);
        add(io->Ysel, (int64_t)Tk * n);
        if (S) {
            add(io->Wg_s, S * nh);
            add(io->Wu_s, S * nh);
            add(io->Wd_s, S * nh);
            add(io->Gs, (int64_t)T * S * h);
            add(io->Us, (int64_t)T * S * h);
        }
        hipLaunchKernelGGL(k_bwd_finite, dim3(1024, (unsigned)c), dim3(256), 0, s, L, err);
        le |= (int)hipGetLastError();
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
    // expert rows in perm order
    hipLaunchKernelGGL(k_bwd_gather, dim3((unsigned)Tk), dim3(256), 0, s, io->perm, io->X,
                       io->dY, io->weights, Tk, k, n, w->ctrl, w->Xp, w->dYp, w->rowq);
    le |= (int)hipGetLastError();
    le |= jtk_make_tiles(w->off32, E, BM_ROWS, w->tiles, w->ntiles, s);
    const unsigned mt = (unsigned)(Tk / BM_ROWS + E);  // bound on the routed tile count
    const int mt_sh = (int)cdiv(T, BM_ROWS);
    // Dg, Du, S = SwiGLU backward of (rows Wd^T): shared experts on all
    // tokens with dY unweighted, routed experts on their perm rows
    GemmP p{};
    p.err = err, p.N = h, p.nsh = S * mt_sh, p.mt_sh = mt_sh;
    {
        Side &a = p.sd[0];
        a.A[0] = io->dY, a.lda = n;
        a.B[0] = io->Wd_s, a.ldb = n, a.sBg = nh;
        a.C[0] = w->SDg, a.C[1] = w->SDu, a.C[2] = w->SSs, a.ldc = h, a.sCg = (int64_t)T * h;
        a.G = io->Gs, a.U = io->Us, a.ldg = S * h, a.sGg = h;
        a.M = T, a.K = n;
        Side &b = p.sd[1];
        b.A[0] = w->dYp, b.lda = n;
        b.B[0] = io->Wd, b.ldb = n, b.sBg = nh;
        b.C[0] = w->Dg, b.C[1] = w->Du, b.C[2] = w->Ss, b.ldc = h;
        b.G = io->Gsel, b.U = io->Usel, b.rowq = w->rowq, b.ldg = h;
        b.K = n, b.tiles = (const int4 *)w->tiles, b.ntiles = w->ntiles;
    }
    le |= launch_gemm<false, true, EPI_DSWIGLU, MODE_ROWS, TM_ROWS, TN_DOT>(
        p, dim3(p.nsh + mt, cdiv(h, 16 * TN_DOT)), s);
    // dx rows = (float)((double)(Dg Wg) + (double)(Du Wu))
    p = GemmP{};
    p.err = err, p.N = n, p.nsh = S * mt_sh, p.mt_sh = mt_sh;
    {
        Side &a = p.sd[0];
        a.A[0] = w->SDg, a.A[1] = w->SDu, a.lda = h, a.sAg = (int64_t)T * h;
        a.B[0] = io->Wg_s, a.B[1] = io->Wu_s, a.ldb = n, a.sBg = nh;
        a.C[0] = w->SDxe, a.ldc = n, a.sCg = (int64_t)T * n;
        a.M = T, a.K = h;
        Side &b = p.sd[1];
        b.A[0] = w->Dg, b.A[1] = w->Du, b.lda = h;
        b.B[0] = io->Wg, b.B[1] = io->Wu, b.ldb = n, b.sBg = nh;
        b.C[0] = w->Dxe, b.ldc = n;
        b.K = h, b.tiles = (const int4 *)w->tiles, b.ntiles = w->ntiles;
    }
    le |= launch_gemm<false, false, EPI_DUAL, MODE_ROWS, TM_ROWS, TN_DX>(
        p, dim3(p.nsh + mt, cdiv(n, 16 * TN_DX)), s);
    // weight gradients D^T rows: dWg = Dg^T X, dWu = Du^T X, dWd = S^T dY
    // (routed: weighted dY rows, over the expert's rows in perm order)
    p = GemmP{};
    p.err = err, p.N = n, p.nsh = 3 * S;
    {
        Side &a = p.sd[0];
        a.A[0] = w->SDg, a.A[1] = w->SDu, a.A[2] = w->SSs, a.lda = h, a.sAg = (int64_t)T * h;
        a.B[0] = io->X, a.B[1] = io->X, a.B[2] = io->dY, a.ldb = n;
        a.C[0] = io->dWg_s, a.C[1] = io->dWu_s, a.C[2] = io->dWd_s, a.ldc = n, a.sCg = nh;
        a.M = h, a.K = T;
        Side &b = p.sd[1];
        b.A[0] = w->Dg, b.A[1] = w->Du, b.A[2] = w->Ss, b.lda = h, b.sAk = h;
        b.B[0] = w->Xp, b.B[1] = w->Xp, b.B[2] = w->dYp, b.ldb = n, b.sBk = n;
        b.C[0] = io->dWg, b.C[1] = io->dWu, b.C[2] = io->dWd, b.ldc = n, b.sCg = nh;
        b.M = h, b.koff = w->off32;
    }
    le |= launch_gemm<true, false, EPI_STORE, MODE_WGRAD, TM_WG, TN_WG>(
        p, dim3(cdiv(h, 16 * TM_WG), cdiv(n, 16 * TN_WG), (unsigned)(3 * (S + E))), s);
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
