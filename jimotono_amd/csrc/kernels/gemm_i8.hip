// int8 GEMM kernels for gfx950: W8A8 (per-channel weights, per-row
// activations) and the grouped low-bit routed-expert GEMM.
//
// Arithmetic:
//   acc   = sum_k A[m][k] * W[n][k] in int32 (order-free, exact);
//   W8A8  : C = (float)((double)acc * ((double)sA[m] * (double)sB[n]))
//           -- the reference's epilogue, src/w8a8.c:664-676;
//   low-bit: per 64-K group g the int32 partial acc_g is taken out of the
//           MFMA and T = fmaf((float)acc_g, scale[n][g], T) in g order
//           (|acc_g| < 2^24, so the float conversion is exact);
//           C = T * sA[m].
// The matrix instruction is v_mfma_i32_16x16x64_i8 (4.3 POPS sustained per
// MI355X). Weights arrive in the 16-channel x 64-K panel layout of jt_dev.h,
// whose byte order equals the MFMA operand layout, so operand panels are
// copied global -> LDS with global_load_lds_dwordx4 (lane i's 16 bytes land
// at LDS base + 16*i) and read back with one ds_read_b128 per lane.
#include <type_traits>

#include "gemm_w8a8.h"
#include "jt_launch.h"
#include "topk_dev.h"
#include "sort_dev.h"
#include "quant_dev.h"

// Output fragment layout of v_mfma_i32_16x16x64_i8 (4 int32 per lane):
// element r of lane l is row 4*(l/16)+r, column l%16 of the 16x16 tile.

// ===================== skinny GEMM (decode, M <= 16) =====================
// One block of 16 waves per unit of NP panels (NP = 2 for SwiGLU: a gate
// block and its up block; NP = 1 otherwise). Wave w takes the 64-K blocks
// w, w+16, w+32, ... and issues all their loads before any math, so the
// whole weight matrix is in flight across the grid at once (decode shapes
// are bound by HBM latency and bandwidth). The M <= 16 activation rows are
// the A operand of one v_mfma_i32_16x16x64_i8 per panel (rows >= M read as
// zero); the 16 waves' int32 partial tiles are summed through LDS (exact).
#define SK_WAVES 16
#define SK_UNROLL 4

//
// QA (quantised activations made here): A is fp32 X [M][lda] with K valid
// columns. Every block first issues its weight loads, then quantises the M
// rows into LDS with the row quantiser's arithmetic (wave m on row m: the
// same scale and codes as k_quant_rows) and reads its A fragments from
// there, so a decode-sized expert needs no separate quantiser launch. The
// rows are re-quantised by every block; at M <= 16 that is at most 16 * K
// floats read from L2 per block.
//
// SkBatch (all zero for one GEMM): blockIdx.y selects one of gridDim.y
// GEMMs whose A (bytes), weight panels (bytes), sB and C (floats) lie at
// fixed strides (the shared experts' down projections in one launch), and
// hpl > 0 sends SwiGLU hidden column x to C[(x / hpl) * plane + m * ldc +
// x % hpl] (the shared experts' gate/ups over concatenated panels).
// rt16 != 0 instead makes blockIdx.y a 16-row tile of one GEMM of up to
// 16 * gridDim.y rows (rows 16y .. 16y+15 of A, sA and C): a GEMM of 17 to
// 64 rows then spreads over 4 x the blocks, each with one weight panel
// unit, and the blocks of one panel unit (x fixed) sit on one XCD when
// gridDim.x is a multiple of 8, so the panel is fetched once per XCD.
struct SkBatch {
    int hpl;
    int64_t plane, bsA, bsW;
    int bsB;
    int64_t bsC;
    int rt16;
};

// One block's work, for block (bx, by) of the grid: k_w8a8_skinny below, and
// the decode launches that run these blocks beside other work.
template <int EPI, int NP, int QV>  // QV > 0: QA with K <= 256 * QV
__device__ __forceinline__ void w8a8_skinny_block(
    int bx, int by, const void *__restrict__ Ain, int lda, const float *__restrict__ sAin,
    const int8_t *__restrict__ Wp, const float *__restrict__ sB, int M, int N, int Kp, int K,
    float *__restrict__ C, int ldc, uint32_t *err, SkBatch bt) {
    constexpr bool QA = QV > 0;
    if (bt.rt16) {  // rows 16 by .. 16 by + 15 of one GEMM
        const int r0 = 16 * by;
        if (QA)
            Ain = (const float *)Ain + (int64_t)r0 * lda;
        else
            Ain = (const int8_t *)Ain + (int64_t)r0 * lda;
        if (!QA) sAin += r0;
        C += (int64_t)r0 * ldc;
        M = min(16, M - r0);
    } else if (by) {  // the by-th GEMM of a batch
        Ain = (const int8_t *)Ain + by * bt.bsA;
        Wp += by * bt.bsW;
        sB += (int64_t)by * bt.bsB;
        C += by * bt.bsC;
    }
    __shared__ v4i red[SK_WAVES][NP][64];
    extern __shared__ __attribute__((aligned(16))) int8_t sk_aq[];  // QA: [16][Kp + 16]
    __shared__ float sk_sa[16];
    constexpr int NV = QA ? QV : 1;
    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform in a scalar register: guards on it then branch, which
    // matters because v_mfma ignores EXEC (an exec-masked MFMA still runs)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KB = Kp / 64;
    const int p0 = bx * NP;
    const int row = lane & 15, kc = lane >> 4;
    const int astr = Kp + 16;
    const int8_t *arow = QA ? sk_aq + row * astr + kc * 16
                            : (const int8_t *)Ain + (int64_t)min(row, M - 1) * lda + kc * 16;
    const float *sA = QA ? sk_sa : sAin;
    v4i acc[NP];
#pragma unroll
    for (int q = 0; q < NP; q++) acc[q] = (v4i){0, 0, 0, 0};
    // wave 0's epilogue scales, requested now so that their latency hides
    // behind the weight stream instead of following the reduction
    // (element r of lane l: row 4*(l/16) + r, channel l%16 of each panel)
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    float sbf[NP], saf[4];
    if (wave == 0) {
#pragma unroll
        for (int q = 0; q < NP; q++) sbf[q] = sB[min((p0 + q) * 16 + lc, N - 1)];
        if (!QA) {
#pragma unroll
            for (int r = 0; r < 4; r++) saf[r] = sAin[min(lr + r, M - 1)];
        }
    }
    v4i b0[SK_UNROLL][NP];  // QA: the first round's weights
    if (QA) {
        // the row loads go first: they are L2 hits and the quantiser needs
        // them, while the weights stream in behind them (loads return in
        // issue order, so the wait for the rows does not wait for weights)
        const int n4 = K >> 2;
        float4 v[NV];
        if (wave < M) {
            // (K % 4 == 0, K <= 256 * QV, 16-byte aligned rows: checked at launch)
            const float4 *x4 = (const float4 *)((const float *)Ain + (int64_t)wave * lda);
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int c = lane + 64 * j;
                v[j] = c < n4 ? x4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        const int kb0 = wave;
#pragma unroll
        for (int u = 0; u < SK_UNROLL; u++) {
            const int kb = kb0 + u * SK_WAVES;
            if (kb < KB) {
#pragma unroll
                for (int q = 0; q < NP; q++)
                    b0[u][q] = *(const v4i *)(Wp + ((int64_t)(p0 + q) * KB + kb) * 1024 +
                                              lane * 16);
            }
        }
        uint32_t flags = 0;
        if (wave < M) {  // row `wave`: k_quant_rows's scale and codes
            uint32_t mu = 0;
#pragma unroll
            for (int j = 0; j < NV; j++)
                if (64 * j < n4) {
                    mu = max(mu, max(abs_bits(v[j].x), abs_bits(v[j].y)));
                    mu = max(mu, max(abs_bits(v[j].z), abs_bits(v[j].w)));
                }
            mu = wave_max_u(mu);
            const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
            uint32_t *qr = (uint32_t *)(sk_aq + wave * astr);
            for (int c = n4 + lane; c < Kp / 4; c += 64) qr[c] = 0;  // K padding
            if (mu >= 0x7f800000u || !qp.ok) {
                flags = mu >= 0x7f800000u ? EF_NONFINITE_INPUT : EF_RANGE;
            } else {
                const float inv = quant_inv_f(qp.scale_d);
                uint32_t fmask = 0;  // bit j: a code of v[j] needs the exact quotient
#pragma unroll
                for (int j = 0; j < NV; j++) {
                    const int c = lane + 64 * j;
                    if (64 * j < n4) {
                        bool f = false;
                        const uint32_t q0 = (uint8_t)quant_code_try(v[j].x, inv, f);
                        const uint32_t q1 = (uint8_t)quant_code_try(v[j].y, inv, f);
                        const uint32_t q2 = (uint8_t)quant_code_try(v[j].z, inv, f);
                        const uint32_t q3 = (uint8_t)quant_code_try(v[j].w, inv, f);
                        fmask |= (uint32_t)(f && c < n4) << j;  // never rewrite past the row
                        if (c < n4) qr[c] = q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
                    }
                }
                while (fmask) {  // rare: redo those words exactly
                    const int j = __builtin_ctz(fmask);
                    fmask &= fmask - 1;
                    float4 u = v[0];
#pragma unroll
                    for (int i = 1; i < NV; i++)
                        if (i == j) u = v[i];
                    qr[lane + 64 * j] = (uint32_t)(uint8_t)quant_code(u.x, qp.scale_d) |
                                        ((uint32_t)(uint8_t)quant_code(u.y, qp.scale_d) << 8) |
                                        ((uint32_t)(uint8_t)quant_code(u.z, qp.scale_d) << 16) |
                                        ((uint32_t)(uint8_t)quant_code(u.w, qp.scale_d) << 24);
                }
            }
            if (lane == 0) sk_sa[wave] = qp.scale_f;
        }
        if (flags && lane == 0 && bx == 0) raise_err(err, flags);
        __syncthreads();
    }
    for (int kb0 = wave; kb0 < KB; kb0 += SK_WAVES * SK_UNROLL) {
        v4i a[SK_UNROLL], b[SK_UNROLL][NP];
#pragma unroll
        for (int u = 0; u < SK_UNROLL; u++) {
            const int kb = kb0 + u * SK_WAVES;
            if (kb < KB) {
                if (QA && kb0 == wave) {
#pragma unroll
                    for (int q = 0; q < NP; q++) b[u][q] = b0[u][q];
                } else {
#pragma unroll
                    for (int q = 0; q < NP; q++)
                        b[u][q] = *(const v4i *)(Wp + ((int64_t)(p0 + q) * KB + kb) * 1024 +
                                                 lane * 16);
                }
                a[u] = *(const v4i *)(arow + kb * 64);
            }
        }
#pragma unroll
        for (int u = 0; u < SK_UNROLL; u++) {
            const int kb = kb0 + u * SK_WAVES;
            if (kb < KB) {
                const v4i av = row < M ? a[u] : (v4i){0, 0, 0, 0};
#pragma unroll
                for (int q = 0; q < NP; q++) acc[q] = mfma16x16x64(av, b[u][q], acc[q]);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NP; q++) red[wave][q][lane] = acc[q];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int q = 0; q < NP; q++) {
        v4i t = red[0][q][lane];
#pragma unroll
        for (int w = 1; w < SK_WAVES; w++) t += red[w][q][lane];
        acc[q] = t;
    }
    double sa[4], sb[NP];
#pragma unroll
    for (int r = 0; r < 4; r++) sa[r] = (double)(QA ? sA[min(lr + r, M - 1)] : saf[r]);
#pragma unroll
    for (int q = 0; q < NP; q++) sb[q] = (double)sbf[q];
    uint32_t bad = 0, badmid = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = lr + r;
        if (m >= M) continue;
        if (EPI == EPI_PLAIN) {
#pragma unroll
            for (int q = 0; q < NP; q++) {
                const int col = (p0 + q) * 16 + lc;
                const float f = (float)((double)acc[q][r] * (sa[r] * sb[q]));
                if (col < N) {
                    bad |= !isfinite(f);
                    C[(int64_t)m * ldc + col] = f;
                }
            }
        } else if ((p0 + 1) * 16 + lc < N) {  // panel p0 = gate block, p0+1 its up block
            const float g = (float)((double)acc[0][r] * (sa[r] * sb[0]));
            const float u = (float)((double)acc[NP - 1][r] * (sa[r] * sb[NP - 1]));
            bad |= (!isfinite(g)) || (!isfinite(u));
            float sv;
            badmid |= !silu_mul(g, u, &sv);
            const int x0 = bx * 16;  // this block's first hidden column
            const int64_t at = bt.hpl > 0 ? (int64_t)(x0 / bt.hpl) * bt.plane + x0 % bt.hpl : x0;
            C[(int64_t)m * ldc + at + lc] = sv;
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

template <int EPI, int NP, int QV>
__global__ __launch_bounds__(64 * SK_WAVES) void k_w8a8_skinny(
    const void *__restrict__ Ain, int lda, const float *__restrict__ sAin,
    const int8_t *__restrict__ Wp, const float *__restrict__ sB, int M, int N, int Kp, int K,
    float *__restrict__ C, int ldc, uint32_t *err, SkBatch bt) {
    w8a8_skinny_block<EPI, NP, QV>((int)blockIdx.x, (int)blockIdx.y, Ain, lda, sAin, Wp, sB, M,
                                   N, Kp, K, C, ldc, err, bt);
}

// Every expert's W8A8 GEMM of the drop-in layer in one launch: block
// (16-channel panel bx, tile blockIdx.y of the 16-row tile list) runs the
// skinny kernel's block on the tile's rows of A (codes [row][lda], row scales
// sA) with its expert's panels P + e pstride and column scales
// sB + e sbstride, into C [row][ldc]. Same block, same sums and epilogue as
// the per-expert launches, so the same outputs.
__global__ __launch_bounds__(64 * SK_WAVES) void k_w8a8_skinny_tiles(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int8_t *__restrict__ P, int64_t pstride, const float *__restrict__ sB,
    int64_t sbstride, int N, int Kp, int K, float *__restrict__ C, int ldc,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ ntiles, uint32_t *err) {
    if ((int)blockIdx.y >= *ntiles) return;  // block-uniform
    const int4 td = tiles[blockIdx.y];        // {expert, first row, rows}
    w8a8_skinny_block<EPI_PLAIN, 1, 0>((int)blockIdx.x, 0, A + (int64_t)td.y * lda, lda,
                                       sA + td.y, P + (int64_t)td.x * pstride,
                                       sB + (int64_t)td.x * sbstride, td.z, N, Kp, K,
                                       C + (int64_t)td.y * ldc, ldc, err, SkBatch{});
}

extern "C" int jtk_w8a8_gemm_tiles(const int8_t *A, int lda, const float *sA, const int8_t *P,
                                   int64_t pstride, const float *sB, int64_t sbstride, int N,
                                   int Np, int Kp, int K, float *C, int ldc, const int32_t *tiles,
                                   const int32_t *ntiles, int max_tiles, uint32_t *err,
                                   hipStream_t s) {
    if (max_tiles <= 0) return 0;
    if (N <= 0 || Np < N || Np % 16 || Kp % 64 || K <= 0 || K > Kp || lda < Kp ||
        max_tiles > 65535)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_w8a8_skinny_tiles, dim3((unsigned)(Np / 16), (unsigned)max_tiles),
                       dim3(64 * SK_WAVES), 0, s, A, lda, sA, P, pstride, sB, sbstride, N, Kp, K,
                       C, ldc, (const int4 *)tiles, ntiles, err);
    return (int)hipGetLastError();
}

template <int QV>
static hipError_t launch_skinny_xq(const float *X, int ldx, int K, const int8_t *Wp,
                                   const float *sB, int M, int N, int Np, int Kp, float *C,
                                   int ldc, int swiglu, uint32_t *err, hipStream_t s,
                                   unsigned nb = 1, SkBatch bt = SkBatch{}) {
    const size_t lds = (size_t)16 * (Kp + 16);
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        if constexpr (QV <= 12)
            e = hipFuncSetAttribute((const void *)k_w8a8_skinny<EPI_SWIGLU, 2, QV>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_w8a8_skinny<EPI_PLAIN, 1, QV>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    if (swiglu) {
        // (the SwiGLU epilogue and 16 float4 per lane do not fit 128 VGPRs)
        if constexpr (QV <= 12)
            hipLaunchKernelGGL((k_w8a8_skinny<EPI_SWIGLU, 2, QV>), dim3((unsigned)(Np / 32)),
                               dim3(64 * SK_WAVES), lds, s, (const void *)X, ldx,
                               (const float *)NULL, Wp, sB, M, N, Kp, K, C, ldc, err, SkBatch{});
        else
            return hipErrorInvalidValue;
    } else
        hipLaunchKernelGGL((k_w8a8_skinny<EPI_PLAIN, 1, QV>), dim3((unsigned)(Np / 16), nb),
                           dim3(64 * SK_WAVES), lds, s, (const void *)X, ldx, (const float *)NULL,
                           Wp, sB, M, N, Kp, K, C, ldc, err, bt);
    return hipGetLastError();
}

extern "C" int jtk_w8a8_gemm_xq(const float *X, int ldx, int K, const int8_t *Wp,
                                const float *sB, int M, int N, int Np, int Kp, float *C, int ldc,
                                int swiglu, uint32_t *err, hipStream_t s) {
    if (M <= 0) return 0;
    if (M > 16 || K <= 0 || K > Kp || Kp % 64 || K % 4 || K > 4096 || ldx % 4 ||
        ((uintptr_t)X & 15) || (size_t)16 * (Kp + 16) > 96 * 1024)
        return (int)hipErrorInvalidValue;
    const int nv = (K + 255) / 256;  // float4 per lane of a row
    hipError_t e;
    if (nv <= 4)
        e = launch_skinny_xq<4>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, swiglu, err, s);
    else if (nv <= 8)
        e = launch_skinny_xq<8>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, swiglu, err, s);
    else if (nv <= 12)
        e = launch_skinny_xq<12>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, swiglu, err, s);
    else
        e = launch_skinny_xq<16>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, swiglu, err, s);
    return (int)e;
}

extern "C" int jtk_w8a8_gemm_ev(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                                const float *sB, int M, int N, int Np, int Kp, float *C,
                                int ldc, int swiglu, uint32_t *err, hipStream_t s,
                                hipEvent_t e0, hipEvent_t e1) {
    if (M <= 0) return 0;
    if (M <= 64 && e0) (void)hipEventRecord(e0, s);
    if (M <= 16) {
        if (swiglu)
            hipLaunchKernelGGL((k_w8a8_skinny<EPI_SWIGLU, 2, 0>), dim3((unsigned)(Np / 32)),
                               dim3(64 * SK_WAVES), 0, s, (const void *)A, lda, sA, Wp, sB, M, N,
                               Kp, Kp, C, ldc, err, SkBatch{});
        else
            hipLaunchKernelGGL((k_w8a8_skinny<EPI_PLAIN, 1, 0>), dim3((unsigned)(Np / 16)),
                               dim3(64 * SK_WAVES), 0, s, (const void *)A, lda, sA, Wp, sB, M, N,
                               Kp, Kp, C, ldc, err, SkBatch{});
    } else if (M <= 64) {
        // 16-row tiles of the skinny GEMM, one per grid row: 4x the blocks
        // of one 64-row block per panel unit
        SkBatch bt{};
        bt.rt16 = 1;
        const unsigned ty = (unsigned)((M + 15) / 16);
        if (swiglu)
            hipLaunchKernelGGL((k_w8a8_skinny<EPI_SWIGLU, 2, 0>), dim3((unsigned)(Np / 32), ty),
                               dim3(64 * SK_WAVES), 0, s, (const void *)A, lda, sA, Wp, sB, M, N,
                               Kp, Kp, C, ldc, err, bt);
        else
            hipLaunchKernelGGL((k_w8a8_skinny<EPI_PLAIN, 1, 0>), dim3((unsigned)(Np / 16), ty),
                               dim3(64 * SK_WAVES), 0, s, (const void *)A, lda, sA, Wp, sB, M, N,
                               Kp, Kp, C, ldc, err, bt);
    } else {
        // Tile choice (measured on MI355X): few 128x128 tiles -> 8 waves per
        // block with an intra-block k-split; otherwise 128 x 256 tiles of
        // 8 waves; SwiGLU pairs need an even number of 16-channel tiles.
        const int mt128 = (M + 127) / 128;
        const bool n256 = (Np % 256) == 0;
        hipError_t e;
        if (swiglu) {
            e = n256 ? launch_w8a8_tile<EPI_SWIGLU, 128, 256, 2, 4, 1, 3, 4>(
                           A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1)
                     : launch_w8a8_tile<EPI_SWIGLU, 128, 128, 2, 2, 2, 2, 4>(
                           A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1);
        } else if (!n256 || mt128 * (Np / 128) <= 512) {
            e = launch_w8a8_tile<EPI_PLAIN, 128, 128, 2, 2, 2, 3, 4>(
                A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1);
        } else {
            e = launch_w8a8_tile<EPI_PLAIN, 128, 256, 2, 4, 1, 3, 4>(
                A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1);
        }
        return (int)e;
    }
    const hipError_t e = hipGetLastError();
    if (e1) (void)hipEventRecord(e1, s);
    return (int)e;
}

extern "C" int jtk_w8a8_swiglu_planes(const int8_t *A, int lda, const float *sA,
                                      const int8_t *Wp, const float *sB, int M, int N, int Kp,
                                      float *C, int ldc, int hpl, int64_t plane, uint32_t *err,
                                      hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if (M <= 64 || N % 256 || hpl <= 0 || hpl % 16 || (N / 2) % hpl)
        return (int)hipErrorInvalidValue;
    return (int)launch_w8a8_tile<EPI_SWIGLU, 128, 256, 2, 4, 1, 3, 4>(
        A, lda, sA, Wp, sB, M, N, N, Kp, C, ldc, err, s, e0, e1, hpl, plane);
}

extern "C" int jtk_w8a8_gemm_batch(const int8_t *A, int lda, int64_t sAq, const float *sA,
                                   int ssA, const int8_t *Wp, int64_t sW, const float *sB,
                                   int ssB, int M, int N, int Np, int Kp, float *C, int ldc,
                                   int64_t sC, int nb, uint32_t *err, hipStream_t s,
                                   hipEvent_t e0, hipEvent_t e1) {
    if (M <= 64 || nb <= 0 || nb > 65535 || Np % 128) return (int)hipErrorInvalidValue;
    TileBatch bt{};
    bt.bsA = sAq;
    bt.bsW = sW;
    bt.bsSA = ssA;
    bt.bsB = ssB;
    bt.bsC = sC;
    // 128 x 256 tiles with a k-split over two groups of 8 waves (16 waves,
    // 3-stage ring of 144 KB: one block per CU) when the batch has at least
    // one such tile per CU: the shared experts' down projections (4096 x 1024
    // x 2816, 2 experts) measured 38.2-38.4 us against 50.4-50.7 us for
    // 128 x 128 tiles of 8 waves. Otherwise 128 x 128 tiles, k-split over
    // two groups of 4 waves, 3-stage ring (one block per CU; a 2-stage ring
    // with two blocks per CU measured 10% faster alone and 3% slower in the
    // layer, where the routed GEMMs run beside it)
    const int64_t wide = (int64_t)((M + 127) / 128) * (Np / 256) * nb;
    if (Np % 256 == 0 && wide >= 256)
        return (int)launch_w8a8_tile<EPI_PLAIN, 128, 256, 2, 4, 2, 3, 4>(
            A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1, 0, 0, (unsigned)nb, bt);
    return (int)launch_w8a8_tile<EPI_PLAIN, 128, 128, 2, 2, 2, 3, 4>(
        A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s, e0, e1, 0, 0, (unsigned)nb, bt);
}

extern "C" int jtk_w8a8_skinny_swiglu_planes(const int8_t *A, int lda, const float *sA,
                                             const int8_t *Wp, const float *sB, int M, int N,
                                             int Kp, float *C, int ldc, int hpl, int64_t plane,
                                             uint32_t *err, hipStream_t s) {
    if (M <= 0 || M > 16 || N % 32 || hpl <= 0 || hpl % 16 || (N / 2) % hpl)
        return (int)hipErrorInvalidValue;
    SkBatch bt{};
    bt.hpl = hpl;
    bt.plane = plane;
    hipLaunchKernelGGL((k_w8a8_skinny<EPI_SWIGLU, 2, 0>), dim3((unsigned)(N / 32)),
                       dim3(64 * SK_WAVES), 0, s, (const void *)A, lda, sA, Wp, sB, M, N, Kp, Kp,
                       C, ldc, err, bt);
    return (int)hipGetLastError();
}

extern "C" int jtk_w8a8_gemm_xq_batch(const float *X, int ldx, int K, int64_t sX,
                                      const int8_t *Wp, int64_t sW, const float *sB, int ssB,
                                      int M, int N, int Np, int Kp, float *C, int ldc,
                                      int64_t sC, int nb, uint32_t *err, hipStream_t s) {
    if (M <= 0 || nb <= 0) return 0;
    if (M > 16 || K <= 0 || K > Kp || Kp % 64 || K % 4 || K > 4096 || ldx % 4 || sX % 4 ||
        ((uintptr_t)X & 15) || (size_t)16 * (Kp + 16) > 96 * 1024 || nb > 65535)
        return (int)hipErrorInvalidValue;
    SkBatch bt{};
    bt.bsA = sX * (int64_t)sizeof(float);
    bt.bsW = sW;
    bt.bsB = ssB;
    bt.bsC = sC;
    const int nv = (K + 255) / 256;
    hipError_t e;
    if (nv <= 4)
        e = launch_skinny_xq<4>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, 0, err, s, nb, bt);
    else if (nv <= 8)
        e = launch_skinny_xq<8>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, 0, err, s, nb, bt);
    else if (nv <= 12)
        e = launch_skinny_xq<12>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, 0, err, s, nb, bt);
    else
        e = launch_skinny_xq<16>(X, ldx, K, Wp, sB, M, N, Np, Kp, C, ldc, 0, err, s, nb, bt);
    return (int)e;
}

extern "C" int jtk_w8a8_gemm(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                             const float *sB, int M, int N, int Np, int Kp, float *C,
                             int ldc, int swiglu, uint32_t *err, hipStream_t s) {
    return jtk_w8a8_gemm_ev(A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, swiglu, err, s, nullptr,
                            nullptr);
}

// ===================== grouped low-bit GEMM =====================
// Work item = (expert e, 64-row tile of that expert's rows) x 128 packed
// channels. A tile descriptor is {e, first sorted row, rows} (int4); rows of
// expert e are the sorted pairs pos = off[e] .. off[e+1]-1.
//   gate/up (BITS 2, EPI_SWIGLU): A row = Xq[perm[pos] / topk], sA = sx[token],
//       output S[pos][hidden] (ldo = h);
//   down    (BITS 4, EPI_SCATTER): A row = Sq[pos], sA = ss[pos],
//       output Ye[perm[pos]][col] (ldo = n).
// Each 64-K group is one pipeline stage in LDS: the 4 gathered A panels
// (one per wave, LDS-DMA with per-lane row addresses) and the 8 weight
// panel-groups of the 128 channels (raw bytes, 256 B per DMA). Waves split
// the 128 channels (32 each = 2 panels); B fragments are unpacked from LDS
// to signed int8 in registers.
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

#ifndef LB_STAGES
#define LB_STAGES 2  // measured on MI355X: 2 stages beat 3-7 (more blocks resident)
#endif
#ifndef LB_GQ_STAGES
#define LB_GQ_STAGES 2  // fused gate/up ring at f = 256 (2-5 stages measured equal)
#endif
#ifndef LB_GQ_PPW
#define LB_GQ_PPW 4  // fused gate/up at f = 256: 8 waves of 4 panels (measured: beats 16 of 2)
#endif

template <int BITS, int EPI, int NST>
__global__ __launch_bounds__(256, 2) void k_lowbit_grouped(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, const int32_t *__restrict__ off, int topk,
    const int32_t *__restrict__ tiles, const int32_t *__restrict__ ntiles,
    const uint8_t *__restrict__ Wp, const uint16_t *__restrict__ Ws, int64_t wp_stride,
    int64_t ws_stride, int N, int K, float *__restrict__ out, int ldo, uint32_t *err) {
    constexpr int PB = BITS == 2 ? 256 : 512;       // bytes per panel-group
    constexpr int BDMA = PB / 256;                  // 256-byte DMAs per panel-group
    constexpr int SOFF = 4096 + 8 * PB;             // scales after A and weight bytes
    constexpr int STAGE = SOFF + 4 * 256;           // + one 256-byte scale slot per wave
    constexpr int PER = 2 + 2 * BDMA;               // DMAs per wave per stage
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];  // NST * STAGE bytes
    __shared__ int rowsrc[64];
    __shared__ float rowscale[64];
    __shared__ int rowdst[64];
    const int tile = blockIdx.y;  // x walks the channel groups of a tile first
    // descriptor and tile count in one round trip (the grid never
    // passes the descriptor array, so the read is in bounds)
    const int4 td = ((const int4 *)tiles)[tile];  // {expert, first sorted row, rows}
    if (tile >= *ntiles) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar addressing
    const int e = td.x, pos0 = td.y, nrows = td.z;
    if (tid < 64) {
        const int r = min(tid, nrows - 1);
        const int pos = pos0 + r;
        int src;
        if (EPI == EPI_SWIGLU) {
            src = perm[pos] / topk;
            rowdst[tid] = pos;
        } else {
            src = pos;
            rowdst[tid] = perm[pos];
        }
        rowsrc[tid] = src;
        rowscale[tid] = sA[src];
    }
    __syncthreads();
    const int G = K / 64;
    const int n0 = blockIdx.x * 128;
    // A: wave w copies panel w (rows 16w..16w+15) of every stage;
    // lane l = kc*16 + r -> row 16w + r, bytes [16kc, 16kc+16) of the group
    const int8_t *a_src = A + (int64_t)rowsrc[wave * 16 + (lane & 15)] * lda + (lane >> 4) * 16;
    // B: wave w copies the panel-groups of panels pb0 + 2w and pb0 + 2w + 1
    const int pb0 = n0 >> 4;
    const uint8_t *wbase = Wp + (int64_t)e * wp_stride;
    // (wave-uniform bases; the lane offset is added at each copy so the
    // compiler keeps one offset register and advances the bases in SGPRs)
    const uint8_t *b_src0 = wbase + (int64_t)(pb0 + 2 * wave) * G * PB;
    const uint8_t *b_src1 = b_src0 + (int64_t)G * PB;
    // this wave's two panels (absolute panel index within the expert)
    const int pan0 = pb0 + wave * 2;
    // fp16 group scales of the two panels: lanes 0-7 copy panel pan0's 16
    // values (2 per lane), lanes 8-15 panel pan0+1's; lanes 16-63 repeat them
    // (the 4-byte DMA always writes 64 lanes)
    const int sl = lane & 15;
    const uint8_t *s_src = (const uint8_t *)(Ws + (int64_t)e * ws_stride + (int64_t)pan0 * G * 16);
    const int s_off = (sl >> 3) * G * 32 + (sl & 7) * 4;
    auto issue = [&](int g) {
        int8_t *st = smem + (g % NST) * STAGE;
        dma<16>(a_src + (int64_t)g * 64, st + wave * 1024);
#pragma unroll
        for (int d = 0; d < BDMA; d++) {
            dma<4>(b_src0 + (int64_t)g * PB + d * 256 + lane * 4,
                   st + 4096 + (2 * wave) * PB + d * 256);
            dma<4>(b_src1 + (int64_t)g * PB + d * 256 + lane * 4,
                   st + 4096 + (2 * wave + 1) * PB + d * 256);
        }
        dma<4>(s_src + (int64_t)g * 32 + s_off, st + SOFF + wave * 256);
    };
#pragma unroll
    for (int s = 0; s < NST - 1; s++)
        if (s < G) issue(s);

    float T[4][2][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) T[i][j][r] = 0.0f;

    for (int g = 0; g < G; g++) {
        wait_stage<PER>(min(NST - 2, G - 1 - g));
        barrier_lds();
        if (g + NST - 1 < G) issue(g + NST - 1);
        const int8_t *st = smem + (g % NST) * STAGE;
        const uint16_t *ss = (const uint16_t *)(st + SOFF + wave * 256);
        const float s0 = f16_to_f32(ss[lane & 15]);
        const float s1 = f16_to_f32(ss[16 + (lane & 15)]);
        v4i b[2];
        if (BITS == 2) {
            b[0] = unpack_int2(*(const uint32_t *)(st + 4096 + (2 * wave) * PB + lane * 4));
            b[1] = unpack_int2(*(const uint32_t *)(st + 4096 + (2 * wave + 1) * PB + lane * 4));
        } else {
            const uint2 w0 = *(const uint2 *)(st + 4096 + (2 * wave) * PB + lane * 8);
            const uint2 w1 = *(const uint2 *)(st + 4096 + (2 * wave + 1) * PB + lane * 8);
            b[0] = unpack_int4(w0.x, w0.y);
            b[1] = unpack_int4(w1.x, w1.y);
        }
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i *)(st + i * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (16 * i >= nrows) continue;  // wave-uniform: padding rows of a short tile
            const v4i z = {0, 0, 0, 0};
            const v4i c0 = mfma16x16x64(af[i], b[0], z);
            const v4i c1 = mfma16x16x64(af[i], b[1], z);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                T[i][0][r] = __builtin_fmaf((float)c0[r], s0, T[i][0][r]);
                T[i][1][r] = __builtin_fmaf((float)c1[r], s1, T[i][1][r]);
            }
        }
    }

    const int lr = (lane >> 4) * 4, lc = lane & 15;
    uint32_t bad = 0, badmid = 0;
    if (EPI == EPI_SWIGLU) {
        // wave's panels: pan0 = gate block, pan0+1 = matching up block
        const int hid = (pan0 / 2) * 16 + lc;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int rr = i * 16 + lr + r;
                if (rr >= nrows) continue;
                const float sa = rowscale[rr];
                const float gv = T[i][0][r] * sa;
                const float uv = T[i][1][r] * sa;
                bad |= (!isfinite(gv)) || (!isfinite(uv));
                float sv;
                badmid |= !silu_mul(gv, uv, &sv);
                out[(int64_t)rowdst[rr] * ldo + hid] = sv;
            }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = (pan0 + j) * 16 + lc;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int rr = i * 16 + lr + r;
                    if (rr >= nrows) continue;
                    const float f = T[i][j][r] * rowscale[rr];
                    bad |= !isfinite(f);
                    out[(int64_t)rowdst[rr] * ldo + col] = f;
                }
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

// ============ routed gate/up + SwiGLU + row codes, 64-row tiles ============
// A block covers all 2f gate/up channels of one (expert, 64-row) tile, so
// the SwiGLU rows are complete inside the block and leave it as int8 codes:
// no fp32 hidden rows in memory and no separate quantiser launch. NW waves
// of PPW panels each (NW * PPW = 2f/16); wave w owns panels PPW*w ..
// PPW*w+PPW-1, i.e. PPW/2 gate/up pairs (2j, 2j+1). One slot of an NST-stage
// ring per 64-K group holds the 4 gathered A panels (waves 0-3 copy one
// each), every wave's INT2 panel-groups and its fp16 scales. The folds are
// k_lowbit_grouped's. Epilogue: SwiGLU, the
// row max |h| (DPP over a panel's 16 channels, then LDS over the waves), the
// row quantiser's parameters once per row, and the codes of
// k_quant_rows written straight to Sq with the scale to ss.
template <int NW, int PPW, int NST>
__global__ __launch_bounds__(64 * NW) void k_lowbit_gu_q(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, int topk, const int32_t *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, const uint8_t *__restrict__ Wp,
    const uint16_t *__restrict__ Ws, int64_t wp_stride, int64_t ws_stride, int K,
    int8_t *__restrict__ Sq, float *__restrict__ ss, int h, uint32_t *err) {
    constexpr int PB = 256;                     // INT2 bytes per panel-group
    constexpr int SOFF = 4096 + NW * PPW * PB;  // scales after A and weights
    constexpr int NJ = PPW / 2;                 // gate/up pairs per wave
    constexpr int STAGE = SOFF + NW * 256;      // one 256-byte scale slot per wave
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];  // NST * STAGE
    __shared__ int rowsrc[64];
    __shared__ float rowscale[64];
    __shared__ uint32_t pmax[NW][64];
    __shared__ double rsd[64];
    __shared__ float rinv[64];
    __shared__ uint32_t rbad[64];
    __shared__ double exp_tab[64];
    // blocks go to the 8 XCDs round-robin by index: block b takes tile
    // (b % 8) * C + b / 8, C an eighth of the tile count, so each XCD works
    // through a contiguous run of the expert-ordered tile list and the tiles
    // of one expert read its weights through one L2
    const int nt = *ntiles;
    const int chunk = (nt + 7) >> 3, tl = (int)(blockIdx.x >> 3);
    const int tile = (int)(blockIdx.x & 7) * chunk + tl;
    if (tl >= chunk || tile >= nt) return;
    const int4 td = ((const int4 *)tiles)[tile];  // {expert, first sorted row, rows}
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e = td.x, pos0 = td.y, nrows = td.z;
    const double tabv = exp_tab_load(lane);  // staged in LDS for the SwiGLU
    if (tid < 64) {
        const int src = perm[pos0 + min(tid, nrows - 1)] / topk;
        rowsrc[tid] = src;
        rowscale[tid] = sA[src];
    }
    __syncthreads();
    const int G = K / 64;
    const int8_t *a_src =
        A + (int64_t)rowsrc[(wave & 3) * 16 + (lane & 15)] * lda + (lane >> 4) * 16;
    const int pan0 = PPW * wave;  // this wave's first panel within the expert
    const uint8_t *wb = Wp + (int64_t)e * wp_stride + (int64_t)pan0 * G * PB;
    const uint8_t *sbase =
        (const uint8_t *)(Ws + (int64_t)e * ws_stride + (int64_t)pan0 * G * 16);
    // scales: lanes 0..8*PPW-1 copy panel l >> 3's 16 values, 2 per lane;
    // the other lanes repeat them (the 4-byte DMA always writes 64 lanes)
    const int sl = lane & (8 * PPW - 1);
    const int s_off = (sl >> 3) * G * 32 + (sl & 7) * 4;
    auto issue = [&](int g) {
        int8_t *st = smem + (g % NST) * STAGE;
        if (wave < 4) dma<16>(a_src + (int64_t)g * 64, st + wave * 1024);
#pragma unroll
        for (int q = 0; q < PPW; q++)
            dma<4>(wb + ((int64_t)q * G + g) * PB + lane * 4,
                   st + 4096 + (PPW * wave + q) * PB);
        dma<4>(sbase + (int64_t)g * 32 + s_off, st + SOFF + wave * 256);
    };
#pragma unroll
    for (int g = 0; g < NST - 1; g++)
        if (g < G) issue(g);
    float T[4][PPW][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int q = 0; q < PPW; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) T[i][q][r] = 0.0f;
    for (int g = 0; g < G; g++) {
        // this wave's copies of stage g (waves 0-3 issue one more per stage)
        if (wave < 4)
            wait_stage<PPW + 2>(min(NST - 2, G - 1 - g));
        else
            wait_stage<PPW + 1>(min(NST - 2, G - 1 - g));
        barrier_lds();  // ... and every other wave's; stage g-1 is free
        if (g + NST - 1 < G) issue(g + NST - 1);
        const int8_t *st = smem + (g % NST) * STAGE;
        const uint16_t *s16 = (const uint16_t *)(st + SOFF + wave * 256);
        float sc[PPW];
        v4i b[PPW];
#pragma unroll
        for (int q = 0; q < PPW; q++) {
            sc[q] = f16_to_f32(s16[q * 16 + (lane & 15)]);
            b[q] = unpack_int2(
                *(const uint32_t *)(st + 4096 + (PPW * wave + q) * PB + lane * 4));
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (16 * i >= nrows) continue;  // wave-uniform: padding rows of a short tile
            const v4i af = *(const v4i *)(st + i * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < PPW; q++) {
                const v4i c = mfma16x16x64(af, b[q], (v4i){0, 0, 0, 0});
#pragma unroll
                for (int r = 0; r < 4; r++) T[i][q][r] = __builtin_fmaf((float)c[r], sc[q], T[i][q][r]);
            }
        }
    }
    // ---- SwiGLU of rows 16i + 4(l/16) + r, hidden channels (NJ w + jj)*16 + l%16 ----
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    uint32_t flags = 0;
    float sv[4][NJ][4];
    exp_tab_stage(exp_tab, lane, tabv);
    uint32_t gmx = 0;  // max |g|, |u| bits: non-finite iff >= those of +inf
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // wave-uniform: a short tile's padding row groups have no SwiGLU
        // (their pmax entries stay unset and their codes are never written)
        if (16 * i >= nrows) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 16 * i + lr + r;
            const float sa = rowscale[rr < nrows ? rr : 0];
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                sv[i][jj][r] = 0.0f;
                if (rr < nrows) {
                    const float gv = T[i][2 * jj][r] * sa, uv = T[i][2 * jj + 1][r] * sa;
                    gmx = max(gmx, max(abs_bits(gv), abs_bits(uv)));
                    (void)silu_mul(gv, uv, &sv[i][jj][r], exp_tab);
                }
            }
            uint32_t m = 0;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) m = max(m, abs_bits(sv[i][jj][r]));
            m = row16_allmax_u(m);  // over this wave's 16 * NJ channels of the row
            if (lc == 0) pmax[wave][rr] = m;
        }
    }
    if (gmx >= 0x7f800000u) flags |= EF_RANGE | EF_NONFINITE_MID;
    __syncthreads();
    // ---- the row quantiser's parameters, once per row ----
    if (tid < 64) {
        uint32_t mu = pmax[0][tid];
#pragma unroll
        for (int w = 1; w < NW; w++) mu = max(mu, pmax[w][tid]);
        const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
        const uint32_t bad = mu >= 0x7f800000u ? EF_NONFINITE_INPUT : (qp.ok ? 0u : EF_RANGE);
        rsd[tid] = qp.scale_d;
        rinv[tid] = quant_inv_f(qp.scale_d);
        rbad[tid] = bad;
        if (tid < nrows) {
            ss[pos0 + tid] = qp.scale_f;
            flags |= bad;
        }
    }
    __syncthreads();
    // ---- codes, straight to Sq [sorted row][h] ----
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (16 * i >= nrows) continue;  // wave-uniform, as above
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 16 * i + lr + r;
            if (rr >= nrows || rbad[rr]) continue;
            const float inv = rinv[rr];
            int8_t *qrow = Sq + (int64_t)(pos0 + rr) * h + NJ * wave * 16 + lc;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                bool f = false;
                int q = quant_code_try(sv[i][jj][r], inv, f);
                if (f) q = quant_code_call(sv[i][jj][r], rsd[rr]);
                qrow[16 * jj] = (int8_t)q;
            }
        }
    }
    if (flags) raise_err(err, flags);
}

template <int NW, int PPW, int NST>
static hipError_t launch_gu_q(int lds, int max_tiles, hipStream_t s, const int8_t *A, int lda,
                              const float *sA, const int32_t *perm, int topk,
                              const int32_t *tiles, const int32_t *ntiles, const uint8_t *Wp,
                              const uint16_t *Ws, int64_t wp_stride, int64_t ws_stride, int K,
                              int8_t *Sq, float *ss, int h, uint32_t *err) {
    auto kern = k_lowbit_gu_q<NW, PPW, NST>;
    // dynamic LDS above 64 KiB must be enabled per device, once
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                lds);
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    // 8 XCD runs of ceil(max_tiles / 8) tiles
    hipLaunchKernelGGL(kern, dim3(8u * (unsigned)((max_tiles + 7) / 8)), dim3(64 * NW), lds, s, A,
                       lda, sA, perm, topk, tiles, ntiles, Wp, Ws, wp_stride, ws_stride, K, Sq, ss,
                       h, err);
    return hipGetLastError();
}

extern "C" int jtk_lowbit_gateup_q(const int8_t *A, int lda, const float *sA,
                                   const int32_t *perm, int topk, const int32_t *tiles,
                                   const int32_t *ntiles, int max_tiles, const uint8_t *Wp,
                                   const uint16_t *Ws, int64_t wp_stride, int64_t ws_stride,
                                   int K, int8_t *Sq, float *ss, int h, uint32_t *err,
                                   hipStream_t s) {
    if (max_tiles <= 0) return 0;
    if (K % 64 || (h != 256 && h != 512)) return (int)hipErrorInvalidValue;
    if (h == 256) {
        constexpr int PPW = LB_GQ_PPW, NW = 32 / PPW, NST = LB_GQ_STAGES;
        constexpr int STAGE = 4096 + NW * PPW * 256 + NW * 256;
        return (int)launch_gu_q<NW, PPW, NST>(NST * STAGE, max_tiles, s, A, lda, sA, perm, topk,
                                              tiles, ntiles, Wp, Ws, wp_stride, ws_stride, K, Sq,
                                              ss, h, err);
    }
    // f = 512: a third ring stage measured 5-7% faster at 16384 tokens, E = 512
    constexpr int PPW = 4, NW = 16, NST = 3;
    constexpr int STAGE = 4096 + NW * PPW * 256 + NW * 256;
    return (int)launch_gu_q<NW, PPW, NST>(NST * STAGE, max_tiles, s, A, lda, sA, perm, topk, tiles,
                                          ntiles, Wp, Ws, wp_stride, ws_stride, K, Sq, ss, h,
                                          err);
}

// ===================== grouped low-bit GEMM, A tile resident =====================
// Same work and arithmetic as k_lowbit_grouped, with the block's 64 gathered
// A rows (all K) loaded into LDS once and CPB consecutive 128-channel groups
// per block: the pipeline streams only weight panel-groups and scales
// (stage s = channel group s / G, k-group s % G), and each channel group's
// epilogue runs as soon as its G k-groups are summed. This amortises the
// row gathering and the pipeline fill over CPB times more MFMA work.
template <int BITS, int EPI, int NST>
__global__ __launch_bounds__(256, 2) void k_lowbit_grouped_res(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, int topk, const int32_t *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, const uint8_t *__restrict__ Wp,
    const uint16_t *__restrict__ Ws, int64_t wp_stride, int64_t ws_stride, int N, int K,
    int cpb, float *__restrict__ out, int ldo, uint32_t *err) {
    constexpr int PB = BITS == 2 ? 256 : 512;  // bytes per panel-group
    constexpr int BDMA = PB / 256;             // 256-byte DMAs per panel-group
    constexpr int SOFF = 8 * PB;               // scales after the weight bytes
    constexpr int STAGE = SOFF + 4 * 256;      // + one 256-byte scale slot per wave
    constexpr int PER = 2 * BDMA + 1;          // DMAs per wave per stage
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];  // A tile + NST stages
    __shared__ int rowsrc[64];
    __shared__ float rowscale[64];
    __shared__ int rowdst[64];
    const int tile = blockIdx.y;  // x walks the channel groups of a tile first
    // descriptor and tile count in one round trip (the grid never
    // passes the descriptor array, so the read is in bounds)
    const int4 td = ((const int4 *)tiles)[tile];  // {expert, first sorted row, rows}
    if (tile >= *ntiles) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar addressing
    const int e = td.x, pos0 = td.y, nrows = td.z;
    if (tid < 64) {
        const int r = min(tid, nrows - 1);
        const int pos = pos0 + r;
        int src;
        if (EPI == EPI_SWIGLU) {
            src = perm[pos] / topk;
            rowdst[tid] = pos;
        } else {
            src = pos;
            rowdst[tid] = perm[pos];
        }
        rowsrc[tid] = src;
        rowscale[tid] = sA[src];
    }
    __syncthreads();
    const int G = K / 64;
    int8_t *atile = smem;                       // [G][4 panels][1 KiB]
    int8_t *ring = smem + (size_t)G * 4096;
    // A: wave w copies panel w (rows 16w..16w+15) of every k-group, once
    const int8_t *a_src = A + (int64_t)rowsrc[wave * 16 + (lane & 15)] * lda + (lane >> 4) * 16;
    for (int g = 0; g < G; g++) dma<16>(a_src + (int64_t)g * 64, atile + g * 4096 + wave * 1024);
    const int pbb = (blockIdx.x * cpb * 128) >> 4;  // the block's first panel
    const uint8_t *wbase = Wp + (int64_t)e * wp_stride;
    const uint8_t *sbase = (const uint8_t *)(Ws + (int64_t)e * ws_stride);
    const int sl = lane & 15;
    auto issue = [&](int s) {
        int8_t *st = ring + (s % NST) * STAGE;
        const int cg = s / G, g = s % G;
        const int pan0 = pbb + cg * 8 + 2 * wave;  // this wave's first panel
        // wave-uniform bases, the lane offset added at each copy
        const uint8_t *b0 = wbase + ((int64_t)pan0 * G + g) * PB;
        const uint8_t *b1 = b0 + (int64_t)G * PB;
#pragma unroll
        for (int d = 0; d < BDMA; d++) {
            dma<4>(b0 + d * 256 + lane * 4, st + (2 * wave) * PB + d * 256);
            dma<4>(b1 + d * 256 + lane * 4, st + (2 * wave + 1) * PB + d * 256);
        }
        // fp16 group scales of the two panels: lanes 0-7 panel pan0's 16
        // values (2 per lane), lanes 8-15 panel pan0+1's; lanes 16-63 repeat
        dma<4>(sbase + ((int64_t)pan0 * G + g) * 32 + ((sl >> 3) * G * 32 + (sl & 7) * 4),
               st + SOFF + wave * 256);
    };
    const int NS = cpb * G;
#pragma unroll
    for (int s = 0; s < NST - 1; s++)
        if (s < NS) issue(s);

    float T[4][2][4];
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    uint32_t bad = 0, badmid = 0;
    for (int s = 0; s < NS; s++) {
        const int cg = s / G, g = s % G;
        // the A tile was issued before stage 0, so stage waits cover it
        wait_stage<PER>(min(NST - 2, NS - 1 - s));
        barrier_lds();
        if (s + NST - 1 < NS) issue(s + NST - 1);
        if (g == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) T[i][j][r] = 0.0f;
        }
        const int8_t *st = ring + (s % NST) * STAGE;
        const uint16_t *ss = (const uint16_t *)(st + SOFF + wave * 256);
        const float s0 = f16_to_f32(ss[lane & 15]);
        const float s1 = f16_to_f32(ss[16 + (lane & 15)]);
        v4i b[2];
        if (BITS == 2) {
            b[0] = unpack_int2(*(const uint32_t *)(st + (2 * wave) * PB + lane * 4));
            b[1] = unpack_int2(*(const uint32_t *)(st + (2 * wave + 1) * PB + lane * 4));
        } else {
            const uint2 w0 = *(const uint2 *)(st + (2 * wave) * PB + lane * 8);
            const uint2 w1 = *(const uint2 *)(st + (2 * wave + 1) * PB + lane * 8);
            b[0] = unpack_int4(w0.x, w0.y);
            b[1] = unpack_int4(w1.x, w1.y);
        }
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i *)(atile + g * 4096 + i * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (16 * i >= nrows) continue;  // wave-uniform: padding rows of a short tile
            const v4i z = {0, 0, 0, 0};
            const v4i c0 = mfma16x16x64(af[i], b[0], z);
            const v4i c1 = mfma16x16x64(af[i], b[1], z);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                T[i][0][r] = __builtin_fmaf((float)c0[r], s0, T[i][0][r]);
                T[i][1][r] = __builtin_fmaf((float)c1[r], s1, T[i][1][r]);
            }
        }
        if (g != G - 1) continue;
        // epilogue of channel group cg
        const int pan0 = pbb + cg * 8 + 2 * wave;
        if (EPI == EPI_SWIGLU) {
            // wave's panels: pan0 = gate block, pan0+1 = matching up block
            const int hid = (pan0 / 2) * 16 + lc;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int rr = i * 16 + lr + r;
                    if (rr >= nrows) continue;
                    const float sa = rowscale[rr];
                    const float gv = T[i][0][r] * sa;
                    const float uv = T[i][1][r] * sa;
                    bad |= (!isfinite(gv)) || (!isfinite(uv));
                    float sv;
                    badmid |= !silu_mul(gv, uv, &sv);
                    out[(int64_t)rowdst[rr] * ldo + hid] = sv;
                }
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = (pan0 + j) * 16 + lc;
                if (col >= N) continue;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int rr = i * 16 + lr + r;
                        if (rr >= nrows) continue;
                        const float f = T[i][j][r] * rowscale[rr];
                        bad |= !isfinite(f);
                        out[(int64_t)rowdst[rr] * ldo + col] = f;
                    }
            }
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

// ============ routed down projection, weights in registers ============
// 64-row tiles of the INT4 down projection (K = h = 64 * G). The A rows
// are the tile's sorted hidden codes (contiguous rows pos0 .. pos0+nrows-1)
// and output row r goes to out[perm[pos0 + r]]. Block = 4 waves; wave w
// owns the CPW 16-channel panels starting at (4 * blockIdx.x + w) * CPW and
// requests every raw INT4 panel group of them into registers at the start,
// its fp16 group scales and one 16-row panel of the A tile by LDS-DMA, then
// waits once: no per-group ring, so each block pays one memory latency.
// The fold T = fmaf((float)acc_g, scale_g, T) runs in ascending g, the
// arithmetic of k_lowbit_grouped_res, so the outputs are identical.
// Blocks go to the 8 XCDs round-robin by their index: block b works on
// channel block (b / 8) % ncb of tile (b % 8) * C + (b / 8) / ncb, where C is
// an eighth of the tile count, so each XCD takes a contiguous run of the
// expert-ordered tile list and the tiles of one expert read its weights
// through one L2.
template <int G, int CPW>
__global__ __launch_bounds__(256) void k_lowbit_down_rr(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, const uint8_t *__restrict__ Wp,
    const uint16_t *__restrict__ Ws, int64_t wp_stride, int64_t ws_stride,
    float *__restrict__ out, int ldo, uint32_t *err, int ncb) {
    static_assert((CPW * G * 32) % 256 == 0, "scale copies of 256 bytes");
    __shared__ __attribute__((aligned(1024))) int8_t atile[G * 4 * 1024];  // [g][panel][64 x 16 B]
    __shared__ __attribute__((aligned(16))) uint16_t scl[4][CPW * G * 16];   // per wave [q][g][16]
    __shared__ float rsc[64];
    __shared__ int rdst[64];
    const int nt = *ntiles;
    const int chunk = (nt + 7) >> 3, sq = (int)(blockIdx.x >> 3);
    const int tl = sq / ncb, cblk = sq - tl * ncb;
    const int tile = (int)(blockIdx.x & 7) * chunk + tl;
    if (tl >= chunk || tile >= nt) return;
    const int4 td = tiles[tile];  // {expert, first sorted row, rows}
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = td.x, pos0 = td.y, nrows = td.z;
    if (nrows <= 0) return;
    // row scale and destination of row `lane` (wave 0), written to LDS later
    float my_sa = 0.0f;
    int my_dst = 0;
    if (wave == 0) {
        const int r = pos0 + min(lane, nrows - 1);
        my_sa = sA[r];
        my_dst = perm[r];
    }
    const int pan0 = (cblk * 4 + wave) * CPW;
    const uint8_t *wb = Wp + (int64_t)e * wp_stride + (int64_t)pan0 * G * 512;
    uint2 rw[CPW][G];
#pragma unroll
    for (int q = 0; q < CPW; q++)
#pragma unroll
        for (int g = 0; g < G; g++) rw[q][g] = *(const uint2 *)(wb + (q * G + g) * 512 + lane * 8);
    const uint8_t *sb = (const uint8_t *)(Ws + (int64_t)e * ws_stride) + (int64_t)pan0 * G * 32;
#pragma unroll
    for (int c = 0; c < CPW * G * 32 / 256; c++)
        dma<4>(sb + c * 256 + lane * 4, (char *)scl[wave] + c * 256);
    if (16 * wave < nrows) {
        const int row = min(16 * wave + (lane & 15), nrows - 1);
        const int8_t *as = A + (int64_t)(pos0 + row) * lda + (lane >> 4) * 16;
#pragma unroll
        for (int g = 0; g < G; g++) dma<16>(as + g * 64, atile + (g * 4 + wave) * 1024);
    }
    wait_vm<0>();
    if (wave == 0) {
        rsc[lane] = my_sa;
        rdst[lane] = my_dst;
    }
    lds_barrier();
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    float T[4][CPW][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int q = 0; q < CPW; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) T[i][q][r] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        v4i b[CPW];
        float sc[CPW];
#pragma unroll
        for (int q = 0; q < CPW; q++) {
            b[q] = unpack_int4(rw[q][g].x, rw[q][g].y);
            sc[q] = f16_to_f32(scl[wave][(q * G + g) * 16 + lc]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (16 * i >= nrows) continue;  // wave-uniform: padding rows of a short tile
            const v4i af = *(const v4i *)(atile + (g * 4 + i) * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < CPW; q++) {
                const v4i c = mfma16x16x64(af, b[q], (v4i){0, 0, 0, 0});
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    T[i][q][r] = __builtin_fmaf((float)c[r], sc[q], T[i][q][r]);
                    asm volatile("" : "+v"(T[i][q][r]));  // fold now, not after the loop
                }
            }
        }
    }
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 16 * i + lr + r;
            if (rr >= nrows) continue;
            const float sa = rsc[rr];
            float *y = out + (int64_t)rdst[rr] * ldo + pan0 * 16 + lc;
#pragma unroll
            for (int q = 0; q < CPW; q++) {
                const float f = T[i][q][r] * sa;
                bad |= !isfinite(f);
                y[16 * q] = f;
            }
        }
    if (bad) raise_err(err, EF_RANGE);
}

// ===================== grouped low-bit GEMM, few rows per expert =====================
// Decode-sized batches (a handful of rows per expert): work item = (expert
// e, 16 sorted rows) x 64 packed channels (4 panels). A block has
// nw = ceil(G / gpw) waves, gpw = min(4, G) consecutive 64-K groups per
// wave (G = K/64). Each wave issues every load it needs at once -- the raw
// INT2/INT4 bytes and fp16 scales of its groups (which need only the
// expert) before the gathered A rows (which need the permutation) -- and
// runs one MFMA per (group, panel). The group fold
// T = fmaf((float)acc_g, scale_g, T) in ascending g, the same fp32 sequence
// as the 64-row kernel, is then handed from wave to wave through LDS (wave
// w folds its groups onto wave w-1's T); the last wave writes the epilogue.
#define LS_PANELS 4
#define LS_GMAX 64

// raw panel-group bytes of one lane -> signed int8 operand
__device__ __forceinline__ v4i unpack_raw(uint32_t w) { return unpack_int2(w); }
__device__ __forceinline__ v4i unpack_raw(uint2 w) { return unpack_int4(w.x, w.y); }

template <int BITS, int EPI>
__global__ __launch_bounds__(1024) void k_lowbit_skinny(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, int topk, const uint8_t *__restrict__ Wp,
    const uint16_t *__restrict__ Ws, int64_t wp_stride, int64_t ws_stride, int N, int K,
    float *__restrict__ out, int ldo, uint32_t *err) {
    constexpr int PB = BITS == 2 ? 256 : 512;  // bytes per panel-group
    typedef typename std::conditional<BITS == 2, uint32_t, uint2>::type raw_t;
    __shared__ float4 tbuf[LS_PANELS][64];
    const int tile = blockIdx.y;  // x walks the channel groups of a tile first
    // descriptor and tile count in one round trip (the grid never
    // passes the descriptor array, so the read is in bounds)
    const int4 td = tiles[tile];  // {expert, first sorted row, rows}
    if (tile >= *ntiles) return;
    const int G = K / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform in a scalar register: guards on it then branch, which
    // matters because v_mfma ignores EXEC (an exec-masked MFMA still runs)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = blockDim.x >> 6;
    const int gpw = G < 4 ? G : 4;
    const int g0 = wave * gpw;
    const int e = td.x, pos0 = td.y, nrows = td.z;
    const int pan0 = blockIdx.x * LS_PANELS;
    const uint8_t *wb = Wp + (int64_t)e * wp_stride;
    const uint16_t *sb = Ws + (int64_t)e * ws_stride;
    raw_t braw[4][LS_PANELS];
    uint16_t sc[4][LS_PANELS];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        const int g = g0 + gi;
        if (gi < gpw && g < G) {
#pragma unroll
            for (int q = 0; q < LS_PANELS; q++) {
                const uint8_t *pg = wb + ((int64_t)(pan0 + q) * G + g) * PB;
                braw[gi][q] = *(const raw_t *)(pg + lane * sizeof(raw_t));
                sc[gi][q] = sb[((int64_t)(pan0 + q) * G + g) * 16 + (lane & 15)];
            }
        }
    }
    const int r = lane & 15, kc = lane >> 4;
    const int pos = pos0 + min(r, nrows - 1);
    const int src = EPI == EPI_SWIGLU ? perm[pos] / topk : pos;
    const int8_t *arow = A + (int64_t)src * lda + kc * 16;
    v4i a[4];
#pragma unroll
    for (int gi = 0; gi < 4; gi++)
        if (gi < gpw && g0 + gi < G) a[gi] = *(const v4i *)(arow + (int64_t)(g0 + gi) * 64);
    // the last wave also needs the rows' scales and destinations
    const int lc = lane & 15, lr = (lane >> 4) * 4;
    float sa[4];
    int dst[4];
    if (wave == nw - 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = pos0 + min(lr + i, nrows - 1);
            const int s2 = EPI == EPI_SWIGLU ? perm[p] / topk : p;
            sa[i] = sA[s2];
            dst[i] = EPI == EPI_SWIGLU ? p : perm[p];
        }
    }
    v4i acc[4][LS_PANELS];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        if (!(gi < gpw && g0 + gi < G)) continue;
        const v4i av = r < nrows ? a[gi] : (v4i){0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < LS_PANELS; q++) {
            acc[gi][q] = mfma16x16x64(av, unpack_raw(braw[gi][q]), (v4i){0, 0, 0, 0});
        }
    }
    // element q of lane l: row 4*(l/16) + q, channel l%16 of each panel
    float T[LS_PANELS][4];
    for (int ph = 0; ph < nw; ph++) {
        if (wave == ph) {
#pragma unroll
            for (int q = 0; q < LS_PANELS; q++) {
                const float4 t = ph == 0 ? make_float4(0.f, 0.f, 0.f, 0.f) : tbuf[q][lane];
                T[q][0] = t.x;
                T[q][1] = t.y;
                T[q][2] = t.z;
                T[q][3] = t.w;
            }
#pragma unroll
            for (int gi = 0; gi < 4; gi++) {
                if (!(gi < gpw && g0 + gi < G)) continue;
#pragma unroll
                for (int q = 0; q < LS_PANELS; q++) {
                    const float s = f16_to_f32(sc[gi][q]);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        T[q][i] = __builtin_fmaf((float)acc[gi][q][i], s, T[q][i]);
                }
            }
            if (ph + 1 < nw)
#pragma unroll
                for (int q = 0; q < LS_PANELS; q++)
                    tbuf[q][lane] = make_float4(T[q][0], T[q][1], T[q][2], T[q][3]);
        }
        if (ph + 1 < nw) __syncthreads();
    }
    if (wave != nw - 1) return;
    uint32_t bad = 0, badmid = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (lr + i >= nrows) continue;
        if (EPI == EPI_SWIGLU) {
            // panels pan0 + 2j (gate block) and pan0 + 2j + 1 (its up block)
#pragma unroll
            for (int j = 0; j < LS_PANELS / 2; j++) {
                const int hid = (pan0 / 2 + j) * 16 + lc;
                if ((pan0 + 2 * j + 1) * 16 + lc >= N) continue;
                const float gv = T[2 * j][i] * sa[i];
                const float uv = T[2 * j + 1][i] * sa[i];
                bad |= (!isfinite(gv)) || (!isfinite(uv));
                float sv;
                badmid |= !silu_mul(gv, uv, &sv);
                out[(int64_t)dst[i] * ldo + hid] = sv;
            }
        } else {
#pragma unroll
            for (int q = 0; q < LS_PANELS; q++) {
                const int col = (pan0 + q) * 16 + lc;
                if (col >= N) continue;
                const float f = T[q][i] * sa[i];
                bad |= !isfinite(f);
                out[(int64_t)dst[i] * ldo + col] = f;
            }
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

template <int BITS, int EPI>
static hipError_t launch_lowbit_skinny(dim3 grid, int G, hipStream_t s, const int8_t *A,
                                       int lda, const float *sA, const int32_t *perm,
                                       const int4 *tiles, const int32_t *ntiles, int topk,
                                       const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                                       int64_t ws_stride, int N, int K, float *out, int ldo,
                                       uint32_t *err) {
    auto kern = k_lowbit_skinny<BITS, EPI>;
    const int gpw = G < 4 ? G : 4;
    const int nw = (G + gpw - 1) / gpw;  // <= 16 for G <= LS_GMAX
    hipLaunchKernelGGL(kern, grid, dim3(64 * nw), 0, s, A, lda, sA, perm, tiles, ntiles, topk,
                       Wp, Ws, wp_stride, ws_stride, N, K, out, ldo, err);
    return hipGetLastError();
}

// ===================== routed FFN of a 16-row tile, one launch =====================
// Decode-sized batches: one block of 16 waves runs a whole (expert, <= 16
// sorted rows) tile through gate/up, SwiGLU, the per-row int8 quantiser and
// the down projection, so the three steps cost one launch and the
// intermediate rows never leave LDS. Every weight byte of the expert (INT2
// gate/up, INT4 down) and its fp16 scales are requested at the start: the
// raw panels into registers, the scales and the gathered A rows by
// LDS-DMA. Wave w owns h-channel block w (gate panel 2w, up panel 2w+1,
// every 64-K group in ascending order) and then down panels
// DPW*w .. DPW*w+DPW-1. The arithmetic
// is that of k_lowbit_skinny + k_quant_rows + k_lowbit_skinny: the same fp32
// group folds, the same SwiGLU and the same row codes, so the outputs are
// identical. h = 256 (16 blocks of 16 channels); n = 64*G1.
#define RF_H 256
#define RF_WAVES 16
#define RF_HSTR (RF_H + 4)   // fp32 gate/up row stride (floats)
#define RF_QSTR (RF_H + 16)  // int8 h row stride (bytes)
#define DS_QV_MAX 12         // shared down beside the routed FFN: K <= 3072 (LDS)

template <int G1>
__device__ __forceinline__ void routed_ffn16_block(
    int tile, const int8_t *__restrict__ Xq, const float *__restrict__ sx,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, int topk, const uint8_t *__restrict__ guP,
    const uint16_t *__restrict__ guS, int64_t gu_pstride, int64_t gu_sstride,
    const uint8_t *__restrict__ dnP, const uint16_t *__restrict__ dnS, int64_t dn_pstride,
    int64_t dn_sstride, float *__restrict__ Ye, int8_t *__restrict__ Hq,
    float *__restrict__ Hs, uint32_t *err) {
    constexpr int N = 64 * G1;                    // model width
    constexpr int HB = (RF_H / 16) / RF_WAVES;    // h blocks per wave (2)
    constexpr int DPW = (N / 16) / RF_WAVES;      // down panels per wave
    constexpr int ASTR = N + 16;                  // A row stride (bytes)
    constexpr int GUS_B = (2 * RF_H / 16) * G1 * 32;  // gate/up scale bytes of one expert
    constexpr int DNS_B = (N / 16) * (RF_H / 64) * 32;
    static_assert(N % 256 == 0 && N <= 1024, "n = 256, 512, 768 or 1024");
    static_assert(GUS_B % 1024 == 0 && DNS_B % 1024 == 0, "1 KiB scale copies");
    __shared__ __attribute__((aligned(16))) int8_t As[16 * ASTR];
    __shared__ __attribute__((aligned(16))) uint16_t gus[GUS_B / 2];
    __shared__ __attribute__((aligned(16))) uint16_t dns[DNS_B / 2];
    __shared__ __attribute__((aligned(16))) float gb[16 * RF_HSTR];
    __shared__ __attribute__((aligned(16))) float ub[16 * RF_HSTR];
    __shared__ __attribute__((aligned(16))) int8_t hq[16 * RF_QSTR];
    __shared__ float rsa[16], rsq[16];
    __shared__ int rdst[16];
    __shared__ double exp_tab[64];
    // descriptor and tile count in one round trip (the grid never
    // passes the descriptor array, so the read is in bounds)
    const int4 td = tiles[tile];  // {expert, first sorted row, rows}
    if (tile >= *ntiles) return;
    const int lane = threadIdx.x & 63;
    // the SwiGLU's exp table entry, requested before the weights so that its
    // wait does not wait for them
    const double tabv = exp_tab_load(lane);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = td.x, pos0 = td.y, nrows = td.z;
    if (nrows <= 0) return;
    const uint8_t *gp = guP + (int64_t)e * gu_pstride;
    const uint8_t *dp = dnP + (int64_t)e * dn_pstride;
    const uint8_t *gsb = (const uint8_t *)(guS + (int64_t)e * gu_sstride);
    const uint8_t *dsb = (const uint8_t *)(dnS + (int64_t)e * dn_sstride);
    // Requests in an order that lets the gate/up start while the rest of
    // the weights stream in (a wave's vector loads complete in issue order):
    //   1. the wave's share of the fp16 scales,
    //   2. the raw gate/up panels of the first GA 64-K groups,
    //   3. the wave's A row (it needs the permutation, a scalar load issued
    //      first, whose wait the group loads above cover),
    //   4. the raw gate/up panels of the other groups, one group at a time,
    //   5. the raw down panels.
    // Everything lands in registers; the scales and the A row go on to LDS
    // once they are in, and after a barrier the gate/up of groups < GA runs
    // while steps 4-5 are still in flight; group g >= GA waits only for its
    // own loads. (Plain register loads, not LDS-DMA: the compiler keeps an
    // exact count of those and waits for just the load a value needs.)
    // Compiler barriers keep the loads of each step in their place.
    constexpr int GA = G1 / 2;
    static_assert(16 / RF_WAVES == 1, "one A row per wave");
    static_assert(GUS_B / 1024 <= RF_WAVES && DNS_B / 1024 <= RF_WAVES, "one 1 KiB copy per wave");
    const int arow = wave;
    const int pv = perm[pos0 + min(arow, nrows - 1)];  // scalar load, waited for at step 3
    const bool has_gs = wave < GUS_B / 1024, has_ds = wave < DNS_B / 1024;  // wave-uniform
    uint4 gs4 = {0, 0, 0, 0}, ds4 = {0, 0, 0, 0};
    if (has_gs) gs4 = *(const uint4 *)(gsb + wave * 1024 + lane * 16);
    if (has_ds) ds4 = *(const uint4 *)(dsb + wave * 1024 + lane * 16);
    // raw weights into registers (wave-uniform bases and constant offsets:
    // one address register for all)
    const uint8_t *gw = gp + (int64_t)(2 * HB * wave) * G1 * 256;
    const uint8_t *dw = dp + (int64_t)(DPW * wave) * 4 * 512;
    uint32_t rg[HB][G1], ru[HB][G1];
#pragma unroll
    for (int g = 0; g < GA; g++)
#pragma unroll
        for (int j = 0; j < HB; j++) {
            rg[j][g] = *(const uint32_t *)(gw + ((2 * j) * G1 + g) * 256 + lane * 4);
            ru[j][g] = *(const uint32_t *)(gw + ((2 * j + 1) * G1 + g) * 256 + lane * 4);
        }
    asm volatile("" ::: "memory");
    const int src = pv / topk;
    uint4 a4 = {0, 0, 0, 0};
    if (lane < N / 16) a4 = *(const uint4 *)(Xq + (int64_t)src * N + lane * 16);
    const float sxv = sx[src];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int g = GA; g < G1; g++) {
#pragma unroll
        for (int j = 0; j < HB; j++) {
            rg[j][g] = *(const uint32_t *)(gw + ((2 * j) * G1 + g) * 256 + lane * 4);
            ru[j][g] = *(const uint32_t *)(gw + ((2 * j + 1) * G1 + g) * 256 + lane * 4);
        }
        asm volatile("" ::: "memory");
    }
    uint2 rd[DPW][4];
#pragma unroll
    for (int q = 0; q < DPW; q++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            rd[q][g] = *(const uint2 *)(dw + (q * 4 + g) * 512 + lane * 8);
    asm volatile("" ::: "memory");
    // steps 1 and 3 to LDS (each store waits only for its own load), then
    // every wave's
    if (has_gs) *(uint4 *)((char *)gus + wave * 1024 + lane * 16) = gs4;
    if (has_ds) *(uint4 *)((char *)dns + wave * 1024 + lane * 16) = ds4;
    if (lane < N / 16) *(uint4 *)(As + arow * ASTR + lane * 16) = a4;
    if (lane == 0) {
        rsa[arow] = sxv;
        rdst[arow] = pv;
    }
    lds_barrier();
    // ---- gate/up: rows 4*(lane/16)+i, h channel 16*(HB*wave+j) + lane%16 ----
    const int r = lane & 15, kc = lane >> 4, lc = lane & 15, lr = (lane >> 4) * 4;
    float Tg[HB][4], Tu[HB][4];
#pragma unroll
    for (int j = 0; j < HB; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) Tg[j][i] = Tu[j][i] = 0.f;
    // one group at a time; the next group's A fragment and scales are read
    // one group ahead
    v4i an = *(const v4i *)(As + r * ASTR + kc * 16);
    uint16_t sgn[HB], sun[HB];
#pragma unroll
    for (int j = 0; j < HB; j++) {
        sgn[j] = gus[((2 * (HB * wave + j)) * G1) * 16 + lc];
        sun[j] = gus[((2 * (HB * wave + j) + 1) * G1) * 16 + lc];
    }
#pragma unroll
    for (int g = 0; g < G1; g++) {
        // group g's raw panels, pinned here: the compiler then waits for
        // exactly their loads at this point (later groups' and the down
        // panels' loads stay in flight), and the scheduler cannot hoist
        // their unpacking above the last loads
#pragma unroll
        for (int j = 0; j < HB; j++) asm volatile("" : "+v"(rg[j][g]), "+v"(ru[j][g])::"memory");
        const v4i a = an;
        if (g + 1 < G1) an = *(const v4i *)(As + r * ASTR + (g + 1) * 64 + kc * 16);
#pragma unroll
        for (int j = 0; j < HB; j++) {
            const int hb = HB * wave + j;
            const float sg = f16_to_f32(sgn[j]), su = f16_to_f32(sun[j]);
            if (g + 1 < G1) {
                sgn[j] = gus[((2 * hb) * G1 + g + 1) * 16 + lc];
                sun[j] = gus[((2 * hb + 1) * G1 + g + 1) * 16 + lc];
            }
            const v4i cg = mfma16x16x64(a, unpack_int2(rg[j][g]), (v4i){0, 0, 0, 0});
            const v4i cu = mfma16x16x64(a, unpack_int2(ru[j][g]), (v4i){0, 0, 0, 0});
#pragma unroll
            for (int i = 0; i < 4; i++) {
                Tg[j][i] = __builtin_fmaf((float)cg[i], sg, Tg[j][i]);
                Tu[j][i] = __builtin_fmaf((float)cu[i], su, Tu[j][i]);
                // pin the fold here: left alone the compiler keeps every
                // group's MFMA result live and folds after the loop
                asm volatile("" : "+v"(Tg[j][i]), "+v"(Tu[j][i]));
            }
        }
    }
    uint32_t flags = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = lr + i;
        if (row >= nrows) continue;
        const float sa = rsa[row];
#pragma unroll
        for (int j = 0; j < HB; j++) {
            const float gv = Tg[j][i] * sa, uv = Tu[j][i] * sa;
            if (!isfinite(gv) || !isfinite(uv)) flags |= EF_RANGE;
            gb[row * RF_HSTR + 16 * (HB * wave + j) + lc] = gv;
            ub[row * RF_HSTR + 16 * (HB * wave + j) + lc] = uv;
        }
    }
    exp_tab_stage(exp_tab, lane, tabv);
    lds_barrier();
    // ---- SwiGLU and the per-row int8 codes of h, wave w on row w ----
#pragma unroll 1
    for (int row = wave; row < nrows; row += RF_WAVES) {
        const float4 g4 = *(const float4 *)(gb + row * RF_HSTR + lane * 4);
        const float4 u4 = *(const float4 *)(ub + row * RF_HSTR + lane * 4);
        float4 v;
        bool ok = silu_mul(g4.x, u4.x, &v.x, exp_tab);
        ok &= silu_mul(g4.y, u4.y, &v.y, exp_tab);
        ok &= silu_mul(g4.z, u4.z, &v.z, exp_tab);
        ok &= silu_mul(g4.w, u4.w, &v.w, exp_tab);
        if (!ok) flags |= EF_NONFINITE_MID;
        uint32_t mu = max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w)));
        mu = wave_max_u(mu);
        const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
        if (mu >= 0x7f800000u) {
            flags |= EF_NONFINITE_INPUT;
        } else if (!qp.ok) {
            flags |= EF_RANGE;
        } else {
            const float inv = quant_inv_f(qp.scale_d);
            const uint32_t b0 = (uint8_t)quant_code_fast(v.x, qp.scale_d, inv);
            const uint32_t b1 = (uint8_t)quant_code_fast(v.y, qp.scale_d, inv);
            const uint32_t b2 = (uint8_t)quant_code_fast(v.z, qp.scale_d, inv);
            const uint32_t b3 = (uint8_t)quant_code_fast(v.w, qp.scale_d, inv);
            const uint32_t wd = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            *(uint32_t *)(hq + row * RF_QSTR + lane * 4) = wd;
            // the hidden row's codes and scale also go to memory, in sorted
            // row order like the 64-row path's
            *(uint32_t *)(Hq + (int64_t)(pos0 + row) * RF_H + lane * 4) = wd;
            if (lane == 0) {
                rsq[row] = qp.scale_f;
                Hs[pos0 + row] = qp.scale_f;
            }
        }
    }
    lds_barrier();
    // the down panels, pinned after the SwiGLU (see the gate/up)
#pragma unroll
    for (int q = 0; q < DPW; q++)
#pragma unroll
        for (int g = 0; g < 4; g++) asm volatile("" : "+v"(rd[q][g].x), "+v"(rd[q][g].y)::"memory");
    // ---- down: rows 4*(lane/16)+i, channel 16*(DPW*wave+q) + lane%16 ----
    float Td[DPW][4];
#pragma unroll
    for (int q = 0; q < DPW; q++)
#pragma unroll
        for (int i = 0; i < 4; i++) Td[q][i] = 0.f;
#pragma unroll
    for (int g = 0; g < RF_H / 64; g++) {
        const v4i a = *(const v4i *)(hq + r * RF_QSTR + g * 64 + kc * 16);
#pragma unroll
        for (int q = 0; q < DPW; q++) {
            const v4i c = mfma16x16x64(a, unpack_int4(rd[q][g].x, rd[q][g].y),
                                       (v4i){0, 0, 0, 0});
            const float sd = f16_to_f32(dns[((DPW * wave + q) * 4 + g) * 16 + lc]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                Td[q][i] = __builtin_fmaf((float)c[i], sd, Td[q][i]);
                asm volatile("" : "+v"(Td[q][i]));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = lr + i;
        if (row >= nrows) continue;
        const float sa = rsq[row];
        float *y = Ye + (int64_t)rdst[row] * N + 16 * DPW * wave + lc;
#pragma unroll
        for (int q = 0; q < DPW; q++) {
            const float f = Td[q][i] * sa;
            if (!isfinite(f)) flags |= EF_RANGE;
            y[16 * q] = f;
        }
    }
    if (flags) raise_err(err, flags);
}

template <int G1>
__global__ __launch_bounds__(64 * RF_WAVES) void k_routed_ffn16(
    const int8_t *__restrict__ Xq, const float *__restrict__ sx,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, int topk, const uint8_t *__restrict__ guP,
    const uint16_t *__restrict__ guS, int64_t gu_pstride, int64_t gu_sstride,
    const uint8_t *__restrict__ dnP, const uint16_t *__restrict__ dnS, int64_t dn_pstride,
    int64_t dn_sstride, float *__restrict__ Ye, int8_t *__restrict__ Hq,
    float *__restrict__ Hs, uint32_t *err) {
    routed_ffn16_block<G1>((int)blockIdx.x, Xq, sx, perm, tiles, ntiles, topk, guP, guS,
                           gu_pstride, gu_sstride, dnP, dnS, dn_pstride, dn_sstride, Ye, Hq, Hs,
                           err);
}

template <int BITS, int EPI, int NST>
static hipError_t launch_lowbit(dim3 grid, hipStream_t s, const int8_t *A, int lda,
                                const float *sA, const int32_t *perm, const int32_t *off,
                                int topk, const int32_t *tiles, const int32_t *ntiles,
                                const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                                int64_t ws_stride, int N, int K, float *out, int ldo,
                                uint32_t *err) {
    constexpr int PB = BITS == 2 ? 256 : 512;
    constexpr int lds = NST * (4096 + 8 * PB + 4 * 256);
    auto kern = k_lowbit_grouped<BITS, EPI, NST>;
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                lds);
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, A, lda, sA, perm, off, topk, tiles, ntiles,
                       Wp, Ws, wp_stride, ws_stride, N, K, out, ldo, err);
    return hipGetLastError();
}

#define LBR_KMAX 1024  // resident A tile: 64 rows x K bytes of LDS

template <int BITS, int EPI, int NST>
static hipError_t launch_lowbit_res(dim3 grid, int cpb, hipStream_t s, const int8_t *A, int lda,
                                    const float *sA, const int32_t *perm, int topk,
                                    const int32_t *tiles, const int32_t *ntiles,
                                    const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                                    int64_t ws_stride, int N, int K, float *out, int ldo,
                                    uint32_t *err) {
    constexpr int PB = BITS == 2 ? 256 : 512;
    constexpr int lds_max = LBR_KMAX * 64 + NST * (8 * PB + 4 * 256);
    const int lds = K * 64 + NST * (8 * PB + 4 * 256);
    auto kern = k_lowbit_grouped_res<BITS, EPI, NST>;
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                lds_max);
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, A, lda, sA, perm, topk, tiles, ntiles, Wp,
                       Ws, wp_stride, ws_stride, N, K, cpb, out, ldo, err);
    return hipGetLastError();
}

// ============ routed FFN of 16-row tiles over 4 CUs, two launches ============
// A decode tile (one expert, <= 16 sorted rows, f = 256) is VALU-bound on one
// CU: unpacking its INT2/INT4 panels and folding the 64-K groups of 16-row
// MFMA tiles take about 1600 VALU instructions per wave in the one-block
// form above, with the tile's few real rows using a sixteenth of each MFMA.
// Here every tile runs on four blocks in each of two launches, so four CUs
// share that work:
//   k_routed_gu16: block (tile, quarter) = 4 waves; wave w takes h-block
//     hb = 4 quarter + w (gate panel 2 hb, up panel 2 hb + 1), folds every
//     64-K group in order and applies the SwiGLU to its own elements, and
//     writes the fp32 hidden values to S [sorted row][256];
//   k_routed_dn16: block (tile, quarter) = 16 waves; wave w quantises hidden
//     row w (k_quant_rows's scale and codes) into LDS, then takes down
//     panel N/64 quarter + w (waves past N/64 only quantise).
// The arithmetic is that of routed_ffn16_block element for element (the
// same folds, SwiGLU and codes), so Ye, the codes and the scales are
// identical; the fp32 hidden rows pass through memory unchanged.
#define RA_WAVES 8  // 4 h-blocks per block, a gate and an up wave for each

// ---- caller-routed decode: the pair sort inside the gate/up launch ----
// With SORT, k_routed_gu16 also does k_quant_sort_small's work (Tk <=
// SORTF_TK pairs, E <= SORTF_E experts, no drops, 16-row tiles), so the
// routed FFN of a caller-routed decode takes two launches instead of three:
//   blocks 0 .. 4 mt - 1 (mt bounds the tile count): (tile, quarter) as
//     without SORT, except that each block ranks the Tk pairs in LDS itself
//     (tile_of_sort, sort_small_fast's ranks and tile list), which gives its
//     tile's descriptor and rows with no round trip through memory, and that
//     its waves quantise their two token rows from X into LDS (the codes and
//     scales of quant_row_wave);
//   block 4 mt: sort_small_fast with its outputs in memory (off, perm,
//     tiles, ntiles), which the down launch and the combine read;
//   blocks 4 mt + 1 ..: the token codes Xq and scales sx, one row a wave.
// Every block ranks the same ids the same way, so the tiles the gate/up
// blocks take are the tiles the down launch reads.
struct GuSort {
    const float *X;
    const int32_t *ids;
    int8_t *Xq;
    float *sx;
    int32_t *off, *perm, *tiles, *ntiles;
    int T, Tk, E, mt;
};
struct TileSortLds {
    int wcnt[SORTF_TK / 64][SORTF_E];  // pairs of expert x in wave w
    int4 td;       // {expert, first sorted row, rows, first rank within the expert}
    int nt;        // tiles in the list
    int rows[16];  // the tile's pairs, in sorted order
};
union GuSortLds {
    TileSortLds tile;
    SortFastLds fast;
};

// Tile `tile` of the R-row tile list that sort_small_fast builds (cap = Tk,
// so nothing is dropped) for pair t's expert e (-1 for none), into sm.td,
// sm.nt and sm.rows: the same ballot ranks, wave counts and expert scan,
// with only the tile's own entries kept. Ends with a block barrier.
static __device__ void tile_of_sort(int e, int Tk, int E, int R, int tile, TileSortLds &sm) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int NW = (Tk + 63) >> 6;
    int *flat = &sm.wcnt[0][0];
    for (int i = t; i < NW * SORTF_E; i += blockDim.x) flat[i] = 0;
    if (t == 0) {
        sm.td = make_int4(0, 0, 0, 0);
        sm.nt = 0;
    }
    __syncthreads();
    int r = 0;  // stable rank: earlier pairs with the same expert
    if (wave < NW) {
        uint64_t m = __ballot(e >= 0);
        for (int b = 0; (1 << b) < E; b++) {
            const int bit = (e >> b) & 1;
            const uint64_t bb = __ballot(bit);
            m &= bit ? bb : ~bb;
        }
        r = __popcll(m & ((1ull << lane) - 1ull));
        if (e >= 0 && r == 0) sm.wcnt[wave][e] = __popcll(m);
    }
    __syncthreads();
    if (e >= 0)
        for (int w = 0; w < wave; w++) r += sm.wcnt[w][e];
    if (wave == 0) {
        // lane l: experts l*EPL .. l*EPL + EPL - 1 (EPL <= 16; x stays below
        // SORTF_E, and experts past E count zero)
        const int EPL = (E + 63) >> 6, x0 = lane * EPL;
        int ks = 0, ts = 0;
        for (int u = 0; u < EPL; u++) {
            const int x = x0 + u;
            int c = 0;
#pragma unroll
            for (int w = 0; w < SORTF_TK / 64; w++) {
                const int v = sm.wcnt[w][x];
                c += w < NW ? v : 0;
            }
            c = x < E ? c : 0;
            ks += c;
            ts += (c + R - 1) / R;
        }
        const int kin = wave_incl_scan_i(ks, lane), tin = wave_incl_scan_i(ts, lane);
        int kbase = kin - ks, tbase = tin - ts;
        if (tile >= tbase && tile < tin) {  // one lane: its experts hold the tile
            for (int u = 0; u < EPL; u++) {
                const int x = x0 + u;
                int c = 0;
#pragma unroll
                for (int w = 0; w < SORTF_TK / 64; w++) {
                    const int v = sm.wcnt[w][x];
                    c += w < NW ? v : 0;
                }
                c = x < E ? c : 0;
                const int nt = (c + R - 1) / R;
                if (tile < tbase + nt) {
                    const int j = tile - tbase;
                    sm.td = make_int4(x, kbase + j * R, min(R, c - j * R), j * R);
                    break;
                }
                kbase += c;
                tbase += nt;
            }
        }
        if (lane == 63) sm.nt = tin;
    }
    __syncthreads();
    const int4 td = sm.td;
    if (e >= 0 && e == td.x && r >= td.w && r < td.w + td.z) sm.rows[r - td.w] = t;
    __syncthreads();
}

template <int G1, bool SORT>
__global__ __launch_bounds__(64 * RA_WAVES) void k_routed_gu16(
    const int8_t *__restrict__ Xq, const float *__restrict__ sx,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, int topk, const uint8_t *__restrict__ guP,
    const uint16_t *__restrict__ guS, int64_t gu_pstride, int64_t gu_sstride,
    float *__restrict__ S, uint32_t *err, GuSort gs) {
    constexpr int N = 64 * G1;
    constexpr int ASTR = N + 16;
    constexpr int HQ = RF_H / 4;  // hidden channels per quarter (4 h-blocks)
    constexpr int VSTR = HQ + 4;  // LDS row stride of the scaled gate/up values (floats)
    static_assert(N % 256 == 0 && N <= 1024, "n = 256, 512, 768 or 1024");
    static_assert(RA_WAVES == 2 * (RF_H / 16) / 4, "a wave per gate or up panel of a quarter");
    __shared__ __attribute__((aligned(16))) int8_t As[16 * ASTR];
    __shared__ __attribute__((aligned(16))) uint16_t gus[RA_WAVES][G1 * 16];
    __shared__ __attribute__((aligned(16))) float gb[16 * VSTR];
    __shared__ __attribute__((aligned(16))) float ub[16 * VSTR];
    __shared__ float rsa[16];
    __shared__ double exp_tab[64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.x >> 2, quarter = blockIdx.x & 3;
    int4 td;  // {expert, first sorted row, rows}
    int src[2];  // the wave's two A rows (token indices)
    if constexpr (SORT) {
        __shared__ __attribute__((aligned(16))) GuSortLds sl;
        if ((int)blockIdx.x >= 4 * gs.mt) {
            if ((int)blockIdx.x == 4 * gs.mt) {  // the sort, into memory
                const int t = threadIdx.x;
                int pe = -1;
                if (t < gs.Tk) {
                    pe = gs.ids[t];
                    if (pe < 0 || pe >= gs.E) {
                        raise_err(err, EF_BAD_ID);
                        pe = -1;
                    }
                }
                sort_small_fast(pe, gs.Tk, gs.E, (int64_t)gs.Tk, 16, gs.off, NULL, gs.perm, NULL,
                                NULL, gs.tiles, gs.ntiles, sl.fast);
            } else {  // token codes, one row a wave
                const int64_t r = (int64_t)((int)blockIdx.x - 4 * gs.mt - 1) * RA_WAVES + wave;
                if (r < gs.T) quant_row_wave(gs.X, r, N, gs.Xq, N, gs.sx, err, lane);
            }
            return;
        }
        int pe = -1;
        if ((int)threadIdx.x < gs.Tk) {
            pe = gs.ids[threadIdx.x];
            if (pe < 0 || pe >= gs.E) pe = -1;  // reported by the sort block
        }
        tile_of_sort(pe, gs.Tk, gs.E, 16, tile, sl.tile);
        if (tile >= sl.tile.nt) return;
        td = sl.tile.td;
        if (td.z <= 0) return;
#pragma unroll
        for (int j = 0; j < 2; j++) src[j] = sl.tile.rows[min(2 * wave + j, td.z - 1)] / topk;
    } else {
        td = tiles[tile];  // the grid stays in bounds
        if (tile >= *ntiles) return;
        if (td.z <= 0) return;
        // scalar loads of the permutation first
#pragma unroll
        for (int j = 0; j < 2; j++) src[j] = perm[td.y + min(2 * wave + j, td.z - 1)] / topk;
    }
    const double tabv = exp_tab_load(lane);
    const int e = td.x, pos0 = td.y, nrows = td.z;
    const int hl = wave >> 1;             // h-block within the quarter
    const int hb = 4 * quarter + hl;      // h-block within the expert
    const int pan = 2 * hb + (wave & 1);  // gate panel (even wave) or up panel (odd wave)
    // 1. the panel's fp16 scales (G1 * 32 bytes)
    const uint8_t *gsb =
        (const uint8_t *)(guS + (int64_t)e * gu_sstride + (int64_t)pan * G1 * 16);
    constexpr int SC16 = G1 * 32 / 16;  // 16-byte pieces
    uint4 gs4 = {0, 0, 0, 0};
    if (lane < SC16) gs4 = *(const uint4 *)(gsb + lane * 16);
    // 2. raw panel groups, first half
    const uint8_t *gw = guP + (int64_t)e * gu_pstride + (int64_t)pan * G1 * 256;
    constexpr int GA = G1 / 2;
    uint32_t rw[G1];
#pragma unroll
    for (int g = 0; g < GA; g++) rw[g] = *(const uint32_t *)(gw + g * 256 + lane * 4);
    asm volatile("" ::: "memory");
    // 3. the A rows and their token scales (with SORT the fp32 rows, G1/4
    //    float4 a lane each, quantised below)
    constexpr int XV = SORT ? G1 / 4 : 1;
    uint4 a4[2];
    float4 xv[2][XV];
    float sxv = 0.0f;
    if constexpr (SORT) {
        // only the tile's real rows (a decode tile holds one or two): the
        // padding rows' codes are zero and their outputs are never stored
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < XV; i++)
                xv[j][i] = 2 * wave + j < nrows
                               ? *(const float4 *)(gs.X + (int64_t)src[j] * N + (lane + 64 * i) * 4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            a4[j] = (uint4){0, 0, 0, 0};
            if (lane < N / 16) a4[j] = *(const uint4 *)(Xq + (int64_t)src[j] * N + lane * 16);
        }
        if (lane == 0) sxv = sx[src[0]];
        if (lane == 1) sxv = sx[src[1]];
    }
    asm volatile("" ::: "memory");
    // 4. the other groups
#pragma unroll
    for (int g = GA; g < G1; g++) {
        rw[g] = *(const uint32_t *)(gw + g * 256 + lane * 4);
        asm volatile("" ::: "memory");
    }
    if (lane < SC16) *(uint4 *)((char *)gus[wave] + lane * 16) = gs4;
    if constexpr (SORT) {
        // quant_row_wave's codes and scale for each row (a row that is not
        // finite or out of range gets zero codes here; the row's quantiser
        // block reports it)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            uint32_t mu = 0;
#pragma unroll
            for (int i = 0; i < XV; i++) {
                mu = max(mu, max(abs_bits(xv[j][i].x), abs_bits(xv[j][i].y)));
                mu = max(mu, max(abs_bits(xv[j][i].z), abs_bits(xv[j][i].w)));
            }
            mu = wave_max_u(mu);
            const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
            const bool good = mu < 0x7f800000u && qp.ok;
            const float inv = quant_inv_f(qp.scale_d);
#pragma unroll
            for (int i = 0; i < XV; i++) {
                const float4 u = xv[j][i];
                bool f = false;
                uint32_t b0 = (uint8_t)quant_code_try(u.x, inv, f);
                uint32_t b1 = (uint8_t)quant_code_try(u.y, inv, f);
                uint32_t b2 = (uint8_t)quant_code_try(u.z, inv, f);
                uint32_t b3 = (uint8_t)quant_code_try(u.w, inv, f);
                if (f && good) {  // rare: the exact quotients
                    b0 = (uint8_t)quant_code_call(u.x, qp.scale_d);
                    b1 = (uint8_t)quant_code_call(u.y, qp.scale_d);
                    b2 = (uint8_t)quant_code_call(u.z, qp.scale_d);
                    b3 = (uint8_t)quant_code_call(u.w, qp.scale_d);
                }
                const uint32_t wd = good ? b0 | (b1 << 8) | (b2 << 16) | (b3 << 24) : 0u;
                *(uint32_t *)(As + (2 * wave + j) * ASTR + (lane + 64 * i) * 4) = wd;
            }
            if (lane == j) sxv = good ? qp.scale_f : 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++)
            if (lane < N / 16) *(uint4 *)(As + (2 * wave + j) * ASTR + lane * 16) = a4[j];
    }
    if (lane < 2) rsa[2 * wave + lane] = sxv;
    lds_barrier();
    // ---- the panel: rows 4*(lane/16)+i, channel 16*pan + lane%16 ----
    const int r = lane & 15, kc = lane >> 4, lc = lane & 15, lr = (lane >> 4) * 4;
    float T[4] = {0.f, 0.f, 0.f, 0.f};
    v4i an = *(const v4i *)(As + r * ASTR + kc * 16);
#pragma unroll
    for (int g = 0; g < G1; g++) {
        // group g's raw panel, pinned here (see routed_ffn16_block)
        asm volatile("" : "+v"(rw[g])::"memory");
        const v4i a = an;
        if (g + 1 < G1) an = *(const v4i *)(As + r * ASTR + (g + 1) * 64 + kc * 16);
        const float sc = f16_to_f32(gus[wave][g * 16 + lc]);
        const v4i c = mfma16x16x64(a, unpack_int2(rw[g]), (v4i){0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < 4; i++) {
            T[i] = __builtin_fmaf((float)c[i], sc, T[i]);
            asm volatile("" : "+v"(T[i]));
        }
    }
    // the scaled gate (even wave) or up (odd wave) values to LDS
    uint32_t flags = 0;
    float *vb = (wave & 1) ? ub : gb;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = lr + i;
        const float v = T[i] * rsa[row < nrows ? row : 0];
        if (row < nrows && !isfinite(v)) flags |= EF_RANGE;
        vb[row * VSTR + 16 * hl + lc] = v;
    }
    exp_tab_stage(exp_tab, lane, tabv);
    lds_barrier();
    // ---- SwiGLU: 16 rows x HQ hidden over the block, fp32 hidden to S ----
#pragma unroll
    for (int u = 0; u < 16 * HQ / (64 * RA_WAVES); u++) {
        const int x = (wave + RA_WAVES * u) * 64 + lane;  // element of the 16 x HQ tile
        const int row = x / HQ, hc = x % HQ;
        if (row >= nrows) continue;
        float sv;
        if (!silu_mul(gb[row * VSTR + hc], ub[row * VSTR + hc], &sv, exp_tab))
            flags |= EF_NONFINITE_MID;
        S[(int64_t)(pos0 + row) * RF_H + HQ * quarter + hc] = sv;
    }
    if (flags) raise_err(err, flags);
}

template <int G1>
__global__ __launch_bounds__(64 * RF_WAVES) void k_routed_dn16(
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, const float *__restrict__ S,
    const uint8_t *__restrict__ dnP, const uint16_t *__restrict__ dnS, int64_t dn_pstride,
    int64_t dn_sstride, float *__restrict__ Ye, int8_t *__restrict__ Hq,
    float *__restrict__ Hs, uint32_t *err) {
    constexpr int N = 64 * G1;
    constexpr int PQ = N / 64;  // down panels per quarter (one per wave)
    static_assert(PQ <= RF_WAVES, "one panel per wave");
    __shared__ __attribute__((aligned(16))) int8_t hq[16 * RF_QSTR];
    __shared__ float rsq[16];
    __shared__ int rdst[16];
    const int tile = blockIdx.x >> 2, quarter = blockIdx.x & 3;
    const int4 td = tiles[tile];  // the grid stays in bounds
    if (tile >= *ntiles) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = td.x, pos0 = td.y, nrows = td.z;
    if (nrows <= 0) return;
    const int p = PQ * quarter + wave;  // this wave's down panel (wave < PQ)
    const bool has_p = wave < PQ;      // wave-uniform
    // the hidden row first (its quantiser runs before the down), then the
    // panel's raw INT4 groups and scales
    const int row = wave;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < nrows) v = *(const float4 *)(S + (int64_t)(pos0 + row) * RF_H + lane * 4);
    if (row < nrows && lane == 0) rdst[row] = perm[pos0 + row];
    uint2 rd[4];
    uint16_t dsc[4];
    const uint8_t *dw = dnP + (int64_t)e * dn_pstride + (int64_t)p * 4 * 512;
    const uint16_t *dsw = dnS + (int64_t)e * dn_sstride + (int64_t)p * 4 * 16;
    if (has_p) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            rd[g] = *(const uint2 *)(dw + g * 512 + lane * 8);
            dsc[g] = dsw[g * 16 + (lane & 15)];
        }
    }
    // ---- row `wave`: k_quant_rows's scale and codes, into LDS ----
    uint32_t flags = 0;
    if (row < nrows) {
        uint32_t mu = max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w)));
        mu = wave_max_u(mu);
        const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
        if (mu >= 0x7f800000u) {
            flags |= EF_NONFINITE_INPUT;
        } else if (!qp.ok) {
            flags |= EF_RANGE;
        } else {
            const float inv = quant_inv_f(qp.scale_d);
            const uint32_t b0 = (uint8_t)quant_code_fast(v.x, qp.scale_d, inv);
            const uint32_t b1 = (uint8_t)quant_code_fast(v.y, qp.scale_d, inv);
            const uint32_t b2 = (uint8_t)quant_code_fast(v.z, qp.scale_d, inv);
            const uint32_t b3 = (uint8_t)quant_code_fast(v.w, qp.scale_d, inv);
            const uint32_t wd = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            *(uint32_t *)(hq + row * RF_QSTR + lane * 4) = wd;
            if (quarter == 0) {  // one copy of the codes and scale in memory
                *(uint32_t *)(Hq + (int64_t)(pos0 + row) * RF_H + lane * 4) = wd;
                if (lane == 0) Hs[pos0 + row] = qp.scale_f;
            }
            if (lane == 0) rsq[row] = qp.scale_f;
        }
    }
    lds_barrier();
    if (has_p) {
        // ---- down: rows 4*(lane/16)+i, channel 16 p + lane%16 ----
        const int r = lane & 15, kc = lane >> 4, lc = lane & 15, lr = (lane >> 4) * 4;
        float Td[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < RF_H / 64; g++) {
            const v4i a = *(const v4i *)(hq + r * RF_QSTR + g * 64 + kc * 16);
            const v4i c = mfma16x16x64(a, unpack_int4(rd[g].x, rd[g].y), (v4i){0, 0, 0, 0});
            const float sd = f16_to_f32(dsc[g]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                Td[i] = __builtin_fmaf((float)c[i], sd, Td[i]);
                asm volatile("" : "+v"(Td[i]));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = lr + i;
            if (rr >= nrows) continue;
            const float f = Td[i] * rsq[rr];
            if (!isfinite(f)) flags |= EF_RANGE;
            Ye[(int64_t)rdst[rr] * N + 16 * p + lc] = f;
        }
    }
    if (flags) raise_err(err, flags);
}

extern "C" int jtk_routed_ffn16(const int8_t *Xq, const float *sx, const int32_t *perm,
                                const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                                int topk, const uint8_t *guP, const uint16_t *guS,
                                int64_t gu_pstride, int64_t gu_sstride, const uint8_t *dnP,
                                const uint16_t *dnS, int64_t dn_pstride, int64_t dn_sstride, int n,
                                int h, float *Ye, int8_t *Hq, float *Hs, float *S, uint32_t *err,
                                hipStream_t s) {
    if (max_tiles <= 0) return 0;
    if (h != RF_H) return (int)hipErrorInvalidValue;
    if (max_tiles > (1 << 29)) return (int)hipErrorInvalidValue;
    const int4 *t4 = (const int4 *)tiles;
    if (S) {  // four CUs per tile, two launches (S: the fp32 hidden rows)
#define RS_LAUNCH(G)                                                                          \
    hipLaunchKernelGGL((k_routed_gu16<G, false>), dim3((unsigned)(4 * max_tiles)),           \
                       dim3(64 * RA_WAVES), 0, s, Xq, sx, perm, t4, ntiles, topk, guP, guS,     \
                       gu_pstride, gu_sstride, S, err, GuSort{});                              \
    hipLaunchKernelGGL(k_routed_dn16<G>, dim3((unsigned)(4 * max_tiles)), dim3(64 * RF_WAVES), 0, \
                       s, perm, t4, ntiles, S, dnP, dnS, dn_pstride, dn_sstride, Ye, Hq, Hs, err)
        switch (n) {
        case 256: RS_LAUNCH(4); break;
        case 512: RS_LAUNCH(8); break;
        case 768: RS_LAUNCH(12); break;
        case 1024: RS_LAUNCH(16); break;
        default: return (int)hipErrorInvalidValue;
        }
#undef RS_LAUNCH
        return (int)hipGetLastError();
    }
#define RF_LAUNCH(G)                                                                            \
    hipLaunchKernelGGL(k_routed_ffn16<G>, dim3((unsigned)max_tiles), dim3(64 * RF_WAVES), 0, s, Xq, sx, \
                       perm, t4, ntiles, topk, guP, guS, gu_pstride, gu_sstride, dnP, dnS,      \
                       dn_pstride, dn_sstride, Ye, Hq, Hs, err)
    switch (n) {
    case 256: RF_LAUNCH(4); break;
    case 512: RF_LAUNCH(8); break;
    case 768: RF_LAUNCH(12); break;
    case 1024: RF_LAUNCH(16); break;
    default: return (int)hipErrorInvalidValue;
    }
#undef RF_LAUNCH
    return (int)hipGetLastError();
}

// The caller-routed decode's routed FFN from the caller's ids: the token
// codes, the pair sort and the gate/up in one launch (k_routed_gu16 with
// SORT), the down in a second; the outputs are those of
// jtk_quant_sort_small (cap = Tk, R = 16, no drop flags) followed by
// jtk_routed_ffn16 with S. Needs Tk <= SORTF_TK, E <= SORTF_E, h = 256,
// n in {256, 512, 768, 1024} and a 16-byte aligned X; anything else returns
// hipErrorInvalidValue before launching.
extern "C" int jtk_routed_ffn16_sort(const float *X, int T, int8_t *Xq, float *sx,
                                     const int32_t *ids, int Tk, int E, int32_t *off,
                                     int32_t *perm, int32_t *tiles, int32_t *ntiles, int topk,
                                     const uint8_t *guP, const uint16_t *guS,
                                     int64_t gu_pstride, int64_t gu_sstride,
                                     const uint8_t *dnP, const uint16_t *dnS,
                                     int64_t dn_pstride, int64_t dn_sstride, int n, int h,
                                     float *Ye, int8_t *Hq, float *Hs, float *S, uint32_t *err,
                                     hipStream_t s) {
    if (T <= 0 || Tk <= 0 || Tk > SORTF_TK || E <= 0 || E > SORTF_E || topk <= 0 ||
        Tk != T * topk || h != RF_H || ((uintptr_t)X & 15) != 0 || !S)
        return (int)hipErrorInvalidValue;
    // tiles: at most Tk / 16 + the experts that hold a pair
    const int mt = Tk / 16 + (E < Tk ? E : Tk);
    GuSort gs{X, ids, Xq, sx, off, perm, tiles, ntiles, T, Tk, E, mt};
    const dim3 grid((unsigned)(4 * mt + 1 + (T + RA_WAVES - 1) / RA_WAVES));
    const int4 *t4 = (const int4 *)tiles;
#define RSS_LAUNCH(G)                                                                         \
    hipLaunchKernelGGL((k_routed_gu16<G, true>), grid, dim3(64 * RA_WAVES), 0, s, nullptr,     \
                       nullptr, nullptr, nullptr, nullptr, topk, guP, guS, gu_pstride,         \
                       gu_sstride, S, err, gs);                                                \
    hipLaunchKernelGGL(k_routed_dn16<G>, dim3((unsigned)(4 * mt)), dim3(64 * RF_WAVES), 0, s, \
                       perm, t4, ntiles, S, dnP, dnS, dn_pstride, dn_sstride, Ye, Hq, Hs, err)
    switch (n) {
    case 256: RSS_LAUNCH(4); break;
    case 512: RSS_LAUNCH(8); break;
    case 768: RSS_LAUNCH(12); break;
    case 1024: RSS_LAUNCH(16); break;
    default: return (int)hipErrorInvalidValue;
    }
#undef RSS_LAUNCH
    return (int)hipGetLastError();
}

// ===================== decode launches with the shared experts beside =====================
// At decode every launch costs a 2-3 us floor and the routing kernels keep
// a few CUs busy, so the shared experts' skinny GEMM blocks ride in the
// launches of the routed path instead of launches of their own (same
// blocks, same arithmetic, so the same outputs):
//   launch 1: top-k of the T <= 16 rows (blocks 0 .. ntb-1, waves 0-3, one
//             row each), then the pair sort and tile list in whichever of
//             those blocks finishes last, + the shared experts' concatenated
//             gate/up panels with the SwiGLU (blocks ntb ..; they need only
//             the token codes);
//   launch 2: the routed FFN of the 16-row tiles (blocks 0 .. max_tiles-1)
//             + the shared experts' down projections (blocks max_tiles ..,
//             expert j / nbx, channel group j % nbx), which read the hidden
//             rows launch 1 wrote.
// The last top-k block is found with a device counter: each top-k block
// releases its rows' ids with an agent-scope fence and counts itself in;
// the block that counts ntb acquires every block's ids, sorts them (as
// k_sort_small) and returns the counter to zero for the next launch.
static_assert(RF_WAVES == SK_WAVES, "one block size for both kinds of block");
// sort_small_core and its block scan assume a block of exactly SORT_SMALL
// threads (they read every wave's partial sum and clear counts with that stride)
static_assert(64 * SK_WAVES == SORT_SMALL, "the merged sort needs SORT_SMALL threads");

template <int EPL>
__global__ __launch_bounds__(64 * SK_WAVES) void k_decode_route_shared_gu(
    const float *__restrict__ logits, int T, int E, int k, int32_t *__restrict__ ids,
    float *__restrict__ w, int ntb, int R, int32_t *__restrict__ off,
    int32_t *__restrict__ perm, int32_t *__restrict__ tiles, int32_t *__restrict__ ntiles,
    uint32_t *__restrict__ done, const int8_t *__restrict__ Xq, int ldx,
    const float *__restrict__ sx, const int8_t *__restrict__ Wp, const float *__restrict__ sB,
    int N, int Kp, float *__restrict__ C, int ldc, SkBatch bt, uint32_t *err) {
    if ((int)blockIdx.x >= ntb) {
        w8a8_skinny_block<EPI_SWIGLU, 2, 0>((int)blockIdx.x - ntb, 0, Xq, ldx, sx, Wp, sB, T, N,
                                            Kp, Kp, C, ldc, err, bt);
        return;
    }
    __shared__ __attribute__((aligned(16))) SortLds sm;
    __shared__ int is_last;
    const int wave = threadIdx.x >> 6, row = blockIdx.x * 4 + wave;
    if (wave < 4 && row < T)
        (void)topk_wave_reg<EPL>(logits + (int64_t)row * E, E, k, threadIdx.x & 63, row, ids,
                                 NULL, w, err);
    __syncthreads();  // this block's rows are written
    if (threadIdx.x == 0) {
        __threadfence();  // ... and visible to the other blocks
        const bool last = atomicAdd(done, 1u) == (uint32_t)ntb - 1;
        // every block's rows are visible from here on, and through the
        // barrier below to the whole block (one fence: each costs an L2
        // write-back and invalidate)
        if (last) __threadfence();
        is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    const int Tk = T * k, t = threadIdx.x;
    int e = -1;
    if (t < Tk) {
        e = ids[t];
        if (e < 0 || e >= E) {
            raise_err(err, EF_BAD_ID);
            e = -1;
        }
    }
    if (Tk <= SORTF_TK && E <= SORTF_E)  // block-uniform
        sort_small_fast(e, Tk, E, (int64_t)Tk, R, off, NULL, perm, NULL, NULL, tiles, ntiles,
                        sm.fast);
    else
        sort_small_core(e, Tk, E, (int64_t)Tk, R, off, NULL, perm, NULL, NULL, tiles, ntiles,
                        sm.small);
    if (t == 0) *done = 0;  // for the next launch (the counter is this block's alone now)
}

extern "C" int jtk_decode_route_shared_gu(const float *logits, int T, int E, int k,
                                          int32_t *ids, float *w, int R, int32_t *off,
                                          int32_t *perm, int32_t *tiles, int32_t *ntiles,
                                          uint32_t *done, const int8_t *Xq, int ldx,
                                          const float *sx, const int8_t *Wp, const float *sB,
                                          int N, int Kp, float *C, int ldc, int hpl,
                                          int64_t plane, uint32_t *err, hipStream_t s) {
    if (T <= 0) return 0;
    if (T > 16 || k <= 0 || k > 64 || T * k > SORT_SMALL || topk_epl(E) == 0 || R <= 0 ||
        !done || N <= 0 || N % 32 || hpl <= 0 || hpl % 16 || (N / 2) % hpl || Kp <= 0 || Kp % 64)
        return (int)hipErrorInvalidValue;
    SkBatch bt{};
    bt.hpl = hpl;
    bt.plane = plane;
    const int ntb = (T + 3) / 4;
    const dim3 grid((unsigned)(ntb + N / 32));
    switch (topk_epl(E)) {
#define TG_LAUNCH(P)                                                                            \
    case P:                                                                                     \
        hipLaunchKernelGGL(k_decode_route_shared_gu<P>, grid, dim3(64 * SK_WAVES), 0, s, logits, \
                           T, E, k, ids, w, ntb, R, off, perm, tiles, ntiles, done, Xq, ldx, sx, \
                           Wp, sB, N, Kp, C, ldc, bt, err);                                     \
        break;
        TG_LAUNCH(1)
        TG_LAUNCH(2)
        TG_LAUNCH(4)
        TG_LAUNCH(8)
        TG_LAUNCH(16)
#undef TG_LAUNCH
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

template <int G1, int QV>
__global__ __launch_bounds__(64 * SK_WAVES) void k_decode_ffn16_shared_down(
    const int8_t *__restrict__ Xq, const float *__restrict__ sx,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, int max_tiles, int topk,
    const uint8_t *__restrict__ guP, const uint16_t *__restrict__ guS, int64_t gu_pstride,
    int64_t gu_sstride, const uint8_t *__restrict__ dnP, const uint16_t *__restrict__ dnS,
    int64_t dn_pstride, int64_t dn_sstride, float *__restrict__ Ye, int8_t *__restrict__ Hq,
    float *__restrict__ Hs, const float *__restrict__ H, int ldh, int K, int T,
    const int8_t *__restrict__ Wd, const float *__restrict__ sBd, int N, int Kp,
    float *__restrict__ Ys, int ldy, SkBatch bt, int nbx, uint32_t *err) {
    if ((int)blockIdx.x < max_tiles) {
        routed_ffn16_block<G1>((int)blockIdx.x, Xq, sx, perm, tiles, ntiles, topk, guP, guS,
                               gu_pstride, gu_sstride, dnP, dnS, dn_pstride, dn_sstride, Ye, Hq,
                               Hs, err);
        return;
    }
    const int j = (int)blockIdx.x - max_tiles;
    w8a8_skinny_block<EPI_PLAIN, 1, QV>(j % nbx, j / nbx, H, ldh, NULL, Wd, sBd, T, N, Kp, K, Ys,
                                        ldy, err, bt);
}

template <int G1, int QV>
static hipError_t launch_ffn16_down(dim3 grid, size_t lds, hipStream_t s, const int8_t *Xq,
                                    const float *sx, const int32_t *perm, const int4 *tiles,
                                    const int32_t *ntiles, int max_tiles, int topk,
                                    const uint8_t *guP, const uint16_t *guS, int64_t gu_pstride,
                                    int64_t gu_sstride, const uint8_t *dnP, const uint16_t *dnS,
                                    int64_t dn_pstride, int64_t dn_sstride, float *Ye, int8_t *Hq,
                                    float *Hs, const float *H, int ldh, int K, int T,
                                    const int8_t *Wd, const float *sBd, int N, int Kp, float *Ys,
                                    int ldy, SkBatch bt, int nbx, uint32_t *err) {
    auto kern = k_decode_ffn16_shared_down<G1, QV>;
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                16 * (256 * DS_QV_MAX + 16));
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(kern, grid, dim3(64 * SK_WAVES), lds, s, Xq, sx, perm, tiles, ntiles,
                       max_tiles, topk, guP, guS, gu_pstride, gu_sstride, dnP, dnS, dn_pstride,
                       dn_sstride, Ye, Hq, Hs, H, ldh, K, T, Wd, sBd, N, Kp, Ys, ldy, bt, nbx, err);
    return hipGetLastError();
}

extern "C" int jtk_decode_ffn16_shared_down(
    const int8_t *Xq, const float *sx, const int32_t *perm, const int32_t *tiles,
    const int32_t *ntiles, int max_tiles, int topk, const uint8_t *guP, const uint16_t *guS,
    int64_t gu_pstride, int64_t gu_sstride, const uint8_t *dnP, const uint16_t *dnS,
    int64_t dn_pstride, int64_t dn_sstride, int n, int h, float *Ye, int8_t *Hq, float *Hs,
    const float *H, int ldh, int K, int64_t sH, int T, const int8_t *Wd, int64_t sW,
    const float *sBd, int ssB, int Np, int Kp, float *Ys, int ldy, int64_t sY, int nb,
    uint32_t *err, hipStream_t s) {
    if (max_tiles <= 0 || T <= 0 || nb <= 0) return (int)hipErrorInvalidValue;
    if (h != RF_H || T > 16 || K <= 0 || K > Kp || Kp % 64 || K % 4 || Kp > 256 * DS_QV_MAX ||
        ldh % 4 || sH % 4 || ((uintptr_t)H & 15) || Np % 16 || Np < n || nb > 65535 ||
        (int64_t)max_tiles + (int64_t)(Np / 16) * nb > 0x7fffffff)
        return (int)hipErrorInvalidValue;
    SkBatch bt{};
    bt.bsA = sH * (int64_t)sizeof(float);
    bt.bsW = sW;
    bt.bsB = ssB;
    bt.bsC = sY;
    const int nbx = Np / 16;
    const dim3 grid((unsigned)(max_tiles + nbx * nb));
    const size_t lds = (size_t)16 * (Kp + 16);
    const int4 *t4 = (const int4 *)tiles;
    const int qv = (K + 255) / 256 <= 4 ? 4 : (K + 255) / 256 <= 8 ? 8 : 12;
#define DS_LAUNCH(G, Q)                                                                         \
    launch_ffn16_down<G, Q>(grid, lds, s, Xq, sx, perm, t4, ntiles, max_tiles, topk, guP, guS,  \
                            gu_pstride, gu_sstride, dnP, dnS, dn_pstride, dn_sstride, Ye, Hq,   \
                            Hs, H, ldh, K, T, Wd, sBd, n, Kp, Ys, ldy, bt, nbx, err)
#define DS_QV(G)                                                                                \
    (qv == 4 ? DS_LAUNCH(G, 4) : qv == 8 ? DS_LAUNCH(G, 8) : DS_LAUNCH(G, 12))
    hipError_t e;
    switch (n) {
    case 256: e = DS_QV(4); break;
    case 512: e = DS_QV(8); break;
    case 768: e = DS_QV(12); break;
    case 1024: e = DS_QV(16); break;
    default: return (int)hipErrorInvalidValue;
    }
#undef DS_QV
#undef DS_LAUNCH
    return (int)e;
}

extern "C" int jtk_lowbit_grouped(int bits, const int8_t *A, int lda, const float *sA,
                                  const int32_t *perm, const int32_t *off, int topk,
                                  const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                                  int rows_per_tile, const uint8_t *Wp, const uint16_t *Ws,
                                  int64_t wp_stride, int64_t ws_stride, int N, int K, float *out,
                                  int ldo, uint32_t *err, hipStream_t s) {
    if (max_tiles <= 0) return 0;
    if (max_tiles > 65535) return (int)hipErrorInvalidValue;  // tiles run on grid y
    hipError_t e;
    if (rows_per_tile == 16) {
        const int G = K / 64;
        if (G > LS_GMAX || N % (16 * LS_PANELS)) return (int)hipErrorInvalidValue;
        dim3 grid((unsigned)(N / (16 * LS_PANELS)), (unsigned)max_tiles);
        const int4 *t4 = (const int4 *)tiles;
        if (bits == 2)
            e = launch_lowbit_skinny<2, EPI_SWIGLU>(grid, G, s, A, lda, sA, perm, t4, ntiles, topk,
                                                    Wp, Ws, wp_stride, ws_stride, N, K, out, ldo,
                                                    err);
        else
            e = launch_lowbit_skinny<4, EPI_SCATTER>(grid, G, s, A, lda, sA, perm, t4, ntiles,
                                                     topk, Wp, Ws, wp_stride, ws_stride, N, K,
                                                     out, ldo, err);
        return (int)e;
    }
    if (rows_per_tile != 64) return (int)hipErrorInvalidValue;
    if (bits == 4 && (K == 256 || K == 512) && N % 256 == 0) {
        // weights in registers: 4 panels per wave (measured in the overlapped
        // layer at K = 256: 4 panels 0.3525 ms against 2 panels 0.3577; the
        // fewer, longer blocks leave more room to the shared experts)
        const int4 *t4 = (const int4 *)tiles;
        const int ncb = N / 256;
        // 8 XCD runs of ceil(max_tiles / 8) tiles x ncb channel blocks
        const unsigned grid = 8u * (unsigned)(((max_tiles + 7) / 8) * ncb);
        if (K == 256)
            hipLaunchKernelGGL((k_lowbit_down_rr<4, 4>), dim3(grid), dim3(256), 0, s, A, lda, sA,
                               perm, t4, ntiles, Wp, Ws, wp_stride, ws_stride, out, ldo, err,
                               ncb);
        else
            hipLaunchKernelGGL((k_lowbit_down_rr<8, 4>), dim3(grid), dim3(256), 0, s, A, lda, sA,
                               perm, t4, ntiles, Wp, Ws, wp_stride, ws_stride, out, ldo, err,
                               ncb);
        return (int)hipGetLastError();
    }
    if (bits == 4 && K <= LBR_KMAX && N % 128 == 0) {
        // channel groups per block: as many as keep about 1536 blocks
        const int ncg = N / 128;
        int ny = (1536 + max_tiles - 1) / max_tiles;
        if (ny > ncg) ny = ncg;
        while (ncg % ny) ny++;
        dim3 grid((unsigned)ny, (unsigned)max_tiles);
        if (bits == 2)
            e = launch_lowbit_res<2, EPI_SWIGLU, LB_STAGES>(grid, ncg / ny, s, A, lda, sA, perm,
                                                            topk, tiles, ntiles, Wp, Ws, wp_stride,
                                                            ws_stride, N, K, out, ldo, err);
        else
            e = launch_lowbit_res<4, EPI_SCATTER, LB_STAGES>(grid, ncg / ny, s, A, lda, sA, perm,
                                                             topk, tiles, ntiles, Wp, Ws,
                                                             wp_stride, ws_stride, N, K, out, ldo,
                                                             err);
        return (int)e;
    }
    dim3 grid((unsigned)(N / 128), (unsigned)max_tiles);
    if (bits == 2)
        e = launch_lowbit<2, EPI_SWIGLU, LB_STAGES>(grid, s, A, lda, sA, perm, off, topk, tiles,
                                                    ntiles, Wp, Ws, wp_stride, ws_stride, N, K,
                                                    out, ldo, err);
    else
        e = launch_lowbit<4, EPI_SCATTER, LB_STAGES>(grid, s, A, lda, sA, perm, off, topk,
                                                     tiles, ntiles, Wp, Ws, wp_stride, ws_stride,
                                                     N, K, out, ldo, err);
    return (int)e;
}

// Load this file's code object now: the runtime otherwise loads it, and
// allocates device memory for it, at the first launch of one of its kernels.
extern "C" int jtk_preload_gemm_i8(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_w8a8_skinny<EPI_PLAIN, 1, 0>));
}
