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
#include "gemm_w8a8.h"
#include "jt_launch.h"

// Output fragment layout of v_mfma_i32_16x16x64_i8 (4 int32 per lane):
// element r of lane l is row 4*(l/16)+r, column l%16 of the 16x16 tile.

// ===================== decode GEMV (M <= 16) =====================
// One block per pair of panels (32 packed channels); the 4 waves split the K
// blocks round-robin. Lane l owns channel l%16 and k-chunk l/16 of every
// 64-K block, multiplies its 16 weight bytes with the same 16 activation
// bytes of each row (v_dot4_i32_i8), then the partial sums are reduced over
// the 4 k-chunks (lane shuffles) and the 4 waves (LDS) -- integer sums, so
// the result equals the MFMA kernel's bit for bit.
template <int EPI, int MR>
__global__ __launch_bounds__(256) void k_w8a8_gemv(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int8_t *__restrict__ Wp, const float *__restrict__ sB, int M, int N, int Kp,
    float *__restrict__ C, int ldc, uint32_t *err) {
    __shared__ int red[4][MR][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KB = Kp / 64;
    const int p0 = blockIdx.x * 2;  // first of the two panels
    const int kc = lane >> 4;
    int acc[2][MR];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[q][m] = 0;
    const int8_t *w0 = Wp + (int64_t)p0 * KB * 1024 + lane * 16;
    const int8_t *w1 = w0 + (int64_t)KB * 1024;
    for (int kb = wave; kb < KB; kb += 4) {
        const v4i b0 = *(const v4i *)(w0 + (int64_t)kb * 1024);
        const v4i b1 = *(const v4i *)(w1 + (int64_t)kb * 1024);
        const int koff = kb * 64 + kc * 16;
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (m < M) {
                const v4i a = *(const v4i *)(A + (int64_t)m * lda + koff);
                int t0 = acc[0][m], t1 = acc[1][m];
                t0 = __builtin_amdgcn_sdot4(a.x, b0.x, t0, false);
                t0 = __builtin_amdgcn_sdot4(a.y, b0.y, t0, false);
                t0 = __builtin_amdgcn_sdot4(a.z, b0.z, t0, false);
                t0 = __builtin_amdgcn_sdot4(a.w, b0.w, t0, false);
                t1 = __builtin_amdgcn_sdot4(a.x, b1.x, t1, false);
                t1 = __builtin_amdgcn_sdot4(a.y, b1.y, t1, false);
                t1 = __builtin_amdgcn_sdot4(a.z, b1.z, t1, false);
                t1 = __builtin_amdgcn_sdot4(a.w, b1.w, t1, false);
                acc[0][m] = t0;
                acc[1][m] = t1;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int m = 0; m < MR; m++) {
            int v = acc[q][m];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane < 16) red[wave][m][q * 16 + lane] = v;
        }
    __syncthreads();
    // 32 channels x MR rows, one (row, channel) per thread. Scales are read
    // before any store (loads and stores share one vmcnt on gfx9).
    constexpr int PT = (MR * 32 + 255) / 256;
    double sa_t[PT], sg_t[PT], su_t[PT];
#pragma unroll
    for (int q = 0; q < PT; q++) {
        const int idx = tid + q * 256;
        const int m = min(idx >> 5, M - 1), c = idx & 31;
        sa_t[q] = (double)sA[m];
        const int cg = min(p0 * 16 + c, N - 1), cu = min(p0 * 16 + c + 16, N - 1);
        sg_t[q] = (double)sB[cg];
        su_t[q] = (double)sB[cu];
    }
    uint32_t bad = 0, badmid = 0;
#pragma unroll
    for (int q = 0; q < PT; q++) {
        const int idx = tid + q * 256;
        if (idx >= MR * 32) continue;
        const int m = idx >> 5, c = idx & 31;
        if (m >= M) continue;
        const int s = red[0][m][c] + red[1][m][c] + red[2][m][c] + red[3][m][c];
        if (EPI == EPI_PLAIN) {
            const int col = p0 * 16 + c;
            if (col >= N) continue;
            const float f = (float)((double)s * (sa_t[q] * sg_t[q]));
            bad |= !isfinite(f);
            C[(int64_t)m * ldc + col] = f;
        } else {
            if (c >= 16) continue;  // gate lanes combine with their up twin
            const int cg = p0 * 16 + c, cu = cg + 16;
            if (cu >= N) continue;
            const int su = red[0][m][c + 16] + red[1][m][c + 16] + red[2][m][c + 16] +
                           red[3][m][c + 16];
            const float g = (float)((double)s * (sa_t[q] * sg_t[q]));
            const float u = (float)((double)su * (sa_t[q] * su_t[q]));
            bad |= (!isfinite(g)) || (!isfinite(u));
            float sv;
            badmid |= !silu_mul(g, u, &sv);
            C[(int64_t)m * ldc + (p0 / 2) * 16 + c] = sv;
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

extern "C" int jtk_w8a8_gemm(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                             const float *sB, int M, int N, int Np, int Kp, float *C,
                             int ldc, int swiglu, uint32_t *err, hipStream_t s) {
    if (M <= 0) return 0;
    if (M <= 16) {
        dim3 grid((unsigned)(Np / 32));
#define GEMV(E, R)                                                                     \
    hipLaunchKernelGGL((k_w8a8_gemv<E, R>), grid, dim3(256), 0, s, A, lda, sA, Wp, sB, M, N, \
                       Kp, C, ldc, err)
        if (swiglu) {
            if (M <= 1) GEMV(EPI_SWIGLU, 1);
            else if (M <= 4) GEMV(EPI_SWIGLU, 4);
            else GEMV(EPI_SWIGLU, 16);
        } else {
            if (M <= 1) GEMV(EPI_PLAIN, 1);
            else if (M <= 4) GEMV(EPI_PLAIN, 4);
            else GEMV(EPI_PLAIN, 16);
        }
#undef GEMV
    } else {
        // Tile choice (measured on MI355X): few 128x128 tiles -> 8 waves per
        // block with an intra-block k-split; otherwise 128 x 256 tiles of
        // 8 waves; SwiGLU pairs need an even number of 16-channel tiles.
        const int mt128 = (M + 127) / 128;
        const bool n256 = (Np % 256) == 0;
        hipError_t e;
        if (swiglu) {
            e = n256 ? launch_w8a8_tile<EPI_SWIGLU, 128, 256, 2, 4, 1, 3, 4>(
                           A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s)
                     : launch_w8a8_tile<EPI_SWIGLU, 128, 128, 2, 2, 2, 2, 4>(
                           A, lda, sA, Wp, sB, M, N, Np, Kp, C, ldc, err, s);
        } else if (!n256 || mt128 * (Np / 128) <= 512) {
            e = launch_w8a8_tile<EPI_PLAIN, 128, 128, 2, 2, 2, 3, 4>(A, lda, sA, Wp, sB, M, N, Np,
                                                                     Kp, C, ldc, err, s);
        } else {
            e = launch_w8a8_tile<EPI_PLAIN, 128, 256, 2, 4, 1, 3, 4>(A, lda, sA, Wp, sB, M, N, Np,
                                                                     Kp, C, ldc, err, s);
        }
        return (int)e;
    }
    return (int)hipGetLastError();
}

// ===================== grouped low-bit GEMM =====================
// Work item = (expert e, 64-row tile of that expert's rows) x 128 packed
// channels. Rows of expert e are the sorted pairs pos = off[e] .. off[e+1]-1.
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
#define LB_STAGES 4
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
    const int tile = blockIdx.x;
    if (tile >= *ntiles) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int packed = tiles[tile];
    const int e = packed >> 16, row0 = (packed & 0xFFFF) * 64;
    const int base = off[e], Me = off[e + 1] - base;
    const int nrows = min(64, Me - row0);
    if (tid < 64) {
        const int r = min(tid, nrows - 1);
        const int pos = base + row0 + r;
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
    const int n0 = blockIdx.y * 128;
    // A: wave w copies panel w (rows 16w..16w+15) of every stage;
    // lane l = kc*16 + r -> row 16w + r, bytes [16kc, 16kc+16) of the group
    const int8_t *a_src = A + (int64_t)rowsrc[wave * 16 + (lane & 15)] * lda + (lane >> 4) * 16;
    // B: wave w copies the panel-groups of panels pb0 + 2w and pb0 + 2w + 1
    const int pb0 = n0 >> 4;
    const uint8_t *wbase = Wp + (int64_t)e * wp_stride;
    const uint8_t *b_src0 = wbase + (int64_t)(pb0 + 2 * wave) * G * PB + lane * 4;
    const uint8_t *b_src1 = b_src0 + (int64_t)G * PB;
    // this wave's two panels (absolute panel index within the expert)
    const int pan0 = pb0 + wave * 2;
    // fp16 group scales of the two panels: lanes 0-7 copy panel pan0's 16
    // values (2 per lane), lanes 8-15 panel pan0+1's; lanes 16-63 repeat them
    // (the 4-byte DMA always writes 64 lanes)
    const int sl = lane & 15;
    const uint8_t *s_src = (const uint8_t *)(Ws + (int64_t)e * ws_stride +
                                             (int64_t)(pan0 + (sl >> 3)) * G * 16) +
                           (sl & 7) * 4;
    auto issue = [&](int g) {
        int8_t *st = smem + (g % NST) * STAGE;
        dma<16>(a_src + (int64_t)g * 64, st + wave * 1024);
#pragma unroll
        for (int d = 0; d < BDMA; d++) {
            dma<4>(b_src0 + (int64_t)g * PB + d * 256, st + 4096 + (2 * wave) * PB + d * 256);
            dma<4>(b_src1 + (int64_t)g * PB + d * 256, st + 4096 + (2 * wave + 1) * PB + d * 256);
        }
        dma<4>(s_src + (int64_t)g * 32, st + SOFF + wave * 256);
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
    static bool attr_set[64];
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

extern "C" int jtk_lowbit_grouped(int bits, const int8_t *A, int lda, const float *sA,
                                  const int32_t *perm, const int32_t *off, int topk,
                                  const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                                  const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                                  int64_t ws_stride, int N, int K, float *out, int ldo,
                                  uint32_t *err, hipStream_t s) {
    if (max_tiles <= 0) return 0;
    dim3 grid((unsigned)max_tiles, (unsigned)(N / 128));
    hipError_t e;
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
