// int8 GEMM kernels for gfx950: W8A8 (per-channel weights, per-row
// activations) and the grouped low-bit routed-expert GEMM.
//
// Arithmetic (identical in every kernel of this file):
//   acc   = sum_k A[m][k] * W[n][k] in int32 (order-free, exact);
//   W8A8  : C = (float)((double)acc * ((double)sA[m] * (double)sB[n]))
//           -- the reference's epilogue, src/w8a8.c:664-676;
//   low-bit: per 64-K group g the int32 partial acc_g is taken out of the
//           MFMA and T += (double)acc_g * (double)f16 scale[n][g] in g order
//           (the product is exact in fp64, so fma and mul+add agree);
//           C = (float)(T * (double)sA[m]).
// The matrix instruction is v_mfma_i32_16x16x64_i8; weights arrive in the
// 16-channel x 64-K panel layout of jt_dev.h so each operand fragment is one
// coalesced 16-byte (int8), 8-byte (INT4) or 4-byte (INT2) load per lane.
#include "jt_dev.h"
#include "jt_launch.h"

// Output fragment layout of v_mfma_i32_16x16x64_i8 (4 int32 per lane):
// element r of lane l is row 4*(l/16)+r, column l%16 of the 16x16 tile.

enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_SCATTER = 2 };

// ===================== dense W8A8 MFMA GEMM =====================
// Block tile 128 x 128, K step 64, 4 waves in a 2 x 2 grid of 64 x 64 wave
// tiles (4 x 4 MFMA tiles each). A [M][lda] row-major int8 (lda >= Kp,
// Kp % 64 == 0, bytes beyond K are zero), W panels padded to Np (multiple of
// 128) channels.
#define GB_M 128
#define GB_N 128

template <int EPI>
__global__ __launch_bounds__(256, 2) void k_w8a8_mfma(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int8_t *__restrict__ Wp, const float *__restrict__ sB, int M, int N, int Kp,
    float *__restrict__ C, int ldc, uint32_t *err) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][GB_M * 64];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][GB_N * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.x * GB_M, n0 = blockIdx.y * GB_N;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int KB = Kp / 64;

    // A tile loader: thread t covers rows t/4 and t/4+64, 16-byte chunk t%4.
    const int a_r = tid >> 2, a_kc = tid & 3;
    int ra0 = m0 + a_r, ra1 = m0 + a_r + 64;
    ra0 = ra0 < M ? ra0 : M - 1;
    ra1 = ra1 < M ? ra1 : M - 1;
    const int8_t *a_src0 = A + (int64_t)ra0 * lda + a_kc * 16;
    const int8_t *a_src1 = A + (int64_t)ra1 * lda + a_kc * 16;
    // LDS position (panel layout): panel = row/16, lane = kc*16 + row%16
    const int a_dst0 = (a_r >> 4) * 1024 + (a_kc * 16 + (a_r & 15)) * 16;
    const int a_dst1 = a_dst0 + 4 * 1024;
    // B tile loader: 8 panels x 1 KiB; thread t copies bytes [16t, 16t+16) and
    // [16t + 4096, ...), i.e. panels t/64 and t/64 + 4.
    const int64_t panel_stride = (int64_t)KB * 1024;
    const int b_p = tid >> 6;
    const int8_t *b_src0 = Wp + (int64_t)(n0 / 16 + b_p) * panel_stride + lane * 16;
    const int8_t *b_src1 = b_src0 + 4 * panel_stride;

    v4i ra, rb, rc, rd;
    ra = *(const v4i *)(a_src0);
    rb = *(const v4i *)(a_src1);
    rc = *(const v4i *)(b_src0);
    rd = *(const v4i *)(b_src1);
    *(v4i *)(&As[0][a_dst0]) = ra;
    *(v4i *)(&As[0][a_dst1]) = rb;
    *(v4i *)(&Bs[0][tid * 16]) = rc;
    *(v4i *)(&Bs[0][tid * 16 + 4096]) = rd;
    __syncthreads();

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    for (int kb = 0; kb < KB; kb++) {
        const int cur = kb & 1;
        const bool more = kb + 1 < KB;
        if (more) {
            const int64_t koff = (int64_t)(kb + 1) * 64;
            ra = *(const v4i *)(a_src0 + koff);
            rb = *(const v4i *)(a_src1 + koff);
            rc = *(const v4i *)(b_src0 + (kb + 1) * 1024);
            rd = *(const v4i *)(b_src1 + (kb + 1) * 1024);
        }
        v4i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            af[i] = *(const v4i *)(&As[cur][((wm >> 4) + i) * 1024 + lane * 16]);
#pragma unroll
        for (int j = 0; j < 4; j++)
            bf[j] = *(const v4i *)(&Bs[cur][((wn >> 4) + j) * 1024 + lane * 16]);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma16x16x64(af[i], bf[j], acc[i][j]);
        if (more) {
            *(v4i *)(&As[cur ^ 1][a_dst0]) = ra;
            *(v4i *)(&As[cur ^ 1][a_dst1]) = rb;
            *(v4i *)(&Bs[cur ^ 1][tid * 16]) = rc;
            *(v4i *)(&Bs[cur ^ 1][tid * 16 + 4096]) = rd;
        }
        __syncthreads();
    }

    // epilogue
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    uint32_t bad = 0;
    if (EPI == EPI_PLAIN) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = n0 + wn + j * 16 + lc;
            if (col >= N) continue;
            const double sb = (double)sB[col];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = m0 + wm + i * 16 + lr + r;
                    if (row >= M) continue;
                    const float f = (float)((double)acc[i][j][r] * ((double)sA[row] * sb));
                    bad |= !isfinite(f);
                    C[(int64_t)row * ldc + col] = f;
                }
        }
        if (bad) raise_err(err, EF_RANGE);
    } else {
        // packed channels: [gate 16][up 16] per 32; tiles j = 0,2 are gate,
        // j = 1,3 the matching up; output column = hidden unit.
        uint32_t badmid = 0;
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const int cg = n0 + wn + (2 * jj) * 16 + lc;  // packed gate channel
            const int cu = cg + 16;
            const int hid = (n0 + wn) / 2 + jj * 16 + lc;
            if (cu >= N) continue;
            const double sbg = (double)sB[cg], sbu = (double)sB[cu];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = m0 + wm + i * 16 + lr + r;
                    if (row >= M) continue;
                    const double sa = (double)sA[row];
                    const float g = (float)((double)acc[i][2 * jj][r] * (sa * sbg));
                    const float u = (float)((double)acc[i][2 * jj + 1][r] * (sa * sbu));
                    bad |= (!isfinite(g)) || (!isfinite(u));
                    float s;
                    badmid |= !silu_mul(g, u, &s);
                    C[(int64_t)row * ldc + hid] = s;
                }
        }
        if (bad) raise_err(err, EF_RANGE);
        if (badmid) raise_err(err, EF_NONFINITE_MID);
    }
}

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
    // 32 channels x MR rows, one (row, channel) per thread
    uint32_t bad = 0, badmid = 0;
    for (int idx = tid; idx < MR * 32; idx += 256) {
        const int m = idx >> 5, c = idx & 31;
        if (m >= M) continue;
        const int s = red[0][m][c] + red[1][m][c] + red[2][m][c] + red[3][m][c];
        if (EPI == EPI_PLAIN) {
            const int col = p0 * 16 + c;
            if (col >= N) continue;
            const float f = (float)((double)s * ((double)sA[m] * (double)sB[col]));
            bad |= !isfinite(f);
            C[(int64_t)m * ldc + col] = f;
        } else {
            if (c >= 16) continue;  // gate lanes combine with their up twin
            const int cg = p0 * 16 + c, cu = cg + 16;
            if (cu >= N) continue;
            const int su = red[0][m][c + 16] + red[1][m][c + 16] + red[2][m][c + 16] +
                           red[3][m][c + 16];
            const double sa = (double)sA[m];
            const float g = (float)((double)s * (sa * (double)sB[cg]));
            const float u = (float)((double)su * (sa * (double)sB[cu]));
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
        dim3 grid((unsigned)((M + GB_M - 1) / GB_M), (unsigned)(Np / GB_N));
        if (swiglu)
            hipLaunchKernelGGL((k_w8a8_mfma<EPI_SWIGLU>), grid, dim3(256), 0, s, A, lda, sA, Wp,
                               sB, M, N, Kp, C, ldc, err);
        else
            hipLaunchKernelGGL((k_w8a8_mfma<EPI_PLAIN>), grid, dim3(256), 0, s, A, lda, sA, Wp,
                               sB, M, N, Kp, C, ldc, err);
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
// Waves split the 128 channels (32 each = 2 panels); all four share the
// 64-row A tile through LDS (double-buffered per 64-K group).
template <int BITS, int EPI>
__global__ __launch_bounds__(256, 2) void k_lowbit_grouped(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int32_t *__restrict__ perm, const int32_t *__restrict__ off, int topk,
    const int32_t *__restrict__ tiles, const int32_t *__restrict__ ntiles,
    const uint8_t *__restrict__ Wp, const uint16_t *__restrict__ Ws, int64_t wp_stride,
    int64_t ws_stride, int N, int K, float *__restrict__ out, int ldo, uint32_t *err) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][64 * 64];
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
    // A loader: thread t -> row t/4, chunk t%4 (one 16-byte load per group)
    const int a_r = tid >> 2, a_kc = tid & 3;
    const int8_t *a_src = A + (int64_t)rowsrc[a_r] * lda + a_kc * 16;
    const int a_dst = (a_r >> 4) * 1024 + (a_kc * 16 + (a_r & 15)) * 16;
    // this wave's two panels
    const int pan0 = (n0 >> 4) + wave * 2;
    constexpr int PB = BITS == 2 ? 256 : 512;  // bytes per panel-group
    const uint8_t *wbase = Wp + (int64_t)e * wp_stride;
    const uint16_t *sbase = Ws + (int64_t)e * ws_stride;
    const uint8_t *wq0 = wbase + (int64_t)pan0 * G * PB + lane * (PB / 64);
    const uint8_t *wq1 = wq0 + (int64_t)G * PB;
    const uint16_t *sc0 = sbase + (int64_t)pan0 * G * 16 + (lane & 15);
    const uint16_t *sc1 = sc0 + (int64_t)G * 16;

    *(v4i *)(&As[0][a_dst]) = *(const v4i *)(a_src);
    double T[4][2][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) T[i][j][r] = 0.0;
    __syncthreads();

    for (int g = 0; g < G; g++) {
        const int cur = g & 1;
        v4i an;
        if (g + 1 < G) an = *(const v4i *)(a_src + (int64_t)(g + 1) * 64);
        v4i b[2];
        if (BITS == 2) {
            const uint32_t w0 = *(const uint32_t *)(wq0 + (int64_t)g * PB);
            const uint32_t w1 = *(const uint32_t *)(wq1 + (int64_t)g * PB);
            b[0] = unpack_int2(w0);
            b[1] = unpack_int2(w1);
        } else {
            const uint2 w0 = *(const uint2 *)(wq0 + (int64_t)g * PB);
            const uint2 w1 = *(const uint2 *)(wq1 + (int64_t)g * PB);
            b[0] = unpack_int4(w0.x, w0.y);
            b[1] = unpack_int4(w1.x, w1.y);
        }
        const double s0 = f16_to_f64(sc0[g * 16]);
        const double s1 = f16_to_f64(sc1[g * 16]);
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i *)(&As[cur][i * 1024 + lane * 16]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const v4i z = {0, 0, 0, 0};
            const v4i c0 = mfma16x16x64(af[i], b[0], z);
            const v4i c1 = mfma16x16x64(af[i], b[1], z);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                T[i][0][r] = fma((double)c0[r], s0, T[i][0][r]);
                T[i][1][r] = fma((double)c1[r], s1, T[i][1][r]);
            }
        }
        if (g + 1 < G) *(v4i *)(&As[cur ^ 1][a_dst]) = an;
        __syncthreads();
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
                const double sa = (double)rowscale[rr];
                const float gv = (float)(T[i][0][r] * sa);
                const float uv = (float)(T[i][1][r] * sa);
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
                    const float f = (float)(T[i][j][r] * (double)rowscale[rr]);
                    bad |= !isfinite(f);
                    out[(int64_t)rowdst[rr] * ldo + col] = f;
                }
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}

extern "C" int jtk_lowbit_grouped(int bits, const int8_t *A, int lda, const float *sA,
                                  const int32_t *perm, const int32_t *off, int topk,
                                  const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                                  const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                                  int64_t ws_stride, int N, int K, float *out, int ldo,
                                  uint32_t *err, hipStream_t s) {
    if (max_tiles <= 0) return 0;
    dim3 grid((unsigned)max_tiles, (unsigned)(N / 128));
    if (bits == 2)
        hipLaunchKernelGGL((k_lowbit_grouped<2, EPI_SWIGLU>), grid, dim3(256), 0, s, A, lda,
                           sA, perm, off, topk, tiles, ntiles, Wp, Ws, wp_stride, ws_stride,
                           N, K, out, ldo, err);
    else
        hipLaunchKernelGGL((k_lowbit_grouped<4, EPI_SCATTER>), grid, dim3(256), 0, s, A, lda,
                           sA, perm, off, topk, tiles, ntiles, Wp, Ws, wp_stride, ws_stride,
                           N, K, out, ldo, err);
    return (int)hipGetLastError();
}
