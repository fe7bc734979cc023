// Dense W8A8 MFMA GEMM for gfx950, templated on the tile geometry.
//
// C[m][n] = epilogue(acc[m][n]), acc = sum_k A[m][k] * W[n][k] in int32 with
// v_mfma_i32_16x16x64_i8. A is row-major int8 [M][lda] (lda >= Kp,
// Kp % 64 == 0, zero bytes past K); W is in the 16-channel x 64-K panel
// layout of jt_dev.h, padded to Np channels (multiple of BN).
//
// Block tile BM x BN. WGM x WGN waves tile the block with (BM/WGM) x (BN/WGN)
// wave tiles; KS such wave groups split each stage's KS k-blocks of 64
// between them (intra-block split-K; int32 partial sums are exchanged
// through LDS at the end, which is exact). Operand panels (1 KiB each) go
// global -> LDS with global_load_lds_dwordx4 into a ring of NST stages filled
// NST-1 stages ahead; a wave waits only for its own copies of the stage it
// is about to use and the workgroup then meets at a fence-less barrier.
// Tile order: blocks are dealt to the 8 XCDs round-robin (block b on XCD
// b % 8). The tile grid is cut into 8 / cp row parts x cp column parts, one
// an XCD, with cp in {1, 2, 4, 8} chosen so that an XCD's share of the A rows
// plus its share of the weight columns is smallest (the gate/up of both
// shared experts, 32 x 44 tiles at K = 1024: 2 x 4; their down, 32 x 4 tiles
// at K = 2816: 8 x 1); when no cut divides the grid the tiles go in order.
// Inside an XCD's share the tiles walk GM row-tiles at a time (all column
// tiles of a GM-row group before the next group) so its concurrently
// resident blocks share A rows and W columns in its L2.
#pragma once
#include <hip/hip_ext.h>
#include "jt_dev.h"

enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_SCATTER = 2 };

typedef __attribute__((address_space(3))) void lds_void;

// One LDS-DMA copy: each lane moves BYTES bytes from its own global address
// to lds_base + BYTES * lane (lds_base is wave-uniform).
template <int BYTES>
__device__ __forceinline__ void dma(const void *g, void *lds_base);
template <>
__device__ __forceinline__ void dma<16>(const void *g, void *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)lds_base, 16, 0, 0);
}
template <>
__device__ __forceinline__ void dma<4>(const void *g, void *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)lds_base, 4, 0, 0);
}

// The 32-bit LDS address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the memory fence of __syncthreads(): the fence
// would drain every in-flight LDS-DMA stage (s_waitcnt vmcnt(0)). Callers
// first wait for their own stage with wait_vm, after which the DMA data is in
// LDS, which all waves of the workgroup see after the barrier.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// This wave's LDS writes done, then the workgroup barrier (no wait on
// in-flight global loads).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait for the oldest in-flight stage when `later` stages of PER copies each
// were issued after it (the counter field holds at most 63; a smaller bound
// only waits longer).
template <int PER>
__device__ __forceinline__ void wait_stage(int later) {
#define JT_WAIT_CASE(k)                              \
    case k:                                          \
        wait_vm<(k * PER < 63 ? k * PER : 63)>(); \
        break;
    switch (later) {
        JT_WAIT_CASE(0)
        JT_WAIT_CASE(1)
        JT_WAIT_CASE(2)
        JT_WAIT_CASE(3)
        JT_WAIT_CASE(4)
        JT_WAIT_CASE(5)
        JT_WAIT_CASE(6)
        default:
            wait_vm<(7 * PER < 63 ? 7 * PER : 63)>();
    }
#undef JT_WAIT_CASE
}

// Linear tile index -> (row tile, column tile), walking GM row tiles at a
// time: all column tiles of a group of GM row tiles before the next group.
template <int GM>
__device__ __forceinline__ void tile_coords(int lin, int mtiles, int ntiles, int &mt, int &nt) {
    const int per_group = GM * ntiles;
    const int first_m = (lin / per_group) * GM;
    const int gsz = min(mtiles - first_m, GM);
    mt = first_m + (lin % per_group) % gsz;
    nt = (lin % per_group) / gsz;
}

// Epilogue of one wave tile at (r0, c0): acc[i][j] element r of lane l is
// row r0 + 16i + 4(l/16) + r, column c0 + 16j + l%16. With HALF > 0 only the
// rows i / HALF == part are written (the other part belongs to a partner wave).
//   EPI_PLAIN : C[row][col] = (float)((double)acc * ((double)sA[row] * sB[col]))
//   EPI_SWIGLU: channels packed [gate 16][up 16] per 32 (tile 2jj gate, 2jj+1
//               up); C[row][hidden] = silu(g) * u in fp64, rounded to float.
//               With hpl > 0 the hidden columns are hpl-wide planes (one per
//               expert whose gate/up panels are concatenated along N):
//               hidden x goes to C[(x / hpl) * plane + row * ldc + x % hpl].
template <int EPI, int TM, int TN, int HALF>
__device__ __forceinline__ void w8a8_epilogue(const v4i (&acc)[TM][TN], int part, int r0, int c0,
                                              int lane, const float *rs, const float *cs,
                                              int M, int N, float *__restrict__ C, int ldc,
                                              int hpl, int64_t plane, uint32_t *err,
                                              const double *exp_tab) {
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    // The scales (rs: this wave tile's rows, cs: its columns) and the exp
    // table were copied to LDS with the first stage, so the epilogue issues
    // no global load: gfx9 counts stores and loads on one vmcnt, and a load
    // after a store would wait for the store.
    float4 saf[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) saf[i] = *(const float4 *)(rs + i * 16 + lr);
    double sb[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) sb[j] = (double)cs[j * 16 + lc];
#define sa(i, r) ((double)((r) == 0 ? saf[i].x : (r) == 1 ? saf[i].y : (r) == 2 ? saf[i].z : saf[i].w))
    // Wave-uniform bounds: interior tiles store without per-element checks.
    const bool full = r0 + 16 * TM <= M && c0 + 16 * TN <= N;
    uint32_t bad = 0, badmid = 0;
    if (EPI == EPI_SWIGLU) {
        // pointer shift of each 16-wide hidden block into its plane
        // (wave-uniform; hpl is a multiple of 16)
        int64_t pofs[TN / 2];
#pragma unroll
        for (int jj = 0; jj < TN / 2; jj++) {
            const int x0 = c0 / 2 + jj * 16;
            pofs[jj] = hpl > 0 ? (int64_t)(x0 / hpl) * plane + (x0 % hpl) - x0 : 0;
        }
        // A non-finite g or u (the only way silu_mul fails) shows as a
        // maximum of the sign-cleared bit patterns at or above that of +inf.
        uint32_t mx = 0;
        auto one = [&](int i, int r, int jj, float *dst) {
            const float g = (float)((double)acc[i][2 * jj][r] * (sa(i, r) * sb[2 * jj]));
            const float u =
                (float)((double)acc[i][2 * jj + 1][r] * (sa(i, r) * sb[2 * jj + 1]));
            mx = max(mx, max(abs_bits(g), abs_bits(u)));
            float sv;
            (void)silu_mul(g, u, &sv, exp_tab);
            *dst = sv;
        };
        if (full) {  // an interior tile: straight-line code
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (HALF > 0 && i / (HALF > 0 ? HALF : 1) != part) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float *crow = C + (int64_t)(r0 + i * 16 + lr + r) * ldc + c0 / 2 + lc;
#pragma unroll
                    for (int jj = 0; jj < TN / 2; jj++) one(i, r, jj, crow + jj * 16 + pofs[jj]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (HALF > 0 && i / (HALF > 0 ? HALF : 1) != part) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = r0 + i * 16 + lr + r;
                    float *crow = C + (int64_t)row * ldc + c0 / 2 + lc;
#pragma unroll
                    for (int jj = 0; jj < TN / 2; jj++)
                        if (row < M && c0 + (2 * jj + 1) * 16 + lc < N)
                            one(i, r, jj, crow + jj * 16 + pofs[jj]);
                }
            }
        }
        if (mx >= 0x7f800000u) raise_err(err, EF_RANGE | EF_NONFINITE_MID);
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
        if (HALF > 0 && i / (HALF > 0 ? HALF : 1) != part) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = r0 + i * 16 + lr + r;
            float *crow = C + (int64_t)row * ldc;
            if (EPI == EPI_PLAIN) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int col = c0 + j * 16 + lc;
                    const float f = (float)((double)acc[i][j][r] * (sa(i, r) * sb[j]));
                    if (full || (row < M && col < N)) {
                        bad |= !isfinite(f);
                        crow[col] = f;
                    }
                }
            } else {
#pragma unroll
                for (int jj = 0; jj < TN / 2; jj++) {
                    const int cu = c0 + (2 * jj + 1) * 16 + lc;
                    const int hid = c0 / 2 + jj * 16 + lc;
                    const float g =
                        (float)((double)acc[i][2 * jj][r] * (sa(i, r) * sb[2 * jj]));
                    const float u =
                        (float)((double)acc[i][2 * jj + 1][r] * (sa(i, r) * sb[2 * jj + 1]));
                    if (full || (row < M && cu < N)) {
                        bad |= (!isfinite(g)) || (!isfinite(u));
                        float sv;
                        badmid |= !silu_mul(g, u, &sv);
                        crow[hid] = sv;
                    }
                }
            }
        }
    }
    if (bad) raise_err(err, EF_RANGE);
    if (badmid) raise_err(err, EF_NONFINITE_MID);
}
#undef sa

// Strides of a batch of GEMMs in one launch (blockIdx.y = GEMM b): A and the
// weight panels in bytes, sA, sB and C in floats. All zero for one GEMM.
struct TileBatch {
    int64_t bsA, bsW;
    int bsSA, bsB;
    int64_t bsC;
};

template <int EPI, int BM, int BN, int WGM, int WGN, int KS, int NST, int GM>
__global__ __launch_bounds__(64 * WGM * WGN * KS) void k_w8a8_tile(
    const int8_t *__restrict__ A, int lda, const float *__restrict__ sA,
    const int8_t *__restrict__ Wp, const float *__restrict__ sB, int M, int N, int Kp,
    float *__restrict__ C, int ldc, int hpl, int64_t plane, uint32_t *err, int mtiles,
    int ntiles, TileBatch bt) {
    if (blockIdx.y) {  // GEMM blockIdx.y of a batch
        A += blockIdx.y * bt.bsA;
        Wp += blockIdx.y * bt.bsW;
        sA += (int64_t)blockIdx.y * bt.bsSA;
        sB += (int64_t)blockIdx.y * bt.bsB;
        C += blockIdx.y * bt.bsC;
    }
    constexpr int NWG = WGM * WGN;  // waves per k-group
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    constexpr int AP = BM / 16, BP = BN / 16, NP = AP + BP;
    constexpr int PPW = NP / NWG;  // panels copied per wave per stage
    constexpr int STAGE = NP * KS * 1024;
    static_assert(NP % NWG == 0, "panels must split evenly over waves");
    static_assert(NST >= 2 && NST <= 8, "2..8 stages");
    static_assert(KS == 1 || KS == 2, "k-split of 1 or 2");
    static_assert(KS == 1 || TM % 2 == 0, "k-split halves the wave tile rows");
    static_assert(KS == 1 || NST * STAGE >= 2 * NWG * (TM / 2) * TN * 1024,
                  "exchange buffer fits the stage ring");
    static_assert(EPI != EPI_SWIGLU || TN % 2 == 0, "gate/up pairs need even TN");
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform in a scalar register: guards on it then branch, which
    // matters because v_mfma ignores EXEC (an exec-masked MFMA still runs)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = wave % NWG, kg = wave / NWG;
    const int pid = blockIdx.x;
    int mt, nt;
    // the XCD split (8 / cp row parts x cp column parts) whose share of the
    // A rows and weight columns is smallest
    int cp = 0;
    int64_t best = INT64_MAX;
#pragma unroll
    for (int c = 1; c <= 8; c *= 2) {
        const int rp = 8 / c;
        const int64_t cost = (int64_t)mtiles * BM / rp + (int64_t)ntiles * BN / c;
        if (mtiles % rp == 0 && ntiles % c == 0 && cost < best) {
            best = cost;
            cp = c;
        }
    }
    if (cp) {
        const int x8 = pid & 7, sm = mtiles / (8 / cp), sn = ntiles / cp;
        int lm, ln;
        tile_coords<GM>(pid >> 3, sm, sn, lm, ln);
        mt = (x8 / cp) * sm + lm;
        nt = (x8 % cp) * sn + ln;
    } else {
        tile_coords<GM>(pid, mtiles, ntiles, mt, nt);
    }
    const int m0 = mt * BM, n0 = nt * BN;
    const int wm = (wg / WGN) * WTM, wn = (wg % WGN) * WTN;
    const int KB = Kp / 64;
    const int NSG = (KB + KS - 1) / KS;  // stages

    // Copy i of a wave moves panel p = wg*PPW + i of k-block sub = kg.
    const int8_t *src[PPW];
    int step[PPW];
#pragma unroll
    for (int i = 0; i < PPW; i++) {
        const int p = wg * PPW + i;
        if (p < AP) {
            int r = m0 + p * 16 + (lane & 15);
            r = r < M ? r : M - 1;
            src[i] = A + (int64_t)r * lda + (lane >> 4) * 16;
            step[i] = 64;
        } else {
            src[i] = Wp + ((int64_t)(n0 / 16 + p - AP) * KB) * 1024 + lane * 16;
            step[i] = 1024;
        }
    }
    // the epilogue's row and column scales (and the SwiGLU's exp table) go
    // to LDS ahead of the first stage; they are older than every stage copy,
    // so the first stage's wait covers them
    __shared__ __attribute__((aligned(16))) float s_rs[BM];
    __shared__ __attribute__((aligned(16))) float s_cs[BN];
    // The exp table goes to LDS through registers (loaded here, stored by
    // every wave at the epilogue, exp_tab_stage): reads of an LDS-DMA
    // target make the compiler wait for every outstanding vector memory
    // operation, stores included.
    __shared__ __attribute__((aligned(16))) double s_tab[EPI == EPI_SWIGLU ? 64 : 2];
    const double tabv = EPI == EPI_SWIGLU ? exp_tab_load(lane) : 0.0;
    for (int c = wave; c < (BM + BN) / 64; c += NWG * KS) {  // 64 scales per copy
        if (c < BM / 64)
            dma<4>(sA + min(m0 + 64 * c + lane, M - 1), s_rs + 64 * c);
        else
            dma<4>(sB + min(n0 + 64 * (c - BM / 64) + lane, N - 1), s_cs + 64 * (c - BM / 64));
    }
    auto issue = [&](int sg) {
        int8_t *st = smem + (sg % NST) * STAGE + kg * NP * 1024;
        int kb = sg * KS + kg;
        kb = kb < KB ? kb : KB - 1;  // a past-the-end block reloads the last one
#pragma unroll
        for (int i = 0; i < PPW; i++)
            dma<16>(src[i] + (int64_t)kb * step[i], st + (wg * PPW + i) * 1024);
    };
#pragma unroll
    for (int s = 0; s < NST - 1; s++)
        if (s < NSG) issue(s);

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    for (int sg = 0; sg < NSG; sg++) {
        wait_stage<PPW>(min(NST - 2, NSG - 1 - sg));
        barrier_lds();
        if (sg + NST - 1 < NSG) issue(sg + NST - 1);
        if (sg * KS + kg < KB) {
            const int8_t *st = smem + (sg % NST) * STAGE + kg * NP * 1024;
            v4i bf[TN];
#pragma unroll
            for (int j = 0; j < TN; j++)
                bf[j] = *(const v4i *)(st + (AP + (wn >> 4) + j) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const v4i af = *(const v4i *)(st + ((wm >> 4) + i) * 1024 + lane * 16);
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = mfma16x16x64(af, bf[j], acc[i][j]);
            }
        }
    }

    // With a k-split each wave finishes the rows i / TE == kg of its wave
    // tile after adding the partner group's partial sums (register arrays
    // are indexed with constants only).
    constexpr int TE = KS == 1 ? TM : TM / 2;
    if (KS == 2) {
        barrier_lds();  // every wave is done reading the stage ring
        v4i *xbuf = (v4i *)smem;  // slot (writer group, wg, i % TE, j) x 64 lanes
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                if (i / TE != kg)
                    xbuf[(((kg * NWG + wg) * TE + i % TE) * TN + j) * 64 + lane] = acc[i][j];
        __syncthreads();  // LDS writes complete and visible
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                if (i / TE == kg)
                    acc[i][j] += xbuf[((((1 - kg) * NWG + wg) * TE + i % TE) * TN + j) * 64 + lane];
    }
    if (EPI == EPI_SWIGLU) exp_tab_stage(s_tab, lane, tabv);
    w8a8_epilogue<EPI, TM, TN, KS == 2 ? TE : 0>(acc, kg, m0 + wm, n0 + wn, lane, s_rs + wm,
                                                  s_cs + wn, M, N, C, ldc, hpl, plane, err,
                                                  s_tab);
}

// Host-side launch of one configuration (dynamic LDS = NST stages). Non-null
// events e0 / e1 take the timestamps of the kernel's own start and end
// (hipExtLaunchKernelGGL), so their elapsed time is the kernel's duration
// with no marker packet around it.
template <int EPI, int BM, int BN, int WGM, int WGN, int KS, int NST, int GM>
inline hipError_t launch_w8a8_tile(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                                   const float *sB, int M, int N, int Np, int Kp, float *C,
                                   int ldc, uint32_t *err, hipStream_t s,
                                   hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr,
                                   int hpl = 0, int64_t plane = 0, unsigned nb = 1,
                                   TileBatch bt = TileBatch{}) {
    auto kern = k_w8a8_tile<EPI, BM, BN, WGM, WGN, KS, NST, GM>;
    constexpr int lds = NST * (BM + BN) / 16 * KS * 1024;
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
    const int mt = (M + BM - 1) / BM, nt = Np / BN;
    hipExtLaunchKernelGGL(kern, dim3((unsigned)(mt * nt), nb), dim3(64 * WGM * WGN * KS), lds,
                          s, e0, e1, 0, A, lda, sA, Wp, sB, M, N, Kp, C, ldc, hpl, plane, err, mt,
                          nt, bt);
    return hipGetLastError();
}
