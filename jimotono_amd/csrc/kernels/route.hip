// Routing, expert sort, work lists and combine (gfx950).
//
//  k_router_logits : logits[t][e] = (float)dot(X[t], Wgate[e]) in fp64 with
//                    the reference's four lane partials over j % 4, combined
//                    as (l0+l1)+(l2+l3), then the tail (src/moe_layer.c:67-86,
//                    1118-1137). Products of two floats are exact in fp64, so
//                    fma(x, w, l) rounds exactly like the reference's
//                    separate multiply and add.
//  k_topk          : top-k by value with ties to the lower index, softmax
//                    over the selected k in fp64 (src/routing.c:16-76).
//  k_sort_*        : stable counting sort of the (token, slot) pairs by
//                    expert, optional capacity (src/moe_layer.c:895-978).
//  k_combine       : Y[t] = (float)(sum_p w_p*Ye[t,p] + sum_s Ys[s][t]) in
//                    fp64, slot order then shared order
//                    (src/moe_layer.c:1443-1463, 1549-1574).
#include "jt_dev.h"
#include "jt_launch.h"
#include "topk_dev.h"
#include "sort_dev.h"
#include "quant_dev.h"

// ---------------- router logits ----------------
// Block: 64 tokens x 64 experts, 256 threads in 4 groups of 64; group p
// accumulates the reference's lane partial l_p = sum over j = p (mod 4) of
// x_j*w_j (j ascending) for all 64 x 64 outputs, each thread an 8 x 8
// (token, expert) register tile of fp64 accumulators. K is staged through
// LDS as fp32, k-major, in chunks of 32 (double-buffered). At the end the
// partials meet in LDS and are combined as (l0+l1)+(l2+l3), then the tail
// j >= n & ~3 is added in order, as in the reference.
#define RT_T 64
#define RT_E 64
#define RT_KC 32
__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ X,
                                                       const float *__restrict__ Wg, int T,
                                                       int E, int n,
                                                       float *__restrict__ logits,
                                                       uint32_t *err) {
    // [stage][x|w][k][row] fp64 (widened once when staged): 64 KiB, reused
    // as the 64 x 64 fp64 partial buffer
    __shared__ __attribute__((aligned(16))) double lds[2][2][RT_KC][64];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * RT_T, e0 = blockIdx.y * RT_E;
    const int p = tid >> 6;                       // lane partial of this thread
    const int ty = (tid >> 3) & 7, tx = tid & 7;  // tokens ty*8.., experts tx*8..
    double acc[8][8];
#pragma unroll
    for (int a = 0; a < 8; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = 0.0;
    const int n4 = n & ~3;
    // stage loader: thread -> row tid%64, k = 8*(tid/64) .. +7 of the chunk;
    // LDS stores of consecutive threads are consecutive (no bank conflicts)
    const int lr = tid & 63, lk = (tid >> 6) * 8;
    const float *xrow = X + (int64_t)min(t0 + lr, T - 1) * n;
    const float *wrow = Wg + (int64_t)min(e0 + lr, E - 1) * n;
    const bool vec = (n & 3) == 0;
    float xv[8], wv[8];
    auto gload = [&](int k0) {
        const int kb = k0 + lk;
        if (vec && kb + 8 <= n4) {
            const float4 a0 = *(const float4 *)(xrow + kb), a1 = *(const float4 *)(xrow + kb + 4);
            const float4 b0 = *(const float4 *)(wrow + kb), b1 = *(const float4 *)(wrow + kb + 4);
            xv[0] = a0.x; xv[1] = a0.y; xv[2] = a0.z; xv[3] = a0.w;
            xv[4] = a1.x; xv[5] = a1.y; xv[6] = a1.z; xv[7] = a1.w;
            wv[0] = b0.x; wv[1] = b0.y; wv[2] = b0.z; wv[3] = b0.w;
            wv[4] = b1.x; wv[5] = b1.y; wv[6] = b1.z; wv[7] = b1.w;
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int k = kb + c;
                xv[c] = k < n4 ? xrow[k] : 0.0f;
                wv[c] = k < n4 ? wrow[k] : 0.0f;
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            lds[buf][0][lk + c][lr] = (double)xv[c];
            lds[buf][1][lk + c][lr] = (double)wv[c];
        }
    };
    gload(0);
    sstore(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < n4; k0 += RT_KC) {
        const bool more = k0 + RT_KC < n4;
        if (more) gload(k0 + RT_KC);
        const int kend = min(RT_KC, n4 - k0);
        for (int i = p; i < kend; i += 4) {
            double xa[8], wa[8];
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                const double2 xx = *(const double2 *)&lds[buf][0][i][ty * 8 + c];
                const double2 ww = *(const double2 *)&lds[buf][1][i][tx * 8 + c];
                xa[c] = xx.x;
                xa[c + 1] = xx.y;
                wa[c] = ww.x;
                wa[c + 1] = ww.y;
            }
#pragma unroll
            for (int a = 0; a < 8; a++)
#pragma unroll
                for (int b = 0; b < 8; b++) acc[a][b] = fma(xa[a], wa[b], acc[a][b]);
        }
        if (more) sstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    // combine partials through LDS (reusing the staging arrays):
    // l1 -> l0+l1, l3 -> l2+l3, then (l0+l1)+(l2+l3)
    double *red = &lds[0][0][0][0];
    auto put = [&]() {
#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
            for (int b = 0; b < 8; b++) red[(ty * 8 + a) * 64 + tx * 8 + b] = acc[a][b];
    };
    auto add = [&]() {
#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
            for (int b = 0; b < 8; b++) acc[a][b] = acc[a][b] + red[(ty * 8 + a) * 64 + tx * 8 + b];
    };
    if (p == 1) put();
    __syncthreads();
    if (p == 0) add();
    __syncthreads();
    if (p == 3) put();
    __syncthreads();
    if (p == 2) add();
    __syncthreads();
    if (p == 2) put();
    __syncthreads();
    if (p != 0) return;
    add();
    uint32_t bad = 0;
#pragma unroll
    for (int a = 0; a < 8; a++) {
        const int t = t0 + ty * 8 + a;
        if (t >= T) continue;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int e = e0 + tx * 8 + b;
            if (e >= E) continue;
            double s = acc[a][b];
            for (int j = n4; j < n; j++)
                s = s + (double)X[(int64_t)t * n + j] * (double)Wg[(int64_t)e * n + j];
            const float f = (float)s;
            bad |= (!isfinite(s)) || (!isfinite(f));
            logits[(int64_t)t * E + e] = f;
        }
    }
    if (bad) raise_err(err, EF_NONFINITE_MID);
}

extern "C" int jtk_router_logits(const float *X, const float *Wg, int T, int E, int n,
                                 float *logits, uint32_t *err, hipStream_t s) {
    dim3 grid((unsigned)((T + RT_T - 1) / RT_T), (unsigned)((E + RT_E - 1) / RT_E));
    hipLaunchKernelGGL(k_router_logits, grid, dim3(256), 0, s, X, Wg, T, E, n, logits, err);
    return (int)hipGetLastError();
}

// ---------------- top-k + softmax ----------------
// Top-k and softmax of one row, one wavefront: the row is copied to the
// wave's LDS row l (E floats), then selected; lanes p < k write id p and
// weight p. Returns false (and raises the error) on a NaN logit or a
// non-finite softmax; *id gets lane p's id (-1 on other lanes / failure).
__device__ bool topk_wave(const float *__restrict__ lg, float *l, int E, int k, int lane,
                          int64_t row, int32_t *__restrict__ ids, int64_t *__restrict__ ids64,
                          float *__restrict__ w, uint32_t *err, int *id) {
    *id = -1;
    int nan = 0;
    for (int i = lane; i < E; i += 64) {
        const float v = lg[i];
        nan |= isnan(v);
        l[i] = v;
    }
    // the row is written and read by this wavefront only
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    nan = wave_or_i(nan);
    if (nan) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return false;
    }
    // Lane l owns elements i = l + 64*j (j < 64, E <= 4096); bit j of
    // `taken` marks an element already selected. Each round takes the wave
    // maximum of 64-bit keys (order-preserving bits of the value, -0 folded
    // into +0 since the reference's comparisons treat them as equal, then
    // ~i so that ties go to the lower index) with DPP moves. A taken
    // element keys as -inf, as in the reference's scan, so when only -inf
    // is left the lowest index wins even if already taken.
    uint64_t taken = 0;
    int mysel = -1;
    for (int p = 0; p < k; p++) {
        uint64_t best = 0;
        for (int i = lane, j = 0; i < E; i += 64, j++) {
            const float v = ((taken >> j) & 1ull) ? -__builtin_inff() : l[i] + 0.0f;
            uint32_t u = __builtin_bit_cast(uint32_t, v);
            u ^= (u >> 31) ? 0xffffffffu : 0x80000000u;
            const uint64_t key = ((uint64_t)u << 32) | (uint32_t)~i;
            best = key > best ? key : best;
        }
        const int bi = (int)~(uint32_t)wave_max_u64(best);
        if ((bi & 63) == lane) taken |= 1ull << (bi >> 6);
        if (lane == p) mysel = bi;
    }
    // softmax over the selected, in selection order; the first selected is
    // the maximum
    const float lv = lane < k ? l[mysel] : -__builtin_inff();
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                   __builtin_bit_cast(int, lv), 0));
    const double e = lane < k ? exp((double)lv - (double)mx) : 0.0;
    double sum = 0.0;
    for (int p = 0; p < k; p++) sum += readlane_f64(e, p);
    const bool ok = (sum > 0.0) && isfinite(sum);
    if (!ok) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return false;
    }
    const float inv = (float)(1.0 / sum);
    if (lane < k) {
        const float wv = (float)e * inv;
        ids[row * k + lane] = mysel;
        if (ids64) ids64[row * k + lane] = mysel;
        w[row * k + lane] = wv;
        if (!(wv >= 0.0f) || !isfinite(wv)) raise_err(err, EF_NONFINITE_MID);
        *id = mysel;
    }
    return true;
}

// One wavefront per row of logits [rows][E]. Selection is an argmax by
// (value desc, index asc) with already-selected entries treated as -INF,
// which is exactly the reference's strict-greater linear scan. NaN logits
// are rejected (EF_NONFINITE_MID). ids are written as int32 and, when ids64
// is non-NULL, also as 64-bit values (the reference's size_t). The row is
// read from memory once into LDS (4 * E floats per block), so the k rounds
// pay LDS rather than memory latency.
__global__ __launch_bounds__(256) void k_topk(const float *__restrict__ logits, int rows,
                                              int E, int k, int32_t *__restrict__ ids,
                                              int64_t *__restrict__ ids64,
                                              float *__restrict__ w, uint32_t *err) {
    extern __shared__ float tk_smem[];
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    int id;
    (void)topk_wave(logits + (int64_t)row * E, tk_smem + (threadIdx.x >> 6) * E, E, k, lane, row,
                    ids, ids64, w, err, &id);
}

// The same with the row's keys in registers (E <= 1024): no LDS round trip
// per element and round (measured 7.3 -> 4.4 us for 16 rows of 256).
template <int EPL>
__global__ __launch_bounds__(256) void k_topk_reg(const float *__restrict__ logits, int rows,
                                                  int E, int k, int32_t *__restrict__ ids,
                                                  int64_t *__restrict__ ids64,
                                                  float *__restrict__ w, uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    (void)topk_wave_reg<EPL>(logits + (int64_t)row * E, E, k, lane, row, ids, ids64, w, err);
}

extern "C" int jtk_topk(const float *logits, int rows, int E, int k, int32_t *ids,
                        int64_t *ids64, float *w, uint32_t *err, hipStream_t s) {
    if (rows <= 0) return 0;
    if (E > 4096 || k > 64) return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch (topk_epl(E)) {
#define TK_REG(P)                                                                          \
    case P:                                                                                \
        hipLaunchKernelGGL(k_topk_reg<P>, grid, dim3(256), 0, s, logits, rows, E, k, ids, \
                           ids64, w, err);                                                 \
        return (int)hipGetLastError();
        TK_REG(1)
        TK_REG(2)
        TK_REG(4)
        TK_REG(8)
        TK_REG(16)
#undef TK_REG
    default: break;
    }
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)k_topk, hipFuncAttributeMaxDynamicSharedMemorySize,
                                4 * 4096 * 4);
        if (e != hipSuccess) return (int)e;
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(k_topk, dim3((unsigned)((rows + 3) / 4)), dim3(256), (size_t)4 * E * 4, s,
                       logits, rows, E, k, ids, ids64, w, err);
    return (int)hipGetLastError();
}

// Top-k of one row of any length n (< 2^31) and any k <= n, in one block
// of 1024 threads: the reference's selection order is the descending order
// of the keys (order-preserving value bits with -0 folded into +0, then ~i
// so ties go to the lower index), so round p takes the largest key below
// round p-1's key with a streaming block max and needs no taken-set.
// Elements at -inf never beat the masked ones: once only -inf remains
// (p >= c, c = number of values above -inf) the reference's scan keeps its
// first index, 0. The softmax then runs over the k selected logits in
// selection order as in topk_wave (one thread: the fp64 sum is sequential).
#define TKB_THREADS 1024
__global__ __launch_bounds__(TKB_THREADS) void k_topk_block(const float *__restrict__ lg,
                                                            int64_t n, int64_t k,
                                                            int64_t *__restrict__ ids64,
                                                            float *__restrict__ w,
                                                            uint32_t *err) {
    __shared__ uint64_t red[TKB_THREADS / 64];
    __shared__ int64_t sh_c;
    __shared__ int sh_nan;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // NaN check and c
    int nan = 0;
    int64_t c = 0;
    for (int64_t i = tid; i < n; i += TKB_THREADS) {
        const float v = lg[i];
        nan |= isnan(v);
        c += v > -__builtin_inff();
    }
    if (tid == 0) {
        sh_c = 0;
        sh_nan = 0;
    }
    __syncthreads();
    nan = wave_or_i(nan);
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if (lane == 0) {
        atomicAdd((unsigned long long *)&sh_c, (unsigned long long)c);
        if (nan) atomicOr(&sh_nan, 1);
    }
    __syncthreads();
    if (sh_nan) {
        if (tid == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    const int64_t cnt = sh_c, kk = k < cnt ? k : cnt;
    uint64_t prev = ~0ull;
    for (int64_t p = 0; p < kk; p++) {
        uint64_t best = 0;
        for (int64_t i = tid; i < n; i += TKB_THREADS) {
            uint32_t u = __builtin_bit_cast(uint32_t, lg[i] + 0.0f);
            u ^= (u >> 31) ? 0xffffffffu : 0x80000000u;
            const uint64_t key = ((uint64_t)u << 32) | (uint32_t)~(uint32_t)i;
            best = (key < prev && key > best) ? key : best;
        }
        best = wave_max_u64(best);
        if (lane == 0) red[wv] = best;
        __syncthreads();
        best = red[0];
        for (int j = 1; j < TKB_THREADS / 64; j++) best = red[j] > best ? red[j] : best;
        __syncthreads();  // red[] is rewritten next round
        prev = best;
        if (tid == 0) ids64[p] = (int64_t)(uint32_t)~(uint32_t)best;
    }
    for (int64_t p = kk + tid; p < k; p += TKB_THREADS) ids64[p] = 0;
    __syncthreads();
    if (tid != 0) return;
    // softmax over the selected, in selection order (src/routing.c:56-75);
    // ids from kk on are 0 (written by other threads: not read back)
    const float mx = lg[kk > 0 ? ids64[0] : 0];
    double sum = 0.0;
    for (int64_t p = 0; p < k; p++) {
        const double e = exp((double)lg[p < kk ? ids64[p] : 0] - (double)mx);
        sum += e;
        w[p] = (float)e;
    }
    if (!(sum > 0.0) || !isfinite(sum)) {
        raise_err(err, EF_NONFINITE_MID);
        return;
    }
    const float inv = (float)(1.0 / sum);
    for (int64_t p = 0; p < k; p++) w[p] = w[p] * inv;
}

extern "C" int jtk_topk_block(const float *logits, int64_t n, int64_t k, int64_t *ids64,
                              float *w, uint32_t *err, hipStream_t s) {
    if (n <= 0 || k <= 0 || k > n || n > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_topk_block, dim3(1), dim3(TKB_THREADS), 0, s, logits, n, k, ids64, w,
                       err);
    return (int)hipGetLastError();
}

// ---------------- stable expert sort ----------------
// Pairs q = 0..Tk-1 with expert ids[q]. Blocks of 256 consecutive pairs.
//  hist   : rank[q] = #{q' < q in the block : ids[q'] == ids[q]},
//           cnt[b][e] = number of pairs of expert e in block b;
//  scan_e : cnt[b][e] -> exclusive prefix over b (per expert), tot[e];
//  off    : off[e] = sum_{e' < e} min(tot[e'], cap);
//  scatter: global rank g = cnt[b][e] + rank[q]; kept iff g < cap;
//           perm[off[e] + g] = q.
#define SQ 256
#define SORT_MID_NB 256  // medium-batch sort: up to 256 blocks of 256 pairs
__global__ __launch_bounds__(256) void k_sort_hist(const int32_t *__restrict__ ids, int Tk,
                                                   int E, int32_t *__restrict__ rank,
                                                   int32_t *__restrict__ cnt, uint32_t *err) {
    __shared__ int sid[SQ];
    const int b = blockIdx.x, t = threadIdx.x;
    const int q = b * SQ + t;
    int e = -1;
    if (q < Tk) {
        e = ids[q];
        if (e < 0 || e >= E) {
            raise_err(err, EF_BAD_ID);
            e = -1;
        }
    }
    sid[t] = e;
    for (int i = t; i < E; i += 256) cnt[(int64_t)b * E + i] = 0;
    __syncthreads();
    int r = 0;
    bool last = true;
    for (int i = 0; i < SQ; i++) {
        const int o = sid[i];
        r += (i < t && o == e);
        last &= !(i > t && o == e);
    }
    if (q < Tk) rank[q] = r;
    __syncthreads();  // zeroing above must land before the counts
    if (q < Tk && e >= 0 && last) cnt[(int64_t)b * E + e] = r + 1;
}

__global__ __launch_bounds__(256) void k_sort_scan_e(int32_t *__restrict__ cnt, int NB, int E,
                                                     int32_t *__restrict__ tot) {
    // one block per expert; sequential prefix in chunks of 256 with a block scan
    __shared__ int buf[256];
    const int e = blockIdx.x, t = threadIdx.x;
    int carry = 0;
    for (int b0 = 0; b0 < NB; b0 += 256) {
        const int b = b0 + t;
        const int v = b < NB ? cnt[(int64_t)b * E + e] : 0;
        buf[t] = v;
        __syncthreads();
        for (int o = 1; o < 256; o <<= 1) {
            const int x = t >= o ? buf[t - o] : 0;
            __syncthreads();
            buf[t] += x;
            __syncthreads();
        }
        if (b < NB) cnt[(int64_t)b * E + e] = carry + buf[t] - v;
        carry += buf[255];
        __syncthreads();
    }
    if (t == 0) tot[e] = carry;
}

__global__ __launch_bounds__(1024) void k_sort_off(const int32_t *__restrict__ tot, int E,
                                                   int64_t cap, int32_t *__restrict__ off,
                                                   int64_t *__restrict__ off64) {
    __shared__ int buf[1024];
    const int t = threadIdx.x;
    int carry = 0;
    if (t == 0) {
        off[0] = 0;
        if (off64) off64[0] = 0;
    }
    for (int e0 = 0; e0 < E; e0 += 1024) {
        const int e = e0 + t;
        const int v = e < E ? (int)min((int64_t)tot[e], cap) : 0;
        buf[t] = v;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int x = t >= o ? buf[t - o] : 0;
            __syncthreads();
            buf[t] += x;
            __syncthreads();
        }
        if (e < E) {
            off[e + 1] = carry + buf[t];
            if (off64) off64[e + 1] = carry + buf[t];
        }
        carry += buf[1023];
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_sort_scatter(
    const int32_t *__restrict__ ids, int Tk, int E, const int32_t *__restrict__ rank,
    const int32_t *__restrict__ cnt, const int32_t *__restrict__ off, int64_t cap,
    int32_t *__restrict__ perm, int64_t *__restrict__ perm64, uint8_t *__restrict__ drop) {
    const int q = blockIdx.x * SQ + threadIdx.x;
    if (q >= Tk) return;
    const int e = ids[q];
    if (e < 0 || e >= E) return;
    const int64_t g = (int64_t)cnt[(int64_t)blockIdx.x * E + e] + rank[q];
    const bool kept = g < cap;
    if (drop) drop[q] = kept ? 0 : 1;
    if (kept) {
        perm[off[e] + g] = q;
        if (perm64) perm64[off[e] + g] = q;
    }
}

extern "C" int jtk_sort_mid(const int32_t *ids, int Tk, int E, int64_t cap, int R,
                            int32_t *rank, int32_t *cnt, int32_t *off, int64_t *off64,
                            int32_t *perm, int64_t *perm64, uint8_t *drop, int32_t *tiles,
                            int32_t *ntiles, uint32_t *err, hipStream_t s);

extern "C" int jtk_sort(const int32_t *ids, int Tk, int E, int64_t cap, int32_t *rank,
                        int32_t *cnt, int32_t *tot, int32_t *off, int64_t *off64,
                        int32_t *perm, int64_t *perm64, uint8_t *drop, uint32_t *err,
                        hipStream_t s) {
    if (Tk > 0 && E <= 1024 && (Tk + SQ - 1) / SQ <= SORT_MID_NB)
        return jtk_sort_mid(ids, Tk, E, cap, 0, rank, cnt, off, off64, perm, perm64, drop, NULL,
                            NULL, err, s);
    const int NB = (Tk + SQ - 1) / SQ;
    hipLaunchKernelGGL(k_sort_hist, dim3((unsigned)NB), dim3(256), 0, s, ids, Tk, E, rank,
                       cnt, err);
    hipLaunchKernelGGL(k_sort_scan_e, dim3((unsigned)E), dim3(256), 0, s, cnt, NB, E, tot);
    hipLaunchKernelGGL(k_sort_off, dim3(1), dim3(1024), 0, s, tot, E, cap, off, off64);
    hipLaunchKernelGGL(k_sort_scatter, dim3((unsigned)NB), dim3(256), 0, s, ids, Tk, E, rank,
                       cnt, off, cap, perm, perm64, drop);
    return (int)hipGetLastError();
}

// ---------------- grouped-GEMM work list ----------------
__global__ __launch_bounds__(1024) void k_make_tiles(const int32_t *__restrict__ off, int E,
                                                     int R, int4 *__restrict__ tiles,
                                                     int32_t *__restrict__ ntiles) {
    __shared__ int buf[1024];
    const int t = threadIdx.x;
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 1024) {
        const int e = e0 + t;
        const int nt = e < E ? (off[e + 1] - off[e] + R - 1) / R : 0;
        buf[t] = nt;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int x = t >= o ? buf[t - o] : 0;
            __syncthreads();
            buf[t] += x;
            __syncthreads();
        }
        const int start = carry + buf[t] - nt;
        if (e < E) put_tiles(tiles, start, e, off[e], off[e + 1] - off[e], R);
        carry += buf[1023];
        __syncthreads();
    }
    if (t == 0) *ntiles = carry;
}

extern "C" int jtk_make_tiles(const int32_t *off, int E, int R, int32_t *tiles,
                              int32_t *ntiles, hipStream_t s) {
    hipLaunchKernelGGL(k_make_tiles, dim3(1), dim3(1024), 0, s, off, E, R, (int4 *)tiles,
                       ntiles);
    return (int)hipGetLastError();
}

// ---------------- small-batch sort + work list in one block ----------------
// The same stable counting sort (rank of pair q = number of earlier pairs
// with its expert; kept iff rank < cap) and the same R-row tile list, for
// Tk <= SORT_SMALL pairs: one workgroup, everything in LDS, one launch
// instead of five. Each of the 1024 threads owns one pair and 4 experts.
__global__ __launch_bounds__(1024) void k_sort_small(
    const int32_t *__restrict__ ids, int Tk, int E, int64_t cap, int R,
    int32_t *__restrict__ off, int64_t *__restrict__ off64, int32_t *__restrict__ perm,
    int64_t *__restrict__ perm64, uint8_t *__restrict__ drop, int32_t *__restrict__ tiles,
    int32_t *__restrict__ ntiles, uint32_t *err) {
    __shared__ __attribute__((aligned(16))) SortLds sm;
    const int t = threadIdx.x;
    int e = -1;
    if (t < Tk) {
        e = ids[t];
        if (e < 0 || e >= E) {
            raise_err(err, EF_BAD_ID);
            e = -1;
        }
    }
    if (Tk <= SORTF_TK && E <= SORTF_E)  // block-uniform
        sort_small_fast(e, Tk, E, cap, R, off, off64, perm, perm64, drop, tiles, ntiles, sm.fast);
    else
        sort_small_core(e, Tk, E, cap, R, off, off64, perm, perm64, drop, tiles, ntiles, sm.small);
}

extern "C" int jtk_sort_small(const int32_t *ids, int Tk, int E, int64_t cap, int R,
                              int32_t *off, int64_t *off64, int32_t *perm, int64_t *perm64,
                              uint8_t *drop, int32_t *tiles, int32_t *ntiles, uint32_t *err,
                              hipStream_t s) {
    if (Tk > SORT_SMALL || E > SORT_EMAX) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sort_small, dim3(1), dim3(1024), 0, s, ids, Tk, E, cap, R, off, off64,
                       perm, perm64, drop, tiles, ntiles, err);
    return (int)hipGetLastError();
}

// ------- caller-routed decode: token codes and the pair sort, one launch -------
// Blocks 0 .. gridDim.x-2 quantise the T token rows (16 per block, one
// wavefront per row, k_quant_rows's codes); the last block sorts the pairs
// as k_sort_small does. The two only share the launch: the sort reads the
// caller's ids, not the codes.
__global__ __launch_bounds__(1024) void k_quant_sort_small(
    const float *__restrict__ X, int T, int n, int8_t *__restrict__ Xq, float *__restrict__ sx,
    const int32_t *__restrict__ ids, int Tk, int E, int64_t cap, int R,
    int32_t *__restrict__ off, int64_t *__restrict__ off64, int32_t *__restrict__ perm,
    int64_t *__restrict__ perm64, uint8_t *__restrict__ drop, int32_t *__restrict__ tiles,
    int32_t *__restrict__ ntiles, uint32_t *err) {
    __shared__ __attribute__((aligned(16))) SortLds sm;
    if (blockIdx.x + 1 < gridDim.x) {
        const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 6);
        if (r < T) quant_row_wave(X, r, n, Xq, n, sx, err, threadIdx.x & 63);
        return;
    }
    const int t = threadIdx.x;
    int e = -1;
    if (t < Tk) {
        e = ids[t];
        if (e < 0 || e >= E) {
            raise_err(err, EF_BAD_ID);
            e = -1;
        }
    }
    if (Tk <= SORTF_TK && E <= SORTF_E)  // block-uniform
        sort_small_fast(e, Tk, E, cap, R, off, off64, perm, perm64, drop, tiles, ntiles, sm.fast);
    else
        sort_small_core(e, Tk, E, cap, R, off, off64, perm, perm64, drop, tiles, ntiles, sm.small);
}

extern "C" int jtk_quant_sort_small(const float *X, int T, int n, int8_t *Xq, float *sx,
                                    const int32_t *ids, int Tk, int E, int64_t cap, int R,
                                    int32_t *off, int64_t *off64, int32_t *perm,
                                    int64_t *perm64, uint8_t *drop, int32_t *tiles,
                                    int32_t *ntiles, uint32_t *err, hipStream_t s) {
    if (T <= 0 || n <= 0 || Tk > SORT_SMALL || E > SORT_EMAX || T > (1 << 24))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_quant_sort_small, dim3((unsigned)((T + 15) / 16 + 1)), dim3(1024), 0,
                       s, X, T, n, Xq, sx, ids, Tk, E, cap, R, off, off64, perm, perm64, drop,
                       tiles, ntiles, err);
    return (int)hipGetLastError();
}

// ---------------- medium-batch sort: two launches ----------------
// The same stable counting sort and tile list for E <= 1024 experts and up
// to SORT_MID_NB blocks of 256 pairs. Launch 1 (one block per 256 pairs):
// each wave finds the lanes holding its lane's expert with one ballot per
// expert-id bit, so a pair's rank is its rank in its wave plus the counts
// of its expert in the block's earlier waves; the block's per-expert
// counts go to cnt. Launch 2 (same blocks, 1024 threads): the per-expert
// sums over all blocks and over the earlier blocks (1024 / E threads per
// expert, each over a segment of the blocks), the scan of the kept counts
// into the expert offsets, and the placement of the block's own pairs;
// block 0 also writes off[] and the tile list. Replaces hist, per-expert
// scan, offsets, scatter and tile launches.
__global__ __launch_bounds__(256) void k_sort_mid_rank(const int32_t *__restrict__ ids, int Tk,
                                                       int E, int32_t *__restrict__ rank,
                                                       int32_t *__restrict__ cnt,
                                                       uint32_t *err) {
    __shared__ int wc[4][1024];  // per-wave counts of each expert
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, b = blockIdx.x;
    const int q = b * SQ + t;
    int e = -1;
    if (q < Tk) {
        e = ids[q];
        if (e < 0 || e >= E) {
            raise_err(err, EF_BAD_ID);
            e = -1;
        }
    }
    for (int i = t; i < 4 * E; i += 256) wc[i / E][i % E] = 0;
    __syncthreads();
    // lanes of this wave with expert e: agree on every bit of the id
    uint64_t m = __ballot(e >= 0);
    const int nbits = E > 1 ? 32 - __builtin_clz((unsigned)(E - 1)) : 1;
    for (int bit = 0; bit < nbits; bit++) {
        const bool one = (e >> bit) & 1;
        const uint64_t bm = __ballot(one);
        m &= one ? bm : ~bm;
    }
    const int rw = __popcll(m & ((1ull << lane) - 1ull));
    if (e >= 0 && rw == __popcll(m) - 1) wc[wave][e] = rw + 1;  // the group's last lane
    __syncthreads();
    if (e >= 0) {
        int r = rw;
        for (int w = 0; w < wave; w++) r += wc[w][e];
        rank[q] = r;
    }
    for (int x = t; x < E; x += 256)
        cnt[(int64_t)b * E + x] = wc[0][x] + wc[1][x] + wc[2][x] + wc[3][x];
}

__global__ __launch_bounds__(1024) void k_sort_mid_place(
    const int32_t *__restrict__ ids, int Tk, int E, int64_t cap, int NB,
    const int32_t *__restrict__ rank, const int32_t *__restrict__ cnt, int R,
    int32_t *__restrict__ off, int64_t *__restrict__ off64, int32_t *__restrict__ perm,
    int64_t *__restrict__ perm64, uint8_t *__restrict__ drop, int32_t *__restrict__ tiles,
    int32_t *__restrict__ ntiles) {
    __shared__ int eoff[1024], epre[1024], ps[1024], ts[1024], wsum[16];
    const int t = threadIdx.x, b = blockIdx.x;
    // thread (segment s, expert x) sums the blocks [s NB / seg, (s+1) NB / seg)
    const int seg = 1024 / E;
    const int x = t % E, sgi = t / E;
    if (sgi < seg) {
        int pre = 0, tot = 0;
        const int b0 = sgi * NB / seg, b1 = (sgi + 1) * NB / seg;
#pragma unroll 8
        for (int bb = b0; bb < b1; bb++) {
            const int c = cnt[(int64_t)bb * E + x];
            pre += bb < b ? c : 0;
            tot += c;
        }
        ps[t] = pre;
        ts[t] = tot;
    }
    __syncthreads();
    int pre = 0, tot = 0;  // pairs of expert t in earlier blocks, in all blocks
    if (t < E)
        for (int si = 0; si < seg; si++) {
            pre += ps[si * E + t];
            tot += ts[si * E + t];
        }
    const int kc = t < E ? (int)min((int64_t)tot, cap) : 0;
    int ktot;
    const int kbase = block_excl_scan_1024(kc, wsum, &ktot);
    if (t < E) {
        eoff[t] = kbase;
        epre[t] = pre;
    }
    if (b == 0) {
        if (t < E) {
            off[t] = kbase;
            if (off64) off64[t] = kbase;
        }
        if (t == 0) {
            off[E] = ktot;
            if (off64) off64[E] = ktot;
        }
        if (tiles) {
            const int nt = (kc + R - 1) / R;
            int ttot;
            const int tbase = block_excl_scan_1024(nt, wsum, &ttot);
            if (t < E) put_tiles((int4 *)tiles, tbase, t, kbase, kc, R);
            if (t == 0) *ntiles = ttot;
        }
    }
    __syncthreads();
    if (t >= SQ) return;
    const int q = b * SQ + t;
    if (q >= Tk) return;
    const int e = ids[q];
    if (e < 0 || e >= E) return;
    const int64_t g = (int64_t)epre[e] + rank[q];
    const bool kept = g < cap;
    if (drop) drop[q] = kept ? 0 : 1;
    if (kept) {
        perm[eoff[e] + g] = q;
        if (perm64) perm64[eoff[e] + g] = q;
    }
}

// Sort (and, with tiles != NULL, the R-row tile list) in two launches;
// returns hipErrorInvalidValue when E > 1024 or Tk > SORT_MID_NB * 256.
// cnt holds ceil(Tk / 256) * E ints.
extern "C" int jtk_sort_mid(const int32_t *ids, int Tk, int E, int64_t cap, int R,
                            int32_t *rank, int32_t *cnt, int32_t *off, int64_t *off64,
                            int32_t *perm, int64_t *perm64, uint8_t *drop, int32_t *tiles,
                            int32_t *ntiles, uint32_t *err, hipStream_t s) {
    const int NB = (Tk + SQ - 1) / SQ;
    if (Tk <= 0 || E <= 0 || E > 1024 || NB > SORT_MID_NB || (tiles && R <= 0))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sort_mid_rank, dim3((unsigned)NB), dim3(256), 0, s, ids, Tk, E, rank,
                       cnt, err);
    hipLaunchKernelGGL(k_sort_mid_place, dim3((unsigned)NB), dim3(1024), 0, s, ids, Tk, E, cap,
                       NB, rank, cnt, R, off, off64, perm, perm64, drop, tiles, ntiles);
    return (int)hipGetLastError();
}

// ---------------- combine ----------------
// One thread per 4 consecutive outputs of a token. drop may be NULL
// (dropless); dropped slots contribute nothing (src/moe_layer.c:1449-1451).
// With a residual R [T][n] (may alias Y: each thread reads its 4 values
// before it writes them) the output is the training loop's
// (float)((double)R + (double)(float)moe), rounded twice as there
// (bench/kernel/train_tinystories.c:1147-1160); a non-finite sum is an
// error there too.
__device__ __forceinline__ float res_add(const float *R, int64_t at, float y, bool &bad) {
    const double v = (double)R[at] + (double)y;
    bad |= !isfinite(v);
    return (float)v;
}
__device__ __forceinline__ void combine_store(float *Y, const float *R, int64_t at, double a0,
                                              double a1, double a2, double a3, uint32_t *err) {
    bool bad = !isfinite(a0) || !isfinite(a1) || !isfinite(a2) || !isfinite(a3);
    float4 o = make_float4((float)a0, (float)a1, (float)a2, (float)a3);
    if (R) {  // kernel-uniform
        const float4 r = *(const float4 *)(R + at);
        o = make_float4(res_add(&r.x, 0, o.x, bad), res_add(&r.y, 0, o.y, bad),
                        res_add(&r.z, 0, o.z, bad), res_add(&r.w, 0, o.w, bad));
    }
    if (bad) raise_err(err, EF_NONFINITE_MID);
    *(float4 *)(Y + at) = o;
}
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ w,
                                                 const float *__restrict__ Ye,
                                                 const uint8_t *__restrict__ drop,
                                                 const float *__restrict__ Ys, int S, int T,
                                                 int k, int n, const float *R, float *Y,
                                                 uint32_t *err) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nq = n / 4;
    if (idx >= (int64_t)T * nq) return;
    const int t = (int)(idx / nq), j = (int)(idx % nq) * 4;
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    for (int p = 0; p < k; p++) {
        const int64_t q = (int64_t)t * k + p;
        if (drop && drop[q]) continue;
        const double wp = (double)w[q];
        const float4 y = *(const float4 *)(Ye + q * n + j);
        a0 = fma(wp, (double)y.x, a0);
        a1 = fma(wp, (double)y.y, a1);
        a2 = fma(wp, (double)y.z, a2);
        a3 = fma(wp, (double)y.w, a3);
    }
    for (int s = 0; s < S; s++) {
        const float4 y = *(const float4 *)(Ys + ((int64_t)s * T + t) * n + j);
        a0 += (double)y.x;
        a1 += (double)y.y;
        a2 += (double)y.z;
        a3 += (double)y.w;
    }
    combine_store(Y, R, (int64_t)t * n + j, a0, a1, a2, a3, err);
}

// The same sum with the top-k K a compile-time constant: every load of a
// thread (its K expert rows, the K weights and drop flags, up to 8 shared
// rows) is issued before the first FMA, so a thread waits for memory once
// instead of once per slot (the runtime-k loop above issues one row, waits,
// adds, and only then loads the next). The sums run in the same order.
#define CMB_SMAX 8
// SN: shared rows loaded per thread, S itself when S <= 2, else CMB_SMAX
// (rows past S - 1 then repeat the last one and are not summed).
// The expert and shared rows are read once, so their loads are non-temporal
// (measured at 4096 tokens, d = 1024, top-8 and two shared rows: 32.3
// against 34.5 us for the plain loads, 185 MB a launch).
typedef float cmb_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 cmb_ld(const float *p) {
    const cmb_f4 v = __builtin_nontemporal_load((const cmb_f4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
template <int K, int SN, bool DROP>
__global__ __launch_bounds__(256) void k_combine_k(const float *__restrict__ w,
                                                   const float *__restrict__ Ye,
                                                   const uint8_t *__restrict__ drop,
                                                   const float *__restrict__ Ys, int S, int T,
                                                   int n, const float *R, float *Y,
                                                   uint32_t *err) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nq = n / 4;
    if (idx >= (int64_t)T * nq) return;
    const int t = (int)(idx / nq), j = (int)(idx % nq) * 4;
    const int64_t q0 = (int64_t)t * K;
    // all loads first, with no branch between them
    float wv[K];
    float4 yv[K];
    uint8_t dr[K];
#pragma unroll
    for (int p = 0; p < K; p++) {
        wv[p] = w[q0 + p];
        yv[p] = cmb_ld(Ye + (q0 + p) * n + j);
        if (DROP) dr[p] = drop[q0 + p];
    }
    float4 ys[SN > 0 ? SN : 1];
    if (S > 0) {  // kernel-uniform
#pragma unroll
        for (int s = 0; s < SN; s++)
            ys[s] = cmb_ld(Ys + ((int64_t)min(s, S - 1) * T + t) * n + j);
    }
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
#pragma unroll
    for (int p = 0; p < K; p++) {
        if (DROP && dr[p]) continue;
        const double wp = (double)wv[p];
        a0 = fma(wp, (double)yv[p].x, a0);
        a1 = fma(wp, (double)yv[p].y, a1);
        a2 = fma(wp, (double)yv[p].z, a2);
        a3 = fma(wp, (double)yv[p].w, a3);
    }
#pragma unroll
    for (int s = 0; s < SN; s++) {
        if (s >= S) break;
        a0 += (double)ys[s].x;
        a1 += (double)ys[s].y;
        a2 += (double)ys[s].z;
        a3 += (double)ys[s].w;
    }
    combine_store(Y, R, (int64_t)t * n + j, a0, a1, a2, a3, err);
}

// Scalar variant for n % 4 != 0 (legacy shapes).
__global__ __launch_bounds__(256) void k_combine1(const float *__restrict__ w,
                                                  const float *__restrict__ Ye,
                                                  const uint8_t *__restrict__ drop,
                                                  const float *__restrict__ Ys, int S, int T,
                                                  int k, int n, const float *R, float *Y,
                                                  uint32_t *err) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)T * n) return;
    const int t = (int)(idx / n), j = (int)(idx % n);
    double a = 0.0;
    for (int p = 0; p < k; p++) {
        const int64_t q = (int64_t)t * k + p;
        if (drop && drop[q]) continue;
        a = fma((double)w[q], (double)Ye[q * n + j], a);
    }
    for (int s = 0; s < S; s++) a += (double)Ys[((int64_t)s * T + t) * n + j];
    bool bad = !isfinite(a);
    float o = (float)a;
    if (R) o = res_add(R, idx, o, bad);
    if (bad) raise_err(err, EF_NONFINITE_MID);
    Y[idx] = o;
}

extern "C" int jtk_combine(const float *w, const float *Ye, const uint8_t *drop,
                           const float *Ys, int S, int T, int k, int n, const float *R, float *Y,
                           uint32_t *err, hipStream_t s) {
    if (n % 4 == 0) {
        const int64_t th = (int64_t)T * (n / 4);
        const dim3 grid((unsigned)((th + 255) / 256));
#define CMB_KS(KK, SN)                                                                     \
    if (drop)                                                                              \
        hipLaunchKernelGGL((k_combine_k<KK, SN, true>), grid, dim3(256), 0, s, w, Ye, drop, \
                           Ys, S, T, n, R, Y, err);                                        \
    else                                                                                   \
        hipLaunchKernelGGL((k_combine_k<KK, SN, false>), grid, dim3(256), 0, s, w, Ye,      \
                           drop, Ys, S, T, n, R, Y, err);
#define CMB_K(KK)                                                                          \
    case KK:                                                                               \
        if (S == 0) {                                                                      \
            CMB_KS(KK, 0)                                                                  \
        } else if (S == 1) {                                                               \
            CMB_KS(KK, 1)                                                                  \
        } else if (S == 2) {                                                               \
            CMB_KS(KK, 2)                                                                  \
        } else {                                                                           \
            CMB_KS(KK, CMB_SMAX)                                                           \
        }                                                                                  \
        break;
        if (S <= CMB_SMAX && k >= 1 && k <= 8) {
            switch (k) {
                CMB_K(1) CMB_K(2) CMB_K(3) CMB_K(4) CMB_K(5) CMB_K(6) CMB_K(7) CMB_K(8)
            }
        } else {
            hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, s, w, Ye, drop, Ys, S, T, k, n, R,
                               Y, err);
        }
#undef CMB_K
#undef CMB_KS
    } else {
        const int64_t th = (int64_t)T * n;
        hipLaunchKernelGGL(k_combine1, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, w,
                           Ye, drop, Ys, S, T, k, n, R, Y, err);
    }
    return (int)hipGetLastError();
}

// ---------------- helpers for the legacy layer ----------------
// Renormalise kept weights of tokens with drops (src/moe_layer.c:1171-1201).
__global__ __launch_bounds__(256) void k_renorm(float *__restrict__ w,
                                                const uint8_t *__restrict__ drop, int T,
                                                int k, uint32_t *err) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    double s = 0.0;
    int nd = 0;
    for (int p = 0; p < k; p++) {
        const int64_t q = (int64_t)t * k + p;
        if (drop[q]) nd++;
        else s += (double)w[q];
    }
    if (nd > 0 && s > 0.0) {
        if (!isfinite(s)) {
            raise_err(err, EF_NONFINITE_MID);
            return;
        }
        for (int p = 0; p < k; p++) {
            const int64_t q = (int64_t)t * k + p;
            if (drop[q]) continue;
            const double rw = (double)w[q] / s;
            if (!isfinite(rw) || rw < 0.0) raise_err(err, EF_NONFINITE_MID);
            w[q] = (float)rw;
        }
    }
}

extern "C" int jtk_renorm(float *w, const uint8_t *drop, int T, int k, uint32_t *err,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_renorm, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, s, w, drop,
                       T, k, err);
    return (int)hipGetLastError();
}

// dst[r][:] = src[idx(r)][:] with idx(r) = perm[base + r] / div (fp32 rows).
__global__ __launch_bounds__(256) void k_gather_rows(const float *__restrict__ src, int n,
                                                     const int32_t *__restrict__ perm,
                                                     int base, int div, int rows,
                                                     float *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * n) return;
    const int r = (int)(i / n), c = (int)(i % n);
    const int sr = perm[base + r] / div;
    dst[i] = src[(int64_t)sr * n + c];
}

// dst[perm[base + r]][:] = src[r][:].
__global__ __launch_bounds__(256) void k_scatter_rows(const float *__restrict__ src, int n,
                                                      const int32_t *__restrict__ perm,
                                                      int base, int rows,
                                                      float *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * n) return;
    const int r = (int)(i / n), c = (int)(i % n);
    dst[(int64_t)perm[base + r] * n + c] = src[i];
}

extern "C" int jtk_gather_rows(const float *src, int n, const int32_t *perm, int base,
                               int div, int rows, float *dst, hipStream_t s) {
    const int64_t th = (int64_t)rows * n;
    if (th <= 0) return 0;
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, src,
                       n, perm, base, div, rows, dst);
    return (int)hipGetLastError();
}

extern "C" int jtk_scatter_rows(const float *src, int n, const int32_t *perm, int base,
                                int rows, float *dst, hipStream_t s) {
    const int64_t th = (int64_t)rows * n;
    if (th <= 0) return 0;
    hipLaunchKernelGGL(k_scatter_rows, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s,
                       src, n, perm, base, rows, dst);
    return (int)hipGetLastError();
}

// Elementwise SwiGLU of two fp32 tiles (src/moe_layer.c:129-157).
__global__ __launch_bounds__(256) void k_silu_tile(const float *__restrict__ G,
                                                   const float *__restrict__ U, int64_t n,
                                                   float *__restrict__ S, uint32_t *err) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s;
    if (!silu_mul(G[i], U[i], &s)) raise_err(err, EF_NONFINITE_MID);
    S[i] = s;
}

extern "C" int jtk_silu_tile(const float *G, const float *U, int64_t n, float *S,
                             uint32_t *err, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_silu_tile, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, G, U,
                       n, S, err);
    return (int)hipGetLastError();
}

// Fill with zero (graph-safe replacement for a memset).
__global__ __launch_bounds__(256) void k_zero_u32(uint32_t *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

extern "C" int jtk_zero_u32(uint32_t *p, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return (int)hipGetLastError();
}

// dst[i] = *src for i < n (a device scalar broadcast, e.g. one per-tensor
// scale repeated per row).
__global__ __launch_bounds__(256) void k_bcast_f32(float *__restrict__ dst, int64_t n,
                                                   const float *__restrict__ src) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = *src;
}

extern "C" int jtk_bcast_f32(float *dst, int64_t n, const float *src, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_bcast_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, n,
                       src);
    return (int)hipGetLastError();
}

// Load this file's code object now: the runtime otherwise loads it, and
// allocates device memory for it, at the first launch of one of its kernels.
extern "C" int jtk_preload_route(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_topk));
}
