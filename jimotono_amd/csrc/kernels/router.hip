// Fast router for gfx950: int8 MFMA candidates, exact fp64 verification.
//
// The reference's gate logit is l = (float)dot(x, w) summed in fp64 in its
// AVX2 lane order (src/moe_layer.c:67-86) and top-k selects by (value desc,
// index asc) (src/routing.c:39-74). Computing all T x E logits that way is
// fp64 vector work. This path computes an approximation with a proven
// error bound on the int8 matrix cores and evaluates the reference's exact
// sum only for the experts the bound cannot rule out:
//
//  1. k_router_codes: each row r (tokens, and the expert rows of Wgate at
//     prepare) is written as x = s*(qh + ql/254) + eps with the row
//     quantiser's scale s = max|x|/127, qh = round(x/s) (the very codes the
//     experts consume), ql = round((x - s*qh)*254/s), |eps| <= s/508; also
//     l1 = sum|x|.
//  2. k_router_approx: a = s_x s_w (HH + (HL + LH)/254 + LL/254^2) from four
//     exact int32 MFMA sums. |dot - a| <= m with
//     m = (s_w/508) l1_x + (s_x/508) l1_w + 3n (s_x/508)(s_w/508)
//     (plus slack for the fp64 evaluation of a and of the reference sum).
//  3. k_router_select (one wave per token): L = a - m, U = a + m; thr <=
//     the k-th largest L; candidates are the experts with U >= thr - delta,
//     delta = 2^-22 |thr| (so a non-candidate's float logit is strictly
//     below k candidates' float logits).
//  4. k_router_exact (one lane per token and candidate): the reference's
//     exact lane-order fp64 sum for each candidate; top-k and softmax then
//     run on those exact float logits exactly as the reference does. Every
//     expert outside the candidate set is provably outside the reference's
//     top-k.
// logits[t][e] holds the exact float logit for candidates and the float of
// the approximation for the others.
#include <atomic>

#include "gemm_w8a8.h"
#include "jt_launch.h"

// ---- 1. codes of a row ----
// One wavefront per row; blockDim = 256 (4 rows). qh/sf follow the row
// quantiser (k_quant_rows) bit for bit; info = {s (fp64), l1}. The residual
// code rounds (x - s qh) * (254 / s) to nearest: |x - s (qh + ql/254)| <=
// s/508 up to the fp64 rounding of the product, which the bound's slack
// covers. Rows of up to 64 * 4 * RC float4 registers (n % 4 == 0) are read
// once into registers with all loads in flight: RC = 4 up to n = 1024 (52
// registers, 16.4 -> 15.0 us for 4096 rows of 1024 against RC = 16), else 16.

__device__ __forceinline__ uint32_t router_lo_code(float v, int q, double sd, double inv_lo) {
    double t = rint(((double)v - sd * (double)q) * inv_lo);
    t = t > 127.0 ? 127.0 : (t < -127.0 ? -127.0 : t);
    return (uint32_t)(uint8_t)(int8_t)(int)t;
}

// The codes of one row held whole in registers (n % 4 == 0, n <= 256 RC,
// x 16-byte aligned), by one wavefront: put(c, hi, lo) receives the 4 codes
// of float4 c as two words. On success *info = {s, l1} and *scale =
// (float)s (all lanes); false (error raised) for a row the quantiser
// rejects, whose codes are then not put.
template <int RC, typename Put>
__device__ __forceinline__ bool router_row_regs(const float *__restrict__ x, int n, int lane,
                                                uint32_t *err, double2 *info, float *scale,
                                                Put put) {
    const float4 *x4 = (const float4 *)x;
    const int n4 = n >> 2;
    float4 v[RC];
    float m = 0.0f;
    double l1 = 0.0;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < RC; i++) {
        const int c = lane + 64 * i;
        v[i] = c < n4 ? x4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < RC; i++) {
        if (64 * i < n4) {  // wave-uniform; constant indices keep v[] in registers
            bad |= (!isfinite(v[i].x)) || (!isfinite(v[i].y)) || (!isfinite(v[i].z)) ||
                   (!isfinite(v[i].w));
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)),
                               fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
            l1 += (fabs((double)v[i].x) + fabs((double)v[i].y)) +
                  (fabs((double)v[i].z) + fabs((double)v[i].w));
        }
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l1 += __shfl_xor(l1, o, 64);
    const QuantParams p = quant_params(m);
    if (bad || !p.ok) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return false;
    }
    *info = make_double2(p.scale_d, l1);
    *scale = p.scale_f;
    const float inv = quant_inv_f(p.scale_d);
    const double inv_lo = p.scale_d != 0.0 ? 254.0 / p.scale_d : 0.0;
    uint32_t fmask = 0;  // bit i: a code of v[i] needs the exact quotient
#pragma unroll
    for (int i = 0; i < RC; i++) {
        const int c = lane + 64 * i;
        if (64 * i < n4 && c < n4) {
            bool f = false;
            const int q0 = quant_code_try(v[i].x, inv, f);
            const int q1 = quant_code_try(v[i].y, inv, f);
            const int q2 = quant_code_try(v[i].z, inv, f);
            const int q3 = quant_code_try(v[i].w, inv, f);
            fmask |= (uint32_t)f << i;
            put(c,
                (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) |
                    ((uint32_t)(uint8_t)q2 << 16) | ((uint32_t)(uint8_t)q3 << 24),
                router_lo_code(v[i].x, q0, p.scale_d, inv_lo) |
                    (router_lo_code(v[i].y, q1, p.scale_d, inv_lo) << 8) |
                    (router_lo_code(v[i].z, q2, p.scale_d, inv_lo) << 16) |
                    (router_lo_code(v[i].w, q3, p.scale_d, inv_lo) << 24));
        }
    }
    // rare: put those words again, exactly, picking v[j] out of the
    // registers with selects (a dynamic index would spill v[] to scratch)
    while (fmask) {
        const int j = __builtin_ctz(fmask);
        fmask &= fmask - 1;
        float4 u = v[0];
#pragma unroll
        for (int i = 1; i < RC; i++)
            if (i == j) u = v[i];
        const int q0 = quant_code(u.x, p.scale_d);
        const int q1 = quant_code(u.y, p.scale_d);
        const int q2 = quant_code(u.z, p.scale_d);
        const int q3 = quant_code(u.w, p.scale_d);
        put(lane + 64 * j,
            (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) | ((uint32_t)(uint8_t)q2 << 16) |
                ((uint32_t)(uint8_t)q3 << 24),
            router_lo_code(u.x, q0, p.scale_d, inv_lo) |
                (router_lo_code(u.y, q1, p.scale_d, inv_lo) << 8) |
                (router_lo_code(u.z, q2, p.scale_d, inv_lo) << 16) |
                (router_lo_code(u.w, q3, p.scale_d, inv_lo) << 24));
    }
    return true;
}

template <int RC_REG>
__global__ __launch_bounds__(256) void k_router_codes(const float *__restrict__ X, int rows,
                                                      int n, int8_t *__restrict__ qh,
                                                      int8_t *__restrict__ ql,
                                                      float *__restrict__ sf,
                                                      double2 *__restrict__ info,
                                                      uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float *x = X + (int64_t)r * n;
    float m = 0.0f;
    double l1 = 0.0;
    int bad = 0;
    const bool vec = (n & 3) == 0 && ((uintptr_t)x & 15) == 0 &&
                     (((uintptr_t)qh | (uintptr_t)ql) & 3) == 0;
    if (vec && n <= 64 * 4 * RC_REG) {
        uint32_t *qh4 = (uint32_t *)(qh + (int64_t)r * n);
        uint32_t *ql4 = (uint32_t *)(ql + (int64_t)r * n);
        double2 inf;
        float scl;
        if (router_row_regs<RC_REG>(x, n, lane, err, &inf, &scl,
                                    [&](int c, uint32_t h, uint32_t l) {
                                        qh4[c] = h;
                                        ql4[c] = l;
                                    }) &&
            lane == 0) {
            if (sf) sf[r] = scl;
            info[r] = inf;
        }
        return;
    }
    for (int c = lane; c < n; c += 64) {
        const float v = x[c];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
        l1 += fabs((double)v);
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l1 += __shfl_xor(l1, o, 64);
    const QuantParams p = quant_params(m);
    if (bad || !p.ok) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    if (lane == 0) {
        if (sf) sf[r] = p.scale_f;
        info[r] = make_double2(p.scale_d, l1);
    }
    const float inv = quant_inv_f(p.scale_d);
    const double inv_lo = p.scale_d != 0.0 ? 254.0 / p.scale_d : 0.0;
    for (int c = lane; c < n; c += 64) {
        const float v = x[c];
        const int q = quant_code_fast(v, p.scale_d, inv);
        qh[(int64_t)r * n + c] = (int8_t)q;
        ql[(int64_t)r * n + c] = (int8_t)router_lo_code(v, q, p.scale_d, inv_lo);
    }
}

extern "C" int jtk_router_codes(const float *X, int rows, int n, int8_t *qh, int8_t *ql,
                                float *sf, double *info, uint32_t *err, hipStream_t s) {
    if (rows <= 0) return 0;
    if (n <= 64 * 4 * 4)
        hipLaunchKernelGGL(k_router_codes<4>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                           X, rows, n, qh, ql, sf, (double2 *)info, err);
    else
        hipLaunchKernelGGL(k_router_codes<16>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                           X, rows, n, qh, ql, sf, (double2 *)info, err);
    return (int)hipGetLastError();
}

// ---- 2. approximate logits ----
// Block = 64 tokens x 64 experts, 8 waves: 4 waves of 16 tokens times 2
// k-groups (group g takes the k-blocks of parity g, one per step). Per step
// each wave copies by DMA, into an RA_NST-step LDS ring, its own 16 token
// rows' hi and lo fragments and one of the group's 4 expert panel pairs
// (hi and lo codes); the group's 4 token waves then read the 4 panel pairs
// there. Only LDS-DMA copies are in flight in the loop, so each wait covers
// exactly the stage it needs. Per step a wave runs 16 MFMAs into three
// int32 sums per 16x16 tile; group 1's sums are added to group 0's through
// LDS (exact), so the result does not depend on how K was split.
#define RA_NST 3
// per step slot and group: A hi of waves 0-3, A lo of waves 0-3, B hi of
// panels 0-3, B lo of panels 0-3, each 64 lanes x 16 B
#define RA_LDS (RA_NST * 2 * 16 * 1024)
static_assert(RA_LDS >= 4 * 3 * 4 * 64 * 16, "the sums fit the ring");
__global__ __launch_bounds__(512) void k_router_approx(
    const int8_t *__restrict__ Xh, const int8_t *__restrict__ Xl, int n,
    const double2 *__restrict__ xinfo, const int8_t *__restrict__ Wh,
    const int8_t *__restrict__ Wl, const double2 *__restrict__ winfo, int T, int E,
    double *__restrict__ approx) {
    // [step slot][group][16 fragments][64 lanes x 16 B] (RA_LDS bytes of
    // dynamic LDS); after the k-loop the same bytes hold group 1's sums
    // [token wave][hh|mid|ll][j]
    extern __shared__ __attribute__((aligned(1024))) int8_t ra_lds[];
    int8_t(*ring)[2][16][1024] = (int8_t(*)[2][16][1024])ra_lds;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: MFMA guards branch
    const int wave = wv & 3, kg = wv >> 2;
    const int t0 = blockIdx.x * 64 + wave * 16, e0 = blockIdx.y * 64;
    const int KB = n / 64;
    const int NS = (KB + 1) / 2;  // steps of both groups (group 1 idles in an odd KB's last)
    const int r = lane & 15, kc = lane >> 4;
    const int64_t arow = (int64_t)min(t0 + r, T - 1) * n + kc * 16;
    const int pb = e0 / 16;
    // this wave's panel pair: panel pb + wave of the group's k-block
    const int8_t *bh_src = Wh + (int64_t)(pb + wave) * KB * 1024 + lane * 16;
    const int8_t *bl_src = Wl + (int64_t)(pb + wave) * KB * 1024 + lane * 16;
    auto kb_of = [&](int st) { return min(2 * st + kg, KB - 1); };  // clamped: in bounds
    auto issue = [&](int st) {
        const int kb = kb_of(st);
        int8_t(*slot)[1024] = ring[st % RA_NST][kg];
        dma<16>(Xh + arow + kb * 64, slot[wave]);
        dma<16>(Xl + arow + kb * 64, slot[4 + wave]);
        dma<16>(bh_src + (int64_t)kb * 1024, slot[8 + wave]);
        dma<16>(bl_src + (int64_t)kb * 1024, slot[12 + wave]);
    };
    // HL and LH share their scale, so one int32 sum holds both (|sum| <
    // 2 n 127^2 < 2^31 for n <= 4096)
    v4i hh[4], mid[4], ll[4];
#pragma unroll
    for (int j = 0; j < 4; j++) hh[j] = mid[j] = ll[j] = (v4i){0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < RA_NST - 1; st++)
        if (st < NS) issue(st);
    for (int st = 0; st < NS; st++) {
        wait_stage<4>(min(RA_NST - 2, NS - 1 - st));  // this wave's copies of stage st
        barrier_lds();  // ... and every other wave's; slot st - 1 is free
        if (st + RA_NST - 1 < NS) issue(st + RA_NST - 1);
        if (2 * st + kg < KB) {  // wave-uniform
            const int8_t(*slot)[1024] = ring[st % RA_NST][kg];
            const v4i ah = *(const v4i *)(slot[wave] + lane * 16);
            const v4i al = *(const v4i *)(slot[4 + wave] + lane * 16);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v4i bh = *(const v4i *)(slot[8 + j] + lane * 16);
                const v4i bl = *(const v4i *)(slot[12 + j] + lane * 16);
                hh[j] = mfma16x16x64(ah, bh, hh[j]);
                mid[j] = mfma16x16x64(ah, bl, mid[j]);
                mid[j] = mfma16x16x64(al, bh, mid[j]);
                ll[j] = mfma16x16x64(al, bl, ll[j]);
            }
        }
    }
    v4i(*part)[3][4][64] = (v4i(*)[3][4][64])ra_lds;
    barrier_lds();  // every wave is done with the ring
    if (kg == 1) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            part[wave][0][j][lane] = hh[j];
            part[wave][1][j][lane] = mid[j];
            part[wave][2][j][lane] = ll[j];
        }
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        hh[j] += part[wave][0][j][lane];
        mid[j] += part[wave][1][j][lane];
        ll[j] += part[wave][2][j][lane];
    }
    const int lr = (lane >> 4) * 4, lc = lane & 15;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = e0 + j * 16 + lc;
        if (e >= E) continue;
        const double sw = winfo[e].x;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int t = t0 + lr + q;
            if (t >= T) continue;
            const double v =
                (double)hh[j][q] + (double)mid[j][q] / 254.0 + (double)ll[j][q] / 64516.0;
            approx[(int64_t)t * E + e] = xinfo[t].x * sw * v;
        }
    }
}

// Few tokens (decode): block = 16 tokens x 16 experts, RA_W waves splitting
// the k-blocks (wave w takes kb = w, w + RA_W, ...; all its loads of a batch
// of 4 issued at once), int32 partial sums added in LDS (exact) by wave 0.
// Many small blocks instead of a few long ones: the latency of one k-block
// chain is what bounds a decode-sized call.
#define RA_W 8
__global__ __launch_bounds__(64 * RA_W) void k_router_approx_small(
    const int8_t *__restrict__ Xh, const int8_t *__restrict__ Xl, int n,
    const double2 *__restrict__ xinfo, const int8_t *__restrict__ Wh,
    const int8_t *__restrict__ Wl, const double2 *__restrict__ winfo, int T, int E,
    double *__restrict__ approx) {
    __shared__ v4i part[RA_W][3][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: MFMA guards branch
    const int t0 = blockIdx.x * 16, pan = blockIdx.y;
    const int KB = n / 64;
    const int r = lane & 15, kc = lane >> 4;
    const int64_t arow = (int64_t)min(t0 + r, T - 1) * n + kc * 16;
    v4i hh = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, ll = {0, 0, 0, 0};
    for (int kb0 = wave; kb0 < KB; kb0 += 4 * RA_W) {
        v4i ah[4], al[4], bh[4], bl[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int kb = kb0 + u * RA_W;
            if (kb < KB) {
                ah[u] = *(const v4i *)(Xh + arow + kb * 64);
                al[u] = *(const v4i *)(Xl + arow + kb * 64);
                const int64_t po = ((int64_t)pan * KB + kb) * 1024 + lane * 16;
                bh[u] = *(const v4i *)(Wh + po);
                bl[u] = *(const v4i *)(Wl + po);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (kb0 + u * RA_W < KB) {
                hh = mfma16x16x64(ah[u], bh[u], hh);
                mid = mfma16x16x64(ah[u], bl[u], mid);
                mid = mfma16x16x64(al[u], bh[u], mid);
                ll = mfma16x16x64(al[u], bl[u], ll);
            }
        }
    }
    part[wave][0][lane] = hh;
    part[wave][1][lane] = mid;
    part[wave][2][lane] = ll;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < RA_W; w++) {
        hh += part[w][0][lane];
        mid += part[w][1][lane];
        ll += part[w][2][lane];
    }
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    const int e = pan * 16 + lc;
    if (e >= E) return;
    const double sw = winfo[e].x;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int t = t0 + lr + q;
        if (t >= T) continue;
        const double v = (double)hh[q] + (double)mid[q] / 254.0 + (double)ll[q] / 64516.0;
        approx[(int64_t)t * E + e] = xinfo[t].x * sw * v;
    }
}

extern "C" int jtk_router_approx(const int8_t *Xh, const int8_t *Xl, int n, const double *xinfo,
                                 const int8_t *Wh, const int8_t *Wl, const double *winfo, int T,
                                 int E, double *approx, hipStream_t s) {
    if (T <= 0) return 0;
    if (T <= 256) {
        dim3 g((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16));
        hipLaunchKernelGGL(k_router_approx_small, g, dim3(64 * RA_W), 0, s, Xh, Xl, n,
                           (const double2 *)xinfo, Wh, Wl, (const double2 *)winfo, T, E,
                           approx);
        return (int)hipGetLastError();
    }
    // dynamic LDS above 64 KiB must be enabled per device, once
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)k_router_approx,
                                hipFuncAttributeMaxDynamicSharedMemorySize, RA_LDS);
        if (e != hipSuccess) return (int)e;
        attr_set[dev] = true;
    }
    dim3 grid((unsigned)((T + 63) / 64), (unsigned)((E + 63) / 64));
    hipLaunchKernelGGL(k_router_approx, grid, dim3(512), RA_LDS, s, Xh, Xl, n,
                       (const double2 *)xinfo, Wh, Wl, (const double2 *)winfo, T, E, approx);
    return (int)hipGetLastError();
}

// ---- 3. candidates ----
#define RV_EMAX 512    // experts per token: RV_EMAX / 64 per lane
#define RV_WPB 4       // waves (tokens) per block
#define RV_KEYBITS 24  // leading key bits resolved by the threshold select

// order-preserving map of a float to an unsigned 32-bit key
__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unkey(uint32_t k) {
    return __builtin_bit_cast(float, (k >> 31) ? (k & 0x7fffffffu) : ~k);
}
// largest float <= d
__device__ __forceinline__ float float_rd(double d) {
    float f = (float)d;
    if ((double)f > d) f = nextafterf(f, -__builtin_inff());
    return f;
}

// One wavefront per token: bounds L = a - m, U = a + m, thr <= the k-th
// largest L, candidates = {U >= thr - delta} in ascending expert order into
// cand[t][0..nc), nc into ncand[t]; the others' logits get the float of a.
//
// thr: each lane keeps the largest of its RV_EMAX / 64 lower bounds (as
// floats rounded down); the k-th largest of those 64 lane maxima is a
// subset's k-th largest, hence <= the k-th largest L. It is found as the
// largest RV_KEYBITS-bit key prefix with at least k lane maxima at or above
// it, one wave ballot per bit (k <= min(E, 64) lanes hold a bound).
// The candidates of token t into cand[0..nc) (ascending expert order) and
// the float of the approximation into the logits of the others; returns nc
// (wave-uniform). Called by one whole wavefront.
// select_token on one row: ap = the token's E approximate logits (global
// memory or LDS), {sx, l1x} its row info, cand / lg its rows of the candidate
// list and of the logits.
__device__ __forceinline__ int select_row(const double *ap_row, double sx, double l1x,
                                          const double2 *__restrict__ winfo, int E, int n,
                                          int k, int lane, int16_t *cand, float *lg) {
    constexpr int EPL = RV_EMAX / 64;
    const double ux = sx * (1.0 / 508.0);
    double ap[EPL], hi[EPL];
    uint32_t kmax = 0;  // below every real key
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        ap[j] = 0.0;
        hi[j] = -__builtin_inf();
        if (e < E) {
            const double a = ap_row[e];
            const double sw = winfo[e].x, l1w = winfo[e].y;
            const double uw = sw * (1.0 / 508.0);
            double m = uw * l1x + ux * l1w + 3.0 * n * ux * uw;
            m = m * (1.0 + 1e-9) + 1e-9 * sx * sw * n * 16641.0 + 1e-12 * l1x * 128.0 * sw;
            ap[j] = a;
            hi[j] = a + m;
            kmax = max(kmax, okey(float_rd(a - m)));
        }
    }
    uint32_t kappa = 0;
    for (int bit = 31; bit >= 32 - RV_KEYBITS; bit--) {
        const uint32_t trial = kappa | (1u << bit);
        if (__popcll(__ballot(kmax >= trial)) >= k) kappa = trial;
    }
    const double thr = (double)unkey(kappa);
    // a prefix of the key of -inf decodes to a NaN: every expert is then a
    // candidate
    const double cut = thr == thr ? thr - (fabs(thr) * 0x1p-22 + 1e-300) : -__builtin_inf();
    int nc = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        const bool c = e < E && hi[j] >= cut;
        const uint64_t mask = __ballot(c);
        if (c) cand[nc + __popcll(mask & ((1ull << lane) - 1ull))] = (int16_t)e;
        else if (e < E) lg[e] = (float)ap[j];
        nc += __popcll(mask);
    }
    return nc;
}
__device__ __forceinline__ int select_token(const double *__restrict__ approx,
                                            const double2 *__restrict__ xinfo,
                                            const double2 *__restrict__ winfo, int t, int E,
                                            int n, int k, int lane, int16_t *cand,
                                            float *__restrict__ logits) {
    return select_row(approx + (int64_t)t * E, xinfo[t].x, xinfo[t].y, winfo, E, n, k, lane,
                      cand, logits + (int64_t)t * E);
}

__global__ __launch_bounds__(64 * RV_WPB) void k_router_select(
    const double *__restrict__ approx, const double2 *__restrict__ xinfo,
    const double2 *__restrict__ winfo, int T, int E, int n, int k,
    int16_t *__restrict__ cand, int32_t *__restrict__ ncand, float *__restrict__ logits) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * RV_WPB + (threadIdx.x >> 6);
    if (t >= T) return;
    const int nc =
        select_token(approx, xinfo, winfo, t, E, n, k, lane, cand + (int64_t)t * E, logits);
    if (lane == 0) ncand[t] = nc;
}

// ---- 1-3 in one launch: codes, approximate logits and candidates ----
// Block = RF_TOK = 16 tokens x every expert (E <= 256, E % 16 == 0, n = 64 KB
// with KB <= 16), 16 waves. Wave w writes the codes of token row w as
// k_router_codes does (qh, the row scale and {s, l1}; the residual codes ql
// stay in LDS), the block's hi and lo code rows go to LDS (row stride n + 16
// bytes: the 16 rows of an MFMA fragment hit distinct banks), and wave w
// then runs k_router_approx's four int32 products for expert panel w
// against all 16 tokens, the panel's codes read straight into registers
// four k-blocks ahead (the 2 x 256 KB of expert codes stay in L2). The
// approximate logits, formed as k_router_approx forms them, go to LDS, and
// wave w runs k_router_select's candidate selection for token w from there.
// Outputs are those of the three launches it replaces, except that the
// residual codes and the approximate logits never reach memory.
#define RF_TOK 16
template <int KB>
__global__ __launch_bounds__(64 * RF_TOK) void k_router_front(
    const float *__restrict__ X, int T, int8_t *__restrict__ qh, float *__restrict__ sf,
    double2 *__restrict__ xinfo, const int8_t *__restrict__ Wh, const int8_t *__restrict__ Wl,
    const double2 *__restrict__ winfo, int E, int k, int16_t *__restrict__ cand,
    int32_t *__restrict__ ncand, float *__restrict__ logits, uint32_t *err) {
    constexpr int n = 64 * KB, AS = n + 16;
    extern __shared__ __attribute__((aligned(16))) int8_t rf_smem[];
    int8_t *ah_s = rf_smem;                               // [16][AS]
    int8_t *al_s = rf_smem + RF_TOK * AS;                 // [16][AS]
    double *ap_s = (double *)(rf_smem + 2 * RF_TOK * AS);  // [16][E]
    __shared__ double2 xi_s[RF_TOK];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: MFMA guards branch
    const int t0 = blockIdx.x * RF_TOK;
    // ---- codes of token row `wave` ----
    {
        const int tl = wave, t = t0 + tl;
        uint32_t *hs = (uint32_t *)(ah_s + tl * AS), *ls = (uint32_t *)(al_s + tl * AS);
        double2 inf = make_double2(0.0, 0.0);
        float scl = 0.0f;
        bool ok = false;
        if (t < T) {
            uint32_t *qg = (uint32_t *)(qh + (int64_t)t * n);
            ok = router_row_regs<(KB + 3) / 4>(X + (int64_t)t * n, n, lane, err, &inf, &scl,
                                               [&](int c, uint32_t h, uint32_t l) {
                                                   qg[c] = h;
                                                   hs[c] = h;
                                                   ls[c] = l;
                                               });
        }
        if (!ok) {  // a rejected row (error raised) or past T: zero codes
            for (int c = lane; c < n / 4; c += 64) hs[c] = ls[c] = 0u;
            inf = make_double2(0.0, 0.0);
        }
        if (lane == 0) {
            xi_s[tl] = inf;
            if (ok) {
                xinfo[t] = inf;
                if (sf) sf[t] = scl;
            }
        }
    }
    __syncthreads();
    // ---- approximate logits of expert panel `wave` ----
    const int lr = (lane >> 4) * 4, lc = lane & 15;
    if (16 * wave < E) {  // wave-uniform
        const int r = lane & 15, kc = lane >> 4;
        const int8_t *bh = Wh + (int64_t)wave * KB * 1024 + lane * 16;
        const int8_t *bl = Wl + (int64_t)wave * KB * 1024 + lane * 16;
        v4i hh = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, ll = {0, 0, 0, 0};
        constexpr int D = KB < 4 ? KB : 4;  // k-blocks of expert codes in flight
        v4i b[D][2];                        // [slot][hi, lo]
#pragma unroll
        for (int d = 0; d < D; d++) {
            b[d][0] = *(const v4i *)(bh + (int64_t)d * 1024);
            b[d][1] = *(const v4i *)(bl + (int64_t)d * 1024);
        }
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const v4i a_h = *(const v4i *)(ah_s + r * AS + kb * 64 + kc * 16);
            const v4i a_l = *(const v4i *)(al_s + r * AS + kb * 64 + kc * 16);
            v4i(&c)[2] = b[kb % D];
            hh = mfma16x16x64(a_h, c[0], hh);
            mid = mfma16x16x64(a_h, c[1], mid);
            mid = mfma16x16x64(a_l, c[0], mid);
            ll = mfma16x16x64(a_l, c[1], ll);
            if (kb + D < KB) {
                c[0] = *(const v4i *)(bh + (int64_t)(kb + D) * 1024);
                c[1] = *(const v4i *)(bl + (int64_t)(kb + D) * 1024);
            }
        }
        const int e = 16 * wave + lc;
        const double sw = winfo[e].x;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int tl = lr + q;
            const double v =
                (double)hh[q] + (double)mid[q] / 254.0 + (double)ll[q] / 64516.0;
            ap_s[tl * E + e] = xi_s[tl].x * sw * v;
        }
    }
    __syncthreads();
    // ---- candidates of token `wave` ----
    const int t = t0 + wave;
    if (t < T) {  // wave-uniform
        const int nc = select_row(ap_s + wave * E, xi_s[wave].x, xi_s[wave].y, winfo, E,
                                  64 * KB, k, lane, cand + (int64_t)t * E,
                                  logits + (int64_t)t * E);
        if (lane == 0) ncand[t] = nc;
    }
}

template <int KB>
static hipError_t launch_router_front(const float *X, int T, int8_t *qh, float *sf,
                                      double *xinfo, const int8_t *Wh, const int8_t *Wl,
                                      const double *winfo, int E, int k, int16_t *cand,
                                      int32_t *ncand, float *logits, uint32_t *err,
                                      hipStream_t s) {
    auto kern = k_router_front<KB>;
    const int lds = 2 * RF_TOK * (64 * KB + 16) + RF_TOK * E * 8;
    // dynamic LDS above 64 KiB must be enabled per device, once
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                2 * RF_TOK * (64 * KB + 16) + RF_TOK * 256 * 8);
        if (e != hipSuccess) return e;
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)((T + RF_TOK - 1) / RF_TOK)), dim3(64 * RF_TOK), lds, s,
                       X, T,
                       qh, sf, (double2 *)xinfo, Wh, Wl, (const double2 *)winfo, E, k, cand,
                       ncand, logits, err);
    return hipGetLastError();
}

extern "C" int jtk_router_front(const float *X, int T, int n, int8_t *qh, float *sf,
                                double *xinfo, const int8_t *Wh, const int8_t *Wl,
                                const double *winfo, int E, int k, int16_t *cand, int32_t *ncand,
                                float *logits, uint32_t *err, hipStream_t s) {
    if (T <= 0 || E <= 0 || E > 256 || E % 16 || k < 1 || k > E || ((uintptr_t)X & 15) ||
        ((uintptr_t)qh & 3))
        return (int)hipErrorInvalidValue;
    switch (n) {
        case 1024:
            return (int)launch_router_front<16>(X, T, qh, sf, xinfo, Wh, Wl, winfo, E, k, cand,
                                                ncand, logits, err, s);
        case 512:
            return (int)launch_router_front<8>(X, T, qh, sf, xinfo, Wh, Wl, winfo, E, k, cand,
                                               ncand, logits, err, s);
        case 256:
            return (int)launch_router_front<4>(X, T, qh, sf, xinfo, Wh, Wl, winfo, E, k, cand,
                                               ncand, logits, err, s);
        default:
            return (int)hipErrorInvalidValue;
    }
}

// ---- 4. exact logits of the candidates, top-k, softmax ----
#define RX_G 16       // lanes per token (4 tokens per wavefront)
#define RX_WPB 4      // wavefronts per block
#define RX_EMAX 256   // experts (the candidate values of a token sit in LDS)
#define RX_CH 32      // row elements per stage (8 float4 steps)
#define RX_SL 9       // 16-byte LDS slots per staged gate row: 8 + 1 pad
#define RX_NBUF 3     // stages per wavefront (two in flight while one is summed)
#define RX_WDMA RX_SL // gate-row DMA instructions per stage: 64 rows x 9 slots / 64
#define RX_STAGE_B (64 * RX_SL * 16 + 1024)  // 64 gate rows + the 4 token rows

typedef float f4 __attribute__((ext_vector_type(4)));

// One stage of a wavefront: for each lane's gate row (64 rows, padded to 9
// slots so that lanes reading their own rows hit distinct banks) and the
// wave's 4 token rows, elements [h0, h0 + RX_CH). Every lane issues every
// DMA, so each stage is exactly RX_WDMA + 1 vector-memory instructions.
// The bases are wave-uniform and the per-lane byte offsets 32-bit, so the
// DMAs take the scalar-base addressing form with no per-stage vector math.
__device__ __forceinline__ void rx_issue(const char *wbase, const uint32_t *woff,
                                         const char *xbase, uint32_t xoff, char *stage) {
#pragma unroll
    for (int m = 0; m < RX_WDMA; m++) dma<16>(wbase + woff[m], stage + m * 1024);
    dma<16>(xbase + xoff, stage + 64 * RX_SL * 16);
}

// A lane owns a (token, candidate) pair and runs the reference's four lane
// partials (element j into partial j % 4, src/moe_layer.c:67-86) as four
// independent fp64 chains over float4 steps; the final sum is
// (p0 + p1) + (p2 + p3). The gate rows of the wave's 64 lanes and its 4
// token rows stream through a 3-stage LDS ring filled by LDS-DMA (coalesced
// 1 KiB requests; rows read straight from global memory by 64 lanes at once
// would touch 64 cache lines per load). Then top-k by (value desc, index
// asc) over the candidates and softmax exactly as k_topk
// (src/routing.c:39-74).
__global__ __launch_bounds__(64 * RX_WPB) void k_router_exact(
    const int16_t *__restrict__ cand, const int32_t *__restrict__ ncand,
    const float *__restrict__ X, const float *__restrict__ Wg, int T, int E, int n, int k,
    int32_t *__restrict__ ids, float *__restrict__ w, float *__restrict__ logits,
    uint32_t *err) {
    constexpr int TPB = RX_WPB * 64 / RX_G;  // tokens per block
    constexpr int TPW = 64 / RX_G;           // tokens per wavefront
    extern __shared__ __attribute__((aligned(16))) char rx_smem[];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tl = threadIdx.x / RX_G, slot = threadIdx.x % RX_G;
    char *ring = rx_smem + (size_t)wid * RX_NBUF * RX_STAGE_B;
    float *cval = (float *)(rx_smem + (size_t)RX_WPB * RX_NBUF * RX_STAGE_B);  // [TPB][RX_EMAX]
    double *exl = (double *)(cval + TPB * RX_EMAX);                              // [TPB][64]
    short *sel = (short *)(exl + TPB * 64);                                      // [TPB][64]
    const int t = blockIdx.x * TPB + tl;
    const bool valid = t < T;
    const int nc = valid ? ncand[t] : 0;
    int ncw = nc;  // the largest count among the wave's tokens
    ncw = max(ncw, __shfl_xor(ncw, 16, 64));
    ncw = max(ncw, __shfl_xor(ncw, 32, 64));
    const int16_t *ct = cand + (int64_t)t * E;
    // token rows: lane l < 32 fetches 16 B of token l / 8 (slot l % 8); the
    // upper half repeats it into the unused half of the token area
    const int t0 = blockIdx.x * TPB + wid * TPW;  // the wave's first token
    const int xt = min(t0 + ((lane & 31) >> 3), T - 1);
    const uint32_t xoff = (uint32_t)(((xt - t0) * n + (lane & 7) * 4) * 4);
    float *cv = cval + tl * RX_EMAX;
    const int nch = n / RX_CH;
    int bad = 0;
    for (int c0 = 0; c0 < ncw; c0 += RX_G) {
        const int c = c0 + slot;
        const bool act = c < nc;
        const int e = act ? ct[c] : 0;
        // DMA m, lane l fills slot q = 64 m + l: row q / 9 (the gate row of
        // lane q / 9), step q % 9 (step 8 is the pad: a repeat of step 7)
        uint32_t woff[RX_WDMA];  // bytes from the stage's column of Wg
#pragma unroll
        for (int m = 0; m < RX_WDMA; m++) {
            const int q = 64 * m + lane, r = q / RX_SL, j = q % RX_SL;
            woff[m] = (uint32_t)((__shfl(e, r, 64) * n + 4 * min(j, RX_SL - 2)) * 4);
        }
        // stage s covers columns [s RX_CH, (s + 1) RX_CH)
        auto issue = [&](int sidx, char *st) {
            rx_issue((const char *)(Wg + sidx * RX_CH), woff,
                     (const char *)(X + (int64_t)t0 * n + sidx * RX_CH), xoff, st);
        };
        double p0 = 0.0, p1 = 0.0, p2 = 0.0, p3 = 0.0;
        constexpr int PER = RX_WDMA + 1;  // vector-memory instructions per stage
        const uint32_t wrow = lane * RX_SL * 16;
        const uint32_t xrow = 64 * RX_SL * 16 + (tl % TPW) * 128;
        auto stage = [&](int sidx) { return ring + (sidx % RX_NBUF) * RX_STAGE_B; };
        // LDS reads of a stage in asm (the compiler cannot tell them from
        // the stages still in flight and would drain every DMA before them);
        // their wait is a separate statement that takes the registers as
        // in/out operands, so the summing of the previous stage overlaps
        // the reads
        auto rd = [&](f4 *wv, f4 *xv, int sidx) {
            if (!act) return;
            const uint32_t wa = lds_addr(stage(sidx)) + wrow, xa = lds_addr(stage(sidx)) + xrow;
            asm volatile(
                "ds_read_b128 %0, %16 offset:0\n\tds_read_b128 %1, %17 offset:0\n\t"
                "ds_read_b128 %2, %16 offset:16\n\tds_read_b128 %3, %17 offset:16\n\t"
                "ds_read_b128 %4, %16 offset:32\n\tds_read_b128 %5, %17 offset:32\n\t"
                "ds_read_b128 %6, %16 offset:48\n\tds_read_b128 %7, %17 offset:48\n\t"
                "ds_read_b128 %8, %16 offset:64\n\tds_read_b128 %9, %17 offset:64\n\t"
                "ds_read_b128 %10, %16 offset:80\n\tds_read_b128 %11, %17 offset:80\n\t"
                "ds_read_b128 %12, %16 offset:96\n\tds_read_b128 %13, %17 offset:96\n\t"
                "ds_read_b128 %14, %16 offset:112\n\tds_read_b128 %15, %17 offset:112"
                : "=&v"(wv[0]), "=&v"(xv[0]), "=&v"(wv[1]), "=&v"(xv[1]), "=&v"(wv[2]),
                  "=&v"(xv[2]), "=&v"(wv[3]), "=&v"(xv[3]), "=&v"(wv[4]), "=&v"(xv[4]),
                  "=&v"(wv[5]), "=&v"(xv[5]), "=&v"(wv[6]), "=&v"(xv[6]), "=&v"(wv[7]),
                  "=&v"(xv[7])
                : "v"(wa), "v"(xa)
                : "memory");
        };
        auto wt = [&](f4 *wv, f4 *xv) {
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(wv[0]), "+v"(xv[0]), "+v"(wv[1]), "+v"(xv[1]), "+v"(wv[2]),
                           "+v"(xv[2]), "+v"(wv[3]), "+v"(xv[3]), "+v"(wv[4]), "+v"(xv[4]),
                           "+v"(wv[5]), "+v"(xv[5]), "+v"(wv[6]), "+v"(xv[6]), "+v"(wv[7]),
                           "+v"(xv[7])
                         :
                         : "memory");
        };
        auto fm = [&](const f4 *wv, const f4 *xv) {
            if (!act) return;
#pragma unroll
            for (int u = 0; u < RX_CH / 4; u++) {
                p0 = fma((double)xv[u].x, (double)wv[u].x, p0);
                p1 = fma((double)xv[u].y, (double)wv[u].y, p1);
                p2 = fma((double)xv[u].z, (double)wv[u].z, p2);
                p3 = fma((double)xv[u].w, (double)wv[u].w, p3);
            }
        };
        auto sync = [&]() {
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        };
        static_assert(RX_CH / 4 == 8, "eight steps per stage");
        f4 wA[8], xA[8], wB[8], xB[8];
        // stage s lives in ring slot s % 3; nch is even and >= 2. The stage
        // waits count this pass's DMAs only: retire the previous pass's
        // logit stores first.
        wait_vm<0>();
        issue(0, stage(0));
        issue(1, stage(1));
        if (nch > 2) {
            issue(2, stage(2));
            wait_vm<2 * PER>();
        } else {
            wait_vm<PER>();
        }
        sync();
        rd(wA, xA, 0);
        for (int ch = 0; ch < nch; ch += 2) {
            // stage ch (A) is summed while stage ch + 1 (B) is read
            wt(wA, xA);  // slot ch % 3 is free again
            if (ch + 2 < nch) wait_vm<PER>();
            else wait_vm<0>();
            sync();
            rd(wB, xB, ch + 1);
            if (ch + 3 < nch) issue(ch + 3, stage(ch + 3));
            fm(wA, xA);
            // stage ch + 1 (B) is summed while stage ch + 2 (A) is read
            wt(wB, xB);  // slot (ch + 1) % 3 is free again
            if (ch + 2 < nch) {
                if (ch + 3 < nch) wait_vm<PER>();
                else wait_vm<0>();
                sync();
                rd(wA, xA, ch + 2);
                if (ch + 4 < nch) issue(ch + 4, stage(ch + 4));
            }
            fm(wB, xB);
        }
        // every read of the ring is complete (wt) before the next pass
        // refills it
        if (act) {
            const double tot = (p0 + p1) + (p2 + p3);
            const float f = (float)tot;
            bad |= (!isfinite(tot)) || (!isfinite(f));
            cv[c] = f;
            logits[(int64_t)t * E + e] = f;
        }
    }
    // a non-finite logit is the reference's error (src/routing.c:39-54)
    if (__ballot(bad != 0)) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    // cval written by some lanes is read by others below
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // rank of each candidate = candidates before it in (value desc, index
    // asc) order; the list is in ascending expert order
    short *sl = sel + tl * 64;
    double *xl2 = exl + tl * 64;
    for (int c = slot; c < nc; c += RX_G) {
        const float f = cv[c];
        int rank = 0;
        for (int j = 0; j < nc; j++) {
            const float g = cv[j];
            rank += (g > f) || (g == f && j < c);
        }
        if (rank < k) sl[rank] = (short)c;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // the rank-0 value is the maximum
    const bool ok = valid && nc >= k;
    const float mx = ok ? cv[sl[0]] : 0.0f;
    for (int r = slot; r < k; r += RX_G)
        if (ok) xl2[r] = exp((double)cv[sl[r]] - (double)mx);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (!valid) return;
    double sum = 0.0;
    for (int r = 0; r < k; r++) sum += xl2[r];
    if (!ok || !((sum > 0.0) && isfinite(sum))) {
        if (slot == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    const float inv = (float)(1.0 / sum);
    for (int r = slot; r < k; r += RX_G) {
        const float wv = (float)xl2[r] * inv;
        ids[(int64_t)t * k + r] = ct[sl[r]];
        w[(int64_t)t * k + r] = wv;
        if (!(wv >= 0.0f) || !isfinite(wv)) raise_err(err, EF_NONFINITE_MID);
    }
}

// ---- 3+4 for few tokens: one wavefront per token ----
// Decode-sized calls have too few tokens to fill the GPU with the 16-token
// blocks above, and one wave's four fp64 chains per lane are then the
// latency. Here a wavefront owns one token: it selects the candidates as
// k_router_select does, then gives each of up to 16 candidates four lanes,
// lane p running the reference's partial p (element j into partial j % 4,
// src/moe_layer.c:67-86) as one fp64 chain over rows staged in LDS by
// LDS-DMA, 1024 elements at a time (rows padded by 4 floats so the 16
// candidates' lanes hit different banks). (l0 + l1) + (l2 + l3) is formed
// with lane shuffles; top-k and softmax as k_router_exact.
#define RS_CH 1024
#define RS_STRIDE (RS_CH + 4)
__global__ __launch_bounds__(64) void k_router_topk_small(
    const double *__restrict__ approx, const double2 *__restrict__ xinfo,
    const double2 *__restrict__ winfo, const float *__restrict__ X,
    const float *__restrict__ Wg, int T, int E, int n, int k, int32_t *__restrict__ ids,
    float *__restrict__ w, float *__restrict__ logits, uint32_t *err) {
    extern __shared__ __attribute__((aligned(16))) char rs_smem[];
    float *xs = (float *)rs_smem;                          // [RS_CH]
    float *ws = xs + RS_CH;                                // [16][RS_STRIDE]
    float *cval = ws + 16 * RS_STRIDE;                     // [RV_EMAX]
    double *exl = (double *)(cval + RV_EMAX);              // [64]
    int16_t *cand = (int16_t *)(exl + 64);                 // [RV_EMAX]
    int16_t *sel = cand + RV_EMAX;                         // [64]
    const int lane = threadIdx.x, t = blockIdx.x;
    const int nc = select_token(approx, xinfo, winfo, t, E, n, k, lane, cand, logits);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const int slot = lane >> 2, p = lane & 3;
    int bad = 0;
    for (int c0 = 0; c0 < nc; c0 += 16) {
        const int c = c0 + slot;
        const bool act = c < nc;
        double sp = 0.0;
        for (int h0 = 0; h0 < n; h0 += RS_CH) {
            const int ch = min(RS_CH, n - h0);  // a multiple of 256
            // row of slot r: expert cand[c0 + r] (inactive slots stage
            // expert cand[0]); 1 KiB of a row per DMA
            for (int r = 0; r < 16; r++) {
                const int er = cand[c0 + r < nc ? c0 + r : 0];
                const float *src = Wg + (int64_t)er * n + h0 + lane * 4;
                for (int q = 0; q < ch / 256; q++)
                    dma<16>(src + q * 256, ws + r * RS_STRIDE + q * 256);
            }
            for (int q = 0; q < ch / 256; q++)
                dma<16>(X + (int64_t)t * n + h0 + q * 256 + lane * 4, xs + q * 256);
            wait_vm<0>();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            if (act) {
                const float *wr = ws + slot * RS_STRIDE;
                for (int i = p; i < ch; i += 64) {
                    float xv[16], wv[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        xv[u] = xs[i + 4 * u];
                        wv[u] = wr[i + 4 * u];
                    }
#pragma unroll
                    for (int u = 0; u < 16; u++) sp = fma((double)xv[u], (double)wv[u], sp);
                }
            }
            // the next chunk overwrites the staged rows
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        const double s1 = __shfl_down(sp, 1, 64), s2 = __shfl_down(sp, 2, 64),
                     s3 = __shfl_down(sp, 3, 64);
        if (act && p == 0) {
            const double tot = (sp + s1) + (s2 + s3);
            const float f = (float)tot;
            bad |= (!isfinite(tot)) || (!isfinite(f));
            cval[c] = f;
            logits[(int64_t)t * E + cand[c]] = f;
        }
    }
    if (__ballot(bad != 0)) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int c = lane; c < nc; c += 64) {
        const float f = cval[c];
        int rank = 0;
        for (int j = 0; j < nc; j++) {
            const float g = cval[j];
            rank += (g > f) || (g == f && j < c);
        }
        if (rank < k) sel[rank] = (int16_t)c;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (nc < k) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    // the rank-0 value is the maximum
    const float mx = cval[sel[0]];
    const double ex = lane < k ? exp((double)cval[sel[lane]] - (double)mx) : 0.0;
    double sum = 0.0;
    for (int r = 0; r < k; r++) sum += readlane_f64(ex, r);
    if (!((sum > 0.0) && isfinite(sum))) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return;
    }
    const float inv = (float)(1.0 / sum);
    if (lane < k) {
        const float wv = (float)ex * inv;
        ids[(int64_t)t * k + lane] = cand[sel[lane]];
        w[(int64_t)t * k + lane] = wv;
        if (!(wv >= 0.0f) || !isfinite(wv)) raise_err(err, EF_NONFINITE_MID);
    }
}

extern "C" int jtk_topk_verify(const double *approx, const double *xinfo, const double *winfo,
                               const float *X, const float *Wg, int T, int E, int n, int k,
                               int16_t *cand, int32_t *ncand, int32_t *ids, float *w,
                               float *logits, uint32_t *err, int stages, hipStream_t s) {
    if (T <= 0 || !(stages & 3)) return 0;
    if (T <= 256 && E <= RV_EMAX && k >= 1 && k <= 64 && k <= E && n % 256 == 0) {
        if (!(stages & 2)) return 0;  // one launch: runs with the second stage
        constexpr size_t lds_s = (size_t)(RS_CH + 16 * RS_STRIDE + RV_EMAX) * 4 + 64 * 8 +
                                 (RV_EMAX + 64) * 2;
        static std::atomic<bool> attr_small[64];
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return (int)e;
        if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
        if (!attr_small[dev]) {
            e = hipFuncSetAttribute((const void *)k_router_topk_small,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_s);
            if (e != hipSuccess) return (int)e;
            attr_small[dev] = true;
        }
        hipLaunchKernelGGL(k_router_topk_small, dim3((unsigned)T), dim3(64), lds_s, s, approx,
                           (const double2 *)xinfo, (const double2 *)winfo, X, Wg, T, E, n, k,
                           ids, w, logits, err);
        return (int)hipGetLastError();
    }
    if (E > RX_EMAX || k < 1 || k > 64 || k > E || n % (2 * RX_CH) != 0 ||
        (int64_t)E * n > 0x1fffffff || (int64_t)4 * n * 4 > 0x7fffffff)
        return (int)hipErrorInvalidValue;
    constexpr int TPB = RX_WPB * 64 / RX_G;
    constexpr size_t lds =
        (size_t)RX_WPB * RX_NBUF * RX_STAGE_B + (size_t)TPB * (RX_EMAX * 4 + 64 * 8 + 64 * 2);
    static_assert(lds <= 160 * 1024, "LDS budget");
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)k_router_exact,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        attr_set[dev] = true;
    }
    if (stages & 1)
        hipLaunchKernelGGL(k_router_select, dim3((unsigned)((T + RV_WPB - 1) / RV_WPB)),
                           dim3(64 * RV_WPB), 0, s, approx, (const double2 *)xinfo,
                           (const double2 *)winfo, T, E, n, k, cand, ncand, logits);
    if (stages & 2)
        hipLaunchKernelGGL(k_router_exact, dim3((unsigned)((T + TPB - 1) / TPB)),
                           dim3(64 * RX_WPB), lds, s, (const int16_t *)cand,
                           (const int32_t *)ncand, X, Wg, T, E, n, k, ids, w, logits, err);
    return (int)hipGetLastError();
}

// ---- decode-sized router: every logit exact, plus the token codes ----
// For T <= 16 tokens the bound/candidate stages cost more launches than the
// fp64 work they save, so every (token, expert) logit is computed exactly:
// a block stages the T token rows (fp32, rows padded by 4 floats so the 16
// token rows hit different banks) and 4 gate rows by LDS-DMA; wave w owns
// expert 4*blockIdx.x + w and lane 4t + p runs the reference's partial p of
// token t (element j into partial j % 4, src/moe_layer.c:67-86) as one fp64
// chain, then (l0 + l1) + (l2 + l3) by lane shuffles. Blocks nb .. nb+T-1
// (nb = the logit blocks) each write one token's int8 codes and scale (the
// row quantiser, src/w8a8.c:787-855) from its row in memory, beside the
// logit blocks instead of after their chains (measured 8.3 -> 6.1 us at
// T = 16, E = 256, n = 1024). n % 256 == 0, T * (n + 4) * 4 +
// 4 * (n + 4) * 4 bytes of LDS.
#define RL_TMAX 16
__global__ __launch_bounds__(256) void k_router_logits_small(
    const float *__restrict__ X, const float *__restrict__ Wg, int T, int E, int n, int nb,
    float *__restrict__ logits, int8_t *__restrict__ Xq, float *__restrict__ sx,
    uint32_t *err) {
    extern __shared__ __attribute__((aligned(16))) float rl_smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if ((int)blockIdx.x >= nb) {  // token blockIdx.x - nb's codes (wave 0)
        const int r = blockIdx.x - nb;
        if (wave != 0 || r >= T) return;
        const float *xr = X + (int64_t)r * n;
        uint32_t mu = 0;
        for (int c = lane; c < n; c += 64) mu = max(mu, abs_bits(xr[c]));
        mu = wave_max_u(mu);
        const QuantParams qp = quant_params(__builtin_bit_cast(float, mu));
        if (mu >= 0x7f800000u || !qp.ok) {
            if (lane == 0) raise_err(err, mu >= 0x7f800000u ? EF_NONFINITE_INPUT : EF_RANGE);
            return;
        }
        if (lane == 0) sx[r] = qp.scale_f;
        const float inv = quant_inv_f(qp.scale_d);
        for (int c = lane * 4; c < n; c += 256) {
            const uint32_t b0 = (uint8_t)quant_code_fast(xr[c], qp.scale_d, inv);
            const uint32_t b1 = (uint8_t)quant_code_fast(xr[c + 1], qp.scale_d, inv);
            const uint32_t b2 = (uint8_t)quant_code_fast(xr[c + 2], qp.scale_d, inv);
            const uint32_t b3 = (uint8_t)quant_code_fast(xr[c + 3], qp.scale_d, inv);
            *(uint32_t *)(Xq + (int64_t)r * n + c) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        return;
    }
    const int stride = n + 4;
    float *xs = rl_smem;                  // [T][n + 4]
    float *ws = rl_smem + T * stride;     // [4][n + 4]
    const int e = blockIdx.x * 4 + wave;
    const int nc = n / 256;  // 1 KiB copies per row
    for (int c = wave; c < T * nc; c += 4) {
        const int t = c / nc, q = c % nc;
        dma<16>(X + (int64_t)t * n + q * 256 + lane * 4, xs + t * stride + q * 256);
    }
    const int er = min(e, E - 1);
    for (int q = 0; q < nc; q++)
        dma<16>(Wg + (int64_t)er * n + q * 256 + lane * 4, ws + wave * stride + q * 256);
    wait_vm<0>();
    __syncthreads();
    const int t = lane >> 2, p = lane & 3;
    const bool act = t < T && e < E;
    double acc = 0.0;
    if (act) {
        const float *xr = xs + t * stride + p;
        const float *wr = ws + wave * stride + p;
        for (int j = 0; j < n; j += 64) {
            float xv[16], wv[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                xv[u] = xr[j + 4 * u];
                wv[u] = wr[j + 4 * u];
            }
#pragma unroll
            for (int u = 0; u < 16; u++) acc = fma((double)xv[u], (double)wv[u], acc);
        }
    }
    const double a1 = __shfl_down(acc, 1, 64), a2 = __shfl_down(acc, 2, 64),
                 a3 = __shfl_down(acc, 3, 64);
    uint32_t bad = 0;
    if (act && p == 0) {
        const double tot = (acc + a1) + (a2 + a3);
        const float f = (float)tot;
        bad = (!isfinite(tot)) || (!isfinite(f));
        logits[(int64_t)t * E + e] = f;
    }
    if (__ballot(bad != 0) && lane == 0) raise_err(err, EF_NONFINITE_MID);
}

extern "C" int jtk_router_logits_small(const float *X, const float *Wg, int T, int E, int n,
                                       float *logits, int8_t *Xq, float *sx, uint32_t *err,
                                       hipStream_t s) {
    if (T <= 0) return 0;
    if (T > RL_TMAX || n % 256 != 0 || E <= 0) return (int)hipErrorInvalidValue;
    const size_t lds = (size_t)(T + 4) * (n + 4) * 4;
    if (lds > 160 * 1024) return (int)hipErrorInvalidValue;
    static std::atomic<bool> attr_set[64];  // set once per device; a repeat is harmless
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    if (!attr_set[dev]) {
        e = hipFuncSetAttribute((const void *)k_router_logits_small,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return (int)e;
        attr_set[dev] = true;
    }
    const int nb = (E + 3) / 4;  // logit blocks; then one block per token's codes
    hipLaunchKernelGGL(k_router_logits_small, dim3((unsigned)(nb + T)), dim3(256), lds, s, X, Wg,
                       T, E, n, nb, logits, Xq, sx, err);
    return (int)hipGetLastError();
}

// Load this file's code object now: the runtime otherwise loads it, and
// allocates device memory for it, at the first launch of one of its kernels.
extern "C" int jtk_preload_router(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_router_codes<4>));
}
