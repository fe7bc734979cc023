// Quantisation, dequantisation and weight-packing kernels (gfx950).
//
// k_quant_rows is the reference's per-row int8 quantiser
// (src/w8a8.c:787-855, per tensor = one row src/w8a8.c:688-747): one
// wavefront per row, fp32 max-abs reduction (exact: the reference takes the
// max of exact fp64 widenings), fp64 divide, round half away from zero.
#include "jt_dev.h"
#include "jt_launch.h"
#include "quant_dev.h"

// One wavefront per row; blockDim = 256 (4 rows per block).
__global__ __launch_bounds__(256) void k_quant_rows(
    const float *__restrict__ X, int64_t rows, int cols, int8_t *__restrict__ Q,
    int64_t ldq, float *__restrict__ scale, const int32_t *__restrict__ row_count,
    uint32_t *err) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t nrows = row_count ? (int64_t)*row_count : rows;
    if (r >= nrows) return;
    quant_row_wave(X, r, cols, Q, ldq, scale, err, threadIdx.x & 63);
}

// Short rows (cols <= 512, a multiple of 64, 16-byte aligned): 16 lanes
// (one DPP row) per row, 4 rows per wavefront, every lane's cols/64 float4
// loads in flight at once. A row of 256 floats (the routed hidden rows) is
// then one float4 per lane of four, not one per lane of a whole wavefront,
// so a launch needs a quarter of the wavefronts and each has four times the
// loads in flight. The row maximum is an all-reduce over the 16 lanes with
// DPP row rotations; the codes are k_quant_rows's.
#define QS_MAXV 8  // float4 per lane: cols <= 512
__global__ __launch_bounds__(256) void k_quant_rows16(const float *__restrict__ X, int64_t rows,
                                                      int cols, int8_t *__restrict__ Q,
                                                      int64_t ldq, float *__restrict__ scale,
                                                      const int32_t *__restrict__ row_count,
                                                      uint32_t *err) {
    const int lane = threadIdx.x & 63, sub = lane & 15;
    const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int64_t nrows = row_count ? (int64_t)*row_count : rows;
    if (r >= nrows) return;  // whole DPP rows leave together
    const float4 *x4 = (const float4 *)(X + r * cols);
    const int nv = cols >> 6;  // float4 per lane
    float4 v[QS_MAXV];
#pragma unroll
    for (int j = 0; j < QS_MAXV; j++)
        if (j < nv) v[j] = x4[sub + 16 * j];  // uniform bound: v[] stays in registers
    uint32_t mu = 0;
#pragma unroll
    for (int j = 0; j < QS_MAXV; j++)
        if (j < nv) {
            mu = max(mu, max(abs_bits(v[j].x), abs_bits(v[j].y)));
            mu = max(mu, max(abs_bits(v[j].z), abs_bits(v[j].w)));
        }
    mu = row16_allmax_u(mu);
    const QuantParams p = quant_params(__builtin_bit_cast(float, mu));
    if (mu >= 0x7f800000u || !p.ok) {
        if (sub == 0) raise_err(err, mu >= 0x7f800000u ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    const float inv = quant_inv_f(p.scale_d);
    uint32_t *q4 = (uint32_t *)(Q + r * ldq);
    uint32_t fmask = 0;  // bit j: a code of v[j] needs the exact quotient
    uint32_t wd[QS_MAXV];  // every word first, then the stores (as in k_quant_rows)
#pragma unroll
    for (int j = 0; j < QS_MAXV; j++) {
        wd[j] = 0;
        if (j < nv) {
            bool f = false;
            const uint32_t b0 = (uint8_t)quant_code_try(v[j].x, inv, f);
            const uint32_t b1 = (uint8_t)quant_code_try(v[j].y, inv, f);
            const uint32_t b2 = (uint8_t)quant_code_try(v[j].z, inv, f);
            const uint32_t b3 = (uint8_t)quant_code_try(v[j].w, inv, f);
            fmask |= (uint32_t)f << j;
            wd[j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
    }
#pragma unroll
    for (int j = 0; j < QS_MAXV; j++)
        if (j < nv) q4[sub + 16 * j] = wd[j];
    if (sub == 0) scale[r] = p.scale_f;
    while (fmask) {  // rare: rewrite those words exactly
        const int j = __builtin_ctz(fmask);
        fmask &= fmask - 1;
        float4 u = v[0];
#pragma unroll
        for (int i = 1; i < QS_MAXV; i++)
            if (i == j) u = v[i];
        const uint32_t b0 = (uint8_t)quant_code(u.x, p.scale_d);
        const uint32_t b1 = (uint8_t)quant_code(u.y, p.scale_d);
        const uint32_t b2 = (uint8_t)quant_code(u.z, p.scale_d);
        const uint32_t b3 = (uint8_t)quant_code(u.w, p.scale_d);
        q4[sub + 16 * j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
}

extern "C" int jtk_quant_rows(const float *X, int64_t rows, int cols, int8_t *Q,
                              int64_t ldq, float *scale, const int32_t *row_count,
                              uint32_t *err, hipStream_t s) {
    if (rows <= 0) return 0;
    // (measured: faster than one row per wavefront up to 512 columns,
    // slower at 1024)
    if (cols > 0 && cols <= 512 && cols % 64 == 0 && ldq % 4 == 0 &&
        ((uintptr_t)X & 15) == 0 && ((uintptr_t)Q & 3) == 0) {
        hipLaunchKernelGGL(k_quant_rows16, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s,
                           X, rows, cols, Q, ldq, scale, row_count, err);
        return (int)hipGetLastError();
    }
    hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, X,
                       rows, cols, Q, ldq, scale, row_count, err);
    return (int)hipGetLastError();
}

// Whole-array (per-tensor) quantisation: pass 1 reduces max|x| and the
// non-finite flag into *amax (float bits, atomicMax on non-negative floats
// is monotone in their bit patterns), pass 2 quantises.
__global__ __launch_bounds__(256) void k_absmax(const float *__restrict__ x, int64_t n,
                                                uint32_t *amax, uint32_t *err) {
    float m = 0.0f;
    int bad = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        float v = x[i];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if ((threadIdx.x & 63) == 0) {
        atomicMax(amax, __float_as_uint(m));
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_quant_tensor(const float *__restrict__ x, int64_t n,
                                                      const uint32_t *amax,
                                                      int8_t *__restrict__ q,
                                                      float *scale, uint32_t *err) {
    QuantParams p = quant_params(__uint_as_float(*amax));
    if (!p.ok) {
        if (blockIdx.x == 0 && threadIdx.x == 0) raise_err(err, EF_RANGE);
        return;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = p.scale_f;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256)
        q[i] = (int8_t)quant_code(x[i], p.scale_d);
}

static unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > 8192) b = 8192;
    if (b < 1) b = 1;
    return (unsigned)b;
}

extern "C" int jtk_quant_tensor(const float *x, int64_t n, int8_t *q, float *scale,
                                uint32_t *amax_scratch, uint32_t *err, hipStream_t s) {
    (void)hipMemsetAsync(amax_scratch, 0, sizeof(uint32_t), s);
    hipLaunchKernelGGL(k_absmax, dim3(grid_for(n)), dim3(256), 0, s, x, n, amax_scratch,
                       err);
    hipLaunchKernelGGL(k_quant_tensor, dim3(grid_for(n)), dim3(256), 0, s, x, n,
                       amax_scratch, q, scale, err);
    return (int)hipGetLastError();
}

// Fake-quant of each row (rows = 1 for per tensor), src/w8a8.c:1074-1200:
// dst = (float)(clamp(round(x/scale_d)) * scale_d) computed in fp64.
__global__ __launch_bounds__(256) void k_fakequant_rows(const float *__restrict__ X,
                                                        int64_t rows, int64_t cols,
                                                        float *__restrict__ D,
                                                        const uint32_t *amax,
                                                        uint32_t *err) {
    int lane = threadIdx.x & 63;
    int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float *x = X + r * cols;
    float *d = D + r * cols;
    float m;
    if (amax) {
        m = __uint_as_float(*amax);
    } else {
        m = 0.0f;
        for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, fabsf(x[c]));
        m = wave_max_f(m);
    }
    if (m == 0.0f) {
        for (int64_t c = lane; c < cols; c += 64) d[c] = 0.0f;
        return;
    }
    double scale_d = (double)m / 127.0;
    for (int64_t c = lane; c < cols; c += 64) {
        double qd = round((double)x[c] / scale_d);
        qd = qd > 127.0 ? 127.0 : (qd < -127.0 ? -127.0 : qd);
        float f = (float)(qd * scale_d);
        if (!isfinite(f)) raise_err(err, EF_RANGE);
        d[c] = f;
    }
}

// Whole-array fake-quant: the block-strided loop covers all n elements with
// one max from k_absmax.
__global__ __launch_bounds__(256) void k_fakequant_tensor(const float *__restrict__ x,
                                                          int64_t n, float *__restrict__ d,
                                                          const uint32_t *amax,
                                                          uint32_t *err) {
    float m = __uint_as_float(*amax);
    double scale_d = (double)m / 127.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        if (m == 0.0f) {
            d[i] = 0.0f;
            continue;
        }
        double qd = round((double)x[i] / scale_d);
        qd = qd > 127.0 ? 127.0 : (qd < -127.0 ? -127.0 : qd);
        float f = (float)(qd * scale_d);
        if (!isfinite(f)) raise_err(err, EF_RANGE);
        d[i] = f;
    }
}

extern "C" int jtk_fakequant(const float *x, int64_t rows, int64_t cols, float *d,
                             uint32_t *amax_scratch, uint32_t *err, hipStream_t s) {
    if (rows == 1) {
        int64_t n = cols;
        (void)hipMemsetAsync(amax_scratch, 0, sizeof(uint32_t), s);
        hipLaunchKernelGGL(k_absmax, dim3(grid_for(n)), dim3(256), 0, s, x, n,
                           amax_scratch, err);
        hipLaunchKernelGGL(k_fakequant_tensor, dim3(grid_for(n)), dim3(256), 0, s, x, n, d,
                           amax_scratch, err);
    } else {
        (void)hipMemsetAsync(amax_scratch, 0, sizeof(uint32_t), s);
        hipLaunchKernelGGL(k_absmax, dim3(grid_for(rows * cols)), dim3(256), 0, s, x,
                           rows * cols, amax_scratch, err);
        hipLaunchKernelGGL(k_fakequant_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                           s, x, rows, cols, d, (const uint32_t *)nullptr, err);
    }
    return (int)hipGetLastError();
}

// dst = (float)((double)q * (double)scale[row]) (src/w8a8.c:890-903); a code
// of -128 raises EF_QRANGE, a non-finite product EF_RANGE.
__global__ __launch_bounds__(256) void k_dequant_rows(const int8_t *__restrict__ q,
                                                      const float *__restrict__ scale,
                                                      int64_t rows, int64_t cols,
                                                      int per_row, float *__restrict__ d,
                                                      uint32_t *err) {
    int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        int v = q[i];
        if (v < -127) raise_err(err, EF_QRANGE);
        double sc = (double)scale[per_row ? i / cols : 0];
        float f = (float)((double)v * sc);
        if (!isfinite(f)) raise_err(err, EF_RANGE);
        d[i] = f;
    }
}

extern "C" int jtk_dequant(const int8_t *q, const float *scale, int64_t rows,
                           int64_t cols, int per_row, float *d, uint32_t *err,
                           hipStream_t s) {
    hipLaunchKernelGGL(k_dequant_rows, dim3(grid_for(rows * cols)), dim3(256), 0, s, q,
                       scale, rows, cols, per_row, d, err);
    return (int)hipGetLastError();
}

// Flags any int8 code of -128 (the reference rejects it, src/w8a8.c:979-999).
__global__ __launch_bounds__(256) void k_check_q(const int8_t *__restrict__ q, int64_t n,
                                                 uint32_t *err) {
    int bad = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256)
        bad |= (q[i] == (int8_t)-128);
    bad = wave_or_i(bad);
    if (bad && (threadIdx.x & 63) == 0) raise_err(err, EF_QRANGE);
}

extern "C" int jtk_check_q(const int8_t *q, int64_t n, uint32_t *err, hipStream_t s) {
    hipLaunchKernelGGL(k_check_q, dim3(grid_for(n)), dim3(256), 0, s, q, n, err);
    return (int)hipGetLastError();
}

// Flags non-finite fp32 values (the reference's finiteness pre-scans).
__global__ __launch_bounds__(256) void k_check_finite(const float *__restrict__ x, int64_t n,
                                                      uint32_t *err) {
    int bad = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256)
        bad |= !isfinite(x[i]);
    bad = wave_or_i(bad);
    if (bad && (threadIdx.x & 63) == 0) raise_err(err, EF_NONFINITE_INPUT);
}

extern "C" int jtk_check_finite(const float *x, int64_t n, uint32_t *err, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_check_finite, dim3(grid_for(n)), dim3(256), 0, s, x, n, err);
    return (int)hipGetLastError();
}

// ---- int8 panel packing ----
// Q is int8 [N][K] (ldq = K) or, when kn != 0, the reference's [K][N] layout.
// Output panels as described in jt_dev.h; N padded to Np (multiple of 16) and
// K to Kp (multiple of 64) with zero codes. One thread per 16-byte lane slot.
__global__ __launch_bounds__(256) void k_pack_i8(const int8_t *__restrict__ Q, int N, int K,
                                                 int kn, int Np, int Kp,
                                                 int8_t *__restrict__ P) {
    int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte slot
    int kblocks = Kp / 64;
    int64_t nslots = (int64_t)(Np / 16) * kblocks * 64;
    if (slot >= nslots) return;
    int lane = (int)(slot & 63);
    int64_t pk = slot >> 6;
    int kb = (int)(pk % kblocks);
    int p = (int)(pk / kblocks);
    int c = lane & 15, kc = lane >> 4;
    int n = p * 16 + c;
    int k0 = kb * 64 + kc * 16;
    union {
        int8_t b[16];
        v4i v;
    } u;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int k = k0 + j;
        int8_t v = 0;
        if (n < N && k < K) v = kn ? Q[(int64_t)k * N + n] : Q[(int64_t)n * K + k];
        u.b[j] = v;
    }
    *(v4i *)(P + slot * 16) = u.v;
}

extern "C" int jtk_pack_i8(const int8_t *Q, int N, int K, int kn, int Np, int Kp,
                           int8_t *P, hipStream_t s) {
    int64_t nslots = (int64_t)(Np / 16) * (Kp / 64) * 64;
    hipLaunchKernelGGL(k_pack_i8, dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, s,
                       Q, N, K, kn, Np, Kp, P);
    return (int)hipGetLastError();
}

// Inverse of k_pack_i8 into the [K][N] layout (tests/export only).
__global__ __launch_bounds__(256) void k_unpack_i8_kn(const int8_t *__restrict__ P, int N,
                                                      int K, int Kp, int8_t *__restrict__ Q) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)N * K) return;
    int k = (int)(i / N), n = (int)(i % N);
    int p = n / 16, c = n % 16, kb = k / 64, kc = (k % 64) / 16, j = k % 16;
    int64_t off = ((int64_t)p * (Kp / 64) + kb) * 1024 + (kc * 16 + c) * 16 + j;
    Q[i] = P[off];
}

extern "C" int jtk_unpack_i8_kn(const int8_t *P, int N, int K, int Kp, int8_t *Q,
                                hipStream_t s) {
    int64_t n = (int64_t)N * K;
    hipLaunchKernelGGL(k_unpack_i8_kn, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       P, N, K, Kp, Q);
    return (int)hipGetLastError();
}

// ---- low-bit packing (prepared routed-expert format) ----
// Expert e's source element (row i, k) is W[e*w_estride + i*ld_n + k*ld_k].
// Packed channel n (0..N-1) takes row n of W0, or, when W1 != NULL, the
// gate/up interleave in blocks of 16: n -> (W0 if (n/16) even else W1),
// row (n/32)*16 + n%16. One wavefront per (expert, channel, 64-K group):
// maxabs over the group (the exact fp64 max via the fp32 max), codes by the
// reference's level formula (src/lowbit.c:78-86), scale
// f16(maxabs / (2^bits - 1)). Writes the panel codes and fp16 scales, and
// optionally plain copies for export: codes_out [E][src][row][K] and
// scales_out [E][src][row][K/64] (src = 0/1 for W0/W1).
__global__ __launch_bounds__(256) void k_pack_lowbit(
    const float *__restrict__ W0, const float *__restrict__ W1, int64_t w_estride,
    int64_t ld_n, int64_t ld_k, int N, int K, int bits, uint8_t *__restrict__ P,
    int64_t p_estride, uint16_t *__restrict__ S, int64_t s_estride,
    uint8_t *__restrict__ codes_out, uint16_t *__restrict__ scales_out, uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int e = blockIdx.y;
    const int G = K / 64;
    if (wid >= (int64_t)N * G) return;
    const int n = (int)(wid / G), g = (int)(wid % G);
    int row = n, src = 0;
    const float *W = W0;
    if (W1) {
        src = (n >> 4) & 1;
        row = (n >> 5) * 16 + (n & 15);
        W = src ? W1 : W0;
    }
    const int k = g * 64 + lane;
    const float w = W[(int64_t)e * w_estride + (int64_t)row * ld_n + (int64_t)k * ld_k];
    const int bad = wave_or_i(!isfinite(w));
    const float m = wave_max_f(fabsf(w));
    const double maxabs = (double)m;
    const double nn = (double)((1 << bits) - 1);
    const uint16_t s16 = f64_to_f16(maxabs / nn);
    if (bad || (s16 & 0x7c00u) == 0x7c00u) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    const int li = lowbit_code((double)w, maxabs, bits);
    const int p = n / 16, c = n % 16;
    const int kc = lane >> 4, kap = lane & 15;
    const int o = kap >> 2, j = kap & 3;
    const int plane = kc * 16 + c;
    uint8_t *Pe = P + (int64_t)e * p_estride;
    if (bits == 2) {
        uint32_t *dw = (uint32_t *)(Pe + ((int64_t)p * G + g) * 256 + plane * 4);
        atomicOr(dw, (uint32_t)li << (8 * j + 2 * o));
    } else {
        uint32_t *dw = (uint32_t *)(Pe + ((int64_t)p * G + g) * 512 + plane * 8 + (o >> 1) * 4);
        atomicOr(dw, (uint32_t)li << (8 * j + 4 * (o & 1)));
    }
    if (lane == 0) S[(int64_t)e * s_estride + ((int64_t)p * G + g) * 16 + c] = s16;
    const int rows_per_src = W1 ? N / 2 : N;
    const int64_t plain_row = ((int64_t)e * (W1 ? 2 : 1) + src) * rows_per_src + row;
    if (codes_out) codes_out[plain_row * K + k] = (uint8_t)li;
    if (scales_out && lane == 0) scales_out[plain_row * G + g] = s16;
}

extern "C" int jtk_pack_lowbit(const float *W0, const float *W1, int64_t w_estride,
                               int64_t ld_n, int64_t ld_k, int E, int N, int K, int bits,
                               uint8_t *P, uint16_t *S, uint8_t *codes_out,
                               uint16_t *scales_out, uint32_t *err, hipStream_t s) {
    const int G = K / 64;
    const int64_t p_estride = (int64_t)(N / 16) * G * (bits == 2 ? 256 : 512);
    const int64_t s_estride = (int64_t)(N / 16) * G * 16;
    (void)hipMemsetAsync(P, 0, (size_t)(p_estride * E), s);
    const int64_t waves = (int64_t)N * G;
    hipLaunchKernelGGL(k_pack_lowbit, dim3((unsigned)((waves + 3) / 4), (unsigned)E), dim3(256),
                       0, s, W0, W1, w_estride, ld_n, ld_k, N, K, bits, P, p_estride, S,
                       s_estride, codes_out, scales_out, err);
    return (int)hipGetLastError();
}

// Row interleave of two [h][cols] byte matrices into [2h][cols] with the
// gate/up 16-block order of the packed layout (dst row 32*(i/16)+16*s+i%16).
__global__ __launch_bounds__(256) void k_interleave_rows(const uint8_t *__restrict__ A,
                                                         const uint8_t *__restrict__ B, int h,
                                                         int64_t row_bytes,
                                                         uint8_t *__restrict__ D) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= 2 * (int64_t)h * row_bytes) return;
    const int64_t drow = id / row_bytes, c = id % row_bytes;
    const int sel = (int)((drow >> 4) & 1);
    const int64_t i = (drow >> 5) * 16 + (drow & 15);
    D[id] = (sel ? B : A)[i * row_bytes + c];
}

extern "C" int jtk_interleave_rows(const void *A, const void *B, int h, int64_t row_bytes,
                                   void *D, hipStream_t s) {
    const int64_t n = 2 * (int64_t)h * row_bytes;
    hipLaunchKernelGGL(k_interleave_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)A, (const uint8_t *)B, h, row_bytes, (uint8_t *)D);
    return (int)hipGetLastError();
}

// Per-row int8 quantisation of a strided fp32 weight matrix (shared experts:
// gate/up rows are contiguous, down columns are strided), writing int8 rows
// [N][K] and scales [N]. One wavefront per row.
__global__ __launch_bounds__(256) void k_quant_weight_rows(
    const float *__restrict__ W, int64_t ld_n, int64_t ld_k, int N, int K,
    int8_t *__restrict__ Q, float *__restrict__ scale, uint32_t *err) {
    int lane = threadIdx.x & 63;
    int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    float m = 0.0f;
    int bad = 0;
    for (int k = lane; k < K; k += 64) {
        float v = W[n * ld_n + (int64_t)k * ld_k];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    QuantParams p = quant_params(m);
    if (bad || !p.ok) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    if (lane == 0) scale[n] = p.scale_f;
    for (int k = lane; k < K; k += 64)
        Q[n * K + k] = (int8_t)quant_code(W[n * ld_n + (int64_t)k * ld_k], p.scale_d);
}

extern "C" int jtk_quant_weight_rows(const float *W, int64_t ld_n, int64_t ld_k, int N,
                                     int K, int8_t *Q, float *scale, uint32_t *err,
                                     hipStream_t s) {
    hipLaunchKernelGGL(k_quant_weight_rows, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s,
                       W, ld_n, ld_k, N, K, Q, scale, err);
    return (int)hipGetLastError();
}

// ---- W8A8 quantisation of every expert at once (the drop-in layer) ----
// The reference's W8A8 expert steps (src/moe_layer.c:185-274) quantise, per
// call and per expert, the expert's gathered activation rows per tensor (one
// scale over its rows) and its weights per output row (gate/up) or per
// tensor (down). These kernels do that for all experts in a few launches
// with k_absmax/k_quant_tensor's and k_quant_weight_rows's arithmetic.
// Experts that hold no pair (off[e + 1] == off[e]) are skipped, as the
// per-expert steps skip them: their weights are neither quantised nor
// checked. Activation rows come in the sorted order, one 16-row tile list
// entry {expert, first row, rows} per block.

// max|x| of each expert's rows of A [row][cols] into amax[expert] (float
// bits; amax zeroed before)
__global__ __launch_bounds__(256) void k_absmax_tiles(const float *__restrict__ A, int cols,
                                                      const int4 *__restrict__ tiles,
                                                      const int32_t *__restrict__ ntiles,
                                                      uint32_t *amax, uint32_t *err) {
    if ((int)blockIdx.x >= *ntiles) return;
    const int4 td = tiles[blockIdx.x];
    const float *a = A + (int64_t)td.y * cols;
    const int64_t n = (int64_t)td.z * cols;
    float m = 0.0f;
    int bad = 0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = a[i];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if ((threadIdx.x & 63) == 0) {
        atomicMax(amax + td.x, __float_as_uint(m));
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

// codes of each tile's rows with their expert's per-tensor scale, into Q
// [row][Kp] (K padding zero) and the row scales sA [row]
__global__ __launch_bounds__(256) void k_quant_tiles(const float *__restrict__ A, int cols,
                                                     const int4 *__restrict__ tiles,
                                                     const int32_t *__restrict__ ntiles,
                                                     const uint32_t *__restrict__ amax,
                                                     int8_t *__restrict__ Q, int Kp,
                                                     float *__restrict__ sA, uint32_t *err) {
    if ((int)blockIdx.x >= *ntiles) return;
    const int4 td = tiles[blockIdx.x];
    const QuantParams p = quant_params(__uint_as_float(amax[td.x]));
    if (!p.ok) {
        if (threadIdx.x == 0) raise_err(err, EF_RANGE);
        return;
    }
    const int64_t n = (int64_t)td.z * Kp;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const int64_t r = i / Kp;
        const int c = (int)(i % Kp);
        const int64_t row = td.y + r;
        Q[row * Kp + c] = c < cols ? (int8_t)quant_code(A[row * cols + c], p.scale_d) : 0;
    }
    if (threadIdx.x < td.z) sA[td.y + threadIdx.x] = p.scale_f;
}

extern "C" int jtk_quant_tiles(const float *A, int cols, const int32_t *tiles,
                               const int32_t *ntiles, int max_tiles, uint32_t *amax, int nexp,
                               int8_t *Q, int Kp, float *sA, uint32_t *err, hipStream_t s) {
    if (max_tiles <= 0) return 0;
    if (cols <= 0 || Kp < cols || nexp <= 0) return (int)hipErrorInvalidValue;
    int e = (int)hipMemsetAsync(amax, 0, (size_t)nexp * sizeof(uint32_t), s);
    hipLaunchKernelGGL(k_absmax_tiles, dim3((unsigned)max_tiles), dim3(256), 0, s, A, cols,
                       (const int4 *)tiles, ntiles, amax, err);
    hipLaunchKernelGGL(k_quant_tiles, dim3((unsigned)max_tiles), dim3(256), 0, s, A, cols,
                       (const int4 *)tiles, ntiles, amax, Q, Kp, sA, err);
    return e ? e : (int)hipGetLastError();
}

// Per-row weight codes of every expert's matrix W [E][N][K] (k_quant_weight_rows's
// arithmetic), one wavefront per row, into Q [E][N][K] and scale [E][N].
__global__ __launch_bounds__(256) void k_quant_weight_rows_e(const float *__restrict__ W,
                                                             int64_t rows, int N, int K,
                                                             const int32_t *__restrict__ off,
                                                             int8_t *__restrict__ Q,
                                                             float *__restrict__ scale,
                                                             uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= rows) return;
    const int64_t ex = n / N;
    if (off[ex + 1] == off[ex]) return;
    const float *w = W + n * K;
    float m = 0.0f;
    int bad = 0;
    for (int k = lane; k < K; k += 64) {
        const float v = w[k];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    const QuantParams p = quant_params(m);
    if (bad || !p.ok) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    if (lane == 0) scale[n] = p.scale_f;
    for (int k = lane; k < K; k += 64) Q[n * K + k] = (int8_t)quant_code(w[k], p.scale_d);
}

// Per-tensor codes of every expert's matrix W [E][nel] (k_absmax /
// k_quant_tensor's arithmetic): blockIdx.y is the expert. The scale is also
// broadcast to sBc [E][Np] (the GEMM's per-column scales).
__global__ __launch_bounds__(256) void k_absmax_mats(const float *__restrict__ W, int64_t nel,
                                                     const int32_t *__restrict__ off,
                                                     uint32_t *amax, uint32_t *err) {
    const int e = blockIdx.y;
    if (off[e + 1] == off[e]) return;
    const float *w = W + (int64_t)e * nel;
    float m = 0.0f;
    int bad = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nel;
         i += (int64_t)gridDim.x * 256) {
        const float v = w[i];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if ((threadIdx.x & 63) == 0) {
        atomicMax(amax + e, __float_as_uint(m));
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_quant_mats(const float *__restrict__ W, int64_t nel,
                                                    const int32_t *__restrict__ off,
                                                    const uint32_t *__restrict__ amax,
                                                    int8_t *__restrict__ Q,
                                                    float *__restrict__ sBc, int Np,
                                                    uint32_t *err) {
    const int e = blockIdx.y;
    if (off[e + 1] == off[e]) return;
    const QuantParams p = quant_params(__uint_as_float(amax[e]));
    if (!p.ok) {
        if (blockIdx.x == 0 && threadIdx.x == 0) raise_err(err, EF_RANGE);
        return;
    }
    if (blockIdx.x == 0)
        for (int c = threadIdx.x; c < Np; c += 256) sBc[(int64_t)e * Np + c] = p.scale_f;
    const float *w = W + (int64_t)e * nel;
    int8_t *q = Q + (int64_t)e * nel;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nel;
         i += (int64_t)gridDim.x * 256)
        q[i] = (int8_t)quant_code(w[i], p.scale_d);
}

// The MFMA panels of every expert's codes (k_pack_i8 with blockIdx.y the
// expert): Q [E][N][K] (kn = 0) or [E][K][N] (kn = 1) -> P [E][Np * Kp].
__global__ __launch_bounds__(256) void k_pack_i8_e(const int8_t *__restrict__ Q, int N, int K,
                                                   int kn, int Np, int Kp,
                                                   const int32_t *__restrict__ off,
                                                   int8_t *__restrict__ P) {
    const int e = blockIdx.y;
    if (off[e + 1] == off[e]) return;
    const int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte slot
    const int kblocks = Kp / 64;
    const int64_t nslots = (int64_t)(Np / 16) * kblocks * 64;
    if (slot >= nslots) return;
    const int8_t *q = Q + (int64_t)e * N * K;
    const int lane = (int)(slot & 63);
    const int64_t pk = slot >> 6;
    const int kb = (int)(pk % kblocks);
    const int pn = (int)(pk / kblocks);
    const int c = lane & 15, kc = lane >> 4;
    const int nn = pn * 16 + c;
    const int k0 = kb * 64 + kc * 16;
    union {
        int8_t b[16];
        v4i v;
    } u;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int k = k0 + j;
        int8_t v = 0;
        if (nn < N && k < K) v = kn ? q[(int64_t)k * N + nn] : q[(int64_t)nn * K + k];
        u.b[j] = v;
    }
    *(v4i *)(P + (int64_t)e * Np * Kp + slot * 16) = u.v;
}

// Every touched expert's weights as the W8A8 GEMM's panels: per output row
// (kn = 0, W [E][N][K]) or per tensor (kn = 1, W [E][K][N], amax: E words),
// codes through Q [E][N*K], panels into P [E][Np*Kp], per-column scales
// into sBc [E][Np] (per tensor: the expert's scale in every column).
extern "C" int jtk_w8a8_weights_e(const float *W, int E, int N, int K, int kn,
                                  const int32_t *off, int8_t *Q, int Np, int Kp, int8_t *P,
                                  float *sBc, uint32_t *amax, uint32_t *err, hipStream_t s) {
    if (E <= 0 || N <= 0 || K <= 0) return 0;
    if (E > 65535 || Np < N || Kp < K || Np % 16 || Kp % 64) return (int)hipErrorInvalidValue;
    int e = 0;
    if (!kn) {
        const int64_t rows = (int64_t)E * N;
        hipLaunchKernelGGL(k_quant_weight_rows_e, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                           s, W, rows, N, K, off, Q, sBc, err);
        // sBc [E][N] here; the GEMM reads it with stride N per expert
    } else {
        const int64_t nel = (int64_t)N * K;
        e = (int)hipMemsetAsync(amax, 0, (size_t)E * sizeof(uint32_t), s);
        const unsigned gx = grid_for(nel) > 64 ? 64 : grid_for(nel);
        hipLaunchKernelGGL(k_absmax_mats, dim3(gx, (unsigned)E), dim3(256), 0, s, W, nel, off,
                           amax, err);
        hipLaunchKernelGGL(k_quant_mats, dim3(gx, (unsigned)E), dim3(256), 0, s, W, nel, off,
                           amax, Q, sBc, Np, err);
    }
    const int64_t nslots = (int64_t)(Np / 16) * (Kp / 64) * 64;
    hipLaunchKernelGGL(k_pack_i8_e, dim3((unsigned)((nslots + 255) / 256), (unsigned)E),
                       dim3(256), 0, s, Q, N, K, kn, Np, Kp, off, P);
    return e ? e : (int)hipGetLastError();
}

// Load this file's code object now: the runtime otherwise loads it, and
// allocates device memory for it, at the first launch of one of its kernels.
extern "C" int jtk_preload_quant(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_quant_rows));
}
