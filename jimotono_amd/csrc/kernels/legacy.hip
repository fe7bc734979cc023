// Kernels behind the reference-compatible fp32 / T-MAC entry points (gfx950).
//
//  k_gemm_f32      : C[m][n] = fp32 sum over k ascending of A[m][k]*B[k][n],
//                    one rounded multiply and one rounded add per step (no
//                    contraction), bit-identical to src/moe_gemm.c:47-89.
//  k_transpose_f32 : exact transpose through an LDS tile.
//  k_tmac_ctor     : the reference's activation lookup tables
//                    (src/tmac.c:230-385), one thread per 32-activation block.
//  k_col_to_idx    : weight column -> bit-planes + max-abs (src/lowbit.c:93-141)
//  k_tmac_gemm     : Y[m][j] through lookup + fp64 aggregation + sign fix
//                    (src/lowbit.c:238-253, src/tmac.c:387-506), one thread
//                    per output.
//  k_lowbit_fq     : per-column fake-quant of a [K][H] matrix
//                    (src/moe_layer.c:24-53 with src/lowbit.c:47-91).
#include "jt_dev.h"
#include "jt_launch.h"

// One thread per output; a 16 x 16 output tile per block with A and B
// staged in LDS in k chunks of 16. The k order per output is sequential.
__global__ __launch_bounds__(256) void k_gemm_f32(const float *__restrict__ A,
                                                  const float *__restrict__ B,
                                                  float *__restrict__ C, int M, int N, int K,
                                                  uint32_t *err) {
    __shared__ float as[16][17];
    __shared__ float bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m = blockIdx.y * 16 + ty, n = blockIdx.x * 16 + tx;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 16) {
        const int ka = k0 + tx, kb = k0 + ty;
        as[ty][tx] = (m < M && ka < K) ? A[(int64_t)m * K + ka] : 0.0f;
        bs[ty][tx] = (kb < K && n < N) ? B[(int64_t)kb * N + n] : 0.0f;
        __syncthreads();
        const int kend = min(16, K - k0);
        for (int kk = 0; kk < kend; kk++) {
            const float p = __fmul_rn(as[ty][kk], bs[kk][tx]);
            acc = __fadd_rn(acc, p);
        }
        __syncthreads();
    }
    if (m < M && n < N) {
        if (!isfinite(acc)) raise_err(err, EF_NONFINITE_MID);
        C[(int64_t)m * N + n] = acc;
    }
}

extern "C" int jtk_gemm_f32(const float *A, const float *B, float *C, int M, int N, int K,
                            uint32_t *err, hipStream_t s) {
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
    hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, s, A, B, C, M, N, K, err);
    return (int)hipGetLastError();
}

// dst[c][r] = src[r][c]; 32 x 32 tiles (blockDim 32 x 8).
__global__ __launch_bounds__(256) void k_transpose_f32(const float *__restrict__ src,
                                                       float *__restrict__ dst, int rows,
                                                       int cols) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int j = ty; j < 32; j += 8) {
        const int r = by + j, c = bx + tx;
        if (r < rows && c < cols) tile[j][tx] = src[(int64_t)r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const int c = bx + j, r = by + tx;
        if (r < rows && c < cols) dst[(int64_t)c * rows + r] = tile[tx][j];
    }
}

extern "C" int jtk_transpose_f32(const float *src, float *dst, int rows, int cols,
                                 hipStream_t s) {
    dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(k_transpose_f32, grid, dim3(256), 0, s, src, dst, rows, cols);
    return (int)hipGetLastError();
}

// ---- T-MAC lookup tables ----
__global__ __launch_bounds__(256) void k_tmac_ctor(const float *__restrict__ act,
                                                   int64_t n, int64_t k,
                                                   int8_t *__restrict__ qlut,
                                                   float *__restrict__ scales,
                                                   float *__restrict__ biases, uint32_t *err) {
    const int64_t nb = k / 32;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= n * nb) return;
    const int64_t r = id / nb, bb = id % nb;
    const float *a = act + r * k + bb * 32;
    int8_t *qb = qlut + r * (k / 4) * 8 + bb * 64;
    float av[32];
    bool bad = false;
    for (int i = 0; i < 32; i++) {
        av[i] = a[i];
        bad |= !isfinite(av[i]);
    }
    if (bad) {
        raise_err(err, EF_NONFINITE_INPUT);
        return;
    }
    // F[g][p] = sum_j (bit j of p ? +a : -a) in j order; |F(p)| = |F(15-p)|
    double maxabs = 0.0;
    for (int g = 0; g < 8; g++)
        for (int p = 0; p < 16; p++) {
            double s = 0.0;
            for (int j = 0; j < 4; j++) s += (((p >> j) & 1) ? 1.0 : -1.0) * (double)av[g * 4 + j];
            const double aa = s >= 0.0 ? s : -s;
            if (aa > maxabs) maxabs = aa;
        }
    double asum = 0.0;
    for (int i = 0; i < 32; i++) asum += (double)av[i];
    const float bias_f = (float)asum;
    if (!isfinite(maxabs) || !isfinite(asum)) {
        raise_err(err, EF_NONFINITE_INPUT);
        return;
    }
    if (maxabs == 0.0) {
        if (!isfinite(bias_f)) raise_err(err, EF_RANGE);
        for (int i = 0; i < 64; i++) qb[i] = 0;
        scales[id] = 1.0f;
        biases[id] = bias_f;
        return;
    }
    const double scale_d = maxabs / 127.0;
    const float scale_f = (float)scale_d;
    if (!isfinite(scale_d) || scale_d <= 0.0 || !isfinite(scale_f) || !isfinite(bias_f)) {
        raise_err(err, EF_RANGE);
        return;
    }
    for (int g = 0; g < 8; g++)
        for (int ii = 0; ii < 8; ii++) {
            const int p = 8 + ii;
            double s = 0.0;
            for (int j = 0; j < 4; j++) s += (((p >> j) & 1) ? 1.0 : -1.0) * (double)av[g * 4 + j];
            double qd = round(s / scale_d);
            qd = qd > 127.0 ? 127.0 : (qd < -128.0 ? -128.0 : qd);
            qb[g * 8 + ii] = (int8_t)(int)qd;
        }
    scales[id] = scale_f;
    biases[id] = bias_f;
}

extern "C" int jtk_tmac_ctor(const float *act, int64_t n, int64_t k, int8_t *qlut,
                             float *scales, float *biases, uint32_t *err, hipStream_t s) {
    const int64_t th = n * (k / 32);
    hipLaunchKernelGGL(k_tmac_ctor, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, act,
                       n, k, qlut, scales, biases, err);
    return (int)hipGetLastError();
}

// Bit-planes of the columns of W[k][h] (column j -> idx[j][bits][k/4],
// ws[j] = max|col|). One thread per (column, group of 4).
__global__ __launch_bounds__(256) void k_col_maxabs(const float *__restrict__ W, int k, int h,
                                                    float *__restrict__ ws, uint32_t *err) {
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (j >= h) return;
    float m = 0.0f;
    int bad = 0;
    for (int t = lane; t < k; t += 64) {
        const float v = W[(int64_t)t * h + j];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if (lane == 0) {
        ws[j] = m;
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_col_to_idx(const float *__restrict__ W, int k, int h,
                                                    int bits, const float *__restrict__ ws,
                                                    uint8_t *__restrict__ idx) {
    const int64_t ng = k / 4;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)h * ng) return;
    const int j = (int)(id / ng);
    const int64_t g = id % ng;
    const double maxa = (double)ws[j];
    int li[4];
    for (int q = 0; q < 4; q++) li[q] = lowbit_code((double)W[(g * 4 + q) * h + j], maxa, bits);
    uint8_t *dst = idx + (int64_t)j * bits * ng;
    for (int b = 0; b < bits; b++) {
        unsigned p = 0;
        for (int q = 0; q < 4; q++)
            if ((li[q] >> b) & 1) p |= 1u << q;
        dst[(int64_t)b * ng + g] = (uint8_t)p;
    }
}

extern "C" int jtk_col_to_idx(const float *W, int k, int h, int bits, float *ws,
                              uint8_t *idx, uint32_t *err, hipStream_t s) {
    hipLaunchKernelGGL(k_col_maxabs, dim3((unsigned)((h + 3) / 4)), dim3(256), 0, s, W, k, h,
                       ws, err);
    const int64_t th = (int64_t)h * (k / 4);
    hipLaunchKernelGGL(k_col_to_idx, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, W, k,
                       h, bits, ws, idx);
    return (int)hipGetLastError();
}

// One lookup-accumulate dot (src/tmac.c:387-506, scalar aggregation order).
__device__ bool tmac_dot(const int8_t *qrow, const uint8_t *idx, const float *sc,
                         const float *bi, int64_t ng, int64_t nb, int bits, float w_scale,
                         float *out) {
    double total = 0.0;
    for (int64_t bb = 0; bb < nb; bb++) {
        const double s = (double)sc[bb], b0 = (double)bi[bb];
        const int8_t *qb = qrow + bb * 64;
        for (int b = 0; b < bits; b++) {
            const uint8_t *plane = idx + (int64_t)b * ng + bb * 8;
            int32_t acc = 0;
            for (int gi = 0; gi < 8; gi++) {
                const unsigned p = plane[gi] & 0x0Fu;
                acc += (p >= 8u) ? (int)qb[gi * 8 + (p - 8u)] : -(int)qb[gi * 8 + (7u - p)];
            }
            const double contrib = (s * (double)acc + b0) * 0.5;
            total += contrib * (double)(1 << b);
            if (!isfinite(total)) return false;
        }
    }
    total *= (double)w_scale;
    if (!isfinite(total)) return false;
    const float f = (float)total;
    if (!isfinite(f)) return false;
    *out = f;
    return true;
}

// rowsum[m] = sum_t (double)X[m][t] in t order.
__global__ __launch_bounds__(256) void k_rowsum_f64(const float *__restrict__ X, int me, int k,
                                                    double *__restrict__ rs) {
    const int m = blockIdx.x * 256 + threadIdx.x;
    if (m >= me) return;
    double s = 0.0;
    for (int t = 0; t < k; t++) s += (double)X[(int64_t)m * k + t];
    rs[m] = s;
}

__global__ __launch_bounds__(256) void k_tmac_gemm(const int8_t *__restrict__ qlut,
                                                   const float *__restrict__ sc,
                                                   const float *__restrict__ bi,
                                                   const double *__restrict__ rowsum,
                                                   const uint8_t *__restrict__ idx,
                                                   const float *__restrict__ ws, int me, int h,
                                                   int k, int bits, float *__restrict__ Y,
                                                   uint32_t *err) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)me * h) return;
    const int m = (int)(id / h), j = (int)(id % h);
    const int64_t ng = k / 4, nb = k / 32;
    float o = 0.0f;
    if (!tmac_dot(qlut + (int64_t)m * ng * 8, idx + (int64_t)j * bits * ng, sc + (int64_t)m * nb,
                  bi + (int64_t)m * nb, ng, nb, bits, ws[j], &o)) {
        raise_err(err, EF_RANGE);
        return;
    }
    const double n1 = (double)((1 << bits) - 1);
    Y[id] = (float)((2.0 * (double)o - n1 * (double)ws[j] * rowsum[m]) / n1);
}

extern "C" int jtk_tmac_gemm(const int8_t *qlut, const float *sc, const float *bi,
                             const double *rowsum, const uint8_t *idx, const float *ws, int me,
                             int h, int k, int bits, float *Y, uint32_t *err, hipStream_t s) {
    const int64_t th = (int64_t)me * h;
    hipLaunchKernelGGL(k_tmac_gemm, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, qlut,
                       sc, bi, rowsum, idx, ws, me, h, k, bits, Y, err);
    return (int)hipGetLastError();
}

extern "C" int jtk_rowsum_f64(const float *X, int me, int k, double *rs, hipStream_t s) {
    hipLaunchKernelGGL(k_rowsum_f64, dim3((unsigned)((me + 255) / 256)), dim3(256), 0, s, X, me,
                       k, rs);
    return (int)hipGetLastError();
}

// Single lookup-accumulate (jt_tmac_lookup_accum) on one thread.
__global__ void k_tmac_lookup1(const int8_t *qlut, const uint8_t *idx, const float *sc,
                               const float *bi, int64_t ng, int64_t nb, int bits,
                               float w_scale, float *out, uint32_t *err) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float o = 0.0f;
    if (!tmac_dot(qlut, idx, sc, bi, ng, nb, bits, w_scale, &o)) {
        raise_err(err, EF_RANGE);
        return;
    }
    *out = o;
}

extern "C" int jtk_tmac_lookup1(const int8_t *qlut, const uint8_t *idx, const float *sc,
                                const float *bi, int64_t ng, int64_t nb, int bits,
                                float w_scale, float *out, uint32_t *err, hipStream_t s) {
    hipLaunchKernelGGL(k_tmac_lookup1, dim3(1), dim3(64), 0, s, qlut, idx, sc, bi, ng, nb, bits,
                       w_scale, out, err);
    return (int)hipGetLastError();
}

// fp64-accumulated GEMM (the K % 32 fallback, src/lowbit.c:144-156).
__global__ __launch_bounds__(256) void k_gemm_f64acc(const float *__restrict__ A,
                                                     const float *__restrict__ B,
                                                     float *__restrict__ C, int M, int N,
                                                     int K) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)M * N) return;
    const int m = (int)(id / N), n = (int)(id % N);
    double acc = 0.0;
    for (int t = 0; t < K; t++)
        acc = acc + (double)A[(int64_t)m * K + t] * (double)B[(int64_t)t * N + n];
    C[id] = (float)acc;
}

extern "C" int jtk_gemm_f64acc(const float *A, const float *B, float *C, int M, int N, int K,
                               hipStream_t s) {
    const int64_t th = (int64_t)M * N;
    hipLaunchKernelGGL(k_gemm_f64acc, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, A, B,
                       C, M, N, K);
    return (int)hipGetLastError();
}

// Low-bit fake-quant of each column of W[k][h] in place
// (src/moe_layer.c:24-53 calling src/lowbit.c:47-91); ws holds max|col|.
__global__ __launch_bounds__(256) void k_lowbit_fq_cols(float *__restrict__ W, int k, int h,
                                                        int bits,
                                                        const float *__restrict__ ws) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)k * h) return;
    const int j = (int)(id % h);
    const double maxa = (double)ws[j];
    if (maxa == 0.0) {
        W[id] = 0.0f;
        return;
    }
    const double nn = (double)((1 << bits) - 1);
    const int l = lowbit_code((double)W[id], maxa, bits);
    W[id] = (float)(((2.0 * (double)l - nn) / nn) * maxa);
}

extern "C" int jtk_lowbit_fq_cols(float *W, int k, int h, int bits, float *ws, uint32_t *err,
                                  hipStream_t s) {
    hipLaunchKernelGGL(k_col_maxabs, dim3((unsigned)((h + 3) / 4)), dim3(256), 0, s, W, k, h,
                       ws, err);
    const int64_t th = (int64_t)k * h;
    hipLaunchKernelGGL(k_lowbit_fq_cols, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, W,
                       k, h, bits, ws);
    return (int)hipGetLastError();
}

// ---- fake-quant of every expert's weights at once ----
// The low-bit fake-quant mode of the drop-in layer quantises, per call, each
// routed expert's gate/up matrix per row (a column of the transposed matrix
// that the per-expert sequence hands to jtk_lowbit_fq_cols) and its down
// matrix per column. These two entry points do that for all experts in two
// launches each, with k_col_maxabs's maximum and k_lowbit_fq_cols's value
// formula, so every weight comes out as the per-expert sequence's. With the
// expert offsets off, experts that hold no pair are skipped, as the
// per-expert sequence skips them (their weights are neither quantised nor
// checked).
// Rows of W [rows][cols], one wavefront per row; rpe rows per expert.
__global__ __launch_bounds__(256) void k_row_maxabs(const float *__restrict__ W, int64_t rows,
                                                    int cols, const int32_t *__restrict__ off,
                                                    int rpe, float *__restrict__ ws,
                                                    uint32_t *err) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    if (off && off[r / rpe + 1] == off[r / rpe]) return;
    const float *w = W + r * cols;
    float m = 0.0f;
    int bad = 0;
    for (int t = lane; t < cols; t += 64) {
        const float v = w[t];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if (lane == 0) {
        ws[r] = m;
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_lowbit_fq_rows(float *__restrict__ W, int64_t rows,
                                                        int cols, const int32_t *__restrict__ off,
                                                        int rpe, int bits,
                                                        const float *__restrict__ ws) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= rows * cols) return;
    const int64_t r = id / cols;
    if (off && off[r / rpe + 1] == off[r / rpe]) return;
    const double maxa = (double)ws[r];
    if (maxa == 0.0) {
        W[id] = 0.0f;
        return;
    }
    const double nn = (double)((1 << bits) - 1);
    const int l = lowbit_code((double)W[id], maxa, bits);
    W[id] = (float)(((2.0 * (double)l - nn) / nn) * maxa);
}

// every row of W [rows][cols] (ws: rows floats)
extern "C" int jtk_lowbit_fq_rows(float *W, int64_t rows, int cols, const int32_t *off, int rpe,
                                  int bits, float *ws, uint32_t *err, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return 0;
    if (off && rpe <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_row_maxabs, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, W, rows,
                       cols, off, rpe, ws, err);
    const int64_t th = rows * cols;
    hipLaunchKernelGGL(k_lowbit_fq_rows, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, W,
                       rows, cols, off, rpe, bits, ws);
    return (int)hipGetLastError();
}

// every column of each of nb matrices [k][h] stored back to back (ws: nb * h
// floats); blockIdx.y is the matrix
__global__ __launch_bounds__(256) void k_col_maxabs_b(const float *__restrict__ W, int k, int h,
                                                      const int32_t *__restrict__ off,
                                                      float *__restrict__ ws, uint32_t *err) {
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (j >= h) return;
    if (off && off[blockIdx.y + 1] == off[blockIdx.y]) return;
    const float *w = W + (int64_t)blockIdx.y * k * h;
    float m = 0.0f;
    int bad = 0;
    for (int t = lane; t < k; t += 64) {
        const float v = w[(int64_t)t * h + j];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if (lane == 0) {
        ws[(int64_t)blockIdx.y * h + j] = m;
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_lowbit_fq_cols_b(float *__restrict__ W, int k, int h,
                                                          const int32_t *__restrict__ off,
                                                          int bits,
                                                          const float *__restrict__ ws) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)k * h) return;
    if (off && off[blockIdx.y + 1] == off[blockIdx.y]) return;
    float *w = W + (int64_t)blockIdx.y * k * h;
    const double maxa = (double)ws[(int64_t)blockIdx.y * h + id % h];
    if (maxa == 0.0) {
        w[id] = 0.0f;
        return;
    }
    const double nn = (double)((1 << bits) - 1);
    const int l = lowbit_code((double)w[id], maxa, bits);
    w[id] = (float)(((2.0 * (double)l - nn) / nn) * maxa);
}

extern "C" int jtk_lowbit_fq_cols_batch(float *W, int nb, int k, int h, const int32_t *off,
                                        int bits, float *ws, uint32_t *err, hipStream_t s) {
    if (nb <= 0 || k <= 0 || h <= 0) return 0;
    if (nb > 65535) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_col_maxabs_b, dim3((unsigned)((h + 3) / 4), (unsigned)nb), dim3(256), 0,
                       s, W, k, h, off, ws, err);
    const int64_t th = (int64_t)k * h;
    hipLaunchKernelGGL(k_lowbit_fq_cols_b, dim3((unsigned)((th + 255) / 256), (unsigned)nb),
                       dim3(256), 0, s, W, k, h, off, bits, ws);
    return (int)hipGetLastError();
}

// ---- the T-MAC LUT GEMM of every expert at once (drop-in layer, mode 2) ----
// jt_dev_lowbit_gemm_lut's steps for all experts: the activation tables and
// row sums are per row, so they run over every sorted row in one launch
// each; the weights' bit-plane indices and column maxima come from a strided
// view of each expert's matrix (element t of column j of expert e at
// W[e estride + t tstride + j jstride]: the rows of a [h][n] matrix for the
// transposed gate/up, the columns of [h][n] for the down); the lookup GEMM
// finds each row's expert from the offsets. Same arithmetic per element as
// k_col_maxabs, k_col_to_idx and k_tmac_gemm. Experts that hold no pair are
// skipped (neither indexed nor checked).
__global__ __launch_bounds__(256) void k_col_maxabs_s(const float *__restrict__ W, int k, int h,
                                                      int64_t estride, int64_t tstride,
                                                      int64_t jstride,
                                                      const int32_t *__restrict__ off,
                                                      float *__restrict__ ws, uint32_t *err) {
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int e = blockIdx.y;
    const int lane = threadIdx.x & 63;
    if (j >= h || off[e + 1] == off[e]) return;
    const float *w = W + (int64_t)e * estride + (int64_t)j * jstride;
    float m = 0.0f;
    int bad = 0;
    for (int t = lane; t < k; t += 64) {
        const float v = w[(int64_t)t * tstride];
        bad |= !isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    if (lane == 0) {
        ws[(int64_t)e * h + j] = m;
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

__global__ __launch_bounds__(256) void k_col_to_idx_s(const float *__restrict__ W, int k, int h,
                                                      int64_t estride, int64_t tstride,
                                                      int64_t jstride,
                                                      const int32_t *__restrict__ off, int bits,
                                                      const float *__restrict__ ws,
                                                      uint8_t *__restrict__ idx) {
    const int64_t ng = k / 4;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int e = blockIdx.y;
    if (id >= (int64_t)h * ng || off[e + 1] == off[e]) return;
    const int j = (int)(id / ng);
    const int64_t g = id % ng;
    const double maxa = (double)ws[(int64_t)e * h + j];
    const float *w = W + (int64_t)e * estride + (int64_t)j * jstride;
    int li[4];
    for (int q = 0; q < 4; q++) li[q] = lowbit_code((double)w[(g * 4 + q) * tstride], maxa, bits);
    uint8_t *dst = idx + ((int64_t)e * h + j) * bits * ng;
    for (int b = 0; b < bits; b++) {
        unsigned p = 0;
        for (int q = 0; q < 4; q++)
            if ((li[q] >> b) & 1) p |= 1u << q;
        dst[(int64_t)b * ng + g] = (uint8_t)p;
    }
}

extern "C" int jtk_col_to_idx_e(const float *W, int E, int k, int h, int64_t estride,
                                int64_t tstride, int64_t jstride, const int32_t *off, int bits,
                                float *ws, uint8_t *idx, uint32_t *err, hipStream_t s) {
    if (E <= 0 || k <= 0 || h <= 0) return 0;
    if (E > 65535 || k % 4) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_col_maxabs_s, dim3((unsigned)((h + 3) / 4), (unsigned)E), dim3(256), 0,
                       s, W, k, h, estride, tstride, jstride, off, ws, err);
    const int64_t th = (int64_t)h * (k / 4);
    hipLaunchKernelGGL(k_col_to_idx_s, dim3((unsigned)((th + 255) / 256), (unsigned)E),
                       dim3(256), 0, s, W, k, h, estride, tstride, jstride, off, bits, ws, idx);
    return (int)hipGetLastError();
}

// Y [row][h] for every sorted row (rows < off[E]); the row's expert e is
// the one with off[e] <= row < off[e + 1]
__global__ __launch_bounds__(256) void k_tmac_gemm_e(const int8_t *__restrict__ qlut,
                                                     const float *__restrict__ sc,
                                                     const float *__restrict__ bi,
                                                     const double *__restrict__ rowsum,
                                                     const uint8_t *__restrict__ idx,
                                                     const float *__restrict__ ws,
                                                     const int32_t *__restrict__ off, int E,
                                                     int rows, int h, int k, int bits,
                                                     float *__restrict__ Y, uint32_t *err) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (int64_t)rows * h) return;
    const int m = (int)(id / h), j = (int)(id % h);
    int lo = 0, hi = E;  // the last e with off[e] <= m (off[0] = 0 <= m)
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= m) lo = mid;
        else hi = mid;
    }
    const int e = lo;
    const int64_t ng = k / 4, nb = k / 32;
    const int64_t col = (int64_t)e * h + j;
    float o = 0.0f;
    if (!tmac_dot(qlut + (int64_t)m * ng * 8, idx + col * bits * ng, sc + (int64_t)m * nb,
                  bi + (int64_t)m * nb, ng, nb, bits, ws[col], &o)) {
        raise_err(err, EF_RANGE);
        return;
    }
    const double n1 = (double)((1 << bits) - 1);
    Y[id] = (float)((2.0 * (double)o - n1 * (double)ws[col] * rowsum[m]) / n1);
}

extern "C" int jtk_tmac_gemm_e(const int8_t *qlut, const float *sc, const float *bi,
                               const double *rowsum, const uint8_t *idx, const float *ws,
                               const int32_t *off, int E, int rows, int h, int k, int bits,
                               float *Y, uint32_t *err, hipStream_t s) {
    if (rows <= 0) return 0;
    if (E <= 0 || h <= 0 || k % 32) return (int)hipErrorInvalidValue;
    const int64_t th = (int64_t)rows * h;
    hipLaunchKernelGGL(k_tmac_gemm_e, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, qlut,
                       sc, bi, rowsum, idx, ws, off, E, rows, h, k, bits, Y, err);
    return (int)hipGetLastError();
}

// Load this file's code object now: the runtime otherwise loads it, and
// allocates device memory for it, at the first launch of one of its kernels.
extern "C" int jtk_preload_legacy(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_gemm_f32));
}

// ---- grouped fp32 expert FFN of the drop-in layer (flags off) ----
// The per-expert sequence gather -> transpose -> k_gemm_f32 (gate, up) ->
// SwiGLU -> k_gemm_f32 (down) -> scatter of src/moe_layer.c:1265-1420 (and the
// shared experts of :1468-1560), as two launches over every expert at once:
// a block computes 16 rows x 16 columns, the rows of one (expert, 16-row)
// tile of the sorted pairs (or, dense, 16 token rows of shared expert
// blockIdx.z). Every output is k_gemm_f32's k-ordered fp32 sum (one rounded
// multiply and one rounded add per step; the transpose is a copy, so reading
// W[j][k] directly gives the same products), and the SwiGLU is
// k_silu_tile's, so the results are those of the per-expert launches.
//   gate/up: G, U [row][h] (optional caches, scattered to the pair's row or
//            to [token][S][h]), S [row][h] (sorted rows, or [s][T][h]);
//   down:    Y [pair][n] (routed, scattered by perm) or [s][T][n] (dense).
__global__ __launch_bounds__(256) void k_ffn_gu_f32(
    const float *__restrict__ X, int n, int h, const int32_t *__restrict__ perm, int topk,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ ntiles, int T, int S,
    const float *__restrict__ Wg, const float *__restrict__ Wu, float *__restrict__ Gc,
    float *__restrict__ Uc, float *__restrict__ Sout, int dense, uint32_t *err) {
    __shared__ float as[16][17];
    __shared__ float bg[16][17];
    __shared__ float bu[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    int e, pos0, nrows;
    if (dense) {
        e = blockIdx.z;
        pos0 = blockIdx.y * 16;
        nrows = min(16, T - pos0);
    } else {
        if ((int)blockIdx.y >= *ntiles) return;
        const int4 td = tiles[blockIdx.y];  // {expert, first sorted row, rows}
        e = td.x;
        pos0 = td.y;
        nrows = td.z;
    }
    const int j0 = blockIdx.x * 16;
    const int rr = min(ty, nrows - 1);
    const int q = dense ? pos0 + rr : perm[pos0 + rr];   // token (dense) or pair index
    const int src = dense ? q : q / topk;                // token row of X
    const float *xa = X + (int64_t)src * n;
    const int64_t wo = (int64_t)e * h * n;
    const int jb = min(j0 + ty, h - 1);  // the weight row this thread stages
    float ag = 0.0f, au = 0.0f;
    for (int k0 = 0; k0 < n; k0 += 16) {
        const int ka = k0 + tx;
        as[ty][tx] = ka < n ? xa[ka] : 0.0f;
        bg[ty][tx] = ka < n ? Wg[wo + (int64_t)jb * n + ka] : 0.0f;
        bu[ty][tx] = ka < n ? Wu[wo + (int64_t)jb * n + ka] : 0.0f;
        __syncthreads();
        const int kend = min(16, n - k0);
        for (int kk = 0; kk < kend; kk++) {
            ag = __fadd_rn(ag, __fmul_rn(as[ty][kk], bg[tx][kk]));
            au = __fadd_rn(au, __fmul_rn(as[ty][kk], bu[tx][kk]));
        }
        __syncthreads();
    }
    const int j = j0 + tx;
    if (ty >= nrows || j >= h) return;
    uint32_t f = 0;
    if (!isfinite(ag) || !isfinite(au)) f |= EF_NONFINITE_MID;
    float sv;
    if (!silu_mul(ag, au, &sv)) f |= EF_NONFINITE_MID;
    const int64_t row = dense ? (int64_t)e * T + pos0 + ty : pos0 + ty;
    Sout[row * h + j] = sv;
    const int64_t crow = dense ? ((int64_t)(pos0 + ty) * S + e) : q;
    if (Gc) Gc[crow * h + j] = ag;
    if (Uc) Uc[crow * h + j] = au;
    if (f) raise_err(err, f);
}

__global__ __launch_bounds__(256) void k_ffn_dn_f32(
    const float *__restrict__ Sin, int h, int n, const int32_t *__restrict__ perm,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ ntiles, int T,
    const float *__restrict__ Wd, float *__restrict__ Y, int dense, uint32_t *err) {
    __shared__ float as[16][17];
    __shared__ float bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    int e, pos0, nrows;
    if (dense) {
        e = blockIdx.z;
        pos0 = blockIdx.y * 16;
        nrows = min(16, T - pos0);
    } else {
        if ((int)blockIdx.y >= *ntiles) return;
        const int4 td = tiles[blockIdx.y];
        e = td.x;
        pos0 = td.y;
        nrows = td.z;
    }
    const int c0 = blockIdx.x * 16;
    const int rr = min(ty, nrows - 1);
    const int64_t arow = dense ? (int64_t)e * T + pos0 + rr : pos0 + rr;
    const float *sa = Sin + arow * h;
    const float *wd = Wd + (int64_t)e * h * n;
    const int cb = min(c0 + tx, n - 1);
    float acc = 0.0f;
    for (int k0 = 0; k0 < h; k0 += 16) {
        const int ka = k0 + tx, kb = k0 + ty;
        as[ty][tx] = ka < h ? sa[ka] : 0.0f;
        bs[ty][tx] = kb < h ? wd[(int64_t)kb * n + cb] : 0.0f;
        __syncthreads();
        const int kend = min(16, h - k0);
        for (int kk = 0; kk < kend; kk++) acc = __fadd_rn(acc, __fmul_rn(as[ty][kk], bs[kk][tx]));
        __syncthreads();
    }
    const int c = c0 + tx;
    if (ty >= nrows || c >= n) return;
    if (!isfinite(acc)) raise_err(err, EF_NONFINITE_MID);
    const int64_t orow = dense ? (int64_t)e * T + pos0 + ty : perm[pos0 + ty];
    Y[orow * n + c] = acc;
}

extern "C" int jtk_ffn_f32(const float *X, int T, int n, int h, const int32_t *perm, int topk,
                           const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                           const float *Wg, const float *Wu, const float *Wd, int nexp,
                           float *Gc, float *Uc, float *Sbuf, float *Y, int dense,
                           uint32_t *err, hipStream_t s) {
    if (T <= 0 || n <= 0 || h <= 0 || nexp <= 0) return 0;
    const unsigned gy = dense ? (unsigned)((T + 15) / 16) : (unsigned)max_tiles;
    const unsigned gz = dense ? (unsigned)nexp : 1u;
    if (gy == 0 || gy > 0x7fffffffu || gz > 65535u) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_ffn_gu_f32, dim3((unsigned)((h + 15) / 16), gy, gz), dim3(256), 0, s,
                       X, n, h, perm, topk, (const int4 *)tiles, ntiles, T, nexp, Wg, Wu, Gc,
                       Uc, Sbuf, dense, err);
    hipLaunchKernelGGL(k_ffn_dn_f32, dim3((unsigned)((n + 15) / 16), gy, gz), dim3(256), 0, s,
                       Sbuf, h, n, perm, (const int4 *)tiles, ntiles, T, Wd, Y, dense, err);
    return (int)hipGetLastError();
}
