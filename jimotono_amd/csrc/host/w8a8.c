/*
 * w8a8.c -- host side of the W8A8 path (C11).
 *
 * The jt_w8a8_* functions keep the reference's signatures and fail-closed
 * contract (include/jimotono/w8a8.h:61-121, src/w8a8.c): argument checks run
 * on the host before anything is staged; data checks (non-finite values,
 * -128 codes) and computed-overflow checks run in the kernels and raise bits
 * in the device error word; outputs are copied back only when no bit was
 * raised, so no error leaves an output partially written.
 */
#include <errno.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jimotono/hip_moe.h"
#include "jimotono/w8a8.h"
#include "jt_rt.h"

#define FAIL(code, e) \
    do {              \
        errno = (e);  \
        return (code); \
    } while (0)

static int g_w8a8_enabled = 0; /* reference src/w8a8.c:53 */

int jt_w8a8_set_enabled(int enabled) {
    if (enabled != 0 && enabled != 1) FAIL(JT_ERR_INVAL, EINVAL);
    g_w8a8_enabled = enabled;
    return JT_OK;
}

int jt_w8a8_get_enabled(int *out_enabled) {
    if (!out_enabled) FAIL(JT_ERR_INVAL, EINVAL);
    *out_enabled = g_w8a8_enabled;
    return JT_OK;
}

int jt_w8a8_is_enabled(void) { return g_w8a8_enabled; }

/* ---------------- quantisation ---------------- */

int jt_w8a8_quant_per_tensor(const float *src, size_t n, int8_t *dst, float *out_scale) {
    if (!src || !dst || !out_scale || n == 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dx = jt_rt_buf(rt, JT_SLOT_A, n * sizeof(float), &rc);
    int8_t *dq = jt_rt_buf(rt, JT_SLOT_B, n, &rc);
    float *ds = jt_rt_buf(rt, JT_SLOT_C, sizeof(float), &rc);
    if (!dx || !dq || !ds) return rc;
    if ((rc = jt_rt_h2d(rt, dx, src, n * sizeof(float))) != JT_OK) return rc;
    if (jtk_quant_tensor(dx, (int64_t)n, dq, ds, rt->d_scratch, jt_rt_errw(rt, rt->stream), rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    float s = 0.0f;
    if ((rc = jt_rt_d2h(rt, &s, ds, sizeof(float))) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, dst, dq, n)) != JT_OK) return rc;
    *out_scale = s;
    return JT_OK;
}

int jt_w8a8_quant_per_channel(const float *src, size_t rows, size_t cols, int8_t *dst,
                              float *scales) {
    if (!src || !dst || !scales || rows == 0 || cols == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (rows > SIZE_MAX / cols || cols > INT32_MAX) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    size_t n = rows * cols;
    float *dx = jt_rt_buf(rt, JT_SLOT_A, n * sizeof(float), &rc);
    int8_t *dq = jt_rt_buf(rt, JT_SLOT_B, n, &rc);
    float *ds = jt_rt_buf(rt, JT_SLOT_C, rows * sizeof(float), &rc);
    if (!dx || !dq || !ds) return rc;
    if ((rc = jt_rt_h2d(rt, dx, src, n * sizeof(float))) != JT_OK) return rc;
    /* the reference checks the whole array before any row (src/w8a8.c:803-811) */
    jtk_check_finite(dx, (int64_t)n, jt_rt_errw(rt, rt->stream), rt->stream);
    if (jtk_quant_rows(dx, (int64_t)rows, (int)cols, dq, (int64_t)cols, ds, NULL, jt_rt_errw(rt, rt->stream),
                       rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, dst, dq, n)) != JT_OK) return rc;
    return jt_rt_d2h(rt, scales, ds, rows * sizeof(float));
}

static int dequant_common(const int8_t *src, const float *scales, size_t rows, size_t cols,
                          int per_row, float *dst) {
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    size_t n = rows * cols;
    int8_t *dq = jt_rt_buf(rt, JT_SLOT_A, n, &rc);
    float *ds = jt_rt_buf(rt, JT_SLOT_B, rows * sizeof(float), &rc);
    float *dd = jt_rt_buf(rt, JT_SLOT_C, n * sizeof(float), &rc);
    if (!dq || !ds || !dd) return rc;
    if ((rc = jt_rt_h2d(rt, dq, src, n)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, ds, scales, (per_row ? rows : 1) * sizeof(float))) != JT_OK)
        return rc;
    if (jtk_dequant(dq, ds, (int64_t)rows, (int64_t)cols, per_row, dd, jt_rt_errw(rt, rt->stream), rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    return jt_rt_d2h(rt, dst, dd, n * sizeof(float));
}

int jt_w8a8_dequant_per_tensor(const int8_t *src, float scale, size_t n, float *dst) {
    if (!src || !dst || n == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (!isfinite((double)scale) || scale <= 0.0f) FAIL(JT_ERR_INVAL, EINVAL);
    return dequant_common(src, &scale, 1, n, 0, dst);
}

int jt_w8a8_dequant_per_channel(const int8_t *src, const float *scales, size_t rows,
                                size_t cols, float *dst) {
    if (!src || !scales || !dst || rows == 0 || cols == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (rows > SIZE_MAX / cols) FAIL(JT_ERR_INVAL, EINVAL);
    for (size_t r = 0; r < rows; r++)
        if (!isfinite((double)scales[r]) || scales[r] <= 0.0f) FAIL(JT_ERR_INVAL, EINVAL);
    return dequant_common(src, scales, rows, cols, 1, dst);
}

static int fakequant_common(const float *src, size_t rows, size_t cols, float *dst) {
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    size_t n = rows * cols;
    float *dx = jt_rt_buf(rt, JT_SLOT_A, n * sizeof(float), &rc);
    float *dd = jt_rt_buf(rt, JT_SLOT_B, n * sizeof(float), &rc);
    if (!dx || !dd) return rc;
    if ((rc = jt_rt_h2d(rt, dx, src, n * sizeof(float))) != JT_OK) return rc;
    if (jtk_fakequant(dx, (int64_t)rows, (int64_t)cols, dd, rt->d_scratch, jt_rt_errw(rt, rt->stream),
                      rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    return jt_rt_d2h(rt, dst, dd, n * sizeof(float));
}

int jt_w8a8_fakequant_per_tensor(const float *src, size_t n, float *dst) {
    if (!src || !dst || n == 0) FAIL(JT_ERR_INVAL, EINVAL);
    return fakequant_common(src, 1, n, dst);
}

int jt_w8a8_fakequant_per_channel(const float *src, size_t rows, size_t cols, float *dst) {
    if (!src || !dst || rows == 0 || cols == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (rows > SIZE_MAX / cols) FAIL(JT_ERR_INVAL, EINVAL);
    return fakequant_common(src, rows, cols, dst);
}

/* ---------------- GEMM (host pointers) ---------------- */

/* Shared body of the two reference GEMMs (src/w8a8.c:955-1072). sB has N
 * entries when per_col, else 1. */
static int gemm_host(const int8_t *Aq, const int8_t *Bq, float sA, const float *sB,
                     int per_col, float *C, int M, int N, int K) {
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    const int Kp = (int)jt_round_up((size_t)K, 64);
    const int Np = (int)jt_round_up((size_t)N, 128);
    int8_t *dA = jt_rt_buf(rt, JT_SLOT_A, (size_t)M * Kp, &rc);
    int8_t *dB = jt_rt_buf(rt, JT_SLOT_B, (size_t)K * N, &rc);
    int8_t *dP = jt_rt_buf(rt, JT_SLOT_C, (size_t)Np * Kp, &rc);
    float *dsA = jt_rt_buf(rt, JT_SLOT_D, (size_t)M * sizeof(float), &rc);
    float *dsB = jt_rt_buf(rt, JT_SLOT_E, (size_t)Np * sizeof(float), &rc);
    float *dC = jt_rt_buf(rt, JT_SLOT_F, (size_t)M * N * sizeof(float), &rc);
    float *hs = malloc((size_t)(M > Np ? M : Np) * sizeof(float));
    if (!dA || !dB || !dP || !dsA || !dsB || !dC || !hs) {
        free(hs);
        if (rc == JT_OK) FAIL(JT_ERR_NOMEM, ENOMEM);
        return rc;
    }
    hipError_t e = hipSuccess;
    if (Kp != K) e = hipMemsetAsync(dA, 0, (size_t)M * Kp, rt->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(dA, (size_t)Kp, Aq, (size_t)K, (size_t)K, (size_t)M,
                             hipMemcpyHostToDevice, rt->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dB, Bq, (size_t)K * N, hipMemcpyHostToDevice, rt->stream);
    for (int m = 0; m < M; m++) hs[m] = sA;
    if (e == hipSuccess)
        e = hipMemcpyAsync(dsA, hs, (size_t)M * sizeof(float), hipMemcpyHostToDevice,
                           rt->stream);
    for (int n = 0; n < Np; n++) hs[n] = n < N ? sB[per_col ? n : 0] : 1.0f;
    if (e == hipSuccess)
        e = hipMemcpyAsync(dsB, hs, (size_t)Np * sizeof(float), hipMemcpyHostToDevice,
                           rt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    free(hs);
    if (e != hipSuccess) return jt_rt_err(e);
    /* -128 codes are rejected before anything is computed (src/w8a8.c:979-999) */
    jtk_check_q(dA, (int64_t)M * Kp, jt_rt_errw(rt, rt->stream), rt->stream);
    jtk_check_q(dB, (int64_t)K * N, jt_rt_errw(rt, rt->stream), rt->stream);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    if (jtk_pack_i8(dB, N, K, 1, Np, Kp, dP, rt->stream) ||
        jtk_w8a8_gemm(dA, Kp, dsA, dP, dsB, M, N, Np, Kp, dC, N, 0, jt_rt_errw(rt, rt->stream), rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc;
    return jt_rt_d2h(rt, C, dC, (size_t)M * N * sizeof(float));
}

static int gemm_validate(const int8_t *Aq, const int8_t *Bq, float sA, const float *C, int M,
                         int N, int K) {
    if (!Aq || !Bq || !C) FAIL(JT_ERR_INVAL, EINVAL);
    if (M < 0 || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (M > JT_BWD_MAX_WIDE || N > JT_BWD_MAX_WIDE || K > JT_BWD_MAX_WIDE)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!isfinite((double)sA) || sA <= 0.0f) FAIL(JT_ERR_INVAL, EINVAL);
    return JT_OK;
}

int jt_w8a8_gemm_per_tensor(const int8_t *Aq, const int8_t *Bq, float sA, float sB, float *C,
                            int M, int N, int K) {
    if (M == 0) {
        if (!Aq || !Bq || !C || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
        return JT_OK;
    }
    int rc = gemm_validate(Aq, Bq, sA, C, M, N, K);
    if (rc != JT_OK) return rc;
    if (!isfinite((double)sB) || sB <= 0.0f) FAIL(JT_ERR_INVAL, EINVAL);
    return gemm_host(Aq, Bq, sA, &sB, 0, C, M, N, K);
}

int jt_w8a8_gemm_per_channel(const int8_t *Aq, const int8_t *Bq, float sA,
                             const float *sB_col, float *C, int M, int N, int K) {
    if (M == 0) {
        if (!Aq || !Bq || !C || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
        return JT_OK;
    }
    int rc = gemm_validate(Aq, Bq, sA, C, M, N, K);
    if (rc != JT_OK) return rc;
    if (!sB_col) FAIL(JT_ERR_INVAL, EINVAL);
    for (int n = 0; n < N; n++)
        if (!isfinite((double)sB_col[n]) || sB_col[n] <= 0.0f) FAIL(JT_ERR_INVAL, EINVAL);
    return gemm_host(Aq, Bq, sA, sB_col, 1, C, M, N, K);
}

/* ---------------- device-resident W8A8 ---------------- */

struct jt_hip_w8a8 {
    int N, K, Np, Kp;
    int8_t *P;  /* panels [Np/16][Kp/64][1024] */
    float *sB;  /* [Np] */
};

int jt_hip_quant_rows(const float *dX, int rows, int cols, int8_t *dXq, float *dscale,
                      void *stream) {
    if (!dX || !dXq || !dscale || rows < 0 || cols <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (rows == 0) return JT_OK;
    hipStream_t s = (hipStream_t)stream; /* NULL: the HIP null stream */
    if (jtk_quant_rows(dX, rows, cols, dXq, cols, dscale, NULL, jt_rt_errw(rt, s), s))
        return jt_rt_err(hipErrorLaunchFailure);
    return JT_OK;
}

static int w8a8_alloc(int N, int K, jt_hip_w8a8 **out) {
    jt_hip_w8a8 *W = calloc(1, sizeof(*W));
    if (!W) FAIL(JT_ERR_NOMEM, ENOMEM);
    W->N = N;
    W->K = K;
    W->Np = (int)jt_round_up((size_t)N, 128);
    W->Kp = (int)jt_round_up((size_t)K, 64);
    hipError_t e = hipMalloc((void **)&W->P, (size_t)W->Np * W->Kp);
    if (e == hipSuccess) e = hipMalloc((void **)&W->sB, (size_t)W->Np * sizeof(float));
    if (e != hipSuccess) {
        (void)hipFree(W->P);
        free(W);
        return jt_rt_err(e);
    }
    *out = W;
    return JT_OK;
}

void jt_hip_w8a8_free(jt_hip_w8a8 *W) {
    if (!W) return;
    (void)hipFree(W->P);
    (void)hipFree(W->sB);
    free(W);
}

int jt_hip_w8a8_prepare(const float *dW, int N, int K, jt_hip_w8a8 **out) {
    if (!dW || !out || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    jt_hip_w8a8 *W = NULL;
    int rc = w8a8_alloc(N, K, &W);
    if (rc != JT_OK) return rc;
    int8_t *tmp = NULL;
    hipError_t e = hipMalloc((void **)&tmp, (size_t)N * K);
    if (e == hipSuccess) e = hipMemsetAsync(W->sB, 0, (size_t)W->Np * sizeof(float), rt->stream);
    if (e != hipSuccess) {
        jt_hip_w8a8_free(W);
        return jt_rt_err(e);
    }
    jtk_quant_weight_rows(dW, K, 1, N, K, tmp, W->sB, jt_rt_errw(rt, rt->stream), rt->stream);
    jtk_pack_i8(tmp, N, K, 0, W->Np, W->Kp, W->P, rt->stream);
    uint32_t f = 0;
    rc = jt_rt_flags(rt, rt->stream, &f);
    (void)hipFree(tmp);
    if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    if (rc != JT_OK) {
        jt_hip_w8a8_free(W);
        return rc;
    }
    *out = W;
    return JT_OK;
}

int jt_hip_w8a8_prepare_kn(const int8_t *dBq, const float *dsB, int N, int K,
                           jt_hip_w8a8 **out) {
    if (!dBq || !dsB || !out || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    jt_hip_w8a8 *W = NULL;
    int rc = w8a8_alloc(N, K, &W);
    if (rc != JT_OK) return rc;
    hipError_t e = hipMemsetAsync(W->sB, 0, (size_t)W->Np * sizeof(float), rt->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(W->sB, dsB, (size_t)N * sizeof(float), hipMemcpyDeviceToDevice,
                           rt->stream);
    if (e != hipSuccess) {
        jt_hip_w8a8_free(W);
        return jt_rt_err(e);
    }
    jtk_check_q(dBq, (int64_t)N * K, jt_rt_errw(rt, rt->stream), rt->stream);
    jtk_pack_i8(dBq, N, K, 1, W->Np, W->Kp, W->P, rt->stream);
    uint32_t f = 0;
    rc = jt_rt_flags(rt, rt->stream, &f);
    if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    if (rc != JT_OK) {
        jt_hip_w8a8_free(W);
        return rc;
    }
    *out = W;
    return JT_OK;
}

int jt_hip_w8a8_gemm(const jt_hip_w8a8 *W, const int8_t *dAq, const float *dsA, float *dC,
                     int M, void *stream) {
    if (!W || !dAq || !dsA || !dC || M < 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (W->K % 64 != 0 || ((uintptr_t)dAq & 15u) != 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (M == 0) return JT_OK;
    hipStream_t s = (hipStream_t)stream; /* NULL: the HIP null stream */
    if (jtk_w8a8_gemm(dAq, W->K, dsA, W->P, W->sB, M, W->N, W->Np, W->Kp, dC, W->N, 0,
                      jt_rt_errw(rt, s), s))
        return jt_rt_err(hipErrorLaunchFailure);
    return JT_OK;
}

size_t jt_hip_w8a8_gemm_f32_ws_bytes(const jt_hip_w8a8 *W, int M) {
    if (!W || M < 0) return 0;
    if (M <= 16) return 0;
    return jt_round_up((size_t)M * W->Kp, 256) + (size_t)M * sizeof(float);
}

int jt_hip_w8a8_gemm_f32(const jt_hip_w8a8 *W, const float *dX, float *dC, int M, void *d_ws,
                         size_t ws_bytes, void *stream) {
    if (!W || !dX || !dC || M < 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (M == 0) return JT_OK;
    hipStream_t s = (hipStream_t)stream;
    if (M <= 16) {
        if (W->K % 4 || W->K > 4096 || ((uintptr_t)dX & 15u)) FAIL(JT_ERR_INVAL, EINVAL);
        return jtk_w8a8_gemm_xq(dX, W->K, W->K, W->P, W->sB, M, W->N, W->Np, W->Kp, dC, W->N, 0,
                                jt_rt_errw(rt, s), s)
                   ? jt_rt_err(hipErrorLaunchFailure)
                   : JT_OK;
    }
    if (!d_ws || ws_bytes < jt_hip_w8a8_gemm_f32_ws_bytes(W, M) || ((uintptr_t)d_ws & 255u))
        FAIL(JT_ERR_INVAL, EINVAL);
    /* codes at row stride Kp: the columns K..Kp-1 meet zero weight codes */
    int8_t *Xq = (int8_t *)d_ws;
    float *sx = (float *)((char *)d_ws + jt_round_up((size_t)M * W->Kp, 256));
    if (jtk_quant_rows(dX, M, W->K, Xq, W->Kp, sx, NULL, jt_rt_errw(rt, s), s) ||
        jtk_w8a8_gemm(Xq, W->Kp, sx, W->P, W->sB, M, W->N, W->Np, W->Kp, dC, W->N, 0, jt_rt_errw(rt, s),
                      s))
        return jt_rt_err(hipErrorLaunchFailure);
    return JT_OK;
}

int jt_hip_w8a8_export(const jt_hip_w8a8 *W, int8_t *Bq_kn, float *sB) {
    if (!W || !Bq_kn || !sB) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    int8_t *d = jt_rt_buf(rt, JT_SLOT_A, (size_t)W->N * W->K, &rc);
    if (!d) return rc;
    if (jtk_unpack_i8_kn(W->P, W->N, W->K, W->Kp, d, rt->stream))
        return jt_rt_err(hipErrorLaunchFailure);
    if ((rc = jt_rt_d2h(rt, Bq_kn, d, (size_t)W->N * W->K)) != JT_OK) return rc;
    return jt_rt_d2h(rt, sB, W->sB, (size_t)W->N * sizeof(float));
}
