/*
 * legacy.c -- host side of the reference's fp32 GEMM, low-bit, T-MAC,
 * routing and sort entry points (C11). Signatures, argument checks and
 * return/errno conventions follow the reference functions cited at each
 * definition; the arithmetic runs in the gfx950 kernels of legacy.hip,
 * quant.hip and route.hip, and outputs are copied back only on success.
 */
#include <errno.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jimotono/lowbit.h"
#include "jimotono/moe_gemm.h"
#include "jimotono/moe_layer.h"
#include "jimotono/routing.h"
#include "jimotono/tmac.h"
#include "jt_rt.h"

#define FAIL(code, e) \
    do {              \
        errno = (e);  \
        return (code); \
    } while (0)

#define LAUNCHED(x) \
    if ((x) != 0) return jt_rt_err(hipErrorLaunchFailure)

static int finish(jt_rt *rt) {
    uint32_t f = 0;
    int rc = jt_rt_flags(rt, rt->stream, &f);
    if (rc != JT_OK) return rc;
    return jt_rt_flags_to_rc(f);
}

/* ---------------- src/moe_gemm.c ---------------- */

/* src/moe_gemm.c:92-170 */
int jt_gemm_mat_f32(const float *A, const float *B, float *C, int M, int N, int K) {
    if (!A || !B || !C) FAIL(JT_ERR_INVAL, EINVAL);
    if (M == 0) {
        if (N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
        return JT_OK;
    }
    if (M < 0 || N <= 0 || K <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    if ((size_t)M > SIZE_MAX / (size_t)K || (size_t)M > SIZE_MAX / (size_t)N ||
        (size_t)K > SIZE_MAX / (size_t)N)
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dA = jt_rt_buf(rt, JT_SLOT_A, (size_t)M * K * 4, &rc);
    float *dB = jt_rt_buf(rt, JT_SLOT_B, (size_t)K * N * 4, &rc);
    float *dC = jt_rt_buf(rt, JT_SLOT_C, (size_t)M * N * 4, &rc);
    if (!dA || !dB || !dC) return rc;
    if ((rc = jt_rt_h2d(rt, dA, A, (size_t)M * K * 4)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, dB, B, (size_t)K * N * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_gemm_f32(dA, dB, dC, M, N, K, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    return jt_rt_d2h(rt, C, dC, (size_t)M * N * 4);
}

/* src/moe_gemm.c:17-42 */
int jt_transpose_f32(const float *src, float *dst, int rows, int cols) {
    if (!src || !dst || rows <= 0 || cols <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    if ((size_t)rows > SIZE_MAX / (size_t)cols) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    const size_t n = (size_t)rows * cols;
    float *dS = jt_rt_buf(rt, JT_SLOT_A, n * 4, &rc);
    float *dD = jt_rt_buf(rt, JT_SLOT_B, n * 4, &rc);
    if (!dS || !dD) return rc;
    if ((rc = jt_rt_h2d(rt, dS, src, n * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_transpose_f32(dS, dD, rows, cols, rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    return jt_rt_d2h(rt, dst, dD, n * 4);
}

/* ---------------- src/lowbit.c ---------------- */

static int g_lowbit_mode = 0; /* src/lowbit.c:16 */

int jt_lowbit_set_mode(int mode) {
    if (mode < 0 || mode > 2) FAIL(JT_ERR_INVAL, EINVAL);
    g_lowbit_mode = mode;
    return JT_OK;
}

int jt_lowbit_get_mode(void) { return g_lowbit_mode; }

int jt_lowbit_bits_for(int is_down, int *out_bits) {
    if (!out_bits) FAIL(JT_ERR_INVAL, EINVAL);
    *out_bits = is_down ? 4 : 2;
    return JT_OK;
}

/* src/lowbit.c:47-91: one column of length n, fake-quantised in place on
 * the device (the per-column kernel with h = 1). */
int jt_lowbit_fakequant(const float *w, float *fq, size_t n, int bits) {
    if (!w || !fq || n == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (bits != 2 && bits != 4) FAIL(JT_ERR_INVAL, EINVAL);
    if (n > INT32_MAX) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dW = jt_rt_buf(rt, JT_SLOT_A, n * 4, &rc);
    float *dws = jt_rt_buf(rt, JT_SLOT_B, 4, &rc);
    if (!dW || !dws) return rc;
    if ((rc = jt_rt_h2d(rt, dW, w, n * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_lowbit_fq_cols(dW, (int)n, 1, bits, dws, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    return jt_rt_d2h(rt, fq, dW, n * 4);
}

/* src/lowbit.c:93-141 */
int jt_lowbit_col_to_idx(const float *col, size_t k, int bits, uint8_t *idx,
                         float *w_scale) {
    if (!col || !idx || !w_scale || k == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if ((bits != 2 && bits != 4) || (k % 4u) != 0u || k > INT32_MAX)
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dc = jt_rt_buf(rt, JT_SLOT_A, k * 4, &rc);
    float *dws = jt_rt_buf(rt, JT_SLOT_B, 4, &rc);
    uint8_t *didx = jt_rt_buf(rt, JT_SLOT_C, (size_t)bits * (k / 4), &rc);
    if (!dc || !dws || !didx) return rc;
    if ((rc = jt_rt_h2d(rt, dc, col, k * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_col_to_idx(dc, (int)k, 1, bits, dws, didx, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    float ws = 0.0f;
    if ((rc = jt_rt_d2h(rt, idx, didx, (size_t)bits * (k / 4))) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, &ws, dws, 4)) != JT_OK) return rc;
    *w_scale = ws;
    return JT_OK;
}

/* T-MAC GEMM on device buffers (shared by jt_lowbit_gemm_lut and the legacy
 * layer): Y[me][h] = X[me][k] * W[k][h]. */
int jt_dev_lowbit_gemm_lut(jt_rt *rt, const float *dX, const float *dW, float *dY, int me,
                           int h, int k, int bits) {
    if (me == 0) return JT_OK;
    if (k % 32 != 0) {
        LAUNCHED(jtk_gemm_f64acc(dX, dW, dY, me, h, k, rt->stream));
        return JT_OK;
    }
    int rc = JT_OK;
    const size_t ng = (size_t)k / 4, nb = (size_t)k / 32;
    int8_t *qlut = jt_rt_buf(rt, JT_SLOT_K, (size_t)me * ng * 8, &rc);
    float *sc = jt_rt_buf(rt, JT_SLOT_L, (size_t)me * nb * 4, &rc);
    float *bi = jt_rt_buf(rt, JT_SLOT_M, (size_t)me * nb * 4, &rc);
    double *rs = jt_rt_buf(rt, JT_SLOT_N, (size_t)me * 8, &rc);
    uint8_t *idx = jt_rt_buf(rt, JT_SLOT_O, (size_t)h * bits * ng, &rc);
    float *ws = jt_rt_buf(rt, JT_SLOT_P, (size_t)h * 4, &rc);
    if (!qlut || !sc || !bi || !rs || !idx || !ws) return rc;
    LAUNCHED(jtk_tmac_ctor(dX, me, k, qlut, sc, bi, jt_rt_errw(rt, rt->stream), rt->stream));
    LAUNCHED(jtk_rowsum_f64(dX, me, k, rs, rt->stream));
    LAUNCHED(jtk_col_to_idx(dW, k, h, bits, ws, idx, jt_rt_errw(rt, rt->stream), rt->stream));
    LAUNCHED(jtk_tmac_gemm(qlut, sc, bi, rs, idx, ws, me, h, k, bits, dY, jt_rt_errw(rt, rt->stream),
                           rt->stream));
    return JT_OK;
}

/* src/lowbit.c:158-267 */
int jt_lowbit_gemm_lut(const float *X, const float *W, float *Y, int me, int h, int k,
                       int bits) {
    if (!X || !W || !Y) FAIL(JT_ERR_INVAL, EINVAL);
    if (me < 0 || h <= 0 || k <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (bits != 2 && bits != 4) FAIL(JT_ERR_INVAL, EINVAL);
    if (me == 0) return JT_OK;
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dX = jt_rt_buf(rt, JT_SLOT_A, (size_t)me * k * 4, &rc);
    float *dW = jt_rt_buf(rt, JT_SLOT_B, (size_t)k * h * 4, &rc);
    float *dY = jt_rt_buf(rt, JT_SLOT_C, (size_t)me * h * 4, &rc);
    if (!dX || !dW || !dY) return rc;
    if ((rc = jt_rt_h2d(rt, dX, X, (size_t)me * k * 4)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, dW, W, (size_t)k * h * 4)) != JT_OK) return rc;
    if (k % 32 == 0) {
        /* the reference rejects non-finite inputs in the table build and the
         * column conversion before writing Y */
        jtk_check_finite(dX, (int64_t)me * k, jt_rt_errw(rt, rt->stream), rt->stream);
        jtk_check_finite(dW, (int64_t)k * h, jt_rt_errw(rt, rt->stream), rt->stream);
        if ((rc = finish(rt)) != JT_OK) return rc;
    }
    if ((rc = jt_dev_lowbit_gemm_lut(rt, dX, dW, dY, me, h, k, bits)) != JT_OK) return rc;
    if ((rc = finish(rt)) != JT_OK) return rc;
    return jt_rt_d2h(rt, Y, dY, (size_t)me * h * 4);
}

/* ---------------- src/tmac.c ---------------- */

static int size_mul(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) return 1;
    *out = a * b;
    return 0;
}

/* src/tmac.c:168-197 */
int jt_tmac_qlut_bytes(size_t n, size_t k, size_t *out) {
    if (!out) FAIL(JT_ERR_INVAL, EINVAL);
    *out = 0;
    if (n == 0 || k == 0 || (k % JT_TMAC_G) != 0) FAIL(JT_ERR_INVAL, EINVAL);
    size_t t = 0, bytes = 0;
    if (size_mul(n, k / JT_TMAC_G, &t) || size_mul(t, JT_TMAC_LUT_HALF, &bytes))
        FAIL(JT_ERR_NOMEM, ENOMEM);
    *out = bytes;
    return JT_OK;
}

/* src/tmac.c:199-228 */
int jt_tmac_param_bytes(size_t n, size_t k, size_t *out) {
    if (!out) FAIL(JT_ERR_INVAL, EINVAL);
    *out = 0;
    if (n == 0 || k == 0 || (k % JT_TMAC_ACT_GROUP) != 0) FAIL(JT_ERR_INVAL, EINVAL);
    size_t t = 0, bytes = 0;
    if (size_mul(n, k / JT_TMAC_ACT_GROUP, &t) || size_mul(t, sizeof(float), &bytes))
        FAIL(JT_ERR_NOMEM, ENOMEM);
    *out = bytes;
    return JT_OK;
}

/* src/tmac.c:230-385 */
int jt_tmac_lut_ctor(const float *act, size_t n, size_t k, int8_t *qlut, float *scales,
                     float *biases) {
    if (!act || !qlut || !scales || !biases) FAIL(JT_ERR_INVAL, EINVAL);
    if (n == 0 || k == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if ((k % JT_TMAC_G) != 0 || (k % JT_TMAC_ACT_GROUP) != 0) FAIL(JT_ERR_INVAL, EINVAL);
    size_t t = 0, u = 0;
    if (size_mul(n, k, &t) || size_mul(n, k / 4, &t) || size_mul(t, 8, &u))
        FAIL(JT_ERR_NOMEM, ENOMEM);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    const size_t nb = k / 32;
    float *dA = jt_rt_buf(rt, JT_SLOT_A, n * k * 4, &rc);
    int8_t *dq = jt_rt_buf(rt, JT_SLOT_B, n * (k / 4) * 8, &rc);
    float *ds = jt_rt_buf(rt, JT_SLOT_C, n * nb * 4, &rc);
    float *db = jt_rt_buf(rt, JT_SLOT_D, n * nb * 4, &rc);
    if (!dA || !dq || !ds || !db) return rc;
    if ((rc = jt_rt_h2d(rt, dA, act, n * k * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_tmac_ctor(dA, (int64_t)n, (int64_t)k, dq, ds, db, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, qlut, dq, n * (k / 4) * 8)) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, scales, ds, n * nb * 4)) != JT_OK) return rc;
    return jt_rt_d2h(rt, biases, db, n * nb * 4);
}

/* src/tmac.c:387-506 */
int jt_tmac_lookup_accum(const int8_t *qlut, const uint8_t *idx, const float *scales,
                         const float *biases, size_t ngroups, size_t nblocks, int bits,
                         float w_scale, float *out) {
    if (!qlut || !idx || !scales || !biases || !out) FAIL(JT_ERR_INVAL, EINVAL);
    if (ngroups == 0 || nblocks == 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (nblocks > SIZE_MAX / 8u) FAIL(JT_ERR_NOMEM, ENOMEM);
    if (ngroups != nblocks * 8u) FAIL(JT_ERR_INVAL, EINVAL);
    if (bits < 1 || bits > 4) FAIL(JT_ERR_INVAL, EINVAL);
    if (ngroups > SIZE_MAX / JT_TMAC_LUT_HALF || ngroups > SIZE_MAX / (size_t)bits)
        FAIL(JT_ERR_NOMEM, ENOMEM);
    if (!isfinite((double)w_scale)) FAIL(JT_ERR_INVAL, EINVAL);
    for (size_t bb = 0; bb < nblocks; bb++)
        if (!isfinite((double)scales[bb]) || !isfinite((double)biases[bb]))
            FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    int8_t *dq = jt_rt_buf(rt, JT_SLOT_A, ngroups * 8, &rc);
    uint8_t *di = jt_rt_buf(rt, JT_SLOT_B, ngroups * (size_t)bits, &rc);
    float *ds = jt_rt_buf(rt, JT_SLOT_C, nblocks * 4, &rc);
    float *db = jt_rt_buf(rt, JT_SLOT_D, nblocks * 4, &rc);
    float *dout = jt_rt_buf(rt, JT_SLOT_E, 4, &rc);
    if (!dq || !di || !ds || !db || !dout) return rc;
    if ((rc = jt_rt_h2d(rt, dq, qlut, ngroups * 8)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, di, idx, ngroups * (size_t)bits)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, ds, scales, nblocks * 4)) != JT_OK) return rc;
    if ((rc = jt_rt_h2d(rt, db, biases, nblocks * 4)) != JT_OK) return rc;
    LAUNCHED(jtk_tmac_lookup1(dq, di, ds, db, (int64_t)ngroups, (int64_t)nblocks, bits,
                              w_scale, dout, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    float o = 0.0f;
    if ((rc = jt_rt_d2h(rt, &o, dout, 4)) != JT_OK) return rc;
    *out = o;
    return JT_OK;
}

/* ---------------- src/routing.c ---------------- */

/* src/routing.c:16-76 */
int jt_routing_topk(const float *logits, size_t n, size_t k, size_t *out_ids,
                    float *out_weights) {
    if (!logits || !out_ids || !out_weights) FAIL(JT_ERR_INVAL, EINVAL);
    if (n == 0 || k == 0 || k > n) FAIL(JT_ERR_INVAL, EINVAL);
    /* indices are 31-bit on the device (an 8 GiB row of logits) */
    if (n > 0x7fffffffu) FAIL(JT_ERR_NOSUP, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    float *dl = jt_rt_buf(rt, JT_SLOT_A, n * 4, &rc);
    int32_t *di = jt_rt_buf(rt, JT_SLOT_B, k * 4, &rc);
    int64_t *di64 = jt_rt_buf(rt, JT_SLOT_C, k * 8, &rc);
    float *dw = jt_rt_buf(rt, JT_SLOT_D, k * 4, &rc);
    if (!dl || !di || !di64 || !dw) return rc;
    if ((rc = jt_rt_h2d(rt, dl, logits, n * 4)) != JT_OK) return rc;
    /* one wavefront holds rows up to the layer's limits (moe_layer.h:52-53);
     * longer rows or larger k take the block kernel */
    if (n <= JT_MOE_MAX_EXPERTS && k <= JT_MOE_MAX_TOPK) {
        LAUNCHED(jtk_topk(dl, 1, (int)n, (int)k, di, di64, dw, jt_rt_errw(rt, rt->stream), rt->stream));
    } else {
        LAUNCHED(jtk_topk_block(dl, (int64_t)n, (int64_t)k, di64, dw, jt_rt_errw(rt, rt->stream), rt->stream));
    }
    if ((rc = finish(rt)) != JT_OK) return rc;
    int64_t *tmp = malloc(k * 8);
    if (!tmp) FAIL(JT_ERR_NOMEM, ENOMEM);
    rc = jt_rt_d2h(rt, tmp, di64, k * 8);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, out_weights, dw, k * 4);
    if (rc == JT_OK)
        for (size_t p = 0; p < k; p++) out_ids[p] = (size_t)tmp[p];
    free(tmp);
    return rc;
}

/* ---------------- src/moe_layer.c: sort ---------------- */

/* src/moe_layer.c:895-978 */
int jt_moe_batch_sort(const size_t *ids, int T, int k, int E, float cap_factor, size_t *perm,
                      size_t *off, unsigned char *drop, size_t *out_kept,
                      size_t *out_dropped) {
    if (!ids || !perm || !off || !drop) FAIL(JT_ERR_INVAL, EINVAL);
    if (T <= 0 || k <= 0 || E <= 0 || E > JT_MOE_MAX_EXPERTS || k > E || k > JT_MOE_MAX_TOPK)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!(cap_factor >= 1.0f) || !(cap_factor <= 1.5f) || !isfinite((double)cap_factor))
        FAIL(JT_ERR_INVAL, EINVAL);
    if ((size_t)k > SIZE_MAX / (size_t)T || (int64_t)T * k > INT32_MAX)
        FAIL(JT_ERR_INVAL, EINVAL);
    const size_t Tk = (size_t)T * (size_t)k;
    for (size_t q = 0; q < Tk; q++)
        if (ids[q] >= (size_t)E) FAIL(JT_ERR_INVAL, EINVAL);
    const double capd = ceil((double)cap_factor * (double)Tk / (double)E);
    if (!isfinite(capd) || capd < 1.0) FAIL(JT_ERR_INVAL, EINVAL);
    const int64_t cap = (int64_t)capd;
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    int rc = JT_OK;
    const size_t NB = (Tk + 255) / 256;
    int32_t *dids = jt_rt_buf(rt, JT_SLOT_A, Tk * 4, &rc);
    int32_t *rank = jt_rt_buf(rt, JT_SLOT_B, Tk * 4, &rc);
    int32_t *cnt = jt_rt_buf(rt, JT_SLOT_C, NB * (size_t)E * 4, &rc);
    int32_t *tot = jt_rt_buf(rt, JT_SLOT_D, (size_t)E * 4, &rc);
    int32_t *doff = jt_rt_buf(rt, JT_SLOT_E, ((size_t)E + 1) * 4, &rc);
    int64_t *doff64 = jt_rt_buf(rt, JT_SLOT_F, ((size_t)E + 1) * 8, &rc);
    int32_t *dperm = jt_rt_buf(rt, JT_SLOT_G, Tk * 4, &rc);
    int64_t *dperm64 = jt_rt_buf(rt, JT_SLOT_H, Tk * 8, &rc);
    uint8_t *ddrop = jt_rt_buf(rt, JT_SLOT_I, Tk, &rc);
    int32_t *h32 = malloc(Tk * 4);
    if (!dids || !rank || !cnt || !tot || !doff || !doff64 || !dperm || !dperm64 || !ddrop ||
        !h32) {
        free(h32);
        if (rc == JT_OK) FAIL(JT_ERR_NOMEM, ENOMEM);
        return rc;
    }
    for (size_t q = 0; q < Tk; q++) h32[q] = (int32_t)ids[q];
    rc = jt_rt_h2d(rt, dids, h32, Tk * 4);
    free(h32);
    if (rc != JT_OK) return rc;
    LAUNCHED(jtk_sort(dids, (int)Tk, E, cap, rank, cnt, tot, doff, doff64, dperm, dperm64,
                      ddrop, jt_rt_errw(rt, rt->stream), rt->stream));
    if ((rc = finish(rt)) != JT_OK) return rc;
    int64_t kept = 0;
    if ((rc = jt_rt_d2h(rt, &kept, doff64 + E, 8)) != JT_OK) return rc;
    if (sizeof(size_t) != 8) FAIL(JT_ERR_NOSUP, EINVAL);
    if ((rc = jt_rt_d2h(rt, off, doff64, ((size_t)E + 1) * 8)) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, perm, dperm64, (size_t)kept * 8)) != JT_OK) return rc;
    if ((rc = jt_rt_d2h(rt, drop, ddrop, Tk)) != JT_OK) return rc;
    if (out_kept) *out_kept = (size_t)kept;
    if (out_dropped) *out_dropped = Tk - (size_t)kept;
    return JT_OK;
}
