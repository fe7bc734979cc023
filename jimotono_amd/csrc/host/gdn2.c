/*
 * gdn2.c -- Gated DeltaNet-2 (the reference's src/gdn2.c) on the MI355X:
 * the reference's host-pointer API (include/jimotono/gdn2.h) and the
 * device-resident batched API (include/jimotono/hip_gdn2.h), C11.
 *
 * The state helpers keep the reference's host-memory contract (64-byte
 * aligned, zeroed blocks). The compute entry points check their arguments
 * in the reference's order, stage the state and vectors into HBM, run the
 * kernels of kernels/gdn2.hip and copy S and the outputs back only when
 * the device found every input finite and alpha in [0,1].
 */
#include <errno.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jimotono/gdn2.h"
#include "jimotono/hip_gdn2.h"
#include "jt_rt.h"

#define FAIL(code, e) \
    do {              \
        errno = (e);  \
        return (code); \
    } while (0)

static int dims_ok(int dk, int dv) {
    return dk > 0 && dv > 0 && dk <= JT_GDN2_MAX_D && dv <= JT_GDN2_MAX_D;
}

int jt_gdn2_state_bytes(int dk, int dv, size_t *out_bytes) {
    if (!out_bytes) FAIL(JT_ERR_INVAL, EINVAL);
    *out_bytes = 0;
    if (!dims_ok(dk, dv)) FAIL(JT_ERR_INVAL, EINVAL);
    *out_bytes = (size_t)dk * (size_t)dv * sizeof(float);
    return JT_OK;
}

int jt_gdn2_state_alloc(float **out_S, int dk, int dv) {
    if (!out_S) FAIL(JT_ERR_INVAL, EINVAL);
    *out_S = NULL;
    size_t bytes = 0;
    int rc = jt_gdn2_state_bytes(dk, dv, &bytes);
    if (rc != JT_OK) return rc;
    const size_t alloc = jt_round_up(bytes, JT_CACHELINE);
    void *p = aligned_alloc(JT_CACHELINE, alloc);
    if (!p) FAIL(JT_ERR_NOMEM, ENOMEM);
    memset(p, 0, alloc);
    *out_S = (float *)p;
    return JT_OK;
}

void jt_gdn2_state_free(float *S) { free(S); }

int jt_gdn2_state_reset(float *S, int dk, int dv) {
    if (!S) FAIL(JT_ERR_INVAL, EINVAL);
    size_t bytes = 0;
    int rc = jt_gdn2_state_bytes(dk, dv, &bytes);
    if (rc != JT_OK) return rc;
    memset(S, 0, bytes);
    return JT_OK;
}

int jt_gdn2_scratch_floats(int dk, int dv, size_t *out_n) {
    if (!out_n) FAIL(JT_ERR_INVAL, EINVAL);
    *out_n = 0;
    if (!dims_ok(dk, dv)) FAIL(JT_ERR_INVAL, EINVAL);
    *out_n = 2 * (size_t)dk + 2 * (size_t)dv;
    return JT_OK;
}

/* host arrays -> one staging slot, in order; returns the device copies */
typedef struct {
    const void *src;
    size_t bytes;
    void *dev;
} stage_t;

static int stage_in(jt_rt *rt, stage_t *st, int n, int slot) {
    size_t tot = 0;
    for (int i = 0; i < n; i++) tot += jt_round_up(st[i].bytes, 256);
    int rc = JT_OK;
    char *base = jt_rt_buf(rt, slot, tot, &rc);
    if (!base) return rc;
    size_t at = 0;
    hipError_t e = hipSuccess;
    for (int i = 0; i < n && e == hipSuccess; i++) {
        st[i].dev = base + at;
        if (st[i].src)
            e = hipMemcpyAsync(st[i].dev, st[i].src, st[i].bytes, hipMemcpyHostToDevice,
                               rt->stream);
        at += jt_round_up(st[i].bytes, 256);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    return jt_rt_err(e);
}

int jt_gdn2_l2norm(const float *x, float *y, int n, float eps) {
    if (!x || !y) FAIL(JT_ERR_INVAL, EINVAL);
    if (n <= 0 || n > JT_GDN2_MAX_D) FAIL(JT_ERR_INVAL, EINVAL);
    if (!(eps > 0.0f)) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    stage_t st[2] = {{x, (size_t)n * 4, NULL}, {NULL, (size_t)n * 4, NULL}};
    int rc = stage_in(rt, st, 2, JT_SLOT_A);
    if (rc != JT_OK) return rc;
    if (jtk_gdn2_l2norm(st[0].dev, st[1].dev, 1, n, eps, rt->stream) != 0)
        return jt_rt_err(hipErrorLaunchFailure);
    return jt_rt_d2h(rt, y, st[1].dev, (size_t)n * 4);
}

int jt_gdn2_decode_step(float *S, float *out_o, const float *q, const float *k,
                        const float *v, const float *b, const float *w, const float *alpha,
                        int dk, int dv, float *scratch, size_t scratch_n) {
    if (!S || !out_o || !q || !k || !v || !b || !w || !alpha || !scratch)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!dims_ok(dk, dv)) FAIL(JT_ERR_INVAL, EINVAL);
    if ((uintptr_t)S % JT_CACHELINE) FAIL(JT_ERR_ALIGN, EINVAL);
    if (scratch_n < 2 * (size_t)dk + 2 * (size_t)dv) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    const size_t sb = (size_t)dk * dv * 4, kb = (size_t)dk * 4, vb = (size_t)dv * 4;
    stage_t st[8] = {{S, sb, NULL}, {q, kb, NULL}, {k, kb, NULL}, {b, kb, NULL},
                     {alpha, kb, NULL}, {v, vb, NULL}, {w, vb, NULL}, {NULL, vb, NULL}};
    int rc = stage_in(rt, st, 8, JT_SLOT_A);
    if (rc != JT_OK) return rc;
    if (jtk_gdn2_decode(st[0].dev, st[7].dev, st[1].dev, st[2].dev, st[5].dev, st[3].dev,
                        st[6].dev, st[4].dev, 1, dk, dv, jt_rt_errw(rt, rt->stream), rt->stream) != 0)
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc; /* S, o untouched */
    rc = jt_rt_d2h(rt, out_o, st[7].dev, vb);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, S, st[0].dev, sb);
    return rc;
}

static int prefill_chunk(float *S, float *Out, const float *Q, const float *K, const float *V,
                         const float *B, const float *W, const float *A, int dk, int dv,
                         float *scratch, size_t scratch_n, int C) {
    if (!S || !Out || !Q || !K || !V || !B || !W || !A || !scratch) FAIL(JT_ERR_INVAL, EINVAL);
    if (!dims_ok(dk, dv)) FAIL(JT_ERR_INVAL, EINVAL);
    if ((uintptr_t)S % JT_CACHELINE) FAIL(JT_ERR_ALIGN, EINVAL);
    const size_t need = 4 * (size_t)C * dk + 2 * (size_t)C * dv + (size_t)C * C + (size_t)dk;
    if (scratch_n < need) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    const size_t sb = (size_t)dk * dv * 4, kb = (size_t)C * dk * 4, vb = (size_t)C * dv * 4;
    stage_t st[9] = {{S, sb, NULL}, {Q, kb, NULL}, {K, kb, NULL},   {B, kb, NULL},
                     {A, kb, NULL}, {V, vb, NULL}, {W, vb, NULL},   {NULL, vb, NULL},
                     {NULL, jtk_gdn2_prefill_ws_bytes(1, C, C, dk), NULL}};
    int rc = stage_in(rt, st, 9, JT_SLOT_A);
    if (rc != JT_OK) return rc;
    if (jtk_gdn2_prefill(st[0].dev, st[7].dev, st[1].dev, st[2].dev, st[5].dev, st[3].dev,
                         st[6].dev, st[4].dev, 0, 0, 1, C, C, dk, dv, st[8].dev, jt_rt_errw(rt, rt->stream),
                         rt->stream) != 0)
        return jt_rt_err(hipErrorLaunchFailure);
    uint32_t f = 0;
    if ((rc = jt_rt_flags(rt, rt->stream, &f)) != JT_OK) return rc;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) return rc; /* S, Out untouched */
    rc = jt_rt_d2h(rt, Out, st[7].dev, vb);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, S, st[0].dev, sb);
    return rc;
}

int jt_gdn2_prefill_chunk16(float *S, float *Out, const float *Q, const float *K,
                            const float *V, const float *B, const float *W, const float *Alpha,
                            int dk, int dv, float *scratch, size_t scratch_n) {
    return prefill_chunk(S, Out, Q, K, V, B, W, Alpha, dk, dv, scratch, scratch_n, 16);
}

int jt_gdn2_prefill_chunk32(float *S, float *Out, const float *Q, const float *K,
                            const float *V, const float *B, const float *W, const float *Alpha,
                            int dk, int dv, float *scratch, size_t scratch_n) {
    return prefill_chunk(S, Out, Q, K, V, B, W, Alpha, dk, dv, scratch, scratch_n, 32);
}

/* ---- device-resident batched API ---- */

int jt_hip_gdn2_decode(float *dS, float *dO, const float *dq, const float *dk_,
                       const float *dv_, const float *db, const float *dw, const float *dalpha,
                       int H, int dk, int dv, void *stream) {
    if (!dS || !dO || !dq || !dk_ || !dv_ || !db || !dw || !dalpha || H <= 0)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!dims_ok(dk, dv)) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    return jtk_gdn2_decode(dS, dO, dq, dk_, dv_, db, dw, dalpha, H, dk, dv, jt_rt_errw(rt, (hipStream_t)stream),
                           (hipStream_t)stream)
               ? jt_rt_err(hipErrorLaunchFailure)
               : JT_OK;
}

size_t jt_hip_gdn2_prefill_ws_bytes(int H, int T, int C, int dk) {
    if (H <= 0 || H > JT_HIP_GDN2_MAX_PREFILL_HEADS || (C != 16 && C != 32) || T <= 0 ||
        T % C || dk <= 0 || dk > JT_GDN2_MAX_D)
        return 0;
    return jtk_gdn2_prefill_ws_bytes(H, T, C, dk);
}

int jt_hip_gdn2_prefill(float *dS, float *dOut, const float *dQ, const float *dK,
                        const float *dV, const float *dB, const float *dW, const float *dA,
                        int H, int T, int C, int dk, int dv, void *d_ws, size_t ws_bytes,
                        void *stream) {
    if (!dS || !dOut || !dQ || !dK || !dV || !dB || !dW || !dA || !d_ws || H <= 0 ||
        H > JT_HIP_GDN2_MAX_PREFILL_HEADS)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!dims_ok(dk, dv) || (C != 16 && C != 32) || T <= 0 || T % C) FAIL(JT_ERR_INVAL, EINVAL);
    if ((int64_t)T * (dk > dv ? dk : dv) > INT32_MAX) FAIL(JT_ERR_INVAL, EINVAL);
    if (ws_bytes < jtk_gdn2_prefill_ws_bytes(H, T, C, dk) || ((uintptr_t)d_ws & 15u))
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    return jtk_gdn2_prefill(dS, dOut, dQ, dK, dV, dB, dW, dA, (int64_t)T * dk, (int64_t)T * dv,
                            H, T, C, dk, dv, (float *)d_ws, jt_rt_errw(rt, (hipStream_t)stream), (hipStream_t)stream)
               ? jt_rt_err(hipErrorLaunchFailure)
               : JT_OK;
}
