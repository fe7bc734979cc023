/*
 * moe_bwd.c -- the reference's batched MoE backward (jt_moe_bwd_batch /
 * jt_moe_bwd_batch_unchecked, src/moe_layer.c:1684-2502) on the MI355X,
 * host orchestration in C11.
 *
 * The backward reuses the forward's permutation (perm, off, drop) and never
 * re-sorts. Every step runs as HIP kernels (moe_bwd.hip) in the reference's
 * order of operations, so each output is the reference's to the bit except
 * where its fp64 exp differs from glibc's by an ulp (SwiGLU backward).
 *
 * Checks. Both forms check on the device, before any result is trusted,
 * that ids, drop, off and perm are consistent (off from 0 and monotone,
 * off[E] == number of kept pairs, perm an exact enumeration of the kept
 * pairs): the kernels index with them. The reference's unchecked form skips
 * most of these; a permutation written by the forward always passes them.
 * The checked form adds the reference's finiteness scans and the weight
 * range test (src/moe_layer.c:1766-1880).
 *
 * The host-pointer entry points stage everything into HBM, run the device
 * entry on the library stream and copy the outputs back only when no error
 * bit was raised, so a failed call leaves every output untouched.
 */
#include <errno.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jimotono/hip_moe.h"
#include "jimotono/moe_layer.h"
#include "jt_rt.h"

#define FAIL(code, e) \
    do {              \
        errno = (e);  \
        return (code); \
    } while (0)

static int bwd_dims_ok(int T, int n, int h, int E, int k, int S) {
    if (T <= 0 || n <= 0 || h <= 0 || n > JT_BWD_MAX_WIDE || h > JT_BWD_MAX_WIDE) return 0;
    if (E <= 0 || E > JT_MOE_MAX_EXPERTS) return 0;
    if (k <= 0 || k > E || k > JT_MOE_MAX_TOPK) return 0;
    if (S < 0 || S > JT_MOE_MAX_SHARED) return 0;
    /* pair and row indices are 32-bit on the device */
    if ((int64_t)T * k > INT32_MAX / 2) return 0;
    return 1;
}

size_t jt_hip_moe_bwd_batch_ws_bytes(int T, int n, int h, int n_experts, int topk,
                                     int n_shared) {
    if (!bwd_dims_ok(T, n, h, n_experts, topk, n_shared)) return 0;
    return jtk_bwd_ws_layout(T, n, h, n_experts, topk, n_shared, NULL, NULL);
}

int jt_hip_moe_bwd_batch(const float *dY, const float *X, const float *Wgate, const float *Wg,
                         const float *Wu, const float *Wd, const float *Wg_s,
                         const float *Wu_s, const float *Wd_s, const size_t *ids,
                         const float *weights, const float *Gsel, const float *Usel,
                         const float *Ysel, const float *Gs, const float *Us,
                         const size_t *perm, const size_t *off, const unsigned char *drop,
                         float *dX, float *dWgate, float *dWg, float *dWu, float *dWd,
                         float *dWg_s, float *dWu_s, float *dWd_s, float *dLogits, int T,
                         int n, int h, int n_experts, int topk, int n_shared, int validate,
                         void *d_ws, size_t ws_bytes, void *stream) {
    if (!dY || !X || !Wgate || !Wg || !Wu || !Wd || !ids || !weights || !Gsel || !Usel ||
        !Ysel || !perm || !off || !drop || !dX || !dWgate || !dWg || !dWu || !dWd || !d_ws)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!bwd_dims_ok(T, n, h, n_experts, topk, n_shared)) FAIL(JT_ERR_INVAL, EINVAL);
    if (n_shared > 0 && (!Wg_s || !Wu_s || !Wd_s || !Gs || !Us || !dWg_s || !dWu_s || !dWd_s))
        FAIL(JT_ERR_INVAL, EINVAL);
    if (sizeof(size_t) != 8) FAIL(JT_ERR_NOSUP, EINVAL);
    const size_t need = jtk_bwd_ws_layout(T, n, h, n_experts, topk, n_shared, NULL, NULL);
    if (ws_bytes < need || ((uintptr_t)d_ws & 255u)) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    jtk_bwd_ws w;
    (void)jtk_bwd_ws_layout(T, n, h, n_experts, topk, n_shared, &w, (char *)d_ws);
    const jtk_bwd_io io = {dY,    X,       Wgate,  Wg,   Wu,    Wd,      Wg_s,  Wu_s,
                           Wd_s,  (const uint64_t *)ids, weights, Gsel, Usel,  Ysel,
                           Gs,    Us,      (const uint64_t *)perm, (const uint64_t *)off,
                           drop,  dX,      dWgate, dWg,  dWu,   dWd,     dWg_s, dWu_s,
                           dWd_s, dLogits};
    int le = jtk_bwd_batch(&io, T, n, h, n_experts, topk, n_shared, validate != 0, &w,
                           jt_rt_errw(rt, (hipStream_t)stream), (hipStream_t)stream);
    return le ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

/* device allocations of one host-pointer call */
typedef struct {
    void *p[40];
    int n;
    hipError_t e;
} bwd_arena;

static void *balloc(bwd_arena *a, size_t bytes) {
    void *p = NULL;
    if (a->e != hipSuccess) return NULL;
    if (a->n >= 40) {
        a->e = hipErrorOutOfMemory;
        return NULL;
    }
    a->e = hipMalloc(&p, bytes ? bytes : 256);
    if (a->e != hipSuccess) return NULL;
    a->p[a->n++] = p;
    return p;
}

static int bwd_host(const float *dY, const float *X, const float *Wgate, const float *Wg,
                    const float *Wu, const float *Wd, const float *Wg_s, const float *Wu_s,
                    const float *Wd_s, const size_t *ids, const float *weights,
                    const float *Gsel, const float *Usel, const float *Ysel, const float *Gs,
                    const float *Us, const size_t *perm, const size_t *off,
                    const unsigned char *drop, float *dX, float *dWgate, float *dWg, float *dWu,
                    float *dWd, float *dWg_s, float *dWu_s, float *dWd_s, float *dLogits, int T,
                    int n, int h, int E, int k, int S, int validate) {
    /* argument checks in the reference's order (src/moe_layer.c:1739-1765) */
    if (!dY || !X || !Wgate || !Wg || !Wu || !Wd || !ids || !weights || !Gsel || !Usel ||
        !Ysel || !perm || !off || !drop || !dX || !dWgate || !dWg || !dWu || !dWd)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (!bwd_dims_ok(T, n, h, E, k, S)) FAIL(JT_ERR_INVAL, EINVAL);
    if (S > 0 && (!Wg_s || !Wu_s || !Wd_s || !Gs || !Us || !dWg_s || !dWu_s || !dWd_s))
        FAIL(JT_ERR_INVAL, EINVAL);
    if (sizeof(size_t) != 8) FAIL(JT_ERR_NOSUP, EINVAL);
    const size_t Tk = (size_t)T * k, Tn = (size_t)T * n, nh = (size_t)n * h;
    const size_t kept = off[E];
    if (kept > Tk) FAIL(JT_ERR_INVAL, EINVAL); /* src/moe_layer.c:1875-1880 */
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    hipStream_t s = rt->stream;
    bwd_arena a = {.n = 0, .e = hipSuccess};
    const size_t wsb = jtk_bwd_ws_layout(T, n, h, E, k, S, NULL, NULL);
    const size_t sh = (size_t)T * S * h * 4;
    float *d_dY = balloc(&a, Tn * 4), *d_X = balloc(&a, Tn * 4);
    float *d_Wgate = balloc(&a, (size_t)E * n * 4);
    float *d_Wg = balloc(&a, E * nh * 4), *d_Wu = balloc(&a, E * nh * 4);
    float *d_Wd = balloc(&a, E * nh * 4);
    float *d_Wgs = S ? balloc(&a, S * nh * 4) : NULL, *d_Wus = S ? balloc(&a, S * nh * 4) : NULL;
    float *d_Wds = S ? balloc(&a, S * nh * 4) : NULL;
    size_t *d_ids = balloc(&a, Tk * 8);
    float *d_w = balloc(&a, Tk * 4);
    float *d_G = balloc(&a, Tk * h * 4), *d_U = balloc(&a, Tk * h * 4);
    float *d_Y = balloc(&a, Tk * n * 4);
    float *d_Gs = S ? balloc(&a, sh) : NULL, *d_Us = S ? balloc(&a, sh) : NULL;
    size_t *d_perm = balloc(&a, kept * 8), *d_off = balloc(&a, ((size_t)E + 1) * 8);
    unsigned char *d_drop = balloc(&a, Tk);
    float *o_dX = balloc(&a, Tn * 4), *o_dWgate = balloc(&a, (size_t)E * n * 4);
    float *o_dWg = balloc(&a, E * nh * 4), *o_dWu = balloc(&a, E * nh * 4);
    float *o_dWd = balloc(&a, E * nh * 4);
    float *o_dWgs = S ? balloc(&a, S * nh * 4) : NULL, *o_dWus = S ? balloc(&a, S * nh * 4) : NULL;
    float *o_dWds = S ? balloc(&a, S * nh * 4) : NULL;
    float *o_dL = dLogits ? balloc(&a, (size_t)T * E * 4) : NULL;
    void *ws = balloc(&a, wsb);
    int rc = jt_rt_err(a.e);
#define H2D(d, h_, b) \
    if (rc == JT_OK) rc = jt_rt_h2d(rt, (d), (h_), (b))
    H2D(d_dY, dY, Tn * 4);
    H2D(d_X, X, Tn * 4);
    H2D(d_Wgate, Wgate, (size_t)E * n * 4);
    H2D(d_Wg, Wg, E * nh * 4);
    H2D(d_Wu, Wu, E * nh * 4);
    H2D(d_Wd, Wd, E * nh * 4);
    if (S) {
        H2D(d_Wgs, Wg_s, S * nh * 4);
        H2D(d_Wus, Wu_s, S * nh * 4);
        H2D(d_Wds, Wd_s, S * nh * 4);
        H2D(d_Gs, Gs, sh);
        H2D(d_Us, Us, sh);
    }
    H2D(d_ids, ids, Tk * 8);
    H2D(d_w, weights, Tk * 4);
    H2D(d_G, Gsel, Tk * h * 4);
    H2D(d_U, Usel, Tk * h * 4);
    H2D(d_Y, Ysel, Tk * n * 4);
    H2D(d_perm, perm, kept * 8);
    H2D(d_off, off, ((size_t)E + 1) * 8);
    H2D(d_drop, drop, Tk);
#undef H2D
    if (rc == JT_OK)
        rc = jt_hip_moe_bwd_batch(d_dY, d_X, d_Wgate, d_Wg, d_Wu, d_Wd, d_Wgs, d_Wus, d_Wds,
                                  d_ids, d_w, d_G, d_U, d_Y, d_Gs, d_Us, d_perm, d_off, d_drop,
                                  o_dX, o_dWgate, o_dWg, o_dWu, o_dWd, o_dWgs, o_dWus, o_dWds,
                                  o_dL, T, n, h, E, k, S, validate, ws, wsb, s);
    uint32_t f = 0;
    if (rc == JT_OK) rc = jt_rt_flags(rt, s, &f);
    if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    /* commit (fail-closed: nothing above wrote a host output) */
    if (rc == JT_OK) rc = jt_rt_d2h(rt, dX, o_dX, Tn * 4);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, dWgate, o_dWgate, (size_t)E * n * 4);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, dWg, o_dWg, E * nh * 4);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, dWu, o_dWu, E * nh * 4);
    if (rc == JT_OK) rc = jt_rt_d2h(rt, dWd, o_dWd, E * nh * 4);
    if (rc == JT_OK && S) {
        rc = jt_rt_d2h(rt, dWg_s, o_dWgs, S * nh * 4);
        if (rc == JT_OK) rc = jt_rt_d2h(rt, dWu_s, o_dWus, S * nh * 4);
        if (rc == JT_OK) rc = jt_rt_d2h(rt, dWd_s, o_dWds, S * nh * 4);
    }
    if (rc == JT_OK && dLogits) rc = jt_rt_d2h(rt, dLogits, o_dL, (size_t)T * E * 4);
    (void)hipStreamSynchronize(s);
    if (rc != JT_OK) {
        /* a failed call reports its own code: flags raised by work it had
         * already queued are dropped, not left for the stream's next call */
        const int saved = errno;
        uint32_t dropped = 0;
        (void)jt_rt_flags(rt, s, &dropped);
        errno = saved;
    }
    for (int i = 0; i < a.n; i++) (void)hipFree(a.p[i]);
    return rc;
}

int jt_moe_bwd_batch(const float *dY, const float *X, const float *Wgate, const float *Wg,
                     const float *Wu, const float *Wd, const float *Wg_s, const float *Wu_s,
                     const float *Wd_s, const size_t *ids, const float *weights,
                     const float *Gsel, const float *Usel, const float *Ysel, const float *Gs,
                     const float *Us, const size_t *perm, const size_t *off,
                     const unsigned char *drop, float *dX, float *dWgate, float *dWg,
                     float *dWu, float *dWd, float *dWg_s, float *dWu_s, float *dWd_s,
                     float *dLogits, int T, int n, int h, int n_experts, int topk,
                     int n_shared) {
    return bwd_host(dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, weights, Gsel, Usel, Ysel,
                    Gs, Us, perm, off, drop, dX, dWgate, dWg, dWu, dWd, dWg_s, dWu_s, dWd_s,
                    dLogits, T, n, h, n_experts, topk, n_shared, 1);
}

int jt_moe_bwd_batch_unchecked(const float *dY, const float *X, const float *Wgate,
                               const float *Wg, const float *Wu, const float *Wd,
                               const float *Wg_s, const float *Wu_s, const float *Wd_s,
                               const size_t *ids, const float *weights, const float *Gsel,
                               const float *Usel, const float *Ysel, const float *Gs,
                               const float *Us, const size_t *perm, const size_t *off,
                               const unsigned char *drop, float *dX, float *dWgate, float *dWg,
                               float *dWu, float *dWd, float *dWg_s, float *dWu_s,
                               float *dWd_s, float *dLogits, int T, int n, int h,
                               int n_experts, int topk, int n_shared) {
    return bwd_host(dY, X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, ids, weights, Gsel, Usel, Ysel,
                    Gs, Us, perm, off, drop, dX, dWgate, dWg, dWu, dWd, dWg_s, dWu_s, dWd_s,
                    dLogits, T, n, h, n_experts, topk, n_shared, 0);
}
