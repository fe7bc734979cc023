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

/* The host-pointer call's device buffers are carved out of one grow-only
 * workspace kept between calls (sized in a first pass with a NULL base),
 * 256-byte aligned; a call of the same or a smaller shape allocates
 * nothing. */
typedef struct {
    char *base;
    size_t off;
} bwd_arena;

static void *balloc(bwd_arena *a, size_t bytes) {
    void *p = a->base ? a->base + a->off : NULL;
    a->off += jt_round_up(bytes ? bytes : 16, 256);
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
    int rc = JT_OK;
    const size_t wsb = jtk_bwd_ws_layout(T, n, h, E, k, S, NULL, NULL);
    const size_t sh = (size_t)T * S * h * 4;
    bwd_arena a = {.base = NULL, .off = 0};
carve:;
    /* the inputs first, then the outputs, each group contiguous: one staged
     * copy each way */
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
    char *o_end = (char *)balloc(&a, 0);
    void *ws = balloc(&a, wsb);
    if (!a.base) {
        a.base = jt_rt_buf(rt, JT_SLOT_BWD, a.off, &rc);
        if (!a.base) return rc;
        a.off = 0;
        goto carve;
    }
    /* inputs: gathered into pinned staging at their workspace offsets (gaps
     * zeroed), one copy queued ahead of the kernels */
    {
        const size_t in_bytes = (size_t)((char *)o_dX - (char *)d_dY);
        char *stin = jt_rt_hbuf(rt, 0, in_bytes, &rc);
        if (!stin) return rc;
        size_t at = 0;
#define STAGE_IN(d, h_, b)                                                                 \
    do {                                                                                   \
        if (d) {                                                                           \
            const size_t o_ = (size_t)((char *)(d) - (char *)d_dY);                        \
            memset(stin + at, 0, o_ - at);                                                 \
            memcpy(stin + o_, (h_), (b));                                                  \
            at = o_ + (b);                                                                 \
        }                                                                                  \
    } while (0)
        STAGE_IN(d_dY, dY, Tn * 4);
        STAGE_IN(d_X, X, Tn * 4);
        STAGE_IN(d_Wgate, Wgate, (size_t)E * n * 4);
        STAGE_IN(d_Wg, Wg, E * nh * 4);
        STAGE_IN(d_Wu, Wu, E * nh * 4);
        STAGE_IN(d_Wd, Wd, E * nh * 4);
        if (S) {
            STAGE_IN(d_Wgs, Wg_s, S * nh * 4);
            STAGE_IN(d_Wus, Wu_s, S * nh * 4);
            STAGE_IN(d_Wds, Wd_s, S * nh * 4);
        }
        STAGE_IN(d_ids, ids, Tk * 8);
        STAGE_IN(d_w, weights, Tk * 4);
        STAGE_IN(d_G, Gsel, Tk * h * 4);
        STAGE_IN(d_U, Usel, Tk * h * 4);
        STAGE_IN(d_Y, Ysel, Tk * n * 4);
        if (S) {
            STAGE_IN(d_Gs, Gs, sh);
            STAGE_IN(d_Us, Us, sh);
        }
        STAGE_IN(d_perm, perm, kept * 8);
        STAGE_IN(d_off, off, ((size_t)E + 1) * 8);
        STAGE_IN(d_drop, drop, Tk);
#undef STAGE_IN
        memset(stin + at, 0, in_bytes - at);
        rc = jt_rt_err(hipMemcpyAsync(d_dY, stin, in_bytes, hipMemcpyHostToDevice, s));
    }
    if (rc == JT_OK)
        rc = jt_hip_moe_bwd_batch(d_dY, d_X, d_Wgate, d_Wg, d_Wu, d_Wd, d_Wgs, d_Wus, d_Wds,
                                  d_ids, d_w, d_G, d_U, d_Y, d_Gs, d_Us, d_perm, d_off, d_drop,
                                  o_dX, o_dWgate, o_dWg, o_dWu, o_dWd, o_dWgs, o_dWus, o_dWds,
                                  o_dL, T, n, h, E, k, S, validate, ws, wsb, s);
    /* outputs: one copy into pinned staging behind the kernels, one wait (the
     * error word's read), then the caller's buffers (fail-closed: a failed
     * call writes no host output) */
    const size_t out_bytes = (size_t)(o_end - (char *)o_dX);
    char *stout = rc == JT_OK ? jt_rt_hbuf(rt, 1, out_bytes, &rc) : NULL;
    if (rc == JT_OK)
        rc = jt_rt_err(hipMemcpyAsync(stout, o_dX, out_bytes, hipMemcpyDeviceToHost, s));
    uint32_t f = 0;
    if (rc == JT_OK) rc = jt_rt_flags(rt, s, &f);
    if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    if (rc == JT_OK) {
#define TAKE(h_, d, b) memcpy((h_), stout + ((char *)(d) - (char *)o_dX), (b))
        TAKE(dX, o_dX, Tn * 4);
        TAKE(dWgate, o_dWgate, (size_t)E * n * 4);
        TAKE(dWg, o_dWg, E * nh * 4);
        TAKE(dWu, o_dWu, E * nh * 4);
        TAKE(dWd, o_dWd, E * nh * 4);
        if (S) {
            TAKE(dWg_s, o_dWgs, S * nh * 4);
            TAKE(dWu_s, o_dWus, S * nh * 4);
            TAKE(dWd_s, o_dWds, S * nh * 4);
        }
        if (dLogits) TAKE(dLogits, o_dL, (size_t)T * E * 4);
#undef TAKE
    }
    (void)hipStreamSynchronize(s);
    if (rc != JT_OK) {
        /* a failed call reports its own code: flags raised by work it had
         * already queued are dropped, not left for the stream's next call */
        const int saved = errno;
        uint32_t dropped = 0;
        (void)jt_rt_flags(rt, s, &dropped);
        errno = saved;
    }
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
