/*
 * moe_layer.c -- the reference's batched MoE forward (jt_moe_fwd_batch,
 * src/moe_layer.c:980-1663) on the MI355X, host orchestration in C11.
 *
 * Same stages, same order, same arithmetic as the reference:
 *   gate logits (fp64, AVX2 lane order) -> top-k softmax -> capacity sort ->
 *   renormalisation of tokens with drops -> per expert: gather, gate/up GEMM
 *   (fp32 k-ordered / W8A8 per-tensor x per-channel with per-call weight
 *   quantisation / low-bit fake-quant / T-MAC LUT), SwiGLU, down GEMM
 *   (fp32 / W8A8 per-tensor / low-bit), scatter -> fp64 combine in slot
 *   order -> shared experts (fp32 or W8A8) added in fp64 -> Y.
 * The flag reads and their precedence (low-bit before W8A8) are those of
 * src/moe_layer.c:1068-1071, 1301-1396. Everything runs as kernels on the
 * library stream; Y, ids, weights and the sort outputs are copied back only
 * when the whole forward raised no error bit.
 */
#include <errno.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jimotono/lowbit.h"
#include "jimotono/moe_layer.h"
#include "jimotono/w8a8.h"
#include "jt_rt.h"

#define FAIL(code, e) \
    do {              \
        errno = (e);  \
        return (code); \
    } while (0)

int jt_dev_lowbit_gemm_lut(jt_rt *rt, const float *dX, const float *dW, float *dY, int me,
                           int h, int k, int bits);

/* The forward's device buffers are carved out of one grow-only workspace
 * of the runtime (slot JT_SLOT_LAYER), kept between calls: the buffer list
 * runs once with base == NULL to size the workspace, then again to hand out
 * the pieces, 256-byte aligned. A call of the same or a smaller shape
 * allocates nothing. */
typedef struct {
    char *base;
    size_t off;
} arena_t;

static void *aalloc(arena_t *a, size_t bytes) {
    void *p = a->base ? a->base + a->off : NULL;
    a->off += jt_round_up(bytes ? bytes : 16, 256);
    return p;
}

/* W8A8 expert GEMM scratch, sized for the largest call of one forward */
typedef struct {
    int8_t *Aq, *Bq, *P;
    float *sA1, *sA, *sB1, *sB;
} w8_ws;

/* C[M][N] = A[M][K] x Brow[N][K]^T: A per tensor, B per output row
 * (src/moe_layer.c:228-274). */
static int w8a8_pc(jt_rt *rt, w8_ws *w, const float *A, const float *Brow, float *C, int M,
                   int N, int K) {
    /* the reference's W8A8 GEMM limit, src/w8a8.c:926-929 (EINVAL) */
    if (M > JT_BWD_MAX_WIDE || N > JT_BWD_MAX_WIDE || K > JT_BWD_MAX_WIDE) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    const int Kp = (int)jt_round_up((size_t)K, 64), Np = (int)jt_round_up((size_t)N, 128);
    hipStream_t s = rt->stream;
    int le = jtk_quant_tensor(A, (int64_t)M * K, w->Bq, w->sA1, rt->d_scratch, jt_rt_errw(rt, s), s);
    /* re-stride the activation codes to the padded GEMM layout */
    le |= (int)hipMemsetAsync(w->Aq, 0, (size_t)M * Kp, s);
    le |= (int)hipMemcpy2DAsync(w->Aq, (size_t)Kp, w->Bq, (size_t)K, (size_t)K, (size_t)M,
                                hipMemcpyDeviceToDevice, s);
    le |= jtk_bcast_f32(w->sA, M, w->sA1, s);
    le |= jtk_quant_weight_rows(Brow, K, 1, N, K, w->Bq, w->sB, jt_rt_errw(rt, s), s);
    le |= jtk_pack_i8(w->Bq, N, K, 0, Np, Kp, w->P, s);
    le |= jtk_w8a8_gemm(w->Aq, Kp, w->sA, w->P, w->sB, M, N, Np, Kp, C, N, 0, jt_rt_errw(rt, s), s);
    return le ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

/* C[M][N] = A[M][K] x Bkn[K][N], both per tensor (src/moe_layer.c:185-223). */
static int w8a8_pt(jt_rt *rt, w8_ws *w, const float *A, const float *Bkn, float *C, int M,
                   int N, int K) {
    /* the reference's W8A8 GEMM limit, src/w8a8.c:926-929 (EINVAL) */
    if (M > JT_BWD_MAX_WIDE || N > JT_BWD_MAX_WIDE || K > JT_BWD_MAX_WIDE) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    const int Kp = (int)jt_round_up((size_t)K, 64), Np = (int)jt_round_up((size_t)N, 128);
    hipStream_t s = rt->stream;
    int le = jtk_quant_tensor(A, (int64_t)M * K, w->Bq, w->sA1, rt->d_scratch, jt_rt_errw(rt, s), s);
    le |= (int)hipMemsetAsync(w->Aq, 0, (size_t)M * Kp, s);
    le |= (int)hipMemcpy2DAsync(w->Aq, (size_t)Kp, w->Bq, (size_t)K, (size_t)K, (size_t)M,
                                hipMemcpyDeviceToDevice, s);
    le |= jtk_bcast_f32(w->sA, M, w->sA1, s);
    le |= jtk_quant_tensor(Bkn, (int64_t)K * N, w->Bq, w->sB1, rt->d_scratch + 1, jt_rt_errw(rt, s), s);
    le |= jtk_bcast_f32(w->sB, Np, w->sB1, s);
    le |= jtk_pack_i8(w->Bq, N, K, 1, Np, Kp, w->P, s);
    le |= jtk_w8a8_gemm(w->Aq, Kp, w->sA, w->P, w->sB, M, N, Np, Kp, C, N, 0, jt_rt_errw(rt, s), s);
    return le ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

static int valid_dims(int n, int h, int e, int k, int s) {
    if (n <= 0 || h <= 0 || n > JT_BWD_MAX_WIDE || h > JT_BWD_MAX_WIDE) return 0;
    if (e <= 0 || e > JT_MOE_MAX_EXPERTS) return 0;
    if (k <= 0 || k > e || k > JT_MOE_MAX_TOPK) return 0;
    if (s < 0 || s > JT_MOE_MAX_SHARED) return 0;
    return 1;
}

static int fwd_batch(const float *X, const float *Wgate, const float *Wg, const float *Wu,
                     const float *Wd, const float *Wg_s, const float *Wu_s, const float *Wd_s,
                     float *Y, int T, int n, int h, int E, int k, int S, size_t *out_ids,
                     float *out_weights, float *cache_Gsel, float *cache_Usel,
                     float *cache_Ysel, float *cache_Gs, float *cache_Us, float cap_factor,
                     size_t *out_perm, size_t *out_off, unsigned char *out_drop,
                     size_t *out_kept, size_t *out_dropped, int validate) {
    if (!X || !Wgate || !Wg || !Wu || !Wd || !Y || !out_ids || !out_weights)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (T <= 0 || !valid_dims(n, h, E, k, S)) FAIL(JT_ERR_INVAL, EINVAL);
    if (S > 0 && (!Wg_s || !Wu_s || !Wd_s)) FAIL(JT_ERR_INVAL, EINVAL);
    if (!(cap_factor >= 1.0f) || !(cap_factor <= 1.5f) || !isfinite((double)cap_factor))
        FAIL(JT_ERR_INVAL, EINVAL);
    if ((int64_t)T * k > INT32_MAX / 2 || (int64_t)T * k * n > ((int64_t)1 << 40))
        FAIL(JT_ERR_INVAL, EINVAL);
    if (sizeof(size_t) != 8) FAIL(JT_ERR_NOSUP, EINVAL);
    const int w8a8_on = jt_w8a8_is_enabled();
    const int lbmode = jt_lowbit_get_mode();
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    hipStream_t s = rt->stream;
    uint32_t *err = jt_rt_errw(rt, s);
    const size_t Tk = (size_t)T * k, nh = (size_t)n * h, Tn = (size_t)T * n;
    const size_t NB = (Tk + 255) / 256;
    const int Kpmax = (int)jt_round_up((size_t)(n > h ? n : h), 64);
    const int Npmax = (int)jt_round_up((size_t)(n > h ? n : h), 128);
    const size_t Mmax = Tk > (size_t)T ? Tk : (size_t)T;
    const int32_t soff_h[2] = {0, T}; /* the shared experts' rows as one expert's */
    int rc = JT_OK;
    arena_t a = {.base = NULL, .off = 0};
carve:; /* first pass sizes the workspace (base NULL), the second carves it */
    float *dX = aalloc(&a, Tn * 4), *dWgate = aalloc(&a, (size_t)E * n * 4);
    float *dWg = aalloc(&a, E * nh * 4), *dWu = aalloc(&a, E * nh * 4);
    float *dWd = aalloc(&a, E * nh * 4);
    float *dWgs = S ? aalloc(&a, S * nh * 4) : NULL, *dWus = S ? aalloc(&a, S * nh * 4) : NULL;
    float *dWds = S ? aalloc(&a, S * nh * 4) : NULL;
    float *logits = aalloc(&a, (size_t)T * E * 4);
    int32_t *ids = aalloc(&a, Tk * 4);
    int64_t *ids64 = aalloc(&a, Tk * 8);
    float *w = aalloc(&a, Tk * 4);
    int32_t *rank = aalloc(&a, Tk * 4), *cnt = aalloc(&a, NB * E * 4);
    int32_t *tot = aalloc(&a, (size_t)E * 4), *off = aalloc(&a, ((size_t)E + 1) * 4);
    int64_t *off64 = aalloc(&a, ((size_t)E + 1) * 8);
    int32_t *perm = aalloc(&a, Tk * 4);
    int64_t *perm64 = aalloc(&a, Tk * 8);
    uint8_t *drop = aalloc(&a, Tk);
    float *Xe = aalloc(&a, Mmax * n * 4), *Ge = aalloc(&a, Mmax * h * 4);
    float *Ue = aalloc(&a, Mmax * h * 4), *Se = aalloc(&a, Mmax * h * 4);
    float *Ye = aalloc(&a, Mmax * n * 4);
    float *Ysel = aalloc(&a, Tk * n * 4);
    float *Gsel = cache_Gsel ? aalloc(&a, Tk * h * 4) : NULL;
    float *Usel = cache_Usel ? aalloc(&a, Tk * h * 4) : NULL;
    float *Ys = aalloc(&a, (size_t)(S ? S : 1) * Tn * 4);
    float *Gs = (S && cache_Gs) ? aalloc(&a, (size_t)T * S * h * 4) : NULL;
    float *Us = (S && cache_Us) ? aalloc(&a, (size_t)T * S * h * 4) : NULL;
    float *Wt1 = aalloc(&a, nh * 4), *Wt2 = aalloc(&a, nh * 4);
    float *dY = aalloc(&a, Tn * 4);
    /* the batched fake-quant's maxima: a row of every gate/up matrix, or a
     * column of every down matrix */
    float *fqws = lbmode == 1 ? aalloc(&a, (size_t)E * (n > h ? n : h) * 4) : NULL;
    w8_ws w8 = {0};
    w8.Aq = aalloc(&a, Mmax * Kpmax);
    w8.Bq = aalloc(&a, (Mmax > (size_t)Npmax ? Mmax : (size_t)Npmax) * Kpmax);
    w8.P = aalloc(&a, (size_t)Npmax * Kpmax);
    w8.sA1 = aalloc(&a, 16);
    w8.sB1 = aalloc(&a, 16);
    w8.sA = aalloc(&a, Mmax * 4);
    w8.sB = aalloc(&a, (size_t)Npmax * 4);
    /* the grouped fp32 path's tile list and shared hidden rows */
    const int max_tiles = (int)(Tk / 16) + E + 1;
    /* W8A8: every routed expert's steps in a few launches over the tile list
     * (the launches' grids hold up to 65535 tiles and experts; beyond, the
     * per-expert steps below): the weights' codes, panels, column scales and
     * the experts' per-tensor maxima */
    const int w8b = !lbmode && w8a8_on && max_tiles <= 65535;
    const int Np16 = (int)jt_round_up((size_t)(n > h ? n : h), 16);
    int8_t *wq = w8b ? aalloc(&a, (size_t)E * nh) : NULL;
    int8_t *wpan = w8b ? aalloc(&a, (size_t)E * Np16 * Kpmax) : NULL;
    float *wsb = w8b ? aalloc(&a, (size_t)E * Np16 * 4) : NULL;
    uint32_t *wamax = w8b ? aalloc(&a, (size_t)E * 4) : NULL;
    /* T-MAC LUT mode: every routed expert's lookup GEMMs in a few launches
     * when both reductions are multiples of 32 (else the per-expert steps,
     * whose fp64 fallback takes the other widths): the rows' tables, scales,
     * biases and sums, the experts' bit-plane indices and column maxima */
    const int lutb = lbmode == 2 && n % 32 == 0 && h % 32 == 0 && E <= 65535;
    const size_t nhmax = (size_t)(n > h ? n : h);
    int8_t *lq = lutb ? aalloc(&a, Mmax * nhmax * 2) : NULL;
    float *lsc = lutb ? aalloc(&a, Mmax * (nhmax / 32) * 4) : NULL;
    float *lbi = lutb ? aalloc(&a, Mmax * (nhmax / 32) * 4) : NULL;
    double *lrs = lutb ? aalloc(&a, Mmax * 8) : NULL;
    uint8_t *lidx = lutb ? aalloc(&a, (size_t)E * nh) : NULL;
    float *lws = lutb ? aalloc(&a, (size_t)E * nhmax * 4) : NULL;
    /* the shared experts' W8A8 steps likewise (T <= 4096 rows): the token
     * rows' codes once, their tile list as one expert's */
    const int w8s = w8a8_on && S > 0 && T <= JT_BWD_MAX_WIDE;
    const int mts = T / 16 + 2;
    int8_t *sxq = w8s ? aalloc(&a, (size_t)T * Kpmax) : NULL;
    float *sxa = w8s ? aalloc(&a, (size_t)T * 4) : NULL;
    int32_t *soff = w8s ? aalloc(&a, 16) : NULL;
    int32_t *stiles = w8s ? aalloc(&a, (size_t)mts * 16) : NULL, *snt = w8s ? aalloc(&a, 16) : NULL;
    int8_t *wq_s = w8s ? aalloc(&a, nh) : NULL;
    int8_t *wpan_s = w8s ? aalloc(&a, (size_t)Np16 * Kpmax) : NULL;
    float *wsb_s = w8s ? aalloc(&a, (size_t)Np16 * 4) : NULL;
    uint32_t *wamax_s = w8s ? aalloc(&a, 16) : NULL;
    int32_t *tiles = aalloc(&a, (size_t)max_tiles * 16), *ntiles = aalloc(&a, 16);
    float *Ssh = S ? aalloc(&a, (size_t)S * T * h * 4) : NULL;
    if (!a.base) {
        a.base = jt_rt_buf(rt, JT_SLOT_LAYER, a.off, &rc);
        if (!a.base) return rc;
        a.off = 0;
        goto carve;
    }
    int64_t *hoff = malloc(((size_t)E + 1) * 8);
    if (!hoff) {
        errno = ENOMEM;
        return JT_ERR_NOMEM;
    }
    /* The inputs sit at the front of the workspace, in this order: they are
     * gathered into pinned staging at the same offsets and go over in one
     * copy, queued ahead of the kernels (the staging is rewritten only by a
     * later call, after this one has waited for its stream). */
    const size_t in_bytes = (size_t)((char *)(S ? dWds + S * nh : dWd + E * nh) - (char *)dX);
    {
        char *stin = jt_rt_hbuf(rt, 0, in_bytes, &rc);
        if (!stin) goto out;
        size_t at = 0; /* the alignment gaps are zero, so one check covers the region */
#define STAGE_IN(d, h_, b)                                                                 \
    do {                                                                                   \
        const size_t o_ = (size_t)((char *)(d) - (char *)dX);                              \
        memset(stin + at, 0, o_ - at);                                                     \
        memcpy(stin + o_, (h_), (b));                                                      \
        at = o_ + (b);                                                                     \
    } while (0)
        STAGE_IN(dX, X, Tn * 4);
        STAGE_IN(dWgate, Wgate, (size_t)E * n * 4);
        STAGE_IN(dWg, Wg, E * nh * 4);
        STAGE_IN(dWu, Wu, E * nh * 4);
        STAGE_IN(dWd, Wd, E * nh * 4);
        if (S) {
            STAGE_IN(dWgs, Wg_s, S * nh * 4);
            STAGE_IN(dWus, Wu_s, S * nh * 4);
            STAGE_IN(dWds, Wd_s, S * nh * 4);
        }
#undef STAGE_IN
        rc = jt_rt_err(hipMemcpyAsync(dX, stin, in_bytes, hipMemcpyHostToDevice, s));
        if (rc != JT_OK) goto out;
    }
    int le = 0;
    if (validate) /* src/moe_layer.c:1074-1096: every input, in one launch */
        le |= jtk_check_finite(dX, (int64_t)(in_bytes / 4), err, s);
    /* gate logits + top-k (src/moe_layer.c:1114-1156) */
    le |= jtk_router_logits(dX, dWgate, T, E, n, logits, err, s);
    le |= jtk_topk(logits, T, E, k, ids, ids64, w, err, s);
    /* capacity sort + renormalisation (src/moe_layer.c:1158-1201) */
    const double capd = ceil((double)cap_factor * (double)Tk / (double)E);
    le |= jtk_sort(ids, (int)Tk, E, (int64_t)capd, rank, cnt, tot, off, off64, perm, perm64,
                   drop, err, s);
    le |= jtk_renorm(w, drop, T, k, err, s);
    if (le) {
        rc = jt_rt_err(hipErrorLaunchFailure);
        goto out;
    }
    /* The routed experts' fp32 FFN in two grouped launches over every expert,
     * with the same arithmetic as the per-expert launches below and no wait
     * for the expert offsets: with the flags off, and in the low-bit
     * fake-quant mode after every touched expert's weights are fake-quantised
     * in place (their per-call device copies; per gate/up row at 2 bits, per
     * down column at 4, as the per-expert steps do). The shared experts'
     * fp32 FFN likewise in two launches unless W8A8 is on. W8A8 and the
     * T-MAC LUT mode keep the reference's per-expert steps (per-call
     * quantisation of each expert's weights and activations). */
    const int rgrouped = lbmode == 0 ? !w8a8_on : lbmode == 1;
    const int sgrouped = !w8a8_on;
    uint32_t f = 0;
    if (!rgrouped) {
        if ((rc = jt_rt_flags(rt, s, &f)) != JT_OK) goto out;
        if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) goto out;
        if ((rc = jt_rt_d2h(rt, hoff, off64, ((size_t)E + 1) * 8)) != JT_OK) goto out;
    }
    if (cache_Ysel) le |= (int)hipMemsetAsync(Ysel, 0, Tk * n * 4, s);
    if (Gsel) le |= (int)hipMemsetAsync(Gsel, 0, Tk * h * 4, s);
    if (Usel) le |= (int)hipMemsetAsync(Usel, 0, Tk * h * 4, s);
    if (rgrouped) {
        le |= jtk_make_tiles(off, E, 16, tiles, ntiles, s);
        if (lbmode == 1) { /* src/moe_layer.c:1301-1365, lowbit.c:118-139 */
            le |= jtk_lowbit_fq_rows(dWg, (int64_t)E * h, n, off, h, 2, fqws, err, s);
            le |= jtk_lowbit_fq_rows(dWu, (int64_t)E * h, n, off, h, 2, fqws, err, s);
            le |= jtk_lowbit_fq_cols_batch(dWd, E, h, n, off, 4, fqws, err, s);
        }
        le |= jtk_ffn_f32(dX, T, n, h, perm, k, tiles, ntiles, max_tiles, dWg, dWu, dWd, E, Gsel,
                          Usel, Se, Ysel, 0, err, s);
    }
    if (sgrouped && S)
        le |= jtk_ffn_f32(dX, T, n, h, NULL, k, NULL, NULL, 0, dWgs, dWus, dWds, S, Gs, Us, Ssh,
                          Ys, 1, err, s);
    if (w8b && rc == JT_OK) {
        /* src/moe_layer.c:1265-1420 with the W8A8 steps of :185-274 for
         * every expert at once: the reference's M <= 4096 limit first */
        for (int e = 0; e < E; e++)
            if (hoff[e + 1] - hoff[e] > JT_BWD_MAX_WIDE) {
                errno = EINVAL;
                rc = JT_ERR_INVAL;
                goto out;
            }
        const int kept = (int)hoff[E];
        const int Kpn = (int)jt_round_up((size_t)n, 64), Kph = (int)jt_round_up((size_t)h, 64);
        const int Nph = (int)jt_round_up((size_t)h, 16), Npn = (int)jt_round_up((size_t)n, 16);
        uint32_t *ew = err;
        le |= jtk_make_tiles(off, E, 16, tiles, ntiles, s);
        le |= jtk_gather_rows(dX, n, perm, 0, k, kept, Xe, s);
        le |= jtk_quant_tiles(Xe, n, tiles, ntiles, max_tiles, wamax, E, w8.Aq, Kpn, w8.sA, ew, s);
        le |= jtk_w8a8_weights_e(dWg, E, h, n, 0, off, wq, Nph, Kpn, wpan, wsb, NULL, ew, s);
        le |= jtk_w8a8_gemm_tiles(w8.Aq, Kpn, w8.sA, wpan, (int64_t)Nph * Kpn, wsb, h, h, Nph,
                                  Kpn, n, Ge, h, tiles, ntiles, max_tiles, ew, s);
        le |= jtk_w8a8_weights_e(dWu, E, h, n, 0, off, wq, Nph, Kpn, wpan, wsb, NULL, ew, s);
        le |= jtk_w8a8_gemm_tiles(w8.Aq, Kpn, w8.sA, wpan, (int64_t)Nph * Kpn, wsb, h, h, Nph,
                                  Kpn, n, Ue, h, tiles, ntiles, max_tiles, ew, s);
        le |= jtk_silu_tile(Ge, Ue, (int64_t)kept * h, Se, ew, s);
        le |= jtk_quant_tiles(Se, h, tiles, ntiles, max_tiles, wamax, E, w8.Aq, Kph, w8.sA, ew, s);
        le |= jtk_w8a8_weights_e(dWd, E, n, h, 1, off, wq, Npn, Kph, wpan, wsb, wamax, ew, s);
        le |= jtk_w8a8_gemm_tiles(w8.Aq, Kph, w8.sA, wpan, (int64_t)Npn * Kph, wsb, Npn, n, Npn,
                                  Kph, h, Ye, n, tiles, ntiles, max_tiles, ew, s);
        le |= jtk_scatter_rows(Ye, n, perm, 0, kept, Ysel, s);
        if (Gsel) le |= jtk_scatter_rows(Ge, h, perm, 0, kept, Gsel, s);
        if (Usel) le |= jtk_scatter_rows(Ue, h, perm, 0, kept, Usel, s);
    }
    if (lutb && rc == JT_OK) {
        /* src/moe_layer.c:1265-1420 with jt_lowbit_gemm_lut (lowbit.c:158-267)
         * for every expert at once */
        const int kept = (int)hoff[E];
        le |= jtk_gather_rows(dX, n, perm, 0, k, kept, Xe, s);
        le |= jtk_tmac_ctor(Xe, kept, n, lq, lsc, lbi, err, s);
        le |= jtk_rowsum_f64(Xe, kept, n, lrs, s);
        /* gate/up: column j of the transposed [n][h] matrix is row j of W */
        le |= jtk_col_to_idx_e(dWg, E, n, h, (int64_t)nh, 1, n, off, 2, lws, lidx, err, s);
        le |= jtk_tmac_gemm_e(lq, lsc, lbi, lrs, lidx, lws, off, E, kept, h, n, 2, Ge, err, s);
        le |= jtk_col_to_idx_e(dWu, E, n, h, (int64_t)nh, 1, n, off, 2, lws, lidx, err, s);
        le |= jtk_tmac_gemm_e(lq, lsc, lbi, lrs, lidx, lws, off, E, kept, h, n, 2, Ue, err, s);
        le |= jtk_silu_tile(Ge, Ue, (int64_t)kept * h, Se, err, s);
        le |= jtk_tmac_ctor(Se, kept, h, lq, lsc, lbi, err, s);
        le |= jtk_rowsum_f64(Se, kept, h, lrs, s);
        /* down: W [h][n] as [k = h][n] */
        le |= jtk_col_to_idx_e(dWd, E, h, n, (int64_t)nh, n, 1, off, 4, lws, lidx, err, s);
        le |= jtk_tmac_gemm_e(lq, lsc, lbi, lrs, lidx, lws, off, E, kept, n, h, 4, Ye, err, s);
        le |= jtk_scatter_rows(Ye, n, perm, 0, kept, Ysel, s);
        if (Gsel) le |= jtk_scatter_rows(Ge, h, perm, 0, kept, Gsel, s);
        if (Usel) le |= jtk_scatter_rows(Ue, h, perm, 0, kept, Usel, s);
    }
    /* per-expert forward (src/moe_layer.c:1265-1420): the T-MAC LUT mode
     * (lbmode 2) with other widths, and W8A8 beyond the batched launches'
     * limits */
    for (int e = 0; e < E && rc == JT_OK && !rgrouped && !w8b && !lutb; e++) {
        const int b0 = (int)hoff[e], Me = (int)(hoff[e + 1] - hoff[e]);
        if (Me == 0) continue;
        const float *wg = dWg + e * nh, *wu = dWu + e * nh, *wd = dWd + e * nh;
        le |= jtk_gather_rows(dX, n, perm, b0, k, Me, Xe, s);
        if (lbmode != 0) {
            le |= jtk_transpose_f32(wg, Wt1, h, n, s);
            le |= jtk_transpose_f32(wu, Wt2, h, n, s);
            rc = jt_dev_lowbit_gemm_lut(rt, Xe, Wt1, Ge, Me, h, n, 2);
            if (rc == JT_OK) rc = jt_dev_lowbit_gemm_lut(rt, Xe, Wt2, Ue, Me, h, n, 2);
        } else {
            rc = w8a8_pc(rt, &w8, Xe, wg, Ge, Me, h, n);
            if (rc == JT_OK) rc = w8a8_pc(rt, &w8, Xe, wu, Ue, Me, h, n);
        }
        if (rc != JT_OK) break; /* nothing more runs on the unfilled rows */
        le |= jtk_silu_tile(Ge, Ue, (int64_t)Me * h, Se, err, s);
        if (lbmode != 0)
            rc = jt_dev_lowbit_gemm_lut(rt, Se, wd, Ye, Me, n, h, 4);
        else
            rc = w8a8_pt(rt, &w8, Se, wd, Ye, Me, n, h);
        if (rc != JT_OK) break;
        le |= jtk_scatter_rows(Ye, n, perm, b0, Me, Ysel, s);
        if (Gsel) le |= jtk_scatter_rows(Ge, h, perm, b0, Me, Gsel, s);
        if (Usel) le |= jtk_scatter_rows(Ue, h, perm, b0, Me, Usel, s);
    }
    if (rc == JT_OK && le) rc = jt_rt_err(hipErrorLaunchFailure);
    /* shared experts with W8A8 on (src/moe_layer.c:1468-1560) */
    if (w8s && rc == JT_OK) {
        const int Kpn = (int)jt_round_up((size_t)n, 64), Kph = (int)jt_round_up((size_t)h, 64);
        const int Nph = (int)jt_round_up((size_t)h, 16), Npn = (int)jt_round_up((size_t)n, 16);
        le |= (int)hipMemcpyAsync(soff, soff_h, sizeof(soff_h), hipMemcpyHostToDevice, s);
        le |= jtk_make_tiles(soff, 1, 16, stiles, snt, s);
        le |= jtk_quant_tiles(dX, n, stiles, snt, mts, wamax_s, 1, sxq, Kpn, sxa, err, s);
        for (int sx = 0; sx < S; sx++) {
            const float *wg = dWgs + sx * nh, *wu = dWus + sx * nh, *wd = dWds + sx * nh;
            le |= jtk_w8a8_weights_e(wg, 1, h, n, 0, soff, wq_s, Nph, Kpn, wpan_s, wsb_s, NULL,
                                     err, s);
            le |= jtk_w8a8_gemm_tiles(sxq, Kpn, sxa, wpan_s, 0, wsb_s, 0, h, Nph, Kpn, n, Ge, h,
                                      stiles, snt, mts, err, s);
            le |= jtk_w8a8_weights_e(wu, 1, h, n, 0, soff, wq_s, Nph, Kpn, wpan_s, wsb_s, NULL,
                                     err, s);
            le |= jtk_w8a8_gemm_tiles(sxq, Kpn, sxa, wpan_s, 0, wsb_s, 0, h, Nph, Kpn, n, Ue, h,
                                      stiles, snt, mts, err, s);
            if (Gs) le |= (int)hipMemcpy2DAsync(Gs + (size_t)sx * h, (size_t)S * h * 4, Ge,
                                               (size_t)h * 4, (size_t)h * 4, (size_t)T,
                                               hipMemcpyDeviceToDevice, s);
            if (Us) le |= (int)hipMemcpy2DAsync(Us + (size_t)sx * h, (size_t)S * h * 4, Ue,
                                               (size_t)h * 4, (size_t)h * 4, (size_t)T,
                                               hipMemcpyDeviceToDevice, s);
            le |= jtk_silu_tile(Ge, Ue, (int64_t)T * h, Se, err, s);
            le |= jtk_quant_tiles(Se, h, stiles, snt, mts, wamax_s, 1, w8.Aq, Kph, w8.sA, err, s);
            le |= jtk_w8a8_weights_e(wd, 1, n, h, 1, soff, wq_s, Npn, Kph, wpan_s, wsb_s, wamax_s,
                                     err, s);
            le |= jtk_w8a8_gemm_tiles(w8.Aq, Kph, w8.sA, wpan_s, 0, wsb_s, 0, n, Npn, Kph, h,
                                      Ys + (size_t)sx * Tn, n, stiles, snt, mts, err, s);
        }
    }
    for (int sx = 0; sx < S && rc == JT_OK && !sgrouped && !w8s; sx++) {
        const float *wg = dWgs + sx * nh, *wu = dWus + sx * nh, *wd = dWds + sx * nh;
        float *ys = Ys + (size_t)sx * Tn;
        rc = w8a8_pc(rt, &w8, dX, wg, Ge, T, h, n);
        if (rc == JT_OK) rc = w8a8_pc(rt, &w8, dX, wu, Ue, T, h, n);
        if (rc != JT_OK) break; /* nothing more runs on the unfilled rows */
        if (Gs) le |= (int)hipMemcpy2DAsync(Gs + (size_t)sx * h, (size_t)S * h * 4, Ge,
                                           (size_t)h * 4, (size_t)h * 4, (size_t)T,
                                           hipMemcpyDeviceToDevice, s);
        if (Us) le |= (int)hipMemcpy2DAsync(Us + (size_t)sx * h, (size_t)S * h * 4, Ue,
                                           (size_t)h * 4, (size_t)h * 4, (size_t)T,
                                           hipMemcpyDeviceToDevice, s);
        le |= jtk_silu_tile(Ge, Ue, (int64_t)T * h, Se, err, s);
        rc = w8a8_pt(rt, &w8, Se, wd, ys, T, n, h);
    }
    /* combine (src/moe_layer.c:1443-1463, 1549-1574) */
    if (rc == JT_OK) le |= jtk_combine(w, Ysel, drop, Ys, S, T, k, n, NULL, dY, err, s);
    if (rc == JT_OK && le) rc = jt_rt_err(hipErrorLaunchFailure);
    if (rc != JT_OK) goto out;
    /* The outputs go to pinned staging in copies queued behind the kernels;
     * one wait (the error word's read) covers them all, and only then are
     * the caller's buffers written (fail-closed: a failed call writes no
     * host output). */
    struct {
        void *dst;
        const void *src;
        size_t bytes, at;
    } oc[12];
    int no = 0;
    size_t ob = 0;
#define STAGE_OUT(d, sp, b)                                                                \
    if (d) {                                                                               \
        oc[no].dst = (void *)(d);                                                          \
        oc[no].src = (sp);                                                                 \
        oc[no].bytes = (b);                                                                \
        oc[no].at = ob;                                                                    \
        ob += jt_round_up((size_t)(b) + 1, 256);                                           \
        no++;                                                                              \
    }
    STAGE_OUT(hoff, off64, ((size_t)E + 1) * 8); /* first: the kept count */
    STAGE_OUT(Y, dY, Tn * 4);
    STAGE_OUT(out_ids, ids64, Tk * 8);
    STAGE_OUT(out_weights, w, Tk * 4);
    STAGE_OUT(out_perm, perm64, Tk * 8); /* the kept entries are handed over */
    STAGE_OUT(out_drop, drop, Tk);
    STAGE_OUT(cache_Ysel, Ysel, Tk * n * 4);
    STAGE_OUT(cache_Gsel, Gsel, Tk * h * 4);
    STAGE_OUT(cache_Usel, Usel, Tk * h * 4);
    if (Gs) STAGE_OUT(cache_Gs, Gs, (size_t)T * S * h * 4);
    if (Us) STAGE_OUT(cache_Us, Us, (size_t)T * S * h * 4);
#undef STAGE_OUT
    char *stout = jt_rt_hbuf(rt, 1, ob, &rc);
    if (!stout) goto out;
    for (int i = 0; i < no && rc == JT_OK; i++)
        rc = jt_rt_err(hipMemcpyAsync(stout + oc[i].at, oc[i].src, oc[i].bytes,
                                      hipMemcpyDeviceToHost, s));
    if (rc != JT_OK) goto out;
    if ((rc = jt_rt_flags(rt, s, &f)) != JT_OK) goto out;
    if ((rc = jt_rt_flags_to_rc(f)) != JT_OK) goto out;
    memcpy(hoff, stout, ((size_t)E + 1) * 8);
    const size_t kept = (size_t)hoff[E];
    for (int i = 1; i < no; i++)
        memcpy(oc[i].dst, stout + oc[i].at, oc[i].dst == out_perm ? kept * 8 : oc[i].bytes);
    if (out_off) memcpy(out_off, hoff, ((size_t)E + 1) * 8);
    if (rc == JT_OK) {
        if (out_kept) *out_kept = kept;
        if (out_dropped) *out_dropped = Tk - kept;
    }
out:
    (void)hipStreamSynchronize(s);
    if (rc != JT_OK) {
        /* a failed call reports its own code: flags raised by work it had
         * already queued are dropped, not left for the stream's next call */
        const int saved = errno;
        uint32_t dropped = 0;
        (void)jt_rt_flags(rt, s, &dropped);
        errno = saved;
    }
    free(hoff);
    return rc;
}

int jt_moe_fwd_batch(const float *X, const float *Wgate, const float *Wg, const float *Wu,
                     const float *Wd, const float *Wg_s, const float *Wu_s, const float *Wd_s,
                     float *Y, int T, int n, int h, int n_experts, int topk, int n_shared,
                     size_t *out_ids, float *out_weights, float *cache_Gsel, float *cache_Usel,
                     float *cache_Ysel, float *cache_Gs, float *cache_Us, float cap_factor,
                     size_t *out_perm, size_t *out_off, unsigned char *out_drop,
                     size_t *out_kept, size_t *out_dropped) {
    return fwd_batch(X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, Y, T, n, h, n_experts, topk,
                     n_shared, out_ids, out_weights, cache_Gsel, cache_Usel, cache_Ysel,
                     cache_Gs, cache_Us, cap_factor, out_perm, out_off, out_drop, out_kept,
                     out_dropped, 1);
}

int jt_moe_fwd_batch_unchecked(
    const float *X, const float *Wgate, const float *Wg, const float *Wu, const float *Wd,
    const float *Wg_s, const float *Wu_s, const float *Wd_s, float *Y, int T, int n, int h,
    int n_experts, int topk, int n_shared, size_t *out_ids, float *out_weights,
    float *cache_Gsel, float *cache_Usel, float *cache_Ysel, float *cache_Gs, float *cache_Us,
    float cap_factor, size_t *out_perm, size_t *out_off, unsigned char *out_drop,
    size_t *out_kept, size_t *out_dropped) {
    return fwd_batch(X, Wgate, Wg, Wu, Wd, Wg_s, Wu_s, Wd_s, Y, T, n, h, n_experts, topk,
                     n_shared, out_ids, out_weights, cache_Gsel, cache_Usel, cache_Ysel,
                     cache_Gs, cache_Us, cap_factor, out_perm, out_off, out_drop, out_kept,
                     out_dropped, 0);
}
