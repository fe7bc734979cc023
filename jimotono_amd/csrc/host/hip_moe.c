/*
 * hip_moe.c -- device-resident quantised MoE layer and W8A8 SwiGLU expert
 * (C11 host orchestration of the gfx950 kernels).
 *
 * Forward of the layer (jimotono/hip_moe.h), all on one stream:
 *   1 quant_x        per-token int8 activations            (src/w8a8.c:787-855)
 *   2 router         fp64 gate logits, lane order          (src/moe_layer.c:67-86)
 *   3 topk           top-k + softmax                       (src/routing.c:16-76)
 *   4 sort           dropless stable expert sort           (src/moe_layer.c:895-978)
 *   5 tiles          work list of the sorted pairs: 64-row tiles, or 16-row
 *                    tiles when experts get few rows (decode); up to 1024
 *                    pairs the sort and the list are one launch
 *   6 routed_gateup  INT2 grouped GEMM + SwiGLU            (src/moe_layer.c:1301-1365)
 *   7 routed_quant   per-row int8 requantisation of SwiGLU output
 *   8 routed_down    INT4 grouped GEMM, rows scattered to their (token, slot)
 *   9 shared_gateup  W8A8 GEMM + SwiGLU per shared expert  (src/moe_layer.c:1468-1540)
 *  10 shared_quant
 *  11 shared_down
 *  12 combine        fp64 weighted sum, slot then shared order
 *                                                          (src/moe_layer.c:1443-1574)
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

/* ======================= W8A8 SwiGLU expert ======================= */

struct jt_hip_ffn {
    int n, h, Kpn, Kph, Np_gu, Np_d;
    int8_t *gu_P; /* gate/up interleaved panels, N = 2h */
    float *gu_s;
    int8_t *d_P; /* down panels, N = n, K = h */
    float *d_s;
    /* workspace */
    int cap_T;
    int8_t *Xq;
    float *sx;
    float *S;
    int8_t *Sq;
    float *ss;
};

void jt_hip_ffn_free(jt_hip_ffn *F) {
    if (!F) return;
    void *p[] = {F->gu_P, F->gu_s, F->d_P, F->d_s, F->Xq, F->sx, F->S, F->Sq, F->ss};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) (void)hipFree(p[i]);
    free(F);
}

/* An expert with its weight arrays allocated (scales zeroed, panels not
 * written yet). */
static int ffn_alloc(jt_rt *rt, int n, int h, jt_hip_ffn **out) {
    jt_hip_ffn *F = calloc(1, sizeof(*F));
    if (!F) FAIL(JT_ERR_NOMEM, ENOMEM);
    F->n = n;
    F->h = h;
    F->Kpn = (int)jt_round_up((size_t)n, 64);
    F->Kph = (int)jt_round_up((size_t)h, 64);
    F->Np_gu = (int)jt_round_up((size_t)2 * h, 128);
    F->Np_d = (int)jt_round_up((size_t)n, 128);
    hipError_t e = hipSuccess;
#define ALLOC(p, bytes) \
    if (e == hipSuccess) e = hipMalloc((void **)&(p), (size_t)(bytes))
    ALLOC(F->gu_P, (size_t)F->Np_gu * F->Kpn);
    ALLOC(F->gu_s, (size_t)F->Np_gu * sizeof(float));
    ALLOC(F->d_P, (size_t)F->Np_d * F->Kph);
    ALLOC(F->d_s, (size_t)F->Np_d * sizeof(float));
#undef ALLOC
    if (e == hipSuccess) e = hipMemsetAsync(F->gu_s, 0, (size_t)F->Np_gu * sizeof(float), rt->stream);
    if (e == hipSuccess) e = hipMemsetAsync(F->d_s, 0, (size_t)F->Np_d * sizeof(float), rt->stream);
    if (e != hipSuccess) {
        jt_hip_ffn_free(F);
        return jt_rt_err(e);
    }
    *out = F;
    return JT_OK;
}

static int ffn_prepare_on(jt_rt *rt, const float *dWg, const float *dWu, const float *dWd,
                          int n, int h, jt_hip_ffn **out) {
    jt_hip_ffn *F = NULL;
    int rc = ffn_alloc(rt, n, h, &F);
    if (rc != JT_OK) return rc;
    int8_t *qg = NULL, *qu = NULL, *qgu = NULL, *qd = NULL;
    float *sg = NULL, *su = NULL;
    hipError_t e = hipSuccess;
#define ALLOC(p, bytes) \
    if (e == hipSuccess) e = hipMalloc((void **)&(p), (size_t)(bytes))
    ALLOC(qg, (size_t)h * n);
    ALLOC(qu, (size_t)h * n);
    ALLOC(qgu, (size_t)2 * h * n);
    ALLOC(qd, (size_t)n * h);
    ALLOC(sg, (size_t)h * sizeof(float));
    ALLOC(su, (size_t)h * sizeof(float));
#undef ALLOC
    rc = jt_rt_err(e);
    if (rc == JT_OK) {
        /* gate/up rows are output channels, K = n contiguous */
        jtk_quant_weight_rows(dWg, n, 1, h, n, qg, sg, jt_rt_errw(rt, rt->stream), rt->stream);
        jtk_quant_weight_rows(dWu, n, 1, h, n, qu, su, jt_rt_errw(rt, rt->stream), rt->stream);
        jtk_interleave_rows(qg, qu, h, n, qgu, rt->stream);
        jtk_interleave_rows(sg, su, h, (int64_t)sizeof(float), F->gu_s, rt->stream);
        jtk_pack_i8(qgu, 2 * h, n, 0, F->Np_gu, F->Kpn, F->gu_P, rt->stream);
        /* down: Wd [h][n] is B[K=h][N=n]; output channel j is column j */
        jtk_quant_weight_rows(dWd, 1, n, n, h, qd, F->d_s, jt_rt_errw(rt, rt->stream), rt->stream);
        jtk_pack_i8(qd, n, h, 0, F->Np_d, F->Kph, F->d_P, rt->stream);
        uint32_t f = 0;
        rc = jt_rt_flags(rt, rt->stream, &f);
        if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    }
    (void)hipFree(qg);
    (void)hipFree(qu);
    (void)hipFree(qgu);
    (void)hipFree(qd);
    (void)hipFree(sg);
    (void)hipFree(su);
    if (rc != JT_OK) {
        jt_hip_ffn_free(F);
        return rc;
    }
    *out = F;
    return JT_OK;
}

int jt_hip_ffn_prepare(const float *dWg, const float *dWu, const float *dWd, int n, int h,
                       jt_hip_ffn **out) {
    if (!dWg || !dWu || !dWd || !out || n <= 0 || h <= 0 || h % 16 != 0 ||
        n > JT_BWD_MAX_WIDE || h > JT_BWD_MAX_WIDE)
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    return ffn_prepare_on(rt, dWg, dWu, dWd, n, h, out);
}

static int ffn_reserve(jt_hip_ffn *F, int T, int with_x) {
    if (T <= F->cap_T && (!with_x || F->Xq)) return JT_OK;
    int cap = T > F->cap_T ? T : F->cap_T;
    (void)hipDeviceSynchronize();
    void *olds[] = {F->Xq, F->sx, F->S, F->Sq, F->ss};
    for (size_t i = 0; i < 5; i++) (void)hipFree(olds[i]);
    F->Xq = NULL;
    F->sx = NULL;
    F->S = F->ss = NULL;
    F->Sq = NULL;
    hipError_t e = hipSuccess;
    if (with_x) {
        e = hipMalloc((void **)&F->Xq, (size_t)cap * F->Kpn);
        if (e == hipSuccess) e = hipMemset(F->Xq, 0, (size_t)cap * F->Kpn);
        if (e == hipSuccess) e = hipMalloc((void **)&F->sx, (size_t)cap * sizeof(float));
    }
    if (e == hipSuccess) e = hipMalloc((void **)&F->S, (size_t)cap * F->h * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&F->Sq, (size_t)cap * F->Kph);
    if (e == hipSuccess) e = hipMemset(F->Sq, 0, (size_t)cap * F->Kph);
    if (e == hipSuccess) e = hipMalloc((void **)&F->ss, (size_t)cap * sizeof(float));
    if (e != hipSuccess) {
        F->cap_T = 0;
        return jt_rt_err(e);
    }
    F->cap_T = cap;
    return JT_OK;
}

/* Workspace of one expert forward: Xq [T][Kpn] (zero K padding), sx [T],
 * S [T][h], Sq [T][Kph] (zero K padding), ss [T]. */
typedef struct ffn_ws {
    int8_t *Xq;
    float *sx, *S;
    int8_t *Sq;
    float *ss;
} ffn_ws;

static ffn_ws ffn_own_ws(const jt_hip_ffn *F) {
    ffn_ws w = {F->Xq, F->sx, F->S, F->Sq, F->ss};
    return w;
}

/* Expert on already-quantised activations Xq [T][Kpn] (zero K padding). */
static int ffn_run_q(const jt_hip_ffn *F, const ffn_ws *ws, const int8_t *Xq, const float *sx,
                     int T, float *dY, uint32_t *err, hipStream_t s, hipEvent_t *ev) {
    /* with profiling events the gate/up stage is the kernel's own duration */
    int e = jtk_w8a8_gemm_ev(Xq, F->Kpn, sx, F->gu_P, F->gu_s, T, 2 * F->h, F->Np_gu, F->Kpn,
                             ws->S, F->h, 1, err, s, ev ? ev[0] : NULL,
                             ev ? ev[1] : NULL);
    /* up to 16 rows the down projection quantises the hidden rows itself
     * (timed with the down stage) */
    const int f = T <= 16 ? jtk_w8a8_gemm_xq(ws->S, F->h, F->h, F->d_P, F->d_s, T, F->n,
                                             F->Np_d, F->Kph, dY, F->n, 0, err, s)
                          : (int)hipErrorInvalidValue;
    if (f == (int)hipErrorInvalidValue) {
        e |= jtk_quant_rows(ws->S, T, F->h, ws->Sq, F->Kph, ws->ss, NULL, err, s);
        if (ev) (void)hipEventRecord(ev[2], s);
        e |= jtk_w8a8_gemm(ws->Sq, F->Kph, ws->ss, F->d_P, F->d_s, T, F->n, F->Np_d, F->Kph, dY,
                           F->n, 0, err, s);
    } else {
        if (ev) (void)hipEventRecord(ev[2], s);
        e |= f;
    }
    return e ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

/* The expert on fp32 rows dX with the workspace ws (T > 0). */
static int ffn_fwd_on(const jt_hip_ffn *F, const ffn_ws *ws, const float *dX, float *dY,
                      int T, uint32_t *err, hipStream_t s) {
    if (T <= 16) {
        /* decode: both GEMMs quantise their rows themselves (two launches) */
        int e = jtk_w8a8_gemm_xq(dX, F->n, F->n, F->gu_P, F->gu_s, T, 2 * F->h, F->Np_gu,
                                 F->Kpn, ws->S, F->h, 1, err, s);
        if (e != (int)hipErrorInvalidValue) {
            if (e) return jt_rt_err(hipErrorLaunchFailure);
            e = jtk_w8a8_gemm_xq(ws->S, F->h, F->h, F->d_P, F->d_s, T, F->n, F->Np_d, F->Kph,
                                 dY, F->n, 0, err, s);
            if (e == (int)hipErrorInvalidValue) {
                e = jtk_quant_rows(ws->S, T, F->h, ws->Sq, F->Kph, ws->ss, NULL, err, s);
                e |= jtk_w8a8_gemm(ws->Sq, F->Kph, ws->ss, F->d_P, F->d_s, T, F->n, F->Np_d,
                                   F->Kph, dY, F->n, 0, err, s);
            }
            return e ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
        }
    }
    if (jtk_quant_rows(dX, T, F->n, ws->Xq, F->Kpn, ws->sx, NULL, err, s))
        return jt_rt_err(hipErrorLaunchFailure);
    return ffn_run_q(F, ws, ws->Xq, ws->sx, T, dY, err, s, NULL);
}

int jt_hip_ffn_fwd(jt_hip_ffn *F, const float *dX, float *dY, int T, void *stream) {
    if (!F || !dX || !dY || T < 0) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (T == 0) return JT_OK;
    int rc = ffn_reserve(F, T, 1);
    if (rc != JT_OK) return rc;
    const ffn_ws ws = ffn_own_ws(F);
    const hipStream_t s = (hipStream_t)stream; /* NULL: the null stream */
    return ffn_fwd_on(F, &ws, dX, dY, T, jt_rt_errw(rt, s), s);
}

int jt_hip_ffn_reserve(jt_hip_ffn *F, int T) {
    if (!F || T <= 0) FAIL(JT_ERR_INVAL, EINVAL);
    if (!jt_rt_get()) return JT_ERR_IO;
    return ffn_reserve(F, T, 1);
}

/* Byte offsets of the workspace of a T-row forward inside one buffer, each
 * part 256-byte aligned; returns the total. */
static size_t ffn_ws_layout(const jt_hip_ffn *F, int T, size_t off[5]) {
    const size_t t = (size_t)T;
    const size_t sz[5] = {t * (size_t)F->Kpn, t * 4, t * (size_t)F->h * 4, t * (size_t)F->Kph,
                          t * 4};
    size_t at = 0;
    for (int i = 0; i < 5; i++) {
        off[i] = at;
        at += jt_round_up(sz[i], 256);
    }
    return at;
}

int jt_hip_ffn_fwd_noalloc(jt_hip_ffn *F, const float *dX, float *dY, int T, void *stream) {
    if (!F || !dX || !dY || T < 0) FAIL(JT_ERR_INVAL, EINVAL);
    size_t off[5];
    if (T > 0 && ffn_ws_layout(F, T, off) > JT_SCRATCH_BYTES) FAIL(JT_ERR_NOSUP, E2BIG);
    jt_rt *rt = jt_rt_get(); /* set up already: F was prepared through it */
    if (!rt) return JT_ERR_IO;
    if (T == 0) return JT_OK;
    uint8_t *base = jtk_scratch();
    if (!base) FAIL(JT_ERR_IO, EIO);
    const ffn_ws ws = {(int8_t *)(base + off[0]), (float *)(base + off[1]),
                       (float *)(base + off[2]), (int8_t *)(base + off[3]),
                       (float *)(base + off[4])};
    hipStream_t s = (hipStream_t)stream; /* NULL: the HIP null stream */
    /* the scratch keeps the previous call's bytes: the GEMMs read the K
     * padding of the code rows, which must be zero (a fill kernel, not a
     * memset node, so the call can be captured) */
    int e = 0;
    if (F->Kpn > F->n) e |= jtk_scratch_zero((uint32_t *)ws.Xq, (int64_t)T * F->Kpn / 4, s);
    if (F->Kph > F->h) e |= jtk_scratch_zero((uint32_t *)ws.Sq, (int64_t)T * F->Kph / 4, s);
    if (e) return jt_rt_err(hipErrorLaunchFailure);
    return ffn_fwd_on(F, &ws, dX, dY, T, jt_rt_errw(rt, s), s);
}

/* ======================= MoE layer ======================= */

enum {
    ST_QUANT_X = 0,
    ST_ROUTER,
    ST_TOPK,
    ST_SORT,
    ST_TILES,
    ST_R_GATEUP,
    ST_R_QUANT,
    ST_R_DOWN,
    ST_S_GATEUP,
    ST_S_QUANT,
    ST_S_DOWN,
    ST_COMBINE,
    ST_N
};
static const char *const k_stage_names[ST_N] = {
    "quant_x",       "router_logits", "topk",         "sort",
    "tiles",         "routed_gateup", "routed_quant", "routed_down",
    "shared_gateup", "shared_quant",  "shared_down",  "combine"};

#define PROF_RING 16
/* side streams for the shared experts: one, so the experts run one after
 * the other beside the routed path (measured at 4096 tokens: 0.360 ms per
 * layer against 0.370 with one side stream per expert, which leaves fewer
 * CUs to the routed chain) */
#define MOE_SIDE 1
/* the fork and join events only order work on this device and the host
 * never waits on them, so they skip the system-scope fence */
#define JT_STREAM_EVENT_FLAGS (hipEventDisableTiming | hipEventDisableSystemFence)

struct jt_hip_moe {
    jt_hip_moe_desc d;
    float *Wgate;
    uint8_t *gu_P;
    uint16_t *gu_S;
    uint8_t *dn_P;
    uint16_t *dn_S;
    int64_t gu_pstride, gu_sstride, dn_pstride, dn_sstride;
    jt_hip_ffn *sh[JT_MOE_MAX_SHARED];
    /* workspace (max_tokens) */
    int8_t *Xq;
    float *sx, *logits, *w, *Sr, *ssr, *Ye, *Ys;
    int32_t *ids, *rank, *cnt, *tot, *off, *perm, *tiles, *ntiles;
    uint32_t *route_done; /* decode launch's block counter (zero between launches) */
    const int32_t *cur_ids; /* ids / weights of the last forward (caller's */
    const float *cur_w;     /* arrays after jt_hip_moe_fwd_routed) */
    /* router on the int8 matrix cores with exact verification (E <= 256,
     * d % 64 == 0):
     * residual codes of X and of Wgate, row {scale, l1}, approximate logits */
    int fast_router;
    int8_t *Xl, *rWh, *rWl;
    double *xinfo, *winfo, *approx;
    int16_t *rcand; /* [T][E] candidate experts of each token */
    int32_t *rnc;   /* [T] candidate counts */
    int8_t *Sqr;
    int last_T;
    /* the shared experts as batched GEMMs (S >= 2, 2*h_shared a multiple of
     * 128): gate/up panels and scales concatenated along N, down panels and
     * scales back to back, hidden rows [S][T][h_shared]; for more than 64
     * tokens also their codes [S][T][Kph] and scales [S][T] */
    int sh_cat;
    int8_t *sgu_P, *sd_P;
    float *sgu_s, *sd_s, *sS, *sss;
    int8_t *sSq;
    /* shared experts run on a side stream forked after the input quantiser
     * and joined before the combine; expert e uses side[e % nside] */
    int nside;
    hipStream_t side[MOE_SIDE];
    hipEvent_t ev_fork, ev_join[MOE_SIDE];
    /* profiling: ring of per-forward event sets */
    int prof;
    hipEvent_t ev[PROF_RING][ST_N + 1 + 3 * JT_MOE_MAX_SHARED];
    int ev_fused[PROF_RING]; /* the forward in this slot ran the fused shared path */
    int ev_ready;
    int ring_head, ring_count;
    double acc_ms[ST_N];
    int acc_count;
};

void jt_hip_moe_free(jt_hip_moe *L) {
    if (!L) return;
    void *p[] = {L->Wgate, L->gu_P, L->gu_S, L->dn_P,  L->dn_S, L->Xq,   L->sx,
                 L->logits, L->w,  L->Sr,   L->ssr,  L->Ye,   L->Ys,   L->ids,
                 L->rank,  L->cnt, L->tot,  L->off,  L->perm, L->tiles, L->ntiles,
                 L->Sqr,   L->Xl,  L->rWh,  L->rWl,  L->xinfo, L->winfo, L->approx, L->rcand, L->rnc,
                 L->sgu_P, L->sgu_s, L->sS,  L->sSq,  L->sss,  L->sd_P,  L->sd_s,
                 L->route_done};
    (void)hipDeviceSynchronize();
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) (void)hipFree(p[i]);
    for (int s = 0; s < JT_MOE_MAX_SHARED; s++) jt_hip_ffn_free(L->sh[s]);
    for (int i = 0; i < L->nside; i++) {
        (void)hipEventDestroy(L->ev_join[i]);
        (void)hipStreamDestroy(L->side[i]);
    }
    if (L->nside) (void)hipEventDestroy(L->ev_fork);
    if (L->ev_ready)
        for (int r = 0; r < PROF_RING; r++)
            for (int i = 0; i < ST_N + 1 + 3 * JT_MOE_MAX_SHARED; i++)
                (void)hipEventDestroy(L->ev[r][i]);
    free(L);
}

/* The prepare-time checks of a layer's sizes (jimotono/hip_moe.h). */
static int moe_check_desc(const jt_hip_moe_desc *dp) {
    const jt_hip_moe_desc d = *dp;
    if (d.n <= 0 || d.n % 128 != 0 || d.n > JT_BWD_MAX_WIDE || d.h <= 0 || d.h % 64 != 0 ||
        d.h > JT_BWD_MAX_WIDE || d.n_experts <= 0 || d.n_experts > JT_MOE_MAX_EXPERTS ||
        d.topk <= 0 || d.topk > d.n_experts || d.topk > JT_MOE_MAX_TOPK || d.n_shared < 0 ||
        d.n_shared > JT_MOE_MAX_SHARED || d.group != 64 || d.max_tokens <= 0)
        FAIL(JT_ERR_INVAL, EINVAL);
    if (d.n_shared > 0 &&
        (d.h_shared <= 0 || d.h_shared % 16 != 0 || d.h_shared > JT_BWD_MAX_WIDE))
        FAIL(JT_ERR_INVAL, EINVAL);
    /* the tile list of the largest forward must fit one launch grid
     * (65535 blocks): 64-row tiles plus one short tile per expert */
    if ((int64_t)d.max_tokens * d.topk / 64 + d.n_experts > 65535) FAIL(JT_ERR_INVAL, EINVAL);
    return JT_OK;
}

/* A layer with every device array allocated (weights unwritten) and its
 * workspace sized for d.max_tokens; the shared experts are not created. */
static int moe_alloc(const jt_hip_moe_desc *dp, int has_gate, jt_hip_moe **out) {
    jt_hip_moe *L = calloc(1, sizeof(*L));
    if (!L) FAIL(JT_ERR_NOMEM, ENOMEM);
    const jt_hip_moe_desc d = *dp;
    L->d = d;
    const int n = d.n, h = d.h, E = d.n_experts, T = d.max_tokens;
    const int64_t Tk = (int64_t)T * d.topk;
    const int NB = (int)((Tk + 255) / 256);
    L->gu_pstride = (int64_t)(2 * h / 16) * (n / 64) * 256;
    L->gu_sstride = (int64_t)(2 * h / 16) * (n / 64) * 16;
    L->dn_pstride = (int64_t)(n / 16) * (h / 64) * 512;
    L->dn_sstride = (int64_t)(n / 16) * (h / 64) * 16;
    hipError_t e = hipSuccess;
#define ALLOC(p, bytes) \
    if (e == hipSuccess) e = hipMalloc((void **)&(p), (size_t)(bytes))
    if (has_gate) ALLOC(L->Wgate, (size_t)E * n * sizeof(float));
    ALLOC(L->gu_P, L->gu_pstride * E);
    ALLOC(L->gu_S, L->gu_sstride * E * 2);
    ALLOC(L->dn_P, L->dn_pstride * E);
    ALLOC(L->dn_S, L->dn_sstride * E * 2);
    ALLOC(L->Xq, (size_t)T * n);
    ALLOC(L->sx, (size_t)T * 4);
    ALLOC(L->logits, (size_t)T * E * 4);
    ALLOC(L->ids, (size_t)Tk * 4);
    ALLOC(L->w, (size_t)Tk * 4);
    ALLOC(L->rank, (size_t)Tk * 4);
    ALLOC(L->cnt, (size_t)NB * E * 4);
    ALLOC(L->tot, (size_t)E * 4);
    ALLOC(L->off, (size_t)(E + 1) * 4);
    ALLOC(L->perm, (size_t)Tk * 4);
    ALLOC(L->tiles, (size_t)(Tk / 16 + E + 1) * 16); /* int4 descriptors */
    ALLOC(L->ntiles, 4);
    ALLOC(L->route_done, 64);
    if (e == hipSuccess) e = hipMemset(L->route_done, 0, 64);
    ALLOC(L->Sr, (size_t)Tk * h * 4);
    ALLOC(L->Sqr, (size_t)Tk * h);
    ALLOC(L->ssr, (size_t)Tk * 4);
    ALLOC(L->Ye, (size_t)Tk * n * 4);
    ALLOC(L->Ys, (size_t)(d.n_shared > 0 ? d.n_shared : 1) * T * n * 4);
    L->fast_router = has_gate && E <= 256 && n % 64 == 0;
    if (L->fast_router) {
        const int Ep = (E + 63) / 64 * 64;
        ALLOC(L->Xl, (size_t)T * n);
        ALLOC(L->xinfo, (size_t)T * 16);
        ALLOC(L->approx, (size_t)T * E * 8);
        ALLOC(L->rcand, (size_t)T * E * 2);
        ALLOC(L->rnc, (size_t)T * 4);
        ALLOC(L->rWh, (size_t)Ep * n);
        ALLOC(L->rWl, (size_t)Ep * n);
        ALLOC(L->winfo, (size_t)E * 16);
    }
#undef ALLOC
    if (e != hipSuccess) {
        jt_hip_moe_free(L);
        return jt_rt_err(e);
    }
    *out = L;
    return JT_OK;
}

/* The shared experts' workspace and the side stream of a layer whose
 * weights are in place. */
static int moe_finish(jt_hip_moe *L) {
    int rc = JT_OK;
    const int S = L->d.n_shared, T = L->d.max_tokens;
    const jt_hip_ffn *F0 = S > 0 ? L->sh[0] : NULL;
    /* batched shared experts: whole 256-channel gate/up tiles over the
     * concatenated panels and no padding channels inside an expert's block */
    L->sh_cat = S >= 2 && F0->Np_gu == 2 * F0->h && (S * F0->Np_gu) % 256 == 0;
    if (L->sh_cat) {
        const size_t gub = (size_t)F0->Np_gu * F0->Kpn, gus = (size_t)F0->Np_gu * sizeof(float);
        const size_t db = (size_t)F0->Np_d * F0->Kph, ds = (size_t)F0->Np_d * sizeof(float);
        hipError_t e = hipMalloc((void **)&L->sgu_P, gub * S);
        if (e == hipSuccess) e = hipMalloc((void **)&L->sgu_s, gus * S);
        if (e == hipSuccess) e = hipMalloc((void **)&L->sd_P, db * S);
        if (e == hipSuccess) e = hipMalloc((void **)&L->sd_s, ds * S);
        if (e == hipSuccess) e = hipMalloc((void **)&L->sS, (size_t)S * T * F0->h * 4);
        if (T > 64) {
            if (e == hipSuccess) e = hipMalloc((void **)&L->sSq, (size_t)S * T * F0->Kph);
            if (e == hipSuccess) e = hipMalloc((void **)&L->sss, (size_t)S * T * 4);
            /* K padding of the hidden codes stays zero (the quantiser writes
             * only the h valid columns) */
            if (e == hipSuccess) e = hipMemset(L->sSq, 0, (size_t)S * T * F0->Kph);
        }
        for (int s = 0; s < S && e == hipSuccess; s++) {
            const jt_hip_ffn *F = L->sh[s];
            e = hipMemcpy(L->sgu_P + gub * s, F->gu_P, gub, hipMemcpyDeviceToDevice);
            if (e == hipSuccess)
                e = hipMemcpy((uint8_t *)L->sgu_s + gus * s, F->gu_s, gus,
                              hipMemcpyDeviceToDevice);
            if (e == hipSuccess) e = hipMemcpy(L->sd_P + db * s, F->d_P, db, hipMemcpyDeviceToDevice);
            if (e == hipSuccess)
                e = hipMemcpy((uint8_t *)L->sd_s + ds * s, F->d_s, ds, hipMemcpyDeviceToDevice);
        }
        if (e == hipSuccess) e = hipDeviceSynchronize(); /* before any stream uses them */
        rc = jt_rt_err(e);
    }
    /* an expert's own workspace then serves only forwards of <= 64 tokens */
    for (int s = 0; s < S && rc == JT_OK; s++)
        rc = ffn_reserve(L->sh[s], L->sh_cat ? 64 : T, 0);
    if (rc == JT_OK && L->d.n_shared > 0) {
        const int ns = L->d.n_shared < MOE_SIDE ? L->d.n_shared : MOE_SIDE;
        hipError_t e = hipEventCreateWithFlags(&L->ev_fork, JT_STREAM_EVENT_FLAGS);
        for (int i = 0; i < ns && e == hipSuccess; i++) {
            e = hipStreamCreateWithFlags(&L->side[i], hipStreamNonBlocking);
            if (e != hipSuccess) break;
            e = hipEventCreateWithFlags(&L->ev_join[i], JT_STREAM_EVENT_FLAGS);
            if (e != hipSuccess) {
                (void)hipStreamDestroy(L->side[i]);
                break;
            }
            L->nside = i + 1;
        }
        if (e != hipSuccess && L->nside == 0) (void)hipEventDestroy(L->ev_fork);
        rc = jt_rt_err(e);
    }
    return rc;
}

int jt_hip_moe_prepare(const jt_hip_moe_desc *desc, const float *dWgate, const float *dWg,
                       const float *dWu, const float *dWd, const float *dWg_s,
                       const float *dWu_s, const float *dWd_s, jt_hip_moe **out) {
    if (!desc || !dWg || !dWu || !dWd || !out) FAIL(JT_ERR_INVAL, EINVAL);
    int rc = moe_check_desc(desc);
    if (rc != JT_OK) return rc;
    const jt_hip_moe_desc d = *desc;
    if (d.n_shared > 0 && (!dWg_s || !dWu_s || !dWd_s)) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    jt_hip_moe *L = NULL;
    if ((rc = moe_alloc(desc, dWgate != NULL, &L)) != JT_OK) return rc;
    const int n = d.n, h = d.h, E = d.n_experts;
    const int Ep = (E + 63) / 64 * 64;
    int8_t *wh_rm = NULL, *wl_rm = NULL;
    hipError_t e = hipSuccess;
    if (L->fast_router) {
        e = hipMalloc((void **)&wh_rm, (size_t)E * n);
        if (e == hipSuccess) e = hipMalloc((void **)&wl_rm, (size_t)E * n);
    }
    if (e == hipSuccess && dWgate)
        e = hipMemcpyAsync(L->Wgate, dWgate, (size_t)E * n * sizeof(float),
                           hipMemcpyDeviceToDevice, rt->stream);
    rc = jt_rt_err(e);
    if (rc == JT_OK) {
        jtk_check_finite(dWgate ? L->Wgate : NULL, dWgate ? (int64_t)E * n : 0, jt_rt_errw(rt, rt->stream),
                         rt->stream);
        if (L->fast_router) {
            jtk_router_codes(L->Wgate, E, n, wh_rm, wl_rm, NULL, L->winfo, jt_rt_errw(rt, rt->stream),
                             rt->stream);
            jtk_pack_i8(wh_rm, E, n, 0, Ep, n, L->rWh, rt->stream);
            jtk_pack_i8(wl_rm, E, n, 0, Ep, n, L->rWl, rt->stream);
        }
        /* routed gate/up: rows of Wg/Wu [E][h][n] are channels, K = n */
        jtk_pack_lowbit(dWg, dWu, (int64_t)h * n, n, 1, E, 2 * h, n, 2, L->gu_P, L->gu_S,
                        NULL, NULL, jt_rt_errw(rt, rt->stream), rt->stream);
        /* routed down: Wd [E][h][n] is B[K=h][N=n]; channel j = column j */
        jtk_pack_lowbit(dWd, NULL, (int64_t)h * n, 1, n, E, n, h, 4, L->dn_P, L->dn_S, NULL,
                        NULL, jt_rt_errw(rt, rt->stream), rt->stream);
        uint32_t f = 0;
        rc = jt_rt_flags(rt, rt->stream, &f);
        if (rc == JT_OK) rc = jt_rt_flags_to_rc(f);
    }
    (void)hipFree(wh_rm); /* jt_rt_flags synchronised the stream */
    (void)hipFree(wl_rm);
    const int hs = d.h_shared;
    for (int s = 0; s < d.n_shared && rc == JT_OK; s++) {
        const int64_t so = (int64_t)s * hs * n;
        rc = ffn_prepare_on(rt, dWg_s + so, dWu_s + so, dWd_s + so, n, hs, &L->sh[s]);
    }
    if (rc == JT_OK) rc = moe_finish(L);
    if (rc != JT_OK) {
        jt_hip_moe_free(L);
        return rc;
    }
    *out = L;
    return JT_OK;
}

static void prof_mark(jt_hip_moe *L, int slot, int i, hipStream_t s) {
    if (L->prof) (void)hipEventRecord(L->ev[slot][i], s);
}

/* Accumulate the stage times of the oldest recorded forward. Event i < ST_N
 * marks the start of stage i (ST_N = end of combine); shared expert e has
 * its own three marks at ST_N + 1 + 3e (gate/up, quant, down). */
static void prof_drain_one(jt_hip_moe *L) {
    const int S = L->d.n_shared;
    const int slot = (L->ring_head - L->ring_count + PROF_RING) % PROF_RING;
    hipEvent_t *ev = L->ev[slot];
    (void)hipEventSynchronize(ev[ST_N]);
    float ms = 0.0f;
#define ADD(st, a, b) \
    if (hipEventElapsedTime(&ms, (a), (b)) == hipSuccess) L->acc_ms[st] += ms
    for (int i = ST_QUANT_X; i < ST_R_DOWN; i++) ADD(i, ev[i], ev[i + 1]);
    ADD(ST_R_DOWN, ev[ST_R_DOWN], S > 0 ? ev[ST_N + 1] : ev[ST_COMBINE]);
    for (int e = 0; e < (L->ev_fused[slot] ? 1 : S); e++) { /* fused: one set of marks */
        hipEvent_t *x = &ev[ST_N + 1 + 3 * e];
        hipEvent_t end = (e + 1 < S && !L->ev_fused[slot]) ? ev[ST_N + 1 + 3 * (e + 1)]
                                                          : ev[ST_COMBINE];
        ADD(ST_S_GATEUP, x[0], x[1]);
        ADD(ST_S_QUANT, x[1], x[2]);
        ADD(ST_S_DOWN, x[2], end);
    }
    ADD(ST_COMBINE, ev[ST_COMBINE], ev[ST_N]);
#undef ADD
    L->acc_count++;
    L->ring_count--;
}

static int prof_begin(jt_hip_moe *L, int *slot) {
    if (!L->prof) return JT_OK;
    if (!L->ev_ready) {
        for (int r = 0; r < PROF_RING; r++)
            for (int i = 0; i < ST_N + 1 + 3 * JT_MOE_MAX_SHARED; i++)
                if (hipEventCreate(&L->ev[r][i]) != hipSuccess) return JT_ERR_IO;
        L->ev_ready = 1;
    }
    if (L->ring_count == PROF_RING) prof_drain_one(L);
    *slot = L->ring_head;
    L->ring_head = (L->ring_head + 1) % PROF_RING;
    L->ring_count++;
    return JT_OK;
}

/* The shared experts of a forward of T > 64 tokens with the fused gate/up:
 * one SwiGLU GEMM over all S experts (hidden rows into S planes of T x h),
 * one row quantiser over the S*T hidden rows, then each expert's down
 * projection into its Ys slot. ev (profiling, may be NULL): the gate/up
 * kernel's own start/end, then the end of the quantiser. */
static int shared_fused(jt_hip_moe *L, int T, uint32_t *err, hipStream_t s, hipEvent_t *ev) {
    const int S = L->d.n_shared, n = L->d.n;
    const jt_hip_ffn *F0 = L->sh[0];
    const int h = F0->h;
    int e = jtk_w8a8_swiglu_planes(L->Xq, F0->Kpn, L->sx, L->sgu_P, L->sgu_s, T, S * F0->Np_gu,
                                   F0->Kpn, L->sS, h, h, (int64_t)T * h, err, s,
                                   ev ? ev[0] : NULL, ev ? ev[1] : NULL);
    e |= jtk_quant_rows(L->sS, (int64_t)S * T, h, L->sSq, F0->Kph, L->sss, NULL, err, s);
    if (ev) (void)hipEventRecord(ev[2], s);
    /* every expert's down projection in one launch */
    e |= jtk_w8a8_gemm_batch(L->sSq, F0->Kph, (int64_t)T * F0->Kph, L->sss, T, L->sd_P,
                             (int64_t)F0->Np_d * F0->Kph, L->sd_s, F0->Np_d, T, n, F0->Np_d,
                             F0->Kph, L->Ys, n, (int64_t)T * n, S, err, s, NULL, NULL);
    return e ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

/* The shared experts of a forward of T <= 16 tokens, batched: one skinny
 * SwiGLU GEMM over the concatenated gate/up panels (hidden rows into S
 * planes of T x h), then one launch of the S down projections, each block
 * quantising its expert's hidden rows itself. ev as in shared_fused. */
static int shared_fused16(jt_hip_moe *L, int T, uint32_t *err, hipStream_t s, hipEvent_t *ev) {
    const int S = L->d.n_shared, n = L->d.n;
    const jt_hip_ffn *F0 = L->sh[0];
    const int h = F0->h;
    if (ev) (void)hipEventRecord(ev[0], s);
    int e = jtk_w8a8_skinny_swiglu_planes(L->Xq, F0->Kpn, L->sx, L->sgu_P, L->sgu_s, T,
                                          S * F0->Np_gu, F0->Kpn, L->sS, h, h, (int64_t)T * h,
                                          err, s);
    if (ev) {
        (void)hipEventRecord(ev[1], s);
        (void)hipEventRecord(ev[2], s);
    }
    e |= jtk_w8a8_gemm_xq_batch(L->sS, h, h, (int64_t)T * h, L->sd_P, (int64_t)F0->Np_d * F0->Kph,
                                L->sd_s, F0->Np_d, T, n, F0->Np_d, F0->Kph, L->Ys, n,
                                (int64_t)T * n, S, err, s);
    return e ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}


/* Forks the shared experts onto the side streams after what s holds so
 * far (they read Xq and sx) and records their join events. */
static int fork_shared(jt_hip_moe *L, int T, int fused, uint32_t *err, hipStream_t s) {
    const int S = L->d.n_shared, n = L->d.n;
    int le = (int)hipEventRecord(L->ev_fork, s);
    for (int i = 0; i < L->nside; i++) le |= (int)hipStreamWaitEvent(L->side[i], L->ev_fork, 0);
    if (fused) /* launch errors are collected; the join still happens */
        le |= shared_fused(L, T, err, L->side[0], NULL);
    else
        for (int e = 0; e < S; e++) {
            const ffn_ws ws = ffn_own_ws(L->sh[e]);
            le |= ffn_run_q(L->sh[e], &ws, L->Xq, L->sx, T, L->Ys + (size_t)e * T * n, err,
                            L->side[e % L->nside], NULL);
        }
    for (int i = 0; i < L->nside; i++) le |= (int)hipEventRecord(L->ev_join[i], L->side[i]);
    return le;
}

static int moe_forward(jt_hip_moe *L, const float *dX, const int32_t *d_ids,
                       const float *d_w, const float *dR, float *dY, int T, void *stream) {
    const jt_hip_moe_desc *d = &L->d;
    if (!dX || !dY || T < 0 || T > d->max_tokens) FAIL(JT_ERR_INVAL, EINVAL);
    if (!d_ids && !L->Wgate) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (T == 0) return JT_OK;
    hipStream_t s = (hipStream_t)stream; /* NULL: the HIP null stream */
    const int n = d->n, h = d->h, E = d->n_experts, k = d->topk, S = d->n_shared;
    const int Tk = T * k;
    uint32_t *err = jt_rt_errw(rt, s);
    int slot = 0, rc = prof_begin(L, &slot);
    if (rc != JT_OK) return rc;
    int le = 0;
    L->last_T = T;

    /* up to 16 tokens: every logit exact in one launch (with the codes Xq),
     * then top-k; larger batches: int8 bounds and exact candidates */
    const int small = !d_ids && L->Wgate && T <= 16 && n % 256 == 0 &&
                      (size_t)(T + 4) * (n + 4) * 4 <= 160 * 1024;
    const int fast = !d_ids && !small && L->fast_router;
    /* the router's codes, bounds and candidates as one launch (16 tokens a
     * block against every expert), where the exact stage reads candidate
     * lists (above 256 tokens; up to 256 the verify launch selects from the
     * bounds in memory itself) */
    const int front = fast && T > 256 && E % 16 == 0 && k <= 64 &&
                      (n == 256 || n == 512 || n == 1024) && ((uintptr_t)dX & 15) == 0;
    /* caller-routed decode without a fork: the token codes ride in the sort
     * launch (k_quant_sort_small) */
    const int qsort = d_ids && !L->prof && T * k <= 1024 && E <= 4096 &&
                      !(S > 0 && T > 16);
    /* ... and with 16-row tiles of f = 256 and at most 256 pairs, inside the
     * routed gate/up launch (one launch fewer) */
    const int qsort_gu = qsort && Tk <= 256 && E <= 1024 && Tk <= 16 * E && h == 256 &&
                         n % 256 == 0 && n <= 1024 && ((uintptr_t)dX & 15) == 0;
    prof_mark(L, slot, ST_QUANT_X, s);
    if (qsort) {
        /* quantised with the sort below */
    } else if (small) /* the codes Xq and all T x E logits (timed as quant_x) */
        le |= jtk_router_logits_small(dX, L->Wgate, T, E, n, L->logits, L->Xq, L->sx, err, s);
    else if (front) /* codes, approximate logits and candidates in one launch */
        le |= jtk_router_front(dX, T, n, L->Xq, L->sx, L->xinfo, L->rWh, L->rWl, L->winfo, E, k,
                               L->rcand, L->rnc, L->logits, err, s);
    else if (fast) /* the expert codes Xq plus the router's residual codes */
        le |= jtk_router_codes(dX, T, n, L->Xq, L->Xl, L->sx, L->xinfo, err, s);
    else
        le |= jtk_quant_rows(dX, T, n, L->Xq, n, L->sx, NULL, err, s);
    /* Without profiling the shared experts overlap the routed path on side
     * streams; with profiling every stage runs in order on s so that each
     * stage's events bracket its kernels alone. Up to 16 tokens the
     * experts are two short launches each and the fork/join events cost
     * more than the overlap gains (measured: 80 -> 70 us per decode layer
     * in stream order), so they run in order there too. */
    const int fork = S > 0 && !L->prof && T > 16;
    const int fused = L->sh_cat && T > 64, fused16 = L->sh_cat && T <= 16;
    if (L->prof) L->ev_fused[slot] = fused || fused16;
    /* with the bound-and-verify router the fork comes after its candidate
     * selection: the exact stage is then queued before the shared gate/up,
     * which otherwise holds every CU's registers and leaves the exact
     * stage (21 us alone) waiting for most of its 100 us (measured at 4096
     * tokens: 0.319-0.325 ms per layer against 0.331-0.332 forking after
     * the codes, 0.332-0.334 forking after the approximate logits) */
    const int fork_late = fork && fast;
    if (fork && !fork_late) le |= fork_shared(L, T, fused, err, s);
    /* 16-row tiles when experts average at most 16 rows; the single-launch
     * sort up to 1024 pairs */
    const int R = Tk <= 16 * E ? 16 : 64;
    /* tiles: at most Tk / R plus one per expert that holds a pair */
    const int max_tiles = Tk / R + (E < Tk ? E : Tk);
    /* Decode with the shared experts concatenated: top-k, the pair sort and
     * the shared gate/up blocks share one launch, the routed FFN and the
     * shared down blocks another (three launches fewer; with profiling each
     * stage keeps its own). T <= 16 and k <= 64 keep Tk <= 1024. */
    const jt_hip_ffn *F0 = S > 0 ? L->sh[0] : NULL;
    const int merge16 = !L->prof && small && fused16 && R == 16 && h == 256 &&
                        n % 256 == 0 && n <= 1024 && E <= 1024 && k <= 64 && F0->h % 16 == 0 &&
                        F0->Kph <= 3072 && F0->Np_d >= n;
    prof_mark(L, slot, ST_ROUTER, s);
    const int32_t *ids = L->ids;
    const float *w = L->w;
    if (d_ids) {
        ids = d_ids; /* caller-routed: read in place */
        w = d_w;
        prof_mark(L, slot, ST_TOPK, s);
    } else if (small) {
        prof_mark(L, slot, ST_TOPK, s);
        if (merge16) /* top-k, the pair sort and the shared gate/ups */
            le |= jtk_decode_route_shared_gu(
                L->logits, T, E, k, L->ids, L->w, R, L->off, L->perm, L->tiles, L->ntiles,
                L->route_done, L->Xq, F0->Kpn, L->sx, L->sgu_P, L->sgu_s, S * F0->Np_gu,
                F0->Kpn, L->sS, F0->h, F0->h, (int64_t)T * F0->h, err, s);
        else
            le |= jtk_topk(L->logits, T, E, k, L->ids, NULL, L->w, err, s);
    } else if (fast) {
        if (!front)
            le |= jtk_router_approx(L->Xq, L->Xl, n, L->xinfo, L->rWh, L->rWl, L->winfo, T, E,
                                    L->approx, s);
        prof_mark(L, slot, ST_TOPK, s);
        /* stage 1 (the candidates) ran in the front launch */
        const int st1 = front ? 0 : 1;
        if (st1 || !fork_late)
            le |= jtk_topk_verify(L->approx, L->xinfo, L->winfo, dX, L->Wgate, T, E, n, k,
                                  L->rcand, L->rnc, L->ids, L->w, L->logits, err,
                                  fork_late ? st1 : st1 | 2, s);
        if (fork_late) {
            le |= fork_shared(L, T, fused, err, s);
            le |= jtk_topk_verify(L->approx, L->xinfo, L->winfo, dX, L->Wgate, T, E, n, k,
                                  L->rcand, L->rnc, L->ids, L->w, L->logits, err, 2, s);
        }
    } else {
        le |= jtk_router_logits(dX, L->Wgate, T, E, n, L->logits, err, s);
        prof_mark(L, slot, ST_TOPK, s);
        le |= jtk_topk(L->logits, T, E, k, L->ids, NULL, L->w, err, s);
    }
    L->cur_ids = ids;
    L->cur_w = w;
    prof_mark(L, slot, ST_SORT, s);
    if (merge16) {
        /* sorted in the top-k launch */
    } else if (qsort_gu) {
        /* sorted in the routed gate/up launch below */
    } else if (qsort) {
        le |= jtk_quant_sort_small(dX, T, n, L->Xq, L->sx, ids, Tk, E, (int64_t)Tk, R, L->off,
                                   NULL, L->perm, NULL, NULL, L->tiles, L->ntiles, err, s);
    } else if (Tk <= 1024 && E <= 4096) {
        le |= jtk_sort_small(ids, Tk, E, (int64_t)Tk, R, L->off, NULL, L->perm, NULL, NULL,
                             L->tiles, L->ntiles, err, s);
        prof_mark(L, slot, ST_TILES, s);
    } else {
        /* sort and tile list in two launches when E <= 1024 and Tk <= 65536 */
        const int rs = jtk_sort_mid(ids, Tk, E, (int64_t)Tk, R, L->rank, L->cnt, L->off, NULL,
                                    L->perm, NULL, NULL, L->tiles, L->ntiles, err, s);
        if (rs != (int)hipErrorInvalidValue) {
            le |= rs;
            prof_mark(L, slot, ST_TILES, s);
        } else {
            le |= jtk_sort(ids, Tk, E, (int64_t)Tk, L->rank, L->cnt, L->tot, L->off, NULL,
                           L->perm, NULL, NULL, err, s);
            prof_mark(L, slot, ST_TILES, s);
            le |= jtk_make_tiles(L->off, E, R, L->tiles, L->ntiles, s);
        }
    }
    prof_mark(L, slot, ST_R_GATEUP, s);
    if (R == 16 && h == 256 && n % 256 == 0 && n <= 1024) {
        /* 16-row tiles: gate/up, SwiGLU, row codes and down in one launch
         * (the three stages are timed as one, under routed_gateup) */
        if (qsort_gu)
            le |= jtk_routed_ffn16_sort(dX, T, L->Xq, L->sx, ids, Tk, E, L->off, L->perm,
                                        L->tiles, L->ntiles, k, L->gu_P, L->gu_S, L->gu_pstride,
                                        L->gu_sstride, L->dn_P, L->dn_S, L->dn_pstride,
                                        L->dn_sstride, n, h, L->Ye, L->Sqr, L->ssr, L->Sr, err,
                                        s);
        else if (merge16)
            le |= jtk_decode_ffn16_shared_down(
                L->Xq, L->sx, L->perm, L->tiles, L->ntiles, max_tiles, k, L->gu_P, L->gu_S,
                L->gu_pstride, L->gu_sstride, L->dn_P, L->dn_S, L->dn_pstride, L->dn_sstride, n,
                h, L->Ye, L->Sqr, L->ssr, L->sS, F0->h, F0->h, (int64_t)T * F0->h, T, L->sd_P,
                (int64_t)F0->Np_d * F0->Kph, L->sd_s, F0->Np_d, F0->Np_d, F0->Kph, L->Ys, n,
                (int64_t)T * n, S, err, s);
        else
            le |= jtk_routed_ffn16(L->Xq, L->sx, L->perm, L->tiles, L->ntiles, max_tiles, k,
                                   L->gu_P, L->gu_S, L->gu_pstride, L->gu_sstride, L->dn_P,
                                   L->dn_S, L->dn_pstride, L->dn_sstride, n, h, L->Ye, L->Sqr,
                                   L->ssr, L->Sr, err, s);
        prof_mark(L, slot, ST_R_QUANT, s);
        prof_mark(L, slot, ST_R_DOWN, s);
    } else {
        /* 64-row tiles with f = 256 or 512: the gate/up launch also writes
         * the hidden rows' int8 codes (timed as routed_gateup) */
        const int gq = R == 64 ? jtk_lowbit_gateup_q(L->Xq, n, L->sx, L->perm, k, L->tiles,
                                                     L->ntiles, max_tiles, L->gu_P, L->gu_S,
                                                     L->gu_pstride, L->gu_sstride, n, L->Sqr,
                                                     L->ssr, h, err, s)
                               : (int)hipErrorInvalidValue;
        if (gq == (int)hipErrorInvalidValue) {
            le |= jtk_lowbit_grouped(2, L->Xq, n, L->sx, L->perm, L->off, k, L->tiles,
                                     L->ntiles, max_tiles, R, L->gu_P, L->gu_S, L->gu_pstride,
                                     L->gu_sstride, 2 * h, n, L->Sr, h, err, s);
            prof_mark(L, slot, ST_R_QUANT, s);
            le |= jtk_quant_rows(L->Sr, Tk, h, L->Sqr, h, L->ssr, NULL, err, s);
        } else {
            le |= gq;
            prof_mark(L, slot, ST_R_QUANT, s);
        }
        prof_mark(L, slot, ST_R_DOWN, s);
        le |= jtk_lowbit_grouped(4, L->Sqr, h, L->ssr, L->perm, L->off, k, L->tiles, L->ntiles,
                                 max_tiles, R, L->dn_P, L->dn_S, L->dn_pstride, L->dn_sstride, n,
                                 h, L->Ye, n, err, s);
    }
    if (fork) {
        for (int i = 0; i < L->nside; i++) le |= (int)hipStreamWaitEvent(s, L->ev_join[i], 0);
    } else if (merge16) {
        /* the shared experts ran in the top-k and routed FFN launches */
    } else if (fused || fused16) {
        hipEvent_t *ev = L->prof ? &L->ev[slot][ST_N + 1] : NULL;
        rc = fused ? shared_fused(L, T, err, s, ev) : shared_fused16(L, T, err, s, ev);
        if (rc != JT_OK) return rc;
    } else {
        for (int e = 0; e < S; e++) {
            hipEvent_t *ev = L->prof ? &L->ev[slot][ST_N + 1 + 3 * e] : NULL;
            const ffn_ws ws = ffn_own_ws(L->sh[e]);
            rc = ffn_run_q(L->sh[e], &ws, L->Xq, L->sx, T, L->Ys + (size_t)e * T * n, err, s, ev);
            if (rc != JT_OK) return rc;
        }
    }
    prof_mark(L, slot, ST_COMBINE, s);
    le |= jtk_combine(w, L->Ye, NULL, L->Ys, S, T, k, n, dR, dY, err, s);
    prof_mark(L, slot, ST_N, s);
    return le ? jt_rt_err(hipErrorLaunchFailure) : JT_OK;
}

int jt_hip_moe_fwd(jt_hip_moe *L, const float *dX, float *dY, int T, void *stream) {
    if (!L) FAIL(JT_ERR_INVAL, EINVAL);
    return moe_forward(L, dX, NULL, NULL, NULL, dY, T, stream);
}

int jt_hip_moe_fwd_routed(jt_hip_moe *L, const float *dX, const int32_t *d_ids,
                          const float *d_weights, float *dY, int T, void *stream) {
    if (!L || !d_ids || !d_weights) FAIL(JT_ERR_INVAL, EINVAL);
    return moe_forward(L, dX, d_ids, d_weights, NULL, dY, T, stream);
}

int jt_hip_moe_fwd_residual(jt_hip_moe *L, const float *dX, const int32_t *d_ids,
                            const float *d_weights, float *dY, int T, void *stream) {
    if (!L || (!d_ids) != (!d_weights)) FAIL(JT_ERR_INVAL, EINVAL);
    /* the residual is the layer input; dY may be dX (every kernel that reads
     * dX runs before the combine, which reads each element before writing it) */
    return moe_forward(L, dX, d_ids, d_weights, dX, dY, T, stream);
}

int jt_hip_moe_buffer(const jt_hip_moe *L, int which, void **dptr, size_t *bytes) {
    if (!L || !dptr || !bytes) FAIL(JT_ERR_INVAL, EINVAL);
    const size_t T = (size_t)L->last_T, k = (size_t)L->d.topk, n = (size_t)L->d.n;
    const size_t E = (size_t)L->d.n_experts, S = (size_t)L->d.n_shared;
    switch (which) {
    case JT_HIP_BUF_IDS: *dptr = (void *)(L->cur_ids ? L->cur_ids : L->ids); *bytes = T * k * 4; break;
    case JT_HIP_BUF_WEIGHTS: *dptr = (void *)(L->cur_w ? L->cur_w : L->w); *bytes = T * k * 4; break;
    case JT_HIP_BUF_PERM: *dptr = L->perm; *bytes = T * k * 4; break;
    case JT_HIP_BUF_OFF: *dptr = L->off; *bytes = (E + 1) * 4; break;
    case JT_HIP_BUF_XQ: *dptr = L->Xq; *bytes = T * n; break;
    case JT_HIP_BUF_XSCALE: *dptr = L->sx; *bytes = T * 4; break;
    case JT_HIP_BUF_YE: *dptr = L->Ye; *bytes = T * k * n * 4; break;
    case JT_HIP_BUF_YS: *dptr = L->Ys; *bytes = S * T * n * 4; break;
    case JT_HIP_BUF_LOGITS: *dptr = L->logits; *bytes = T * E * 4; break;
    case JT_HIP_BUF_HQ: *dptr = L->Sqr; *bytes = T * k * (size_t)L->d.h; break;
    case JT_HIP_BUF_HSCALE: *dptr = L->ssr; *bytes = T * k * 4; break;
    default: FAIL(JT_ERR_INVAL, EINVAL);
    }
    return JT_OK;
}

/* Decode one expert's panels back into plain code / scale arrays. */
static void decode_panels(const uint8_t *P, const uint16_t *Sc, int N, int K, int bits,
                          int inter, uint8_t *codes, uint16_t *scales) {
    const int G = K / 64, PB = bits == 2 ? 256 : 512;
    for (int nn = 0; nn < N; nn++) {
        int row = nn, src = 0;
        if (inter) {
            src = (nn >> 4) & 1;
            row = (nn >> 5) * 16 + (nn & 15);
        }
        const int64_t prow = (int64_t)src * (inter ? N / 2 : N) + row;
        const int p = nn / 16, c = nn % 16;
        for (int g = 0; g < G; g++) {
            scales[prow * G + g] = Sc[((int64_t)p * G + g) * 16 + c];
            for (int kk = 0; kk < 64; kk++) {
                const int kc = kk >> 4, kap = kk & 15, o = kap >> 2, j = kap & 3;
                const int plane = kc * 16 + c;
                uint32_t dw;
                int sh;
                if (bits == 2) {
                    memcpy(&dw, P + ((int64_t)p * G + g) * PB + plane * 4, 4);
                    sh = 8 * j + 2 * o;
                    codes[prow * K + g * 64 + kk] = (uint8_t)((dw >> sh) & 3u);
                } else {
                    memcpy(&dw, P + ((int64_t)p * G + g) * PB + plane * 8 + (o >> 1) * 4, 4);
                    sh = 8 * j + 4 * (o & 1);
                    codes[prow * K + g * 64 + kk] = (uint8_t)((dw >> sh) & 15u);
                }
            }
        }
    }
}

int jt_hip_moe_export_routed(const jt_hip_moe *L, int e, uint8_t *gu_codes,
                             uint16_t *gu_scales, uint8_t *d_codes, uint16_t *d_scales) {
    if (!L || e < 0 || e >= L->d.n_experts || !gu_codes || !gu_scales || !d_codes ||
        !d_scales)
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    const int n = L->d.n, h = L->d.h;
    uint8_t *hp = malloc((size_t)(L->gu_pstride > L->dn_pstride ? L->gu_pstride : L->dn_pstride));
    uint16_t *hs = malloc((size_t)(L->gu_sstride > L->dn_sstride ? L->gu_sstride : L->dn_sstride) * 2);
    if (!hp || !hs) {
        free(hp);
        free(hs);
        FAIL(JT_ERR_NOMEM, ENOMEM);
    }
    int rc = jt_rt_d2h(rt, hp, L->gu_P + (int64_t)e * L->gu_pstride, (size_t)L->gu_pstride);
    if (rc == JT_OK)
        rc = jt_rt_d2h(rt, hs, L->gu_S + (int64_t)e * L->gu_sstride, (size_t)L->gu_sstride * 2);
    if (rc == JT_OK) decode_panels(hp, hs, 2 * h, n, 2, 1, gu_codes, gu_scales);
    if (rc == JT_OK)
        rc = jt_rt_d2h(rt, hp, L->dn_P + (int64_t)e * L->dn_pstride, (size_t)L->dn_pstride);
    if (rc == JT_OK)
        rc = jt_rt_d2h(rt, hs, L->dn_S + (int64_t)e * L->dn_sstride, (size_t)L->dn_sstride * 2);
    if (rc == JT_OK) decode_panels(hp, hs, n, h, 4, 0, d_codes, d_scales);
    free(hp);
    free(hs);
    return rc;
}

/* ======================= serialised layer ======================= */
/*
 * Format "JTMOEQ" version 1: a 4 KiB header, then the layer's device arrays
 * byte for byte, each section starting on a 4 KiB boundary, in this order:
 *   gate fp32 [E][n] and, for the int8-bounded router, its hi/lo code
 *   panels and row info (only with a router gate);
 *   routed gate/up INT2 panels [E][2h/16][n/64][256 B], their fp16 scales,
 *   down INT4 panels [E][n/16][h/64][512 B], their fp16 scales;
 *   per shared expert: gate/up int8 panels (gate and up interleaved in
 *   blocks of 16 channels), their fp32 scales, down panels, their scales.
 * Every array is in the order the kernels read it, so a load is a copy.
 * Header (little-endian): magic "JTMOEQ1\0", u32 version, u32 header bytes,
 * i32 n, h, E, k, S, h_shared, group, u32 flags (bit 0: router gate),
 * u32 section count, u64 payload bytes, u64 payload checksum, then one
 * {u64 offset, u64 bytes} per section (offsets from the file start).
 */
#define MQ_HDR 4096u
#define MQ_ALIGN 4096u
#define MQ_MAXSEC (4 + 4 + 4 * JT_MOE_MAX_SHARED)
static const char k_mq_magic[8] = {'J', 'T', 'M', 'O', 'E', 'Q', '1', '\0'};

typedef struct mq_sec {
    void *dev;
    size_t bytes;
} mq_sec;

/* The sections of a layer (device pointers and sizes), in file order. */
static int mq_sections(const jt_hip_moe *L, mq_sec *sec) {
    const jt_hip_moe_desc *d = &L->d;
    const size_t E = (size_t)d->n_experts, n = (size_t)d->n;
    int ns = 0;
    if (L->Wgate) {
        sec[ns++] = (mq_sec){L->Wgate, E * n * 4};
        if (L->fast_router) {
            const size_t Ep = (E + 63) / 64 * 64;
            sec[ns++] = (mq_sec){L->rWh, Ep * n};
            sec[ns++] = (mq_sec){L->rWl, Ep * n};
            sec[ns++] = (mq_sec){L->winfo, E * 16};
        }
    }
    sec[ns++] = (mq_sec){L->gu_P, (size_t)L->gu_pstride * E};
    sec[ns++] = (mq_sec){L->gu_S, (size_t)L->gu_sstride * E * 2};
    sec[ns++] = (mq_sec){L->dn_P, (size_t)L->dn_pstride * E};
    sec[ns++] = (mq_sec){L->dn_S, (size_t)L->dn_sstride * E * 2};
    for (int s = 0; s < d->n_shared; s++) {
        const jt_hip_ffn *F = L->sh[s];
        sec[ns++] = (mq_sec){F->gu_P, (size_t)F->Np_gu * F->Kpn};
        sec[ns++] = (mq_sec){F->gu_s, (size_t)F->Np_gu * 4};
        sec[ns++] = (mq_sec){F->d_P, (size_t)F->Np_d * F->Kph};
        sec[ns++] = (mq_sec){F->d_s, (size_t)F->Np_d * 4};
    }
    return ns;
}

/* 64-bit FNV-1a over 8-byte words (the payload is a multiple of 4 KiB). */
static uint64_t mq_checksum(const uint8_t *p, size_t bytes) {
    uint64_t hsh = 0xcbf29ce484222325ull;
    for (size_t i = 0; i + 8 <= bytes; i += 8) {
        uint64_t w;
        memcpy(&w, p + i, 8);
        hsh = (hsh ^ w) * 0x100000001b3ull;
    }
    return hsh;
}

static void put32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
static void put64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); }
static uint32_t get32(const uint8_t *p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static uint64_t get64(const uint8_t *p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}

static size_t mq_layout(const mq_sec *sec, int ns, size_t *off) {
    size_t at = MQ_HDR;
    for (int i = 0; i < ns; i++) {
        off[i] = at;
        at += jt_round_up(sec[i].bytes, MQ_ALIGN);
    }
    return at;
}

int jt_hip_moe_save(const jt_hip_moe *L, void *buf, size_t cap, size_t *bytes) {
    if (!L || !bytes) FAIL(JT_ERR_INVAL, EINVAL);
    mq_sec sec[MQ_MAXSEC];
    size_t off[MQ_MAXSEC];
    const int ns = mq_sections(L, sec);
    const size_t total = mq_layout(sec, ns, off);
    *bytes = total;
    if (!buf) return JT_OK;
    if (cap < total) FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    uint8_t *b = buf;
    memset(b, 0, total);
    for (int i = 0; i < ns; i++) {
        const int rc = jt_rt_d2h(rt, b + off[i], sec[i].dev, sec[i].bytes);
        if (rc != JT_OK) return rc;
    }
    const jt_hip_moe_desc *d = &L->d;
    memcpy(b, k_mq_magic, 8);
    put32(b + 8, 1);
    put32(b + 12, MQ_HDR);
    const int32_t f[7] = {d->n, d->h, d->n_experts, d->topk, d->n_shared, d->h_shared, d->group};
    memcpy(b + 16, f, sizeof(f));
    put32(b + 44, L->Wgate ? 1u : 0u);
    put32(b + 48, (uint32_t)ns);
    put64(b + 52, (uint64_t)(total - MQ_HDR));
    put64(b + 60, mq_checksum(b + MQ_HDR, total - MQ_HDR));
    for (int i = 0; i < ns; i++) {
        put64(b + 68 + 16 * i, (uint64_t)off[i]);
        put64(b + 76 + 16 * i, (uint64_t)sec[i].bytes);
    }
    return JT_OK;
}

int jt_hip_moe_load(const void *buf, size_t bytes, int max_tokens, jt_hip_moe **out) {
    if (!buf || !out || bytes < MQ_HDR) FAIL(JT_ERR_INVAL, EINVAL);
    const uint8_t *b = buf;
    if (memcmp(b, k_mq_magic, 8) != 0 || get32(b + 8) != 1 || get32(b + 12) != MQ_HDR)
        FAIL(JT_ERR_INVAL, EINVAL);
    int32_t f[7];
    memcpy(f, b + 16, sizeof(f));
    const uint32_t flags = get32(b + 44);
    if (flags > 1u) FAIL(JT_ERR_INVAL, EINVAL);
    const jt_hip_moe_desc d = {f[0], f[1], f[2], f[3], f[4], f[5], f[6], max_tokens};
    int rc = moe_check_desc(&d);
    if (rc != JT_OK) return rc;
    const uint64_t payload = get64(b + 52);
    if (payload != bytes - MQ_HDR || mq_checksum(b + MQ_HDR, bytes - MQ_HDR) != get64(b + 60))
        FAIL(JT_ERR_INVAL, EINVAL);
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    jt_hip_moe *L = NULL;
    if ((rc = moe_alloc(&d, (int)(flags & 1u), &L)) != JT_OK) return rc;
    for (int s = 0; s < d.n_shared && rc == JT_OK; s++) rc = ffn_alloc(rt, d.n, d.h_shared, &L->sh[s]);
    mq_sec sec[MQ_MAXSEC];
    size_t off[MQ_MAXSEC];
    int ns = 0;
    if (rc == JT_OK) {
        ns = mq_sections(L, sec);
        /* the section table must be exactly this layer's layout */
        if (get32(b + 48) != (uint32_t)ns || mq_layout(sec, ns, off) != bytes) rc = JT_ERR_INVAL;
        for (int i = 0; i < ns && rc == JT_OK; i++)
            if (get64(b + 68 + 16 * i) != off[i] || get64(b + 76 + 16 * i) != sec[i].bytes)
                rc = JT_ERR_INVAL;
        if (rc != JT_OK) errno = EINVAL;
    }
    for (int i = 0; i < ns && rc == JT_OK; i++)
        rc = jt_rt_h2d(rt, sec[i].dev, b + off[i], sec[i].bytes);
    if (rc == JT_OK) rc = moe_finish(L);
    if (rc != JT_OK) {
        jt_hip_moe_free(L);
        return rc;
    }
    *out = L;
    return JT_OK;
}

int jt_hip_moe_set_profiling(jt_hip_moe *L, int on) {
    if (!L) FAIL(JT_ERR_INVAL, EINVAL);
    while (L->ring_count > 0) prof_drain_one(L);
    L->prof = on ? 1 : 0;
    return JT_OK;
}

int jt_hip_moe_stage_times(jt_hip_moe *L, const char **names, double *ms, int cap, int *n,
                           int *count) {
    if (!L || !ms || !n || !count) FAIL(JT_ERR_INVAL, EINVAL);
    while (L->ring_count > 0) prof_drain_one(L);
    int m = cap < ST_N ? cap : ST_N;
    for (int i = 0; i < m; i++) {
        if (names) names[i] = k_stage_names[i];
        ms[i] = L->acc_ms[i];
        L->acc_ms[i] = 0.0;
    }
    *n = m;
    *count = L->acc_count;
    L->acc_count = 0;
    return JT_OK;
}
