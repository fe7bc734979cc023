/*
 * jt_oracle.c -- CPU restatement of the reference's quantised MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see jt_oracle.h). Plain scalar C11, built with
 * -ffp-contract=off: each fp64 operation rounds on its own, like the
 * reference build. References are file:line of the reference checkout.
 */
#include "jt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RC_OK 0
#define RC_NOMEM 1
#define RC_INVAL 2

/* ===================== W8A8 ===================== */

/* Shared body of the per-tensor / per-row quantiser: max|x| in fp64, zero
 * input -> scale 1 and codes 0, otherwise scale_d = maxabs/127,
 * q = clamp(round(x/scale_d)) (src/w8a8.c:710-743, 815-850). */
static int quant_span(const float *x, size_t n, int8_t *q, float *scale) {
    double maxabs = 0.0;
    for (size_t i = 0; i < n; i++) {
        double a = fabs((double)x[i]);
        if (a > maxabs) maxabs = a;
    }
    if (maxabs == 0.0) {
        *scale = 1.0f;
        for (size_t i = 0; i < n; i++) q[i] = 0;
        return RC_OK;
    }
    double scale_d = maxabs / 127.0;
    if (!isfinite(scale_d) || scale_d <= 0.0) return RC_INVAL;
    float scale_f = (float)scale_d;
    if (!isfinite((double)scale_f) || scale_f <= 0.0f) return RC_INVAL;
    *scale = scale_f;
    for (size_t i = 0; i < n; i++) {
        double qd = round((double)x[i] / scale_d);
        if (qd > 127.0) qd = 127.0;
        else if (qd < -127.0) qd = -127.0;
        q[i] = (int8_t)(int)qd;
    }
    return RC_OK;
}

int or_quant_row(const float *x, size_t n, int8_t *q, float *scale) {
    if (!x || !q || !scale || n == 0) return RC_INVAL;
    for (size_t i = 0; i < n; i++)
        if (!isfinite((double)x[i])) return RC_INVAL;
    return quant_span(x, n, q, scale);
}

int or_quant_rows(const float *X, size_t rows, size_t cols, int8_t *Q,
                  float *scales) {
    if (!X || !Q || !scales || rows == 0 || cols == 0) return RC_INVAL;
    for (size_t i = 0; i < rows * cols; i++)
        if (!isfinite((double)X[i])) return RC_INVAL;
    for (size_t r = 0; r < rows; r++) {
        int rc = quant_span(X + r * cols, cols, Q + r * cols, scales + r);
        if (rc != RC_OK) return rc;
    }
    return RC_OK;
}

int or_dequant_rows(const int8_t *q, const float *scales, size_t rows,
                    size_t cols, float *dst) {
    if (!q || !scales || !dst || rows == 0 || cols == 0) return RC_INVAL;
    for (size_t r = 0; r < rows; r++) {
        double sc = (double)scales[r];
        if (!isfinite(sc) || sc <= 0.0) return RC_INVAL;
    }
    for (size_t i = 0; i < rows * cols; i++)
        if (q[i] < -127) return RC_INVAL;
    for (size_t r = 0; r < rows; r++) {
        double sc = (double)scales[r];
        for (size_t c = 0; c < cols; c++) {
            float f = (float)((double)(int)q[r * cols + c] * sc);
            if (!isfinite((double)f)) return RC_INVAL;
            dst[r * cols + c] = f;
        }
    }
    return RC_OK;
}

int or_fakequant_rows(const float *src, size_t rows, size_t cols,
                      float *dst) {
    if (!src || !dst || rows == 0 || cols == 0) return RC_INVAL;
    for (size_t i = 0; i < rows * cols; i++)
        if (!isfinite((double)src[i])) return RC_INVAL;
    for (size_t r = 0; r < rows; r++) {
        const float *s = src + r * cols;
        float *d = dst + r * cols;
        double maxabs = 0.0;
        for (size_t c = 0; c < cols; c++) {
            double a = fabs((double)s[c]);
            if (a > maxabs) maxabs = a;
        }
        if (maxabs == 0.0) {
            for (size_t c = 0; c < cols; c++) d[c] = 0.0f;
            continue;
        }
        double scale_d = maxabs / 127.0;
        for (size_t c = 0; c < cols; c++) {
            double qd = round((double)s[c] / scale_d);
            if (qd > 127.0) qd = 127.0;
            else if (qd < -127.0) qd = -127.0;
            float f = (float)(qd * scale_d);
            if (!isfinite((double)f)) return RC_INVAL;
            d[c] = f;
        }
    }
    return RC_OK;
}

int or_w8a8_gemm(const int8_t *Aq, const float *sA, int sA_rows,
                 const int8_t *Bq_kn, const float *sB, int sB_cols, float *C,
                 int32_t *acc_out, int M, int N, int K) {
    int rc = RC_OK;
    for (int m = 0; m < M; m++) {
        double sA_d = (double)sA[sA_rows ? m : 0];
        for (int n = 0; n < N; n++) {
            int32_t acc = 0;
            for (int k = 0; k < K; k++)
                acc += (int32_t)Aq[(size_t)m * K + k] *
                       (int32_t)Bq_kn[(size_t)k * N + n];
            double ss = sA_d * (double)sB[sB_cols ? n : 0];
            float f = (float)((double)acc * ss);
            if (!isfinite((double)f)) rc = RC_INVAL;
            C[(size_t)m * N + n] = f;
            if (acc_out) acc_out[(size_t)m * N + n] = acc;
        }
    }
    return rc;
}

/* ===================== fp32 GEMM ===================== */

void or_gemm_f32(const float *A, const float *B, float *C, int M, int N,
                 int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                float p = A[(size_t)m * K + k] * B[(size_t)k * N + n];
                acc = acc + p;
            }
            C[(size_t)m * N + n] = acc;
        }
}

/* ===================== low-bit levels ===================== */

int or_lowbit_code(double w, double maxabs, int bits) {
    int nl = 1 << bits;
    double t = (maxabs == 0.0) ? 0.0 : w / maxabs;
    double li = floor(t * (double)(nl - 1) / 2.0 + (double)(nl - 1) / 2.0 +
                      0.5);
    long l = (long)li;
    if (l < 0) l = 0;
    if (l > (long)(nl - 1)) l = nl - 1;
    return (int)l;
}

int or_lowbit_fakequant(const float *w, float *fq, size_t n, int bits) {
    if (!w || !fq || n == 0 || (bits != 2 && bits != 4)) return RC_INVAL;
    double maxa = 0.0;
    for (size_t i = 0; i < n; i++) {
        double v = (double)w[i];
        if (!isfinite(v)) return RC_INVAL;
        if (fabs(v) > maxa) maxa = fabs(v);
    }
    if (maxa == 0.0) {
        for (size_t i = 0; i < n; i++) fq[i] = 0.0f;
        return RC_OK;
    }
    double nn = (double)((1 << bits) - 1);
    for (size_t i = 0; i < n; i++) {
        int l = or_lowbit_code((double)w[i], maxa, bits);
        double level = (2.0 * (double)l - nn) / nn; /* src/lowbit.c:42-45 */
        fq[i] = (float)(level * maxa);
    }
    return RC_OK;
}

int or_lowbit_col_to_idx(const float *col, size_t k, int bits, uint8_t *idx,
                         float *w_scale) {
    if (!col || !idx || !w_scale || k == 0) return RC_INVAL;
    if ((bits != 2 && bits != 4) || (k % 4u) != 0u) return RC_INVAL;
    double maxa = 0.0;
    for (size_t i = 0; i < k; i++) {
        double v = (double)col[i];
        if (!isfinite(v)) return RC_INVAL;
        if (fabs(v) > maxa) maxa = fabs(v);
    }
    size_t ng = k / 4u;
    for (int b = 0; b < bits; b++)
        for (size_t g = 0; g < ng; g++) {
            unsigned p = 0u;
            for (unsigned j = 0; j < 4u; j++) {
                int l = or_lowbit_code((double)col[g * 4u + j], maxa, bits);
                if (((unsigned)l >> (unsigned)b) & 1u) p |= 1u << j;
            }
            idx[(size_t)b * ng + g] = (uint8_t)p;
        }
    *w_scale = (float)maxa;
    return RC_OK;
}

uint16_t or_f64_to_f16(double x) {
    uint16_t sign = signbit(x) ? 0x8000u : 0u;
    if (isnan(x)) return (uint16_t)(sign | 0x7e00u);
    double a = fabs(x);
    if (a == 0.0) return sign;
    if (isinf(a)) return (uint16_t)(sign | 0x7c00u);
    int e;
    (void)frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    int E = e - 1;      /* a = 1.x * 2^E */
    if (E < -14) {
        /* subnormal: an integer number of 2^-24 units, ties to even */
        double q = rint(ldexp(a, 24));
        return (uint16_t)(sign | (uint16_t)q); /* q == 1024 -> min normal */
    }
    double q = rint(ldexp(a, 10 - E)); /* in [1024, 2048] */
    if (q >= 2048.0) {
        q = 1024.0;
        E += 1;
    }
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((E + 15) << 10) |
                      (uint16_t)(q - 1024.0));
}

double or_f16_to_f64(uint16_t h) {
    int s = (h >> 15) & 1;
    int e = (h >> 10) & 0x1f;
    int m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m + 1024), e - 25);
    return s ? -v : v;
}

int or_lowbit_pack_rows(const float *W, int N, int K, int bits, int group,
                        uint8_t *codes, uint16_t *scales) {
    if (!W || !codes || !scales || N <= 0 || K <= 0 || group <= 0 ||
        K % group != 0 || (bits != 2 && bits != 4))
        return RC_INVAL;
    int G = K / group;
    double nn = (double)((1 << bits) - 1);
    for (int r = 0; r < N; r++)
        for (int g = 0; g < G; g++) {
            const float *w = W + (size_t)r * K + (size_t)g * group;
            double maxa = 0.0;
            for (int i = 0; i < group; i++) {
                double v = (double)w[i];
                if (!isfinite(v)) return RC_INVAL;
                if (fabs(v) > maxa) maxa = fabs(v);
            }
            uint16_t s16 = or_f64_to_f16(maxa / nn);
            if ((s16 & 0x7c00u) == 0x7c00u) return RC_INVAL;
            scales[(size_t)r * G + g] = s16;
            for (int i = 0; i < group; i++)
                codes[(size_t)r * K + (size_t)g * group + i] =
                    (uint8_t)or_lowbit_code((double)w[i], maxa, bits);
        }
    return RC_OK;
}

int or_gemm_lowbit_group(const int8_t *Aq, const float *sA,
                         const uint8_t *codes, const uint16_t *scales,
                         int bits, int group, float *C, int32_t *acc_out,
                         int M, int N, int K) {
    int rc = RC_OK;
    int G = K / group;
    int nn = (1 << bits) - 1;
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float T = 0.0f;
            for (int g = 0; g < G; g++) {
                int32_t acc = 0;
                for (int i = 0; i < group; i++) {
                    size_t k = (size_t)g * group + i;
                    acc += (int32_t)Aq[(size_t)m * K + k] *
                           (2 * (int32_t)codes[(size_t)n * K + k] - nn);
                }
                if (acc_out) acc_out[((size_t)m * N + n) * G + g] = acc;
                /* |acc| < 2^24, so (float)acc is exact; one rounding per group */
                T = fmaf((float)acc, (float)or_f16_to_f64(scales[(size_t)n * G + g]), T);
            }
            float f = T * sA[m];
            if (!isfinite((double)f)) rc = RC_INVAL;
            C[(size_t)m * N + n] = f;
        }
    return rc;
}

/* ===================== T-MAC ===================== */

int or_tmac_lut_ctor(const float *act, size_t n, size_t k, int8_t *qlut,
                     float *scales, float *biases) {
    if (!act || !qlut || !scales || !biases || n == 0 || k == 0)
        return RC_INVAL;
    if (k % 4u != 0 || k % 32u != 0) return RC_INVAL;
    size_t ngroups = k / 4u, nblocks = k / 32u;
    for (size_t r = 0; r < n; r++)
        for (size_t bb = 0; bb < nblocks; bb++) {
            const float *a = act + r * k + bb * 32u;
            int8_t *qb = qlut + r * ngroups * 8u + bb * 64u;
            double fmat[8][16];
            double maxabs = 0.0, asum = 0.0;
            for (size_t gi = 0; gi < 8u; gi++)
                for (size_t p = 0; p < 16u; p++) {
                    double s = 0.0;
                    for (size_t j = 0; j < 4u; j++) {
                        float av = a[gi * 4u + j];
                        if (!isfinite((double)av)) return RC_INVAL;
                        s += (((p >> j) & 1u) ? 1.0 : -1.0) * (double)av;
                    }
                    fmat[gi][p] = s;
                    double aa = s >= 0.0 ? s : -s;
                    if (aa > maxabs) maxabs = aa;
                }
            for (size_t i = 0; i < 32u; i++) asum += (double)a[i];
            if (!isfinite(maxabs) || !isfinite(asum)) return RC_INVAL;
            float bias_f = (float)asum;
            if (maxabs == 0.0) {
                if (!isfinite((double)bias_f)) return RC_INVAL;
                memset(qb, 0, 64);
                scales[r * nblocks + bb] = 1.0f;
                biases[r * nblocks + bb] = bias_f;
                continue;
            }
            double scale_d = maxabs / 127.0;
            float scale_f = (float)scale_d;
            if (!isfinite(scale_d) || scale_d <= 0.0 ||
                !isfinite((double)scale_f) || !isfinite((double)bias_f))
                return RC_INVAL;
            for (size_t gi = 0; gi < 8u; gi++)
                for (size_t ii = 0; ii < 8u; ii++) {
                    double qd = round(fmat[gi][8u + ii] / scale_d);
                    if (qd > 127.0) qd = 127.0;
                    else if (qd < -128.0) qd = -128.0;
                    qb[gi * 8u + ii] = (int8_t)(int)qd;
                }
            scales[r * nblocks + bb] = scale_f;
            biases[r * nblocks + bb] = bias_f;
        }
    return RC_OK;
}

/* Mirror lookup of one bit-plane over 8 groups, src/tmac.c:80-93. */
static int32_t plane_acc(const int8_t *qblk, const uint8_t *plane) {
    int32_t acc = 0;
    for (size_t gi = 0; gi < 8u; gi++) {
        unsigned p = plane[gi] & 0x0Fu;
        acc += (p >= 8u) ? (int)qblk[gi * 8u + (p - 8u)]
                         : -(int)qblk[gi * 8u + (7u - p)];
    }
    return acc;
}

int or_tmac_lookup_accum(const int8_t *qlut, const uint8_t *idx,
                         const float *scales, const float *biases,
                         size_t ngroups, size_t nblocks, int bits,
                         float w_scale, float *out) {
    if (!qlut || !idx || !scales || !biases || !out) return RC_INVAL;
    if (ngroups == 0 || nblocks == 0 || ngroups != nblocks * 8u)
        return RC_INVAL;
    if (bits < 1 || bits > 4 || !isfinite((double)w_scale)) return RC_INVAL;
    for (size_t bb = 0; bb < nblocks; bb++)
        if (!isfinite((double)scales[bb]) || !isfinite((double)biases[bb]))
            return RC_INVAL;
    double total = 0.0;
    for (size_t bb = 0; bb < nblocks; bb++) {
        double sc = (double)scales[bb], bi = (double)biases[bb];
        for (int b = 0; b < bits; b++) {
            int32_t acc = plane_acc(qlut + bb * 64u,
                                    idx + (size_t)b * ngroups + bb * 8u);
            double contrib = (sc * (double)acc + bi) * 0.5;
            total += contrib * (double)(1 << b);
            if (!isfinite(total)) return RC_INVAL;
        }
    }
    total *= (double)w_scale;
    if (!isfinite(total)) return RC_INVAL;
    float f = (float)total;
    if (!isfinite((double)f)) return RC_INVAL;
    *out = f;
    return RC_OK;
}

int or_lowbit_gemm_lut(const float *X, const float *W, float *Y, int me, int h,
                       int k, int bits) {
    if (!X || !W || !Y || me < 0 || h <= 0 || k <= 0) return RC_INVAL;
    if (bits != 2 && bits != 4) return RC_INVAL;
    if (me == 0) return RC_OK;
    if (k % 32 != 0) { /* src/lowbit.c:144-156, 176-179 */
        for (int i = 0; i < me; i++)
            for (int j = 0; j < h; j++) {
                double acc = 0.0;
                for (int t = 0; t < k; t++)
                    acc += (double)X[(size_t)i * k + t] *
                           (double)W[(size_t)t * h + j];
                Y[(size_t)i * h + j] = (float)acc;
            }
        return RC_OK;
    }
    size_t ng = (size_t)k / 4u, nb = (size_t)k / 32u;
    int rc = RC_NOMEM;
    int8_t *qlut = malloc((size_t)me * ng * 8u);
    float *sc = malloc((size_t)me * nb * sizeof(float));
    float *bi = malloc((size_t)me * nb * sizeof(float));
    uint8_t *idx = malloc((size_t)bits * ng);
    float *col = malloc((size_t)k * sizeof(float));
    double *rowsum = malloc((size_t)me * sizeof(double));
    float *Yt = malloc((size_t)me * h * sizeof(float));
    if (!qlut || !sc || !bi || !idx || !col || !rowsum || !Yt) goto out;
    rc = or_tmac_lut_ctor(X, (size_t)me, (size_t)k, qlut, sc, bi);
    if (rc != RC_OK) goto out;
    for (int m = 0; m < me; m++) {
        double s = 0.0;
        for (int t = 0; t < k; t++) s += (double)X[(size_t)m * k + t];
        rowsum[m] = s;
    }
    double n1 = (double)((1 << bits) - 1);
    for (int j = 0; j < h; j++) {
        float ws = 0.0f;
        for (int t = 0; t < k; t++) col[t] = W[(size_t)t * h + j];
        rc = or_lowbit_col_to_idx(col, (size_t)k, bits, idx, &ws);
        if (rc != RC_OK) goto out;
        for (int m = 0; m < me; m++) {
            float o = 0.0f;
            rc = or_tmac_lookup_accum(qlut + (size_t)m * ng * 8u, idx,
                                      sc + (size_t)m * nb, bi + (size_t)m * nb,
                                      ng, nb, bits, ws, &o);
            if (rc != RC_OK) goto out;
            Yt[(size_t)m * h + j] =
                (float)((2.0 * (double)o - n1 * (double)ws * rowsum[m]) / n1);
        }
    }
    memcpy(Y, Yt, (size_t)me * h * sizeof(float));
    rc = RC_OK;
out:
    free(qlut); free(sc); free(bi); free(idx); free(col); free(rowsum);
    free(Yt);
    return rc;
}

/* ===================== routing ===================== */

double or_logit_lane4(const float *x, const float *w, int n) {
    double l[4] = {0.0, 0.0, 0.0, 0.0};
    int n4 = n & ~3, j = 0;
    for (; j < n4; j += 4)
        for (int i = 0; i < 4; i++) {
            double p = (double)x[j + i] * (double)w[j + i];
            l[i] = l[i] + p;
        }
    double s = (l[0] + l[1]) + (l[2] + l[3]);
    for (; j < n; j++) s += (double)x[j] * (double)w[j];
    return s;
}

int or_topk(const float *logits, size_t n, size_t k, int64_t *ids,
            float *weights) {
    if (!logits || !ids || !weights || n == 0 || k == 0 || k > n)
        return RC_INVAL;
    for (size_t i = 0; i < n; i++)
        if (isnan(logits[i])) return RC_INVAL;
    for (size_t p = 0; p < k; p++) {
        size_t best = n;
        float best_v = 0.0f;
        for (size_t i = 0; i < n; i++) {
            int taken = 0;
            for (size_t q = 0; q < p; q++) taken |= ((size_t)ids[q] == i);
            float v = taken ? -INFINITY : logits[i];
            int better = (best == n) ? 1 : (v > best_v);
            if (better) {
                best = i;
                best_v = v;
            }
        }
        ids[p] = (int64_t)best;
    }
    float mx = logits[ids[0]];
    for (size_t p = 1; p < k; p++)
        if (logits[ids[p]] > mx) mx = logits[ids[p]];
    double sum = 0.0;
    for (size_t p = 0; p < k; p++) {
        double e = exp((double)logits[ids[p]] - (double)mx);
        sum += e;
        weights[p] = (float)e;
    }
    if (!(sum > 0.0) || !isfinite(sum)) return RC_INVAL;
    float inv = (float)(1.0 / sum);
    for (size_t p = 0; p < k; p++) weights[p] = weights[p] * inv;
    return RC_OK;
}

/* Router over T tokens: logits[t][e] = (float)or_logit_lane4(x_t, w_e)
 * (src/moe_layer.c:67-86), then or_topk of each token's row
 * (src/routing.c:16-76); a non-finite logit is an error, as in the
 * reference's layer (src/moe_layer.c:391-399). */
int or_router(const float *X, const float *Wgate, int T, int E, int n, int k,
              int64_t *ids, float *w, float *logits) {
    if (!X || !Wgate || !ids || !w || !logits || T <= 0 || E <= 0 || n <= 0 ||
        k <= 0 || k > E)
        return RC_INVAL;
    for (int t = 0; t < T; t++) {
        float *lg = logits + (size_t)t * E;
        for (int e = 0; e < E; e++) {
            lg[e] = (float)or_logit_lane4(X + (size_t)t * n, Wgate + (size_t)e * n, n);
            if (!isfinite(lg[e])) return RC_INVAL;
        }
        int rc = or_topk(lg, (size_t)E, (size_t)k, ids + (size_t)t * k, w + (size_t)t * k);
        if (rc != RC_OK) return rc;
    }
    return RC_OK;
}

int or_batch_sort(const int64_t *ids, int T, int k, int E, float cap_factor,
                  int64_t *perm, int64_t *off, unsigned char *drop,
                  int64_t *out_kept) {
    if (!ids || !perm || !off || !drop || T <= 0 || k <= 0 || E <= 0 ||
        E > 4096 || k > E || k > 64)
        return RC_INVAL;
    size_t Tk = (size_t)T * (size_t)k;
    size_t cap;
    if (cap_factor > 0.0f) {
        if (!(cap_factor >= 1.0f) || !(cap_factor <= 1.5f)) return RC_INVAL;
        double capd = ceil((double)cap_factor * (double)Tk / (double)E);
        if (!isfinite(capd) || capd < 1.0) return RC_INVAL;
        cap = (size_t)capd;
    } else {
        cap = Tk;
    }
    for (size_t q = 0; q < Tk; q++)
        if (ids[q] < 0 || ids[q] >= E) return RC_INVAL;
    size_t *cnt = calloc((size_t)E, sizeof(size_t));
    if (!cnt) return RC_NOMEM;
    for (size_t q = 0; q < Tk; q++) cnt[ids[q]]++;
    off[0] = 0;
    for (int e = 0; e < E; e++)
        off[e + 1] = off[e] + (int64_t)(cnt[e] < cap ? cnt[e] : cap);
    for (int e = 0; e < E; e++) cnt[e] = (size_t)off[e];
    for (size_t q = 0; q < Tk; q++) {
        int64_t e = ids[q];
        if ((int64_t)cnt[e] < off[e + 1]) {
            perm[cnt[e]++] = (int64_t)q;
            drop[q] = 0;
        } else {
            drop[q] = 1;
        }
    }
    if (out_kept) *out_kept = off[E];
    free(cnt);
    return RC_OK;
}

/* ===================== SwiGLU ===================== */

int or_silu_mul(float g, float u, float *s) {
    double gi = (double)g, ui = (double)u;
    double sig = 1.0 / (1.0 + exp(-gi));
    double silu = gi * sig;
    double v = silu * ui;
    if (!isfinite(v) || !isfinite(sig) || !isfinite(silu)) return RC_INVAL;
    *s = (float)v;
    return RC_OK;
}

/* ===================== legacy batched layer ===================== */

static void transpose_f32(const float *src, float *dst, int rows, int cols) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++)
            dst[(size_t)c * rows + r] = src[(size_t)r * cols + c];
}

static int gemm_f32_checked(const float *A, const float *B, float *C, int M,
                            int N, int K) {
    or_gemm_f32(A, B, C, M, N, K);
    for (size_t i = 0; i < (size_t)M * N; i++)
        if (!isfinite((double)C[i])) return RC_INVAL;
    return RC_OK;
}

/* Per-column fake-quant of W[k][h] (src/moe_layer.c:24-53). */
static int fq_cols(float *W, int k, int h, int bits) {
    float *col = malloc((size_t)k * sizeof(float));
    if (!col) return RC_NOMEM;
    for (int j = 0; j < h; j++) {
        for (int t = 0; t < k; t++) col[t] = W[(size_t)t * h + j];
        if (or_lowbit_fakequant(col, col, (size_t)k, bits) != RC_OK) {
            free(col);
            return RC_INVAL;
        }
        for (int t = 0; t < k; t++) W[(size_t)t * h + j] = col[t];
    }
    free(col);
    return RC_OK;
}

/* A per-tensor, B per-channel, B given as [N][K] (src/moe_layer.c:228-274). */
static int w8a8_pc(const float *A, const float *Brow, float *C, int M, int N,
                   int K) {
    /* M, N, K <= JT_BWD_MAX_WIDE (src/w8a8.c:926-929) */
    if (M > 4096 || N > 4096 || K > 4096) return RC_INVAL;
    int rc = RC_NOMEM;
    int8_t *Aq = malloc((size_t)M * K), *BqT = malloc((size_t)N * K),
           *Bq = malloc((size_t)N * K);
    float *sB = malloc((size_t)N * sizeof(float)), sA = 1.0f;
    if (!Aq || !BqT || !Bq || !sB) goto out;
    if ((rc = or_quant_row(A, (size_t)M * K, Aq, &sA)) != RC_OK) goto out;
    if ((rc = or_quant_rows(Brow, (size_t)N, (size_t)K, BqT, sB)) != RC_OK)
        goto out;
    for (int r = 0; r < N; r++)
        for (int c = 0; c < K; c++) Bq[(size_t)c * N + r] = BqT[(size_t)r * K + c];
    rc = or_w8a8_gemm(Aq, &sA, 0, Bq, sB, 1, C, NULL, M, N, K);
out:
    free(Aq); free(BqT); free(Bq); free(sB);
    return rc;
}

/* Both sides per tensor, B given as [K][N] (src/moe_layer.c:185-223). */
static int w8a8_pt(const float *A, const float *Bkn, float *C, int M, int N,
                   int K) {
    if (M > 4096 || N > 4096 || K > 4096) return RC_INVAL; /* src/w8a8.c:926-929 */
    int rc = RC_NOMEM;
    int8_t *Aq = malloc((size_t)M * K), *Bq = malloc((size_t)K * N);
    float sA = 1.0f, sB = 1.0f;
    if (!Aq || !Bq) goto out;
    if ((rc = or_quant_row(A, (size_t)M * K, Aq, &sA)) != RC_OK) goto out;
    if ((rc = or_quant_row(Bkn, (size_t)K * N, Bq, &sB)) != RC_OK) goto out;
    rc = or_w8a8_gemm(Aq, &sA, 0, Bq, &sB, 0, C, NULL, M, N, K);
out:
    free(Aq); free(Bq);
    return rc;
}

static int silu_tile(const float *G, const float *U, float *S, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (or_silu_mul(G[i], U[i], &S[i]) != RC_OK) return RC_INVAL;
    return RC_OK;
}

int or_moe_fwd_batch(const float *X, const float *Wgate, const float *Wg,
                     const float *Wu, const float *Wd, const float *Wg_s,
                     const float *Wu_s, const float *Wd_s, float *Y, int T,
                     int n, int h, int E, int k, int S, int64_t *out_ids,
                     float *out_weights, float cap_factor, int64_t *out_perm,
                     int64_t *out_off, unsigned char *out_drop,
                     int64_t *out_kept, int w8a8_on, int lowbit_mode,
                     float *cache_Ysel) {
    if (!X || !Wgate || !Wg || !Wu || !Wd || !Y || !out_ids || !out_weights)
        return RC_INVAL;
    if (T <= 0 || n <= 0 || h <= 0 || n > 4096 || h > 4096 || E <= 0 ||
        E > 4096 || k <= 0 || k > E || k > 64 || S < 0 || S > 8)
        return RC_INVAL;
    if (S > 0 && (!Wg_s || !Wu_s || !Wd_s)) return RC_INVAL;
    if (!(cap_factor >= 1.0f) || !(cap_factor <= 1.5f)) return RC_INVAL;
    size_t Tk = (size_t)T * k, nh = (size_t)n * h;
    {
        const float *arrs[5] = {X, Wgate, Wg, Wu, Wd};
        size_t lens[5] = {(size_t)T * n, (size_t)E * n, E * nh, E * nh, E * nh};
        for (int a = 0; a < 5; a++)
            for (size_t i = 0; i < lens[a]; i++)
                if (!isfinite((double)arrs[a][i])) return RC_INVAL;
        if (S > 0) {
            const float *sarr[3] = {Wg_s, Wu_s, Wd_s};
            for (int a = 0; a < 3; a++)
                for (size_t i = 0; i < S * nh; i++)
                    if (!isfinite((double)sarr[a][i])) return RC_INVAL;
        }
    }
    int rc = RC_NOMEM;
    double *yacc = calloc((size_t)T * n, sizeof(double));
    int64_t *perm = malloc(Tk * sizeof(int64_t));
    int64_t *off = malloc(((size_t)E + 1) * sizeof(int64_t));
    unsigned char *drop = malloc(Tk);
    float *Ysel = calloc(Tk * n, sizeof(float));
    float *logits = malloc((size_t)E * sizeof(float));
    float *Wgt = malloc(nh * sizeof(float)), *Wut = malloc(nh * sizeof(float));
    float *Wfq = malloc(nh * sizeof(float));
    float *Xe = NULL, *Ge = NULL, *Ue = NULL, *Se = NULL, *Ye = NULL;
    float *Gs = NULL, *Us = NULL, *Ys = NULL;
    int64_t kept = 0;
    if (!yacc || !perm || !off || !drop || !Ysel || !logits || !Wgt || !Wut ||
        !Wfq)
        goto out;
    rc = RC_INVAL;
    for (int t = 0; t < T; t++) {
        for (int e = 0; e < E; e++) {
            double acc = or_logit_lane4(X + (size_t)t * n, Wgate + (size_t)e * n, n);
            if (!isfinite(acc)) goto out;
            logits[e] = (float)acc;
            if (!isfinite((double)logits[e])) goto out;
        }
        if (or_topk(logits, (size_t)E, (size_t)k, out_ids + (size_t)t * k,
                    out_weights + (size_t)t * k) != RC_OK)
            goto out;
        for (int p = 0; p < k; p++) {
            float w = out_weights[(size_t)t * k + p];
            if (!(w >= 0.0f) || !isfinite((double)w)) goto out;
        }
    }
    if (or_batch_sort(out_ids, T, k, E, cap_factor, perm, off, drop, &kept) !=
        RC_OK)
        goto out;
    for (int t = 0; t < T; t++) { /* src/moe_layer.c:1171-1201 */
        double s = 0.0;
        int nd = 0;
        for (int p = 0; p < k; p++) {
            size_t q = (size_t)t * k + p;
            if (drop[q]) nd++;
            else s += (double)out_weights[q];
        }
        if (nd > 0 && s > 0.0) {
            if (!isfinite(s)) goto out;
            for (int p = 0; p < k; p++) {
                size_t q = (size_t)t * k + p;
                if (drop[q]) continue;
                double rw = (double)out_weights[q] / s;
                if (!isfinite(rw) || rw < 0.0) goto out;
                out_weights[q] = (float)rw;
            }
        }
    }
    {
        size_t maxMe = 0;
        for (int e = 0; e < E; e++)
            if ((size_t)(off[e + 1] - off[e]) > maxMe) maxMe = off[e + 1] - off[e];
        rc = RC_NOMEM;
        if (maxMe > 0) {
            Xe = malloc(maxMe * n * sizeof(float));
            Ye = malloc(maxMe * n * sizeof(float));
            Ge = malloc(maxMe * h * sizeof(float));
            Ue = malloc(maxMe * h * sizeof(float));
            Se = malloc(maxMe * h * sizeof(float));
            if (!Xe || !Ye || !Ge || !Ue || !Se) goto out;
        }
        rc = RC_INVAL;
        for (int e = 0; e < E; e++) {
            size_t b0 = (size_t)off[e];
            int Me = (int)(off[e + 1] - off[e]);
            if (Me == 0) continue;
            for (int m = 0; m < Me; m++) {
                size_t t = (size_t)perm[b0 + m] / (size_t)k;
                memcpy(Xe + (size_t)m * n, X + t * n, (size_t)n * sizeof(float));
            }
            const float *wg = Wg + (size_t)e * nh, *wu = Wu + (size_t)e * nh,
                        *wd = Wd + (size_t)e * nh;
            if (lowbit_mode != 0) {
                transpose_f32(wg, Wgt, h, n);
                transpose_f32(wu, Wut, h, n);
                if (lowbit_mode == 1) {
                    if (fq_cols(Wgt, n, h, 2) != RC_OK ||
                        fq_cols(Wut, n, h, 2) != RC_OK)
                        goto out;
                    if (gemm_f32_checked(Xe, Wgt, Ge, Me, h, n) != RC_OK ||
                        gemm_f32_checked(Xe, Wut, Ue, Me, h, n) != RC_OK)
                        goto out;
                } else {
                    if (or_lowbit_gemm_lut(Xe, Wgt, Ge, Me, h, n, 2) != RC_OK ||
                        or_lowbit_gemm_lut(Xe, Wut, Ue, Me, h, n, 2) != RC_OK)
                        goto out;
                }
            } else if (w8a8_on) {
                if (w8a8_pc(Xe, wg, Ge, Me, h, n) != RC_OK ||
                    w8a8_pc(Xe, wu, Ue, Me, h, n) != RC_OK)
                    goto out;
            } else {
                transpose_f32(wg, Wgt, h, n);
                transpose_f32(wu, Wut, h, n);
                if (gemm_f32_checked(Xe, Wgt, Ge, Me, h, n) != RC_OK ||
                    gemm_f32_checked(Xe, Wut, Ue, Me, h, n) != RC_OK)
                    goto out;
            }
            if (silu_tile(Ge, Ue, Se, (size_t)Me * h) != RC_OK) goto out;
            int grc;
            if (lowbit_mode != 0) {
                if (lowbit_mode == 1) {
                    memcpy(Wfq, wd, nh * sizeof(float));
                    if (fq_cols(Wfq, h, n, 4) != RC_OK) goto out;
                    grc = gemm_f32_checked(Se, Wfq, Ye, Me, n, h);
                } else {
                    grc = or_lowbit_gemm_lut(Se, wd, Ye, Me, n, h, 4);
                }
            } else if (w8a8_on) {
                grc = w8a8_pt(Se, wd, Ye, Me, n, h);
            } else {
                grc = gemm_f32_checked(Se, wd, Ye, Me, n, h);
            }
            if (grc != RC_OK) goto out;
            for (int m = 0; m < Me; m++)
                memcpy(Ysel + (size_t)perm[b0 + m] * n, Ye + (size_t)m * n,
                       (size_t)n * sizeof(float));
        }
    }
    for (int t = 0; t < T; t++) {
        double *ya = yacc + (size_t)t * n;
        for (int p = 0; p < k; p++) {
            size_t q = (size_t)t * k + p;
            if (drop[q]) continue;
            double w = (double)out_weights[q];
            const float *yp = Ysel + q * n;
            for (int j = 0; j < n; j++) ya[j] += w * (double)yp[j];
        }
    }
    if (S > 0) {
        rc = RC_NOMEM;
        Gs = malloc((size_t)T * h * sizeof(float));
        Us = malloc((size_t)T * h * sizeof(float));
        Ys = malloc((size_t)T * n * sizeof(float));
        if (!Gs || !Us || !Ys) goto out;
        rc = RC_INVAL;
        for (int s = 0; s < S; s++) {
            const float *wg = Wg_s + (size_t)s * nh, *wu = Wu_s + (size_t)s * nh,
                        *wd = Wd_s + (size_t)s * nh;
            if (w8a8_on) {
                if (w8a8_pc(X, wg, Gs, T, h, n) != RC_OK ||
                    w8a8_pc(X, wu, Us, T, h, n) != RC_OK)
                    goto out;
            } else {
                transpose_f32(wg, Wgt, h, n);
                transpose_f32(wu, Wut, h, n);
                if (gemm_f32_checked(X, Wgt, Gs, T, h, n) != RC_OK ||
                    gemm_f32_checked(X, Wut, Us, T, h, n) != RC_OK)
                    goto out;
            }
            if (silu_tile(Gs, Us, Gs, (size_t)T * h) != RC_OK) goto out;
            int grc = w8a8_on ? w8a8_pt(Gs, wd, Ys, T, n, h)
                              : gemm_f32_checked(Gs, wd, Ys, T, n, h);
            if (grc != RC_OK) goto out;
            for (size_t i = 0; i < (size_t)T * n; i++) yacc[i] += (double)Ys[i];
        }
    }
    for (size_t i = 0; i < (size_t)T * n; i++)
        if (!isfinite(yacc[i])) goto out;
    for (size_t i = 0; i < (size_t)T * n; i++) Y[i] = (float)yacc[i];
    if (out_perm) memcpy(out_perm, perm, (size_t)kept * sizeof(int64_t));
    if (out_off) memcpy(out_off, off, ((size_t)E + 1) * sizeof(int64_t));
    if (out_drop) memcpy(out_drop, drop, Tk);
    if (out_kept) *out_kept = kept;
    if (cache_Ysel) memcpy(cache_Ysel, Ysel, Tk * n * sizeof(float));
    rc = RC_OK;
out:
    free(yacc); free(perm); free(off); free(drop); free(Ysel); free(logits);
    free(Wgt); free(Wut); free(Wfq); free(Xe); free(Ge); free(Ue); free(Se);
    free(Ye); free(Gs); free(Us); free(Ys);
    return rc;
}

/* ===================== prepared quantised layer ===================== */

void or_moe_q_free(or_moe_q *L) {
    free(L->gu_codes); free(L->gu_scales); free(L->d_codes); free(L->d_scales);
    free(L->sgu_q); free(L->sgu_s); free(L->sd_q); free(L->sd_s);
    memset(L, 0, sizeof(*L));
}

int or_moe_q_prepare(or_moe_q *L, int n, int h, int E, int k, int S, int hs,
                     int group, const float *Wgate, const float *Wg,
                     const float *Wu, const float *Wd, const float *Wg_s,
                     const float *Wu_s, const float *Wd_s) {
    memset(L, 0, sizeof(*L));
    if (n % group || h % group) return RC_INVAL;
    L->n = n; L->h = h; L->E = E; L->k = k; L->S = S; L->hs = hs;
    L->group = group; L->Wgate = Wgate;
    size_t nh = (size_t)n * h;
    L->gu_codes = malloc((size_t)E * 2 * nh);
    L->gu_scales = malloc((size_t)E * 2 * nh / group * sizeof(uint16_t));
    L->d_codes = malloc((size_t)E * nh);
    L->d_scales = malloc((size_t)E * nh / group * sizeof(uint16_t));
    float *tr = malloc(((size_t)n * (hs > h ? hs : h)) * sizeof(float));
    if (S > 0) {
        L->sgu_q = malloc((size_t)S * 2 * hs * n);
        L->sgu_s = malloc((size_t)S * 2 * hs * sizeof(float));
        L->sd_q = malloc((size_t)S * n * hs);
        L->sd_s = malloc((size_t)S * n * sizeof(float));
    }
    if (!L->gu_codes || !L->gu_scales || !L->d_codes || !L->d_scales || !tr ||
        (S > 0 && (!L->sgu_q || !L->sgu_s || !L->sd_q || !L->sd_s))) {
        free(tr);
        or_moe_q_free(L);
        return RC_NOMEM;
    }
    int rc = RC_OK;
    for (int e = 0; e < E && rc == RC_OK; e++) {
        for (int w = 0; w < 2 && rc == RC_OK; w++) {
            const float *src = (w == 0 ? Wg : Wu) + (size_t)e * nh;
            rc = or_lowbit_pack_rows(src, h, n, 2, group,
                                     L->gu_codes + ((size_t)e * 2 + w) * nh,
                                     L->gu_scales + ((size_t)e * 2 + w) * nh / group);
        }
        if (rc != RC_OK) break;
        transpose_f32(Wd + (size_t)e * nh, tr, h, n); /* [n][h] */
        rc = or_lowbit_pack_rows(tr, n, h, 4, group, L->d_codes + (size_t)e * nh,
                                 L->d_scales + (size_t)e * nh / group);
    }
    size_t nhs = (size_t)n * hs;
    for (int s = 0; s < S && rc == RC_OK; s++) {
        rc = or_quant_rows(Wg_s + (size_t)s * nhs, hs, n,
                           L->sgu_q + ((size_t)s * 2) * nhs,
                           L->sgu_s + ((size_t)s * 2) * hs);
        if (rc == RC_OK)
            rc = or_quant_rows(Wu_s + (size_t)s * nhs, hs, n,
                               L->sgu_q + ((size_t)s * 2 + 1) * nhs,
                               L->sgu_s + ((size_t)s * 2 + 1) * hs);
        if (rc == RC_OK) {
            transpose_f32(Wd_s + (size_t)s * nhs, tr, hs, n); /* [n][hs] */
            rc = or_quant_rows(tr, n, hs, L->sd_q + (size_t)s * nhs,
                               L->sd_s + (size_t)s * n);
        }
    }
    free(tr);
    if (rc != RC_OK) or_moe_q_free(L);
    return rc;
}

/* Dot of one int8 activation row with one int8 weight row (both K long),
 * W8A8 epilogue (src/w8a8.c:664-676). */
static int w8a8_row_dot(const int8_t *a, float sa, const int8_t *wrow,
                        float sw, int K, float *out) {
    int32_t acc = 0;
    for (int i = 0; i < K; i++) acc += (int32_t)a[i] * (int32_t)wrow[i];
    float f = (float)((double)acc * ((double)sa * (double)sw));
    if (!isfinite((double)f)) return RC_INVAL;
    *out = f;
    return RC_OK;
}

/* Shared expert s of L on one token (activation row already quantised). */
static int shared_token(const or_moe_q *L, int s, const int8_t *xq, float sx,
                        float *sbuf, int8_t *sq, float *y) {
    int n = L->n, hs = L->hs;
    size_t nhs = (size_t)n * hs;
    const int8_t *gq = L->sgu_q + ((size_t)s * 2) * nhs;
    const int8_t *uq = L->sgu_q + ((size_t)s * 2 + 1) * nhs;
    const float *gs = L->sgu_s + ((size_t)s * 2) * hs;
    const float *us = L->sgu_s + ((size_t)s * 2 + 1) * hs;
    for (int i = 0; i < hs; i++) {
        float g, u;
        if (w8a8_row_dot(xq, sx, gq + (size_t)i * n, gs[i], n, &g) != RC_OK ||
            w8a8_row_dot(xq, sx, uq + (size_t)i * n, us[i], n, &u) != RC_OK ||
            or_silu_mul(g, u, &sbuf[i]) != RC_OK)
            return RC_INVAL;
    }
    float ss;
    if (quant_span(sbuf, (size_t)hs, sq, &ss) != RC_OK) return RC_INVAL;
    const int8_t *dq = L->sd_q + (size_t)s * nhs;
    const float *ds = L->sd_s + (size_t)s * n;
    for (int j = 0; j < n; j++)
        if (w8a8_row_dot(sq, ss, dq + (size_t)j * hs, ds[j], hs, &y[j]) != RC_OK)
            return RC_INVAL;
    return RC_OK;
}

int or_moe_q_fwd(const or_moe_q *L, const float *X, int T,
                 const int32_t *ids_in, const float *w_in, float *Y,
                 int32_t *ids_o, float *w_o, int32_t *perm_o, int32_t *off_o,
                 float *Ye_o, float *Ys_o, int8_t *Hq_o, float *Hs_o) {
    int n = L->n, h = L->h, E = L->E, k = L->k, S = L->S, hs = L->hs;
    int G = L->group;
    size_t Tk = (size_t)T * k, nh = (size_t)n * h;
    int rc = RC_NOMEM;
    int8_t *Xq = malloc((size_t)T * n);
    float *sx = malloc((size_t)T * sizeof(float));
    int64_t *ids = malloc(Tk * sizeof(int64_t));
    float *w = malloc(Tk * sizeof(float));
    int64_t *perm = malloc(Tk * sizeof(int64_t));
    int64_t *off = malloc(((size_t)E + 1) * sizeof(int64_t));
    unsigned char *drop = malloc(Tk);
    float *Ye = malloc(Tk * n * sizeof(float));
    float *Ys = malloc(((size_t)(S > 0 ? S : 1)) * T * n * sizeof(float));
    float *logits = malloc((size_t)E * sizeof(float));
    int hm = hs > h ? hs : h;
    float *g = malloc((size_t)hm * sizeof(float));
    float *u = malloc((size_t)hm * sizeof(float));
    float *sb = malloc((size_t)hm * sizeof(float));
    int8_t *sq = malloc((size_t)hm);
    if (!Xq || !sx || !ids || !w || !perm || !off || !drop || !Ye || !Ys ||
        !logits || !g || !u || !sb || !sq)
        goto out;
    rc = or_quant_rows(X, (size_t)T, (size_t)n, Xq, sx);
    if (rc != RC_OK) goto out;
    rc = RC_INVAL;
    if (ids_in && w_in) {
        for (size_t q = 0; q < Tk; q++) {
            if (ids_in[q] < 0 || ids_in[q] >= E) goto out;
            ids[q] = ids_in[q];
            w[q] = w_in[q];
        }
    } else {
        if (!L->Wgate) goto out;
        for (int t = 0; t < T; t++) {
            for (int e = 0; e < E; e++) {
                double acc = or_logit_lane4(X + (size_t)t * n,
                                            L->Wgate + (size_t)e * n, n);
                logits[e] = (float)acc;
                if (!isfinite(acc) || !isfinite((double)logits[e])) goto out;
            }
            if (or_topk(logits, (size_t)E, (size_t)k, ids + (size_t)t * k,
                        w + (size_t)t * k) != RC_OK)
                goto out;
        }
    }
    if (or_batch_sort(ids, T, k, E, 0.0f, perm, off, drop, NULL) != RC_OK)
        goto out;
    /* routed experts, row by row in perm order */
    for (int e = 0; e < E; e++) {
        const uint8_t *gc = L->gu_codes + ((size_t)e * 2) * nh;
        const uint8_t *uc = L->gu_codes + ((size_t)e * 2 + 1) * nh;
        const uint16_t *gsc = L->gu_scales + ((size_t)e * 2) * nh / G;
        const uint16_t *usc = L->gu_scales + ((size_t)e * 2 + 1) * nh / G;
        const uint8_t *dc = L->d_codes + (size_t)e * nh;
        const uint16_t *dsc = L->d_scales + (size_t)e * nh / G;
        for (int64_t r = off[e]; r < off[e + 1]; r++) {
            int64_t q = perm[r];
            int64_t t = q / k;
            const int8_t *xq = Xq + (size_t)t * n;
            if (or_gemm_lowbit_group(xq, &sx[t], gc, gsc, 2, G, g, NULL, 1, h,
                                     n) != RC_OK ||
                or_gemm_lowbit_group(xq, &sx[t], uc, usc, 2, G, u, NULL, 1, h,
                                     n) != RC_OK)
                goto out;
            for (int i = 0; i < h; i++)
                if (or_silu_mul(g[i], u[i], &sb[i]) != RC_OK) goto out;
            float ss;
            if (quant_span(sb, (size_t)h, sq, &ss) != RC_OK) goto out;
            if (Hq_o) memcpy(Hq_o + (size_t)r * h, sq, (size_t)h);
            if (Hs_o) Hs_o[r] = ss;
            if (or_gemm_lowbit_group(sq, &ss, dc, dsc, 4, G, Ye + (size_t)q * n,
                                     NULL, 1, n, h) != RC_OK)
                goto out;
        }
    }
    for (int s = 0; s < S; s++)
        for (int t = 0; t < T; t++)
            if (shared_token(L, s, Xq + (size_t)t * n, sx[t], sb, sq,
                             Ys + ((size_t)s * T + t) * n) != RC_OK)
                goto out;
    for (int t = 0; t < T; t++)
        for (int j = 0; j < n; j++) {
            double acc = 0.0;
            for (int p = 0; p < k; p++) {
                size_t q = (size_t)t * k + p;
                acc += (double)w[q] * (double)Ye[q * n + j];
            }
            for (int s = 0; s < S; s++)
                acc += (double)Ys[((size_t)s * T + t) * n + j];
            if (!isfinite(acc)) goto out;
            Y[(size_t)t * n + j] = (float)acc;
        }
    if (ids_o) for (size_t q = 0; q < Tk; q++) ids_o[q] = (int32_t)ids[q];
    if (w_o) memcpy(w_o, w, Tk * sizeof(float));
    if (perm_o) for (size_t q = 0; q < Tk; q++) perm_o[q] = (int32_t)perm[q];
    if (off_o) for (int e = 0; e <= E; e++) off_o[e] = (int32_t)off[e];
    if (Ye_o) memcpy(Ye_o, Ye, Tk * n * sizeof(float));
    if (Ys_o && S > 0) memcpy(Ys_o, Ys, (size_t)S * T * n * sizeof(float));
    rc = RC_OK;
out:
    free(Xq); free(sx); free(ids); free(w); free(perm); free(off); free(drop);
    free(Ye); free(Ys); free(logits); free(g); free(u); free(sb); free(sq);
    return rc;
}

int or_ffn_fwd(const float *Wg, const float *Wu, const float *Wd, int n,
               int h, const float *X, int T, float *Y) {
    or_moe_q L;
    memset(&L, 0, sizeof(L));
    L.n = n; L.hs = h; L.S = 1;
    size_t nh = (size_t)n * h;
    int rc = RC_NOMEM;
    int8_t *Xq = malloc((size_t)T * n);
    float *sx = malloc((size_t)T * sizeof(float));
    float *tr = malloc(nh * sizeof(float));
    float *sb = malloc((size_t)h * sizeof(float));
    int8_t *sq = malloc((size_t)h);
    L.sgu_q = malloc(2 * nh);
    L.sgu_s = malloc(2 * (size_t)h * sizeof(float));
    L.sd_q = malloc(nh);
    L.sd_s = malloc((size_t)n * sizeof(float));
    if (!Xq || !sx || !tr || !sb || !sq || !L.sgu_q || !L.sgu_s || !L.sd_q ||
        !L.sd_s)
        goto out;
    if ((rc = or_quant_rows(Wg, h, n, L.sgu_q, L.sgu_s)) != RC_OK) goto out;
    if ((rc = or_quant_rows(Wu, h, n, L.sgu_q + nh, L.sgu_s + h)) != RC_OK)
        goto out;
    transpose_f32(Wd, tr, h, n);
    if ((rc = or_quant_rows(tr, n, h, L.sd_q, L.sd_s)) != RC_OK) goto out;
    if ((rc = or_quant_rows(X, T, n, Xq, sx)) != RC_OK) goto out;
    for (int t = 0; t < T; t++)
        if ((rc = shared_token(&L, 0, Xq + (size_t)t * n, sx[t], sb, sq,
                               Y + (size_t)t * n)) != RC_OK)
            goto out;
out:
    free(Xq); free(sx); free(tr); free(sb); free(sq);
    free(L.sgu_q); free(L.sgu_s); free(L.sd_q); free(L.sd_s);
    return rc;
}

/* Residual add of the reference's training loop after its MoE layer
 * (bench/kernel/train_tinystories.c:1147-1160): y = (float)((double)x +
 * (double)m) per element; rc 2 (y untouched from that element on) when a
 * sum is not finite. */
int or_residual_add(const float *X, const float *Mo, float *Y, size_t n) {
    for (size_t i = 0; i < n; i++) {
        double v = (double)X[i] + (double)Mo[i];
        if (!isfinite(v)) return RC_INVAL;
        Y[i] = (float)v;
    }
    return RC_OK;
}

/* ===================== batched backward ===================== */

/* C[r][c] = fp32 sum over kk ascending of A(r, kk) * B(kk, c), one rounded
 * multiply and one rounded add per step (src/moe_gemm.c:47-61), with
 * A(r, kk) = A[r*ar + kk*ak] and B(kk, c) = B[kk*bk + c*bc]: the strides
 * stand for the reference's exact transposes (src/moe_gemm.c:17-41). */
static void gemm_f32_strided(const float *A, size_t ar, size_t ak,
                             const float *B, size_t bk, size_t bc, float *C,
                             int M, int N, int K) {
    for (int r = 0; r < M; r++)
        for (int c = 0; c < N; c++) {
            float acc = 0.0f;
            for (int kk = 0; kk < K; kk++) {
                float p = A[(size_t)r * ar + (size_t)kk * ak] *
                          B[(size_t)kk * bk + (size_t)c * bc];
                acc = acc + p;
            }
            C[(size_t)r * N + c] = acc;
        }
}

/* SwiGLU backward of one element in fp64 (src/moe_layer.c:1680-1682,
 * 2204-2233): sig = 1/(1+exp(-g)), silu = g*sig,
 * dsilu = sig*(1 + g*(1-sig)); dg = acc*u*dsilu, du = acc*silu,
 * s = silu*u. Returns 0 when acc or a result is not finite. */
static int swiglu_bwd_elem(float g, float u, float dot, float *dg, float *du,
                           float *s) {
    double gi = (double)g, ui = (double)u, acc = (double)dot;
    double sig = 1.0 / (1.0 + exp(-gi));
    double silu = gi * sig;
    double dsilu = sig * (1.0 + gi * (1.0 - sig));
    if (!isfinite(acc)) return 0;
    double gd = acc * ui * dsilu, ud = acc * silu, sv = silu * ui;
    if (!isfinite(gd) || !isfinite(ud) || !isfinite(sv)) return 0;
    *dg = (float)gd;
    *du = (float)ud;
    *s = (float)sv;
    return 1;
}

/* One expert's backward over M rows (src/moe_layer.c:2196-2283 for a routed
 * expert, :2310-2396 for a shared one): Xr, Dy [M][n]; G, U rows of h with
 * row stride ldgu; W* [h][n]. dxe [M][n] = (float)((double)(Dg Wg) +
 * (double)(Du Wu)); oWg = Dg^T Xr, oWu = Du^T Xr, oWd = S^T Dy. */
static int expert_bwd(const float *Xr, const float *Dy, const float *G,
                      const float *U, size_t ldgu, const float *Wg,
                      const float *Wu, const float *Wd, int M, int n, int h,
                      float *dxe, float *oWg, float *oWu, float *oWd) {
    size_t Mh = (size_t)M * h, Mn = (size_t)M * n;
    float *buf = malloc((4 * Mh + 2 * Mn) * sizeof(float));
    if (!buf) return RC_NOMEM;
    float *dot = buf, *dg = dot + Mh, *du = dg + Mh, *ss = du + Mh;
    float *d1 = ss + Mh, *d2 = d1 + Mn;
    int rc = RC_INVAL;
    /* dot[m][i] = sum_j Dy[m][j] * Wd[i][j] */
    gemm_f32_strided(Dy, (size_t)n, 1, Wd, 1, (size_t)n, dot, M, h, n);
    for (int m = 0; m < M; m++)
        for (int i = 0; i < h; i++) {
            size_t a = (size_t)m * ldgu + i, o = (size_t)m * h + i;
            if (!swiglu_bwd_elem(G[a], U[a], dot[o], &dg[o], &du[o], &ss[o]))
                goto out;
        }
    gemm_f32_strided(dg, (size_t)h, 1, Wg, (size_t)n, 1, d1, M, n, h);
    gemm_f32_strided(du, (size_t)h, 1, Wu, (size_t)n, 1, d2, M, n, h);
    for (size_t i = 0; i < Mn; i++) dxe[i] = (float)((double)d1[i] + (double)d2[i]);
    /* dW[i][j] = sum over m ascending of D[m][i] * rows[m][j] */
    gemm_f32_strided(dg, 1, (size_t)h, Xr, (size_t)n, 1, oWg, h, n, M);
    gemm_f32_strided(du, 1, (size_t)h, Xr, (size_t)n, 1, oWu, h, n, M);
    gemm_f32_strided(ss, 1, (size_t)h, Dy, (size_t)n, 1, oWd, h, n, M);
    rc = RC_OK;
out:
    free(buf);
    return rc;
}

static int all_finite_f(const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite((double)x[i])) return 0;
    return 1;
}

/* src/moe_layer.c:1684-2439. Steps, in the reference's order:
 *  0. argument checks (validate: finiteness of every input, ids < E,
 *     weights in [0,1], drop in {0,1}, off monotone from 0, perm an exact
 *     enumeration of the kept pairs; otherwise only off[E] <= T*k);
 *  1. dw[q] = lane-4 fp64 dot(Ysel[q], dY[t]) for kept q, 0 for dropped;
 *  2. per token s = sum_kept (double)w*dw in slot order,
 *     dlog[q] = (double)w*(dw - s), dLogits[t][ids[q]] = (float)dlog;
 *  3. gate-path dX: the first two kept slots of the token, ordered by
 *     expert id, acc = sum dlog*(double)Wgate[e][j], dx[t][j] += acc;
 *  4. dWgate[e][j] += (float)(dlog*(double)X[t][j]) in token/slot order;
 *  5. routed experts in id order on their perm rows, rows weighted
 *     dYe = (float)((double)w*(double)dY); dx[t] += (double)dxe in perm order;
 *  6. shared experts in index order on all tokens, dY unweighted;
 *  7. dX = (float)dx after a finiteness check. */
int or_moe_bwd_batch(const float *dY, const float *X, const float *Wgate,
                     const float *Wg, const float *Wu, const float *Wd,
                     const float *Wg_s, const float *Wu_s, const float *Wd_s,
                     const int64_t *ids, const float *weights,
                     const float *Gsel, const float *Usel, const float *Ysel,
                     const float *Gs, const float *Us, const int64_t *perm,
                     const int64_t *off, const unsigned char *drop, float *dX,
                     float *dWgate, float *dWg, float *dWu, float *dWd,
                     float *dWg_s, float *dWu_s, float *dWd_s, float *dLogits,
                     int T, int n, int h, int E, int k, int S, int validate) {
    if (!dY || !X || !Wgate || !Wg || !Wu || !Wd || !ids || !weights ||
        !Gsel || !Usel || !Ysel || !perm || !off || !drop || !dX ||
        !dWgate || !dWg || !dWu || !dWd)
        return RC_INVAL;
    if (T <= 0 || n <= 0 || h <= 0 || n > 4096 || h > 4096 || E <= 0 ||
        E > 4096 || k <= 0 || k > E || k > 64 || S < 0 || S > 8)
        return RC_INVAL;
    if (S > 0 && (!Wg_s || !Wu_s || !Wd_s || !Gs || !Us || !dWg_s || !dWu_s ||
                  !dWd_s))
        return RC_INVAL;
    const size_t Tk = (size_t)T * k, Tn = (size_t)T * n, nh = (size_t)n * h;
    size_t kept;
    if (validate) {
        if (!all_finite_f(dY, Tn) || !all_finite_f(X, Tn) ||
            !all_finite_f(Wgate, (size_t)E * n) || !all_finite_f(Wg, E * nh) ||
            !all_finite_f(Wu, E * nh) || !all_finite_f(Wd, E * nh) ||
            !all_finite_f(weights, Tk) || !all_finite_f(Gsel, Tk * h) ||
            !all_finite_f(Usel, Tk * h) || !all_finite_f(Ysel, Tk * n))
            return RC_INVAL;
        if (S > 0 && (!all_finite_f(Wg_s, S * nh) || !all_finite_f(Wu_s, S * nh) ||
                      !all_finite_f(Wd_s, S * nh) ||
                      !all_finite_f(Gs, Tk / k * S * h) ||
                      !all_finite_f(Us, Tk / k * S * h)))
            return RC_INVAL;
        for (size_t q = 0; q < Tk; q++) {
            if (ids[q] < 0 || ids[q] >= E) return RC_INVAL;
            if (!(weights[q] >= 0.0f) || !(weights[q] <= 1.0f)) return RC_INVAL;
            if (drop[q] > 1) return RC_INVAL;
        }
        if (off[0] != 0) return RC_INVAL;
        for (int e = 0; e < E; e++)
            if (off[e + 1] < off[e] || (size_t)off[e + 1] > Tk) return RC_INVAL;
        kept = (size_t)off[E];
        unsigned char *seen = calloc(Tk, 1);
        if (!seen) return RC_NOMEM;
        size_t nkept = 0;
        int bad = 0;
        for (size_t i = 0; i < kept && !bad; i++) {
            int64_t q = perm[i];
            if (q < 0 || (size_t)q >= Tk || drop[q] || seen[q]) bad = 1;
            else seen[q] = 1;
        }
        for (size_t q = 0; q < Tk && !bad; q++)
            if (!drop[q]) {
                nkept++;
                if (!seen[q]) bad = 1;
            }
        free(seen);
        if (bad || nkept != kept) return RC_INVAL;
    } else {
        if (off[E] < 0 || (size_t)off[E] > Tk) return RC_INVAL;
        kept = (size_t)off[E];
    }
    (void)kept;
    double *dx = calloc(Tn, sizeof(double));
    double *dw = malloc(Tk * sizeof(double)), *dlog = malloc(Tk * sizeof(double));
    int rc = RC_NOMEM;
    float *Xe = NULL, *Dye = NULL, *Ge = NULL, *Ue = NULL, *dxe = NULL;
    if (!dx || !dw || !dlog) goto out;
    memset(dWgate, 0, (size_t)E * n * sizeof(float));
    memset(dWg, 0, E * nh * sizeof(float));
    memset(dWu, 0, E * nh * sizeof(float));
    memset(dWd, 0, E * nh * sizeof(float));
    if (S > 0) {
        memset(dWg_s, 0, S * nh * sizeof(float));
        memset(dWu_s, 0, S * nh * sizeof(float));
        memset(dWd_s, 0, S * nh * sizeof(float));
    }
    if (dLogits) memset(dLogits, 0, (size_t)T * E * sizeof(float));
    rc = RC_INVAL;
    /* 1 */
    for (size_t q = 0; q < Tk; q++) {
        dlog[q] = 0.0;
        dw[q] = drop[q] ? 0.0 : or_logit_lane4(Ysel + q * n, dY + q / k * n, n);
        if (!isfinite(dw[q])) goto out;
    }
    /* 2 */
    for (int t = 0; t < T; t++) {
        double s = 0.0;
        for (int p = 0; p < k; p++) {
            size_t q = (size_t)t * k + p;
            if (!drop[q]) s = s + (double)weights[q] * dw[q];
        }
        if (!isfinite(s)) goto out;
        for (int p = 0; p < k; p++) {
            size_t q = (size_t)t * k + p;
            if (drop[q]) continue;
            if (ids[q] < 0 || ids[q] >= E) goto out;
            double v = (double)weights[q] * (dw[q] - s);
            if (!isfinite(v)) goto out;
            dlog[q] = v;
            if (dLogits) dLogits[(size_t)t * E + ids[q]] = (float)v;
        }
    }
    /* 3 */
    for (int t = 0; t < T; t++) {
        int64_t es[2] = {0, 0};
        double dl[2] = {0.0, 0.0};
        int nk = 0;
        for (int p = 0; p < k && nk < 2; p++) {
            size_t q = (size_t)t * k + p;
            if (drop[q]) continue;
            es[nk] = ids[q];
            dl[nk] = dlog[q];
            nk++;
        }
        if (nk == 2 && es[0] > es[1]) {
            int64_t te = es[0];
            double td = dl[0];
            es[0] = es[1], dl[0] = dl[1];
            es[1] = te, dl[1] = td;
        }
        for (int j = 0; j < n; j++) {
            double acc = 0.0;
            for (int a = 0; a < nk; a++)
                acc = acc + dl[a] * (double)Wgate[(size_t)es[a] * n + j];
            dx[(size_t)t * n + j] = dx[(size_t)t * n + j] + acc;
        }
    }
    /* 4 */
    for (size_t q = 0; q < Tk; q++) {
        if (drop[q]) continue;
        const float *xt = X + q / k * n;
        float *rg = dWgate + (size_t)ids[q] * n;
        for (int j = 0; j < n; j++) rg[j] = rg[j] + (float)(dlog[q] * (double)xt[j]);
    }
    /* 5 */
    size_t maxMe = 0;
    for (int e = 0; e < E; e++) {
        int64_t me = off[e + 1] - off[e];
        if (me < 0 || me > INT32_MAX) goto out;
        if ((size_t)me > maxMe) maxMe = (size_t)me;
    }
    size_t rows = maxMe > (size_t)T ? maxMe : (size_t)T;
    rc = RC_NOMEM;
    Xe = malloc(rows * n * sizeof(float));
    Dye = malloc(rows * n * sizeof(float));
    Ge = malloc(rows * h * sizeof(float));
    Ue = malloc(rows * h * sizeof(float));
    dxe = malloc(rows * n * sizeof(float));
    if (!Xe || !Dye || !Ge || !Ue || !dxe) goto out;
    rc = RC_INVAL;
    for (int e = 0; e < E; e++) {
        const size_t b0 = (size_t)off[e];
        const int Me = (int)(off[e + 1] - off[e]);
        if (Me == 0) continue;
        for (int m = 0; m < Me; m++) {
            int64_t q = perm[b0 + m];
            if (q < 0 || (size_t)q >= Tk || drop[q]) goto out;
            const size_t t = (size_t)q / k;
            const double w = (double)weights[q];
            memcpy(Xe + (size_t)m * n, X + t * n, n * sizeof(float));
            memcpy(Ge + (size_t)m * h, Gsel + (size_t)q * h, h * sizeof(float));
            memcpy(Ue + (size_t)m * h, Usel + (size_t)q * h, h * sizeof(float));
            for (int j = 0; j < n; j++)
                Dye[(size_t)m * n + j] = (float)(w * (double)dY[t * n + j]);
        }
        int r = expert_bwd(Xe, Dye, Ge, Ue, (size_t)h, Wg + e * nh, Wu + e * nh,
                           Wd + e * nh, Me, n, h, dxe, dWg + e * nh, dWu + e * nh,
                           dWd + e * nh);
        if (r != RC_OK) {
            rc = r;
            goto out;
        }
        for (int m = 0; m < Me; m++) {
            double *xa = dx + (size_t)perm[b0 + m] / k * n;
            for (int j = 0; j < n; j++)
                xa[j] = xa[j] + (double)dxe[(size_t)m * n + j];
        }
    }
    /* 6 */
    for (int s = 0; s < S; s++) {
        int r = expert_bwd(X, dY, Gs + (size_t)s * h, Us + (size_t)s * h,
                           (size_t)S * h, Wg_s + s * nh, Wu_s + s * nh,
                           Wd_s + s * nh, T, n, h, dxe, dWg_s + s * nh,
                           dWu_s + s * nh, dWd_s + s * nh);
        if (r != RC_OK) {
            rc = r;
            goto out;
        }
        for (size_t i = 0; i < Tn; i++) dx[i] = dx[i] + (double)dxe[i];
    }
    /* 7 */
    for (size_t i = 0; i < Tn; i++)
        if (!isfinite(dx[i])) goto out;
    for (size_t i = 0; i < Tn; i++) dX[i] = (float)dx[i];
    rc = RC_OK;
out:
    free(dx);
    free(dw);
    free(dlog);
    free(Xe);
    free(Dye);
    free(Ge);
    free(Ue);
    free(dxe);
    return rc;
}

/* ===================== GDN-2 ===================== */

static int gdn2_dims_ok(int dk, int dv) {
    return dk > 0 && dv > 0 && dk <= 1024 && dv <= 1024;
}

int or_gdn2_l2norm(const float *x, float *y, int n, float eps) {
    if (!x || !y || n <= 0 || n > 1024 || !(eps > 0.0f)) return RC_INVAL;
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
    const double nrm = sqrt(ss);
    if (nrm < (double)eps) {
        for (int i = 0; i < n; i++) y[i] = 0.0f;
        return RC_OK;
    }
    const float inv = (float)(1.0 / nrm);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv;
    return RC_OK;
}

/* the inputs of a decode step / prefill chunk are finite and alpha in [0,1] */
static int gdn2_inputs_ok(const float *q, const float *k, const float *b,
                          const float *alpha, size_t nk, const float *v,
                          const float *w, size_t nv) {
    if (!all_finite_f(q, nk) || !all_finite_f(k, nk) || !all_finite_f(b, nk) ||
        !all_finite_f(alpha, nk) || !all_finite_f(v, nv) || !all_finite_f(w, nv))
        return 0;
    for (size_t i = 0; i < nk; i++)
        if (!(alpha[i] >= 0.0f && alpha[i] <= 1.0f)) return 0;
    return 1;
}

int or_gdn2_decode_step(float *S, float *o, const float *q, const float *k,
                        const float *v, const float *b, const float *w,
                        const float *alpha, int dk, int dv) {
    if (!S || !o || !q || !k || !v || !b || !w || !alpha) return RC_INVAL;
    if (!gdn2_dims_ok(dk, dv)) return RC_INVAL;
    if (!gdn2_inputs_ok(q, k, b, alpha, (size_t)dk, v, w, (size_t)dv)) return RC_INVAL;
    float *buf = malloc((2 * (size_t)dk + 2 * (size_t)dv) * sizeof(float));
    if (!buf) return RC_NOMEM;
    float *qn = buf, *kn = qn + dk, *c = kn + dk, *vw = c + dv;
    or_gdn2_l2norm(q, qn, dk, 1e-6f);
    or_gdn2_l2norm(k, kn, dk, 1e-6f);
    /* pass 1 (one sweep of S): decay each row, then c += (b*kn)_i * row */
    for (int j = 0; j < dv; j++) c[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        float *row = S + (size_t)i * dv;
        const float ke = b[i] * kn[i];
        for (int j = 0; j < dv; j++) row[j] = row[j] * alpha[i];
        for (int j = 0; j < dv; j++) c[j] = c[j] + ke * row[j];
    }
    for (int j = 0; j < dv; j++) vw[j] = w[j] * v[j];
    /* pass 2: erase, write, read out */
    for (int j = 0; j < dv; j++) o[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        float *row = S + (size_t)i * dv;
        for (int j = 0; j < dv; j++) row[j] = row[j] - kn[i] * c[j];
        for (int j = 0; j < dv; j++) row[j] = row[j] + kn[i] * vw[j];
        for (int j = 0; j < dv; j++) o[j] = o[j] + qn[i] * row[j];
    }
    free(buf);
    return RC_OK;
}

/* sum over i of (x[i]*d[i])*y[i] in four chains over i % 4 for
 * i < dk & ~3, the tail into chain 0, then (s0+s1)+(s2+s3)
 * (src/gdn2.c:584-599, 702-713) */
static float gdn2_dot3(const float *x, const float *d, const float *y, int dk) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 3 < dk; i += 4)
        for (int l = 0; l < 4; l++) s[l] = s[l] + (x[i + l] * d[i + l]) * y[i + l];
    for (; i < dk; i++) s[0] = s[0] + (x[i] * d[i]) * y[i];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

int or_gdn2_prefill_chunk(float *S, float *Out, const float *Q,
                          const float *K, const float *V, const float *B,
                          const float *W, const float *Alpha, int dk, int dv,
                          int C) {
    if (!S || !Out || !Q || !K || !V || !B || !W || !Alpha) return RC_INVAL;
    if ((C != 16 && C != 32) || !gdn2_dims_ok(dk, dv)) return RC_INVAL;
    const size_t Ck = (size_t)C * dk, Cv = (size_t)C * dv;
    if (!gdn2_inputs_ok(Q, K, B, Alpha, Ck, V, W, Cv)) return RC_INVAL;
    float *buf = malloc((4 * Ck + 2 * Cv + (size_t)C * C + 2 * (size_t)dk) * sizeof(float));
    if (!buf) return RC_NOMEM;
    float *Qn = buf, *Kn = Qn + Ck, *KE = Kn + Ck, *Wg = KE + Ck;
    float *U = Wg + Ck, *G = U + Cv, *LP = G + Cv, *cum = LP + (size_t)C * C;
    float *cf = cum + dk;
    for (int t = 0; t < C; t++) {
        or_gdn2_l2norm(Q + (size_t)t * dk, Qn + (size_t)t * dk, dk, 1e-6f);
        or_gdn2_l2norm(K + (size_t)t * dk, Kn + (size_t)t * dk, dk, 1e-6f);
    }
    for (size_t n = 0; n < Ck; n++) KE[n] = B[n] * Kn[n];
    for (size_t n = 0; n < Cv; n++) U[n] = W[n] * V[n];
    /* L[t][s] (t > s) = (ke_t * cum(t,s)) . k_s, cum(t,s) = alpha_{s+1..t} */
    for (int s = 0; s < C; s++) {
        for (int i = 0; i < dk; i++) cum[i] = 1.0f;
        for (int t = s + 1; t < C; t++) {
            for (int i = 0; i < dk; i++) cum[i] = cum[i] * Alpha[(size_t)t * dk + i];
            LP[(size_t)t * C + s] =
                gdn2_dot3(KE + (size_t)t * dk, cum, Kn + (size_t)s * dk, dk);
        }
    }
    /* G_t = u_t - sum_i (ke_t * cumfwd(t))[i] S[i], cumfwd(t) = alpha_{0..t} */
    for (int i = 0; i < dk; i++) cum[i] = 1.0f;
    for (int t = 0; t < C; t++) {
        float *g = G + (size_t)t * dv;
        for (int i = 0; i < dk; i++) cum[i] = cum[i] * Alpha[(size_t)t * dk + i];
        for (int j = 0; j < dv; j++) g[j] = U[(size_t)t * dv + j];
        for (int i = 0; i < dk; i++) {
            const float wi = KE[(size_t)t * dk + i] * cum[i];
            for (int j = 0; j < dv; j++) g[j] = g[j] - wi * S[(size_t)i * dv + j];
        }
    }
    /* (I + L) E = G by forward substitution, in place */
    for (int t = 0; t < C; t++)
        for (int s = 0; s < t; s++) {
            const float l = LP[(size_t)t * C + s];
            for (int j = 0; j < dv; j++)
                G[(size_t)t * dv + j] = G[(size_t)t * dv + j] - l * G[(size_t)s * dv + j];
        }
    /* P[t][s] (s <= t) = (q_t * cum(t,s)) . k_s */
    for (int s = 0; s < C; s++) {
        for (int i = 0; i < dk; i++) cum[i] = 1.0f;
        for (int t = s; t < C; t++) {
            if (t != s)
                for (int i = 0; i < dk; i++) cum[i] = cum[i] * Alpha[(size_t)t * dk + i];
            LP[(size_t)t * C + s] =
                gdn2_dot3(Qn + (size_t)t * dk, cum, Kn + (size_t)s * dk, dk);
        }
    }
    /* Out_t = sum_i (q_t * cumfwd(t))[i] S[i] + sum_{s <= t} P[t][s] E_s */
    for (int i = 0; i < dk; i++) cum[i] = 1.0f;
    for (int t = 0; t < C; t++) {
        float *ot = Out + (size_t)t * dv;
        for (int i = 0; i < dk; i++) cum[i] = cum[i] * Alpha[(size_t)t * dk + i];
        for (int j = 0; j < dv; j++) ot[j] = 0.0f;
        for (int i = 0; i < dk; i++) {
            const float wi = Qn[(size_t)t * dk + i] * cum[i];
            for (int j = 0; j < dv; j++) ot[j] = ot[j] + wi * S[(size_t)i * dv + j];
        }
        for (int s = 0; s <= t; s++) {
            const float p = LP[(size_t)t * C + s];
            for (int j = 0; j < dv; j++) ot[j] = ot[j] + p * G[(size_t)s * dv + j];
        }
    }
    /* S <- cumfwd(C-1) * S + sum_s (k_s * suffix_s) E_s^T, suffix_s =
     * alpha_{s+1..C-1} accumulated from the end */
    for (int i = 0; i < dk; i++) cum[i] = 1.0f;
    for (int s = C - 1; s >= 0; s--)
        for (int i = 0; i < dk; i++) {
            Wg[(size_t)s * dk + i] = Kn[(size_t)s * dk + i] * cum[i];
            cum[i] = cum[i] * Alpha[(size_t)s * dk + i];
        }
    for (int i = 0; i < dk; i++) cf[i] = 1.0f;
    for (int t = 0; t < C; t++)
        for (int i = 0; i < dk; i++) cf[i] = cf[i] * Alpha[(size_t)t * dk + i];
    for (int i = 0; i < dk; i++) {
        float *row = S + (size_t)i * dv;
        for (int j = 0; j < dv; j++) row[j] = row[j] * cf[i];
        for (int s = 0; s < C; s++) {
            const float wv = Wg[(size_t)s * dk + i];
            for (int j = 0; j < dv; j++) row[j] = row[j] + wv * G[(size_t)s * dv + j];
        }
    }
    free(buf);
    return RC_OK;
}
