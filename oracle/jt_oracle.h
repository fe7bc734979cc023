/*
 * jt_oracle -- CPU restatement of the reference's quantised MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product library (jimotono_amd/libjimotono_hip.so) does not
 * link, load or call it.
 *
 * Every function restates one reference function (file:line given at each
 * declaration; paths are relative to the reference checkout) in plain C11,
 * scalar, compiled with -ffp-contract=off so every fp64 multiply and add
 * rounds separately, as in the reference build (CMakeLists.txt:14-24).
 * Functions that define the prepared-weight formats of the MI355X build
 * (or_lowbit_pack_rows, or_gemm_lowbit_group, or_moe_q_*) have no reference
 * counterpart as a whole; their pieces cite the reference arithmetic they
 * reuse.
 *
 * How each function is pinned (checked by tests/test_oracle_*.py) is listed
 * in the header of those tests; functions without such a check would say
 * "parity unpinned" here -- there are none.
 */
#ifndef JT_ORACLE_H
#define JT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------- W8A8 (src/w8a8.c) ---------- */

/* Per-tensor quantisation, src/w8a8.c:688-747. rc 0 ok, 2 invalid. */
int or_quant_row(const float *x, size_t n, int8_t *q, float *scale);
/* Per-row (per-channel) quantisation, src/w8a8.c:787-855. */
int or_quant_rows(const float *X, size_t rows, size_t cols, int8_t *Q,
                  float *scales);
/* dst = (float)((double)q * (double)scale[row]), src/w8a8.c:857-907
 * (rows == 1 gives the per-tensor form, src/w8a8.c:749-785). */
int or_dequant_rows(const int8_t *q, const float *scales, size_t rows,
                    size_t cols, float *dst);
/* Fake-quant per tensor (rows=1) or per row, src/w8a8.c:1074-1200. */
int or_fakequant_rows(const float *src, size_t rows, size_t cols, float *dst);
/* int8 GEMM with B in the reference layout Bq[K][N]:
 *   acc = sum_k Aq[m][k]*Bq[k][n] (int32),
 *   C = (float)((double)acc * ((double)sA_m * (double)sB_n)),
 * src/w8a8.c:654-686. sA has M entries if sA_rows, else 1; sB has N entries
 * if sB_cols, else 1. acc_out [M][N] may be NULL. rc 2 + flag on a
 * non-finite result (ERANGE case). */
int or_w8a8_gemm(const int8_t *Aq, const float *sA, int sA_rows,
                 const int8_t *Bq_kn, const float *sB, int sB_cols, float *C,
                 int32_t *acc_out, int M, int N, int K);

/* ---------- fp32 GEMM (src/moe_gemm.c) ---------- */
/* C[m][n] = fp32 sum over k ascending of A[m][k]*B[k][n], separate mul and
 * add, src/moe_gemm.c:47-61 (bit-identical to :68-89). */
void or_gemm_f32(const float *A, const float *B, float *C, int M, int N,
                 int K);

/* ---------- low-bit levels (src/lowbit.c) ---------- */
/* Level index li of w on the 2^bits grid with max-abs scale maxabs,
 * src/lowbit.c:78-86 (maxabs == 0 -> t = 0, src/lowbit.c:122). */
int or_lowbit_code(double w, double maxabs, int bits);
/* src/lowbit.c:47-91. */
int or_lowbit_fakequant(const float *w, float *fq, size_t n, int bits);
/* src/lowbit.c:93-141. */
int or_lowbit_col_to_idx(const float *col, size_t k, int bits, uint8_t *idx,
                         float *w_scale);

/* IEEE binary16 conversions, round to nearest even (no reference
 * counterpart; pinned against numpy.float16). */
uint16_t or_f64_to_f16(double x);
double or_f16_to_f64(uint16_t h);

/* Prepared low-bit format of the MI355X build: row r of W[N][K] (one output
 * channel) is cut into K/group groups; per group maxabs_g = max|w| (fp64),
 * codes[r][k] = or_lowbit_code(w, maxabs_g, bits),
 * scales[r][g] = f16(maxabs_g / (2^bits - 1)). K % group == 0. */
int or_lowbit_pack_rows(const float *W, int N, int K, int bits, int group,
                        uint8_t *codes, uint16_t *scales);

/* Grouped low-bit GEMM on prepared codes, C[M][N]:
 *   acc_g = sum_{k in g} Aq[m][k] * (2*codes[n][k] - (2^bits-1))   (int32)
 *   T     = fmaf((float)acc_g, f16(scales[n][g]), T), fp32, g ascending
 *           from T = 0 (one rounding per group; (float)acc_g is exact)
 *   C     = T * sA[m] (fp32)
 * acc_out [M][N][K/group] may be NULL. rc 2 on a non-finite C. */
int or_gemm_lowbit_group(const int8_t *Aq, const float *sA,
                         const uint8_t *codes, const uint16_t *scales,
                         int bits, int group, float *C, int32_t *acc_out,
                         int M, int N, int K);

/* ---------- T-MAC (src/tmac.c) ---------- */
int or_tmac_lut_ctor(const float *act, size_t n, size_t k, int8_t *qlut,
                     float *scales, float *biases); /* src/tmac.c:230-385 */
/* Scalar aggregation order of the default build (tmac.c has no -mavx2 in
 * CMakeLists.txt:73-81), src/tmac.c:387-506. */
int or_tmac_lookup_accum(const int8_t *qlut, const uint8_t *idx,
                         const float *scales, const float *biases,
                         size_t ngroups, size_t nblocks, int bits,
                         float w_scale, float *out);
/* src/lowbit.c:158-267 (fp64 fallback src/lowbit.c:144-156). */
int or_lowbit_gemm_lut(const float *X, const float *W, float *Y, int me, int h,
                       int k, int bits);

/* ---------- routing (src/routing.c, src/moe_layer.c) ---------- */
/* Gate logit in the reference's AVX2 order, src/moe_layer.c:67-86: four
 * fp64 lane partials over j % 4 (j < n & ~3), (l0+l1)+(l2+l3), then the tail
 * in order. Returns the fp64 sum (caller casts to float). */
double or_logit_lane4(const float *x, const float *w, int n);
/* src/routing.c:16-76. ids as int64 (size_t in the reference). */
int or_topk(const float *logits, size_t n, size_t k, int64_t *ids,
            float *weights);
int or_router(const float *X, const float *Wgate, int T, int E, int n, int k,
              int64_t *ids, float *w, float *logits);
/* src/moe_layer.c:895-978 with cap_factor in [1,1.5]; cap_factor <= 0
 * selects the dropless variant (cap = T*k). */
int or_batch_sort(const int64_t *ids, int T, int k, int E, float cap_factor,
                  int64_t *perm, int64_t *off, unsigned char *drop,
                  int64_t *out_kept);

/* ---------- SwiGLU (src/moe_layer.c:129-157) ---------- */
/* s = (float)((g * (1/(1+exp(-g)))) * u) in fp64; rc 2 if non-finite. */
int or_silu_mul(float g, float u, float *s);

/* ---------- legacy batched layer (src/moe_layer.c:980-1614) ----------
 * w8a8_on / lowbit_mode are the reference's process flags. caches may be
 * NULL. ids/perm/off as int64. Returns 0 or 2. */
int or_moe_fwd_batch(const float *X, const float *Wgate, const float *Wg,
                     const float *Wu, const float *Wd, const float *Wg_s,
                     const float *Wu_s, const float *Wd_s, float *Y, int T,
                     int n, int h, int E, int k, int S, int64_t *out_ids,
                     float *out_weights, float cap_factor, int64_t *out_perm,
                     int64_t *out_off, unsigned char *out_drop,
                     int64_t *out_kept, int w8a8_on, int lowbit_mode,
                     float *cache_Ysel);

/* ---------- batched backward (src/moe_layer.c:1684-2502) ----------
 * jt_moe_bwd_batch (validate = 1) / jt_moe_bwd_batch_unchecked
 * (validate = 0) on the forward's permutation. Shapes as in the reference
 * (moe_layer.h:276-330); ids/perm/off as int64. dLogits may be NULL; the
 * shared arrays may be NULL when S == 0. Returns 0 or 2 (EINVAL cases). On
 * 2 the outputs hold whatever the steps before the failure wrote. */
int or_moe_bwd_batch(const float *dY, const float *X, const float *Wgate,
                     const float *Wg, const float *Wu, const float *Wd,
                     const float *Wg_s, const float *Wu_s, const float *Wd_s,
                     const int64_t *ids, const float *weights,
                     const float *Gsel, const float *Usel, const float *Ysel,
                     const float *Gs, const float *Us, const int64_t *perm,
                     const int64_t *off, const unsigned char *drop, float *dX,
                     float *dWgate, float *dWg, float *dWu, float *dWd,
                     float *dWg_s, float *dWu_s, float *dWd_s, float *dLogits,
                     int T, int n, int h, int E, int k, int S, int validate);

/* ---------- GDN-2 linear attention (src/gdn2.c) ----------
 * State S [dk][dv] fp32 row-major; q, k, b, alpha [dk]; v, w [dv].
 * Returns 0 or 2 (EINVAL cases: dims outside 1..1024, non-finite inputs,
 * alpha outside [0,1]); on 2 nothing is written. */
/* y = x * (float)(1/sqrt(sum x^2 in fp64, i ascending)); y = 0 when the
 * norm is below eps. src/gdn2.c:219-250. */
int or_gdn2_l2norm(const float *x, float *y, int n, float eps);
/* One decode step (src/gdn2.c:252-405): S <- S*alpha (rows), c = (b*kn)^T S,
 * S <- S - kn c^T + kn (w*v)^T, o = S^T qn, fp32 in the reference's order. */
int or_gdn2_decode_step(float *S, float *o, const float *q, const float *k,
                        const float *v, const float *b, const float *w,
                        const float *alpha, int dk, int dv);
/* One prefill chunk of C = 16 or 32 tokens in the WY form
 * (src/gdn2.c:474-842): Q, K, B, Alpha [C][dk]; V, W, Out [C][dv]. */
int or_gdn2_prefill_chunk(float *S, float *Out, const float *Q,
                          const float *K, const float *V, const float *B,
                          const float *W, const float *Alpha, int dk, int dv,
                          int C);

/* ---------- prepared quantised layer (MI355X fast path) ---------- */
typedef struct or_moe_q {
    int n, h, E, k, S, hs, group;
    /* router, fp32 [E][n] (may be NULL for caller-routed use) */
    const float *Wgate;
    /* routed: gate/up codes [E][2][h][n] + scales [E][2][h][n/group],
     * down codes [E][n][h] + scales [E][n][h/group] */
    uint8_t *gu_codes;
    uint16_t *gu_scales;
    uint8_t *d_codes;
    uint16_t *d_scales;
    /* shared: int8 [S][2][hs][n] + scales [S][2][hs]; down int8
     * [S][n][hs] + scales [S][n] */
    int8_t *sgu_q;
    float *sgu_s;
    int8_t *sd_q;
    float *sd_s;
} or_moe_q;

/* Quantise fp32 reference-layout weights into the prepared format.
 * Wg, Wu, Wd [E][h][n]; Wg_s, Wu_s, Wd_s [S][hs][n]. Allocates the arrays
 * of L (free with or_moe_q_free). */
int or_moe_q_prepare(or_moe_q *L, int n, int h, int E, int k, int S, int hs,
                     int group, const float *Wgate, const float *Wg,
                     const float *Wu, const float *Wd, const float *Wg_s,
                     const float *Wu_s, const float *Wd_s);
void or_moe_q_free(or_moe_q *L);

/* Forward of the prepared layer for T tokens (see jimotono/hip_moe.h for
 * the semantics). ids_in/w_in select caller routing (both non-NULL), else
 * the router runs. Outputs ids/w [T][k], perm [T*k], off [E+1], Ye
 * [T*k][n], Ys [S][T][n] may be NULL. */
int or_moe_q_fwd(const or_moe_q *L, const float *X, int T,
                 const int32_t *ids_in, const float *w_in, float *Y,
                 int32_t *ids, float *w, int32_t *perm, int32_t *off,
                 float *Ye, float *Ys, int8_t *Hq, float *Hs);

/* Residual add after the layer, bench/kernel/train_tinystories.c:1147-1160:
 * Y = (float)((double)X + (double)Mo); rc 2 on a non-finite sum. */
int or_residual_add(const float *X, const float *Mo, float *Y, size_t n);

/* One W8A8 SwiGLU expert as used for the shared experts of or_moe_q_fwd:
 * Wg, Wu, Wd [h][n] fp32, prepared on the fly; Y [T][n]. */
int or_ffn_fwd(const float *Wg, const float *Wu, const float *Wd, int n,
               int h, const float *X, int T, float *Y);

#ifdef __cplusplus
}
#endif

#endif /* JT_ORACLE_H */
