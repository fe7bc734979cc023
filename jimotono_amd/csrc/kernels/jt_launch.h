/*
 * Launchers of the gfx950 kernels, callable from the C11 host layer.
 * Each returns the hipError_t of the launch (0 = success). Pointers are
 * device pointers; `err` is the library's device error word (EF_* bits).
 */
#ifndef JT_LAUNCH_H
#define JT_LAUNCH_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* noalloc.hip: a fixed device scratch array of JT_SCRATCH_BYTES per device,
 * for entry points that must not allocate. jtk_scratch_init looks up the
 * current device's address of the array once (at the library's set-up);
 * jtk_scratch returns it (NULL before the set-up on that device). */
#define JT_SCRATCH_BYTES ((size_t)16 << 20)
int jtk_scratch_init(void);
void *jtk_scratch(void);
/* p[0..n) = 0 (a fill kernel whose code object is loaded at set-up) */
int jtk_scratch_zero(uint32_t *p, int64_t n, hipStream_t s);
/* Load every code object of the library on the current device, so that no
 * later launch makes the runtime load one (and allocate device memory). */
int jtk_preload(void);

/* quant.hip */
int jtk_quant_rows(const float *X, int64_t rows, int cols, int8_t *Q, int64_t ldq,
                   float *scale, const int32_t *row_count, uint32_t *err, hipStream_t s);
int jtk_quant_tensor(const float *x, int64_t n, int8_t *q, float *scale,
                     uint32_t *amax_scratch, uint32_t *err, hipStream_t s);
int jtk_fakequant(const float *x, int64_t rows, int64_t cols, float *d,
                  uint32_t *amax_scratch, uint32_t *err, hipStream_t s);
int jtk_dequant(const int8_t *q, const float *scale, int64_t rows, int64_t cols,
                int per_row, float *d, uint32_t *err, hipStream_t s);
int jtk_check_q(const int8_t *q, int64_t n, uint32_t *err, hipStream_t s);
int jtk_check_finite(const float *x, int64_t n, uint32_t *err, hipStream_t s);
int jtk_pack_i8(const int8_t *Q, int N, int K, int kn, int Np, int Kp, int8_t *P,
                hipStream_t s);
int jtk_unpack_i8_kn(const int8_t *P, int N, int K, int Kp, int8_t *Q, hipStream_t s);
int jtk_pack_lowbit(const float *W0, const float *W1, int64_t w_estride, int64_t ld_n,
                    int64_t ld_k, int E, int N, int K, int bits, uint8_t *P, uint16_t *S,
                    uint8_t *codes_out, uint16_t *scales_out, uint32_t *err, hipStream_t s);
int jtk_interleave_rows(const void *A, const void *B, int h, int64_t row_bytes, void *D,
                        hipStream_t s);
int jtk_quant_weight_rows(const float *W, int64_t ld_n, int64_t ld_k, int N, int K,
                          int8_t *Q, float *scale, uint32_t *err, hipStream_t s);
/* W8A8 quantisation of every expert at once (experts with off[e + 1] ==
 * off[e] skipped): the rows of A [row][cols] listed by the 16-row tile
 * list, per tensor per expert (amax: nexp words, zeroed here) into Q
 * [row][Kp] and sA [row]; and each expert's weights W [E][N][K] per output
 * row (kn = 0; sBc [E][N]) or W [E][K][N] per tensor (kn = 1; sBc [E][Np],
 * amax: E words) through the codes Q [E][N*K] into the panels P [E][Np*Kp] */
int jtk_quant_tiles(const float *A, int cols, const int32_t *tiles, const int32_t *ntiles,
                    int max_tiles, uint32_t *amax, int nexp, int8_t *Q, int Kp, float *sA,
                    uint32_t *err, hipStream_t s);
int jtk_w8a8_weights_e(const float *W, int E, int N, int K, int kn, const int32_t *off,
                       int8_t *Q, int Np, int Kp, int8_t *P, float *sBc, uint32_t *amax,
                       uint32_t *err, hipStream_t s);
/* every expert's W8A8 GEMM over the 16-row tile list: C [row][ldc] = A
 * [row][lda] (codes, row scales sA) x the tile's expert's panels
 * P + e pstride (column scales sB + e sbstride) */
int jtk_w8a8_gemm_tiles(const int8_t *A, int lda, const float *sA, const int8_t *P,
                        int64_t pstride, const float *sB, int64_t sbstride, int N, int Np,
                        int Kp, int K, float *C, int ldc, const int32_t *tiles,
                        const int32_t *ntiles, int max_tiles, uint32_t *err, hipStream_t s);

/* gemm_i8.hip */
int jtk_w8a8_gemm(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                  const float *sB, int M, int N, int Np, int Kp, float *C, int ldc,
                  int swiglu, uint32_t *err, hipStream_t s);
/* jtk_w8a8_gemm with events for its duration: above 64 rows e0 / e1 carry
 * the tile kernel's own start and end timestamps; up to 64 rows they are
 * recorded before and after the launch. Either may be NULL. */
int jtk_w8a8_gemm_ev(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                     const float *sB, int M, int N, int Np, int Kp, float *C, int ldc,
                     int swiglu, uint32_t *err, hipStream_t s, hipEvent_t e0, hipEvent_t e1);
/* The SwiGLU GEMM of several experts whose interleaved gate/up panels are
 * concatenated along N (each expert 2*hpl channels, N % 256 == 0): hidden
 * column x of row m goes to C[(x / hpl) * plane + m * ldc + x % hpl], one
 * plane per expert. M > 64 only (128 x 256 tiles); hipErrorInvalidValue
 * (nothing launched) otherwise. e0 / e1 as in jtk_w8a8_gemm_ev. */
int jtk_w8a8_swiglu_planes(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                           const float *sB, int M, int N, int Kp, float *C, int ldc, int hpl,
                           int64_t plane, uint32_t *err, hipStream_t s, hipEvent_t e0,
                           hipEvent_t e1);
/* nb plain W8A8 GEMMs of M > 64 rows in one launch (128 x 128 tiles with a
 * k-split; blockIdx.y = GEMM b): GEMM b reads A + b*sAq (bytes), sA + b*ssA,
 * panels Wp + b*sW (bytes), sB + b*ssB and writes C + b*sC (floats).
 * hipErrorInvalidValue (nothing launched) for M <= 64 or Np % 128 != 0. */
int jtk_w8a8_gemm_batch(const int8_t *A, int lda, int64_t sAq, const float *sA, int ssA,
                        const int8_t *Wp, int64_t sW, const float *sB, int ssB, int M, int N,
                        int Np, int Kp, float *C, int ldc, int64_t sC, int nb, uint32_t *err,
                        hipStream_t s, hipEvent_t e0, hipEvent_t e1);
/* The skinny SwiGLU GEMM (M <= 16) over concatenated gate/up panels with
 * the hidden columns sent to hpl-wide planes, as jtk_w8a8_swiglu_planes. */
int jtk_w8a8_skinny_swiglu_planes(const int8_t *A, int lda, const float *sA, const int8_t *Wp,
                                  const float *sB, int M, int N, int Kp, float *C, int ldc,
                                  int hpl, int64_t plane, uint32_t *err, hipStream_t s);
/* nb plain jtk_w8a8_gemm_xq GEMMs in one launch: GEMM b reads X + b*sX
 * (floats), weight panels Wp + b*sW (bytes), sB + b*ssB and writes
 * C + b*sC (floats). hipErrorInvalidValue under jtk_w8a8_gemm_xq's limits
 * or when sX is not a multiple of 4. */
int jtk_w8a8_gemm_xq_batch(const float *X, int ldx, int K, int64_t sX, const int8_t *Wp,
                           int64_t sW, const float *sB, int ssB, int M, int N, int Np, int Kp,
                           float *C, int ldc, int64_t sC, int nb, uint32_t *err, hipStream_t s);
/* M <= 16 on fp32 activations X [M][ldx] (K valid columns): each block
 * quantises the rows itself with the row quantiser's arithmetic.
 * hipErrorInvalidValue (nothing launched) unless K % 4 == 0, K <= 4096
 * (3072 with SwiGLU), ldx % 4 == 0 and X is 16-byte aligned */
int jtk_w8a8_gemm_xq(const float *X, int ldx, int K, const int8_t *Wp, const float *sB, int M,
                     int N, int Np, int Kp, float *C, int ldc, int swiglu, uint32_t *err,
                     hipStream_t s);
/* 64-row tiles, f = h in {256, 512}: gate/up, SwiGLU and the row codes of
 * the hidden rows in one launch (Sq [Tk][h] int8, ss [Tk]); hipErrorInvalidValue
 * for other shapes */
int jtk_lowbit_gateup_q(const int8_t *A, int lda, const float *sA, const int32_t *perm,
                        int topk, const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                        const uint8_t *Wp, const uint16_t *Ws, int64_t wp_stride,
                        int64_t ws_stride, int K, int8_t *Sq, float *ss, int h, uint32_t *err,
                        hipStream_t s);
/* rows_per_tile 64 (batches) or 16 (few rows per expert) */
int jtk_lowbit_grouped(int bits, const int8_t *A, int lda, const float *sA,
                       const int32_t *perm, const int32_t *off, int topk,
                       const int32_t *tiles, const int32_t *ntiles, int max_tiles,
                       int rows_per_tile, const uint8_t *Wp, const uint16_t *Ws,
                       int64_t wp_stride, int64_t ws_stride, int N, int K, float *out, int ldo,
                       uint32_t *err, hipStream_t s);

/* the routed FFN of 16-row tiles (h = 256, n = 256..1024 in steps of 256;
 * hipErrorInvalidValue for other shapes): with S == NULL one block per tile
 * in one launch; with S (fp32 hidden rows, [sorted row][256]) four blocks per
 * tile in each of two launches (same results) */
int jtk_routed_ffn16(const int8_t *Xq, const float *sx, const int32_t *perm,
                     const int32_t *tiles, const int32_t *ntiles, int max_tiles, int topk,
                     const uint8_t *guP, const uint16_t *guS, int64_t gu_pstride,
                     int64_t gu_sstride, const uint8_t *dnP, const uint16_t *dnS,
                     int64_t dn_pstride, int64_t dn_sstride, int n, int h, float *Ye,
                     int8_t *Hq, float *Hs, float *S, uint32_t *err, hipStream_t s);
/* the caller-routed decode's routed FFN from the caller's ids: the outputs
 * of jtk_quant_sort_small (cap = T*topk, R = 16, no drop flags) and then of
 * jtk_routed_ffn16 with S, in two launches (the token codes and the sort
 * ride in the gate/up launch); Tk = T*topk <= 256, E <= 1024, h = 256, n =
 * 256..1024 in steps of 256, X 16-byte aligned, else hipErrorInvalidValue
 * before any launch */
int jtk_routed_ffn16_sort(const float *X, int T, int8_t *Xq, float *sx, const int32_t *ids,
                          int Tk, int E, int32_t *off, int32_t *perm, int32_t *tiles,
                          int32_t *ntiles, int topk, const uint8_t *guP, const uint16_t *guS,
                          int64_t gu_pstride, int64_t gu_sstride, const uint8_t *dnP,
                          const uint16_t *dnS, int64_t dn_pstride, int64_t dn_sstride, int n,
                          int h, float *Ye, int8_t *Hq, float *Hs, float *S, uint32_t *err,
                          hipStream_t s);
/* decode launches that carry the shared experts' blocks: top-k of T <= 16
 * rows (E <= 1024, k <= 64) and the pair sort / tile list (as
 * jtk_sort_small with cap = T*k; `done` is a zeroed device word the launch
 * leaves zeroed) beside the concatenated SwiGLU gate/up panels (as
 * jtk_w8a8_skinny_swiglu_planes), and the routed FFN of 16-row tiles (as
 * jtk_routed_ffn16) beside the batched down projections (as
 * jtk_w8a8_gemm_xq_batch, Kp <= 3072); hipErrorInvalidValue for other
 * shapes */
int jtk_decode_route_shared_gu(const float *logits, int T, int E, int k, int32_t *ids,
                               float *w, int R, int32_t *off, int32_t *perm, int32_t *tiles,
                               int32_t *ntiles, uint32_t *done, const int8_t *Xq, int ldx,
                               const float *sx, const int8_t *Wp, const float *sB, int N, int Kp,
                               float *C, int ldc, int hpl, int64_t plane, uint32_t *err,
                               hipStream_t s);
int jtk_decode_ffn16_shared_down(
    const int8_t *Xq, const float *sx, const int32_t *perm, const int32_t *tiles,
    const int32_t *ntiles, int max_tiles, int topk, const uint8_t *guP, const uint16_t *guS,
    int64_t gu_pstride, int64_t gu_sstride, const uint8_t *dnP, const uint16_t *dnS,
    int64_t dn_pstride, int64_t dn_sstride, int n, int h, float *Ye, int8_t *Hq, float *Hs,
    const float *H, int ldh, int K, int64_t sH, int T, const int8_t *Wd, int64_t sW,
    const float *sBd, int ssB, int Np, int Kp, float *Ys, int ldy, int64_t sY, int nb,
    uint32_t *err, hipStream_t s);

/* router.hip: int8 MFMA candidates + exact fp64 verification of the gate */
int jtk_router_codes(const float *X, int rows, int n, int8_t *qh, int8_t *ql, float *sf,
                     double *info, uint32_t *err, hipStream_t s);
int jtk_router_approx(const int8_t *Xh, const int8_t *Xl, int n, const double *xinfo,
                      const int8_t *Wh, const int8_t *Wl, const double *winfo, int T, int E,
                      double *approx, hipStream_t s);
/* jtk_router_codes, jtk_router_approx and the candidate selection of
 * jtk_topk_verify (stage 1) in one launch, for E <= 256 with E % 16 == 0 and
 * n in {256, 512, 1024}: writes qh, sf, info, the candidate lists and the
 * non-candidates' logits as those three do (the residual codes and the
 * approximate logits stay on chip). hipErrorInvalidValue (nothing launched)
 * for another shape. */
int jtk_router_front(const float *X, int T, int n, int8_t *qh, float *sf, double *info,
                     const int8_t *Wh, const int8_t *Wl, const double *winfo, int E, int k,
                     int16_t *cand, int32_t *ncand, float *logits, uint32_t *err, hipStream_t s);
/* T <= 16: every logit exact in fp64 (all T x E), plus the tokens' int8
 * codes and scales; n % 256 == 0 */
int jtk_router_logits_small(const float *X, const float *Wg, int T, int E, int n,
                            float *logits, int8_t *Xq, float *sx, uint32_t *err, hipStream_t s);
/* stages: bit 0 the candidate selection, bit 1 the exact logits and top-k
 * (3: both; T <= 256 runs both in one launch, with bit 1) */
int jtk_topk_verify(const double *approx, const double *xinfo, const double *winfo,
                    const float *X, const float *Wg, int T, int E, int n, int k, int16_t *cand,
                    int32_t *ncand, int32_t *ids, float *w, float *logits, uint32_t *err,
                    int stages, hipStream_t s);

/* route.hip */
int jtk_router_logits(const float *X, const float *Wg, int T, int E, int n, float *logits,
                      uint32_t *err, hipStream_t s);
/* one row of any length n < 2^31 and any k <= n (one block; the legacy
 * jt_routing_topk beyond the wavefront kernel's n <= 4096, k <= 64) */
int jtk_topk_block(const float *logits, int64_t n, int64_t k, int64_t *ids64, float *w,
                   uint32_t *err, hipStream_t s);
int jtk_topk(const float *logits, int rows, int E, int k, int32_t *ids, int64_t *ids64,
             float *w, uint32_t *err, hipStream_t s);
int jtk_sort(const int32_t *ids, int Tk, int E, int64_t cap, int32_t *rank, int32_t *cnt,
             int32_t *tot, int32_t *off, int64_t *off64, int32_t *perm, int64_t *perm64,
             uint8_t *drop, uint32_t *err, hipStream_t s);
/* tiles: int4 {expert, first sorted row, rows, 0} per R-row tile */
int jtk_make_tiles(const int32_t *off, int E, int R, int32_t *tiles, int32_t *ntiles,
                   hipStream_t s);
/* one-launch sort + R-row tile list for Tk <= 1024 pairs and E <= 4096 */
int jtk_sort_small(const int32_t *ids, int Tk, int E, int64_t cap, int R, int32_t *off,
                   int64_t *off64, int32_t *perm, int64_t *perm64, uint8_t *drop,
                   int32_t *tiles, int32_t *ntiles, uint32_t *err, hipStream_t s);
/* the T token rows' codes (k_quant_rows) and k_sort_small's sort of the
 * caller's ids in one launch (Tk <= 1024, E <= SORT_EMAX) */
int jtk_quant_sort_small(const float *X, int T, int n, int8_t *Xq, float *sx,
                         const int32_t *ids, int Tk, int E, int64_t cap, int R, int32_t *off,
                         int64_t *off64, int32_t *perm, int64_t *perm64, uint8_t *drop,
                         int32_t *tiles, int32_t *ntiles, uint32_t *err, hipStream_t s);
int jtk_sort_mid(const int32_t *ids, int Tk, int E, int64_t cap, int R, int32_t *rank,
                 int32_t *cnt, int32_t *off, int64_t *off64, int32_t *perm, int64_t *perm64,
                 uint8_t *drop, int32_t *tiles, int32_t *ntiles, uint32_t *err, hipStream_t s);
/* R: optional residual [T][n] (may alias Y): Y = (float)((double)R + (double)(float)sum) */
int jtk_combine(const float *w, const float *Ye, const uint8_t *drop, const float *Ys,
                int S, int T, int k, int n, const float *R, float *Y, uint32_t *err,
                hipStream_t s);
int jtk_renorm(float *w, const uint8_t *drop, int T, int k, uint32_t *err, hipStream_t s);
int jtk_gather_rows(const float *src, int n, const int32_t *perm, int base, int div,
                    int rows, float *dst, hipStream_t s);
int jtk_scatter_rows(const float *src, int n, const int32_t *perm, int base, int rows,
                     float *dst, hipStream_t s);
int jtk_silu_tile(const float *G, const float *U, int64_t n, float *S, uint32_t *err,
                  hipStream_t s);
/* the drop-in layer's expert FFN in fp32 (flags off) for every expert at
 * once: routed (dense = 0: the R = 16 tile list over the sorted pairs, Y
 * scattered to Y[perm[pos]]) or the nexp shared experts (dense = 1: T rows
 * each, S and Y as [nexp][T][.]); Gc/Uc optional caches ([pair][h] or
 * [token][nexp][h]) */
int jtk_ffn_f32(const float *X, int T, int n, int h, const int32_t *perm, int topk,
                const int32_t *tiles, const int32_t *ntiles, int max_tiles, const float *Wg,
                const float *Wu, const float *Wd, int nexp, float *Gc, float *Uc, float *Sbuf,
                float *Y, int dense, uint32_t *err, hipStream_t s);
int jtk_zero_u32(uint32_t *p, int64_t n, hipStream_t s);
int jtk_bcast_f32(float *dst, int64_t n, const float *src, hipStream_t s);

/* legacy.hip */
int jtk_gemm_f32(const float *A, const float *B, float *C, int M, int N, int K,
                 uint32_t *err, hipStream_t s);
int jtk_transpose_f32(const float *src, float *dst, int rows, int cols, hipStream_t s);
int jtk_tmac_ctor(const float *act, int64_t n, int64_t k, int8_t *qlut, float *scales,
                  float *biases, uint32_t *err, hipStream_t s);
int jtk_col_to_idx(const float *W, int k, int h, int bits, float *ws, uint8_t *idx,
                   uint32_t *err, hipStream_t s);
int jtk_tmac_gemm(const int8_t *qlut, const float *sc, const float *bi, const double *rowsum,
                  const uint8_t *idx, const float *ws, int me, int h, int k, int bits,
                  float *Y, uint32_t *err, hipStream_t s);
int jtk_rowsum_f64(const float *X, int me, int k, double *rs, hipStream_t s);
int jtk_tmac_lookup1(const int8_t *qlut, const uint8_t *idx, const float *sc,
                     const float *bi, int64_t ng, int64_t nb, int bits, float w_scale,
                     float *out, uint32_t *err, hipStream_t s);
int jtk_gemm_f64acc(const float *A, const float *B, float *C, int M, int N, int K,
                    hipStream_t s);
int jtk_lowbit_fq_cols(float *W, int k, int h, int bits, float *ws, uint32_t *err,
                       hipStream_t s);
/* the same fake-quant per row of W [rows][cols] (ws: rows floats), and per
 * column of each of nb matrices [k][h] stored back to back (ws: nb * h
 * floats; nb <= 65535); with the expert offsets off (E + 1 entries; rpe
 * rows, or one matrix, per expert) the experts that hold no pair are left
 * as they are */
int jtk_lowbit_fq_rows(float *W, int64_t rows, int cols, const int32_t *off, int rpe, int bits,
                       float *ws, uint32_t *err, hipStream_t s);
int jtk_lowbit_fq_cols_batch(float *W, int nb, int k, int h, const int32_t *off, int bits,
                             float *ws, uint32_t *err, hipStream_t s);
/* the T-MAC LUT GEMM of every expert: the bit-plane indices and maxima of
 * the columns of each touched expert's matrix (element t of column j at
 * W[e estride + t tstride + j jstride]; idx [E][h][bits][k/4], ws [E][h]),
 * and the lookup GEMM of the sorted rows < off[E] with their experts'
 * columns (k % 32 == 0) */
int jtk_col_to_idx_e(const float *W, int E, int k, int h, int64_t estride, int64_t tstride,
                     int64_t jstride, const int32_t *off, int bits, float *ws, uint8_t *idx,
                     uint32_t *err, hipStream_t s);
int jtk_tmac_gemm_e(const int8_t *qlut, const float *sc, const float *bi, const double *rowsum,
                    const uint8_t *idx, const float *ws, const int32_t *off, int E, int rows,
                    int h, int k, int bits, float *Y, uint32_t *err, hipStream_t s);

/* moe_bwd.hip: batched MoE backward on the forward's permutation.
 * Device pointers in the reference's argument order (ids, perm, off as
 * size_t); dLogits and the shared arrays may be NULL (S == 0). */
typedef struct jtk_bwd_io {
    const float *dY, *X, *Wgate, *Wg, *Wu, *Wd, *Wg_s, *Wu_s, *Wd_s;
    const uint64_t *ids;
    const float *weights, *Gsel, *Usel, *Ysel, *Gs, *Us;
    const uint64_t *perm, *off;
    const uint8_t *drop;
    float *dX, *dWgate, *dWg, *dWu, *dWd, *dWg_s, *dWu_s, *dWd_s, *dLogits;
} jtk_bwd_io;
typedef struct jtk_bwd_ws {
    uint32_t *ctrl, *seen;
    int32_t *key, *inv, *rowq, *rank, *cnt, *tot, *off2, *perm2, *off32, *tiles, *ntiles;
    double *dw, *dlog, *gate_dl;
    int32_t *gate_e, *gate_n, *tokpos, *tokcnt;
    float *Xp, *dYp, *Dg, *Du, *Ss, *Dxe, *SDg, *SDu, *SSs, *SDxe;
} jtk_bwd_ws;
/* Bytes of the workspace; with base != NULL also fills *w with its pieces. */
size_t jtk_bwd_ws_layout(int T, int n, int h, int E, int k, int S, jtk_bwd_ws *w, char *base);
/* Enqueues the whole backward; returns nonzero when a launch failed. */
int jtk_bwd_batch(const jtk_bwd_io *io, int T, int n, int h, int E, int k, int S, int validate,
                  const jtk_bwd_ws *w, uint32_t *err, hipStream_t s);

/* gdn2.hip: Gated DeltaNet-2 decode step and prefill chunk over H heads.
 * Decode: S [H][dk][dv], O [H][dv], q/k/b/alpha [H][dk], v/w [H][dv].
 * Prefill: head h's rows of Q/K/B/A start at h*hk, of V/W/Out at h*hv. */
int jtk_gdn2_decode(float *S, float *O, const float *q, const float *k, const float *v,
                    const float *b, const float *w, const float *alpha, int H, int dk, int dv,
                    uint32_t *err, hipStream_t s);
size_t jtk_gdn2_prefill_ws_bytes(int H, int T, int C, int dk);
/* T tokens per head (T % C == 0) in T/C chunks; a head with a bad input
 * value anywhere keeps its S and Out (EF_NONFINITE_INPUT). */
int jtk_gdn2_prefill(float *S, float *Out, const float *Q, const float *K, const float *V,
                     const float *B, const float *W, const float *A, int64_t hk, int64_t hv,
                     int H, int T, int C, int dk, int dv, float *ws, uint32_t *err,
                     hipStream_t s);
int jtk_gdn2_l2norm(const float *x, float *y, int rows, int n, float eps, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* JT_LAUNCH_H */
