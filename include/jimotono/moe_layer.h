#pragma once
#ifndef JIMOTONO_MOE_LAYER_H
#define JIMOTONO_MOE_LAYER_H
/*
 * Batched MoE layer forward and its expert sort, on the MI355X. Drop-in for
 * jt_moe_batch_sort / jt_moe_fwd_batch / jt_moe_fwd_batch_unchecked of the
 * reference's include/jimotono/moe_layer.h, with the same signatures and the
 * same process-wide switches: jt_w8a8_set_enabled(1) selects the W8A8 expert
 * GEMMs and jt_lowbit_set_mode(1|2) the low-bit routed GEMMs (low-bit wins
 * when both are on), exactly as the reference reads them
 * (src/moe_layer.c:1068-1071, 1301, 1333).
 *
 * These are host-pointer entry points: inputs are staged into HBM, every
 * stage (gate logits, top-k, sort, renormalisation, gather, expert GEMMs,
 * SwiGLU, combine, shared experts) runs as HIP kernels, and Y is copied back
 * only after the whole forward succeeded. The batched backward
 * (jt_moe_bwd_batch, jt_moe_bwd_batch_unchecked) runs the same way on the
 * forward's permutation. The single-token training helpers of the reference
 * (jt_moe_fwd, jt_moe_bwd, jt_moe_sticky_seq_loss) are not part of this
 * library.
 */
#include <stddef.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Reference moe_layer.h:52-54. */
#define JT_MOE_MAX_EXPERTS 4096
#define JT_MOE_MAX_TOPK 64
#define JT_MOE_MAX_SHARED 8

/* Stable counting sort of the T*k (token, slot) pairs by expert with
 * capacity cap = ceil(cap_factor*T*k/E), cap_factor in [1.0, 1.5]. perm holds
 * the kept flattened indices q = t*k+p grouped by expert (q ascending inside
 * an expert), off[E+1] the expert boundaries, drop[q] = 1 for pairs over
 * capacity. Reference: moe_layer.h:194-198, src/moe_layer.c:895-978. */
int jt_moe_batch_sort(const size_t *JT_RESTRICT ids, int T, int k, int E,
                      float cap_factor, size_t *JT_RESTRICT perm,
                      size_t *JT_RESTRICT off, unsigned char *JT_RESTRICT drop,
                      size_t *JT_RESTRICT out_kept,
                      size_t *JT_RESTRICT out_dropped);

/* Batched forward of T tokens. Shapes (row-major): X, Y [T][n];
 * Wgate [E][n]; Wg, Wu, Wd [E][h][n]; Wg_s, Wu_s, Wd_s [S][h][n];
 * out_ids/out_weights [T][k]; caches as in the reference (NULL allowed).
 * Reference: moe_layer.h:230-249, src/moe_layer.c:980-1614, 1616-1638. */
int jt_moe_fwd_batch(const float *JT_RESTRICT X, const float *JT_RESTRICT Wgate,
                     const float *JT_RESTRICT Wg, const float *JT_RESTRICT Wu,
                     const float *JT_RESTRICT Wd,
                     const float *JT_RESTRICT Wg_s,
                     const float *JT_RESTRICT Wu_s,
                     const float *JT_RESTRICT Wd_s, float *JT_RESTRICT Y,
                     int T, int n, int h, int n_experts, int topk,
                     int n_shared, size_t *JT_RESTRICT out_ids,
                     float *JT_RESTRICT out_weights,
                     float *JT_RESTRICT cache_Gsel,
                     float *JT_RESTRICT cache_Usel,
                     float *JT_RESTRICT cache_Ysel,
                     float *JT_RESTRICT cache_Gs, float *JT_RESTRICT cache_Us,
                     float cap_factor, size_t *JT_RESTRICT out_perm,
                     size_t *JT_RESTRICT out_off,
                     unsigned char *JT_RESTRICT out_drop,
                     size_t *JT_RESTRICT out_kept,
                     size_t *JT_RESTRICT out_dropped);

/* Same computation without the O(E*h*n) finiteness pre-scan of the weights.
 * Reference: moe_layer.h:252-275, src/moe_layer.c:1640-1663. */
int jt_moe_fwd_batch_unchecked(
    const float *JT_RESTRICT X, const float *JT_RESTRICT Wgate,
    const float *JT_RESTRICT Wg, const float *JT_RESTRICT Wu,
    const float *JT_RESTRICT Wd, const float *JT_RESTRICT Wg_s,
    const float *JT_RESTRICT Wu_s, const float *JT_RESTRICT Wd_s,
    float *JT_RESTRICT Y, int T, int n, int h, int n_experts, int topk,
    int n_shared, size_t *JT_RESTRICT out_ids, float *JT_RESTRICT out_weights,
    float *JT_RESTRICT cache_Gsel, float *JT_RESTRICT cache_Usel,
    float *JT_RESTRICT cache_Ysel, float *JT_RESTRICT cache_Gs,
    float *JT_RESTRICT cache_Us, float cap_factor,
    size_t *JT_RESTRICT out_perm, size_t *JT_RESTRICT out_off,
    unsigned char *JT_RESTRICT out_drop, size_t *JT_RESTRICT out_kept,
    size_t *JT_RESTRICT out_dropped);

/* Batched backward of T tokens on the forward's permutation (no re-sort).
 * dY, X [T][n]; weights as the forward; ids, weights [T][k]; caches Gsel,
 * Usel [T*k][h], Ysel [T*k][n], Gs, Us [T][S][h]; perm [kept], off [E+1],
 * drop [T*k] as the forward wrote them. Outputs (overwritten): dX [T][n],
 * dWgate [E][n], dWg/dWu/dWd [E][h][n], dWg_s/dWu_s/dWd_s [S][h][n],
 * dLogits [T][E] (NULL allowed). JT_OK, or JT_ERR_INVAL with errno EINVAL
 * and no output written. Reference: moe_layer.h:277-329,
 * src/moe_layer.c:1684-2467. */
int jt_moe_bwd_batch(const float *JT_RESTRICT dY, const float *JT_RESTRICT X,
                     const float *JT_RESTRICT Wgate, const float *JT_RESTRICT Wg,
                     const float *JT_RESTRICT Wu, const float *JT_RESTRICT Wd,
                     const float *JT_RESTRICT Wg_s, const float *JT_RESTRICT Wu_s,
                     const float *JT_RESTRICT Wd_s, const size_t *JT_RESTRICT ids,
                     const float *JT_RESTRICT weights, const float *JT_RESTRICT Gsel,
                     const float *JT_RESTRICT Usel, const float *JT_RESTRICT Ysel,
                     const float *JT_RESTRICT Gs, const float *JT_RESTRICT Us,
                     const size_t *JT_RESTRICT perm, const size_t *JT_RESTRICT off,
                     const unsigned char *JT_RESTRICT drop, float *JT_RESTRICT dX,
                     float *JT_RESTRICT dWgate, float *JT_RESTRICT dWg,
                     float *JT_RESTRICT dWu, float *JT_RESTRICT dWd,
                     float *JT_RESTRICT dWg_s, float *JT_RESTRICT dWu_s,
                     float *JT_RESTRICT dWd_s, float *JT_RESTRICT dLogits, int T, int n,
                     int h, int n_experts, int topk, int n_shared);

/* Same computation without the finiteness scans of the weights and caches
 * and without the weight-range test. The index checks the device kernels
 * depend on (ids < E for kept pairs, off monotone from 0 with
 * off[E] == kept, perm an exact enumeration of the kept pairs) still run;
 * a permutation written by the forward always passes them.
 * Reference: moe_layer.h:330-362, src/moe_layer.c:2469-2502. */
int jt_moe_bwd_batch_unchecked(
    const float *JT_RESTRICT dY, const float *JT_RESTRICT X, const float *JT_RESTRICT Wgate,
    const float *JT_RESTRICT Wg, const float *JT_RESTRICT Wu, const float *JT_RESTRICT Wd,
    const float *JT_RESTRICT Wg_s, const float *JT_RESTRICT Wu_s,
    const float *JT_RESTRICT Wd_s, const size_t *JT_RESTRICT ids,
    const float *JT_RESTRICT weights, const float *JT_RESTRICT Gsel,
    const float *JT_RESTRICT Usel, const float *JT_RESTRICT Ysel, const float *JT_RESTRICT Gs,
    const float *JT_RESTRICT Us, const size_t *JT_RESTRICT perm,
    const size_t *JT_RESTRICT off, const unsigned char *JT_RESTRICT drop,
    float *JT_RESTRICT dX, float *JT_RESTRICT dWgate, float *JT_RESTRICT dWg,
    float *JT_RESTRICT dWu, float *JT_RESTRICT dWd, float *JT_RESTRICT dWg_s,
    float *JT_RESTRICT dWu_s, float *JT_RESTRICT dWd_s, float *JT_RESTRICT dLogits, int T,
    int n, int h, int n_experts, int topk, int n_shared);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_MOE_LAYER_H */
