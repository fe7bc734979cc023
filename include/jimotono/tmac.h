#pragma once
#ifndef JIMOTONO_TMAC_H
#define JIMOTONO_TMAC_H
/*
 * T-MAC activation lookup tables (the reference's low-bit GEMM core) on the
 * MI355X. Drop-in for the reference's include/jimotono/tmac.h.
 *
 * Layout (identical to the reference, tmac.h:19-27):
 *   act    [N][K] float
 *   qlut   [N][K/4][8] int8: entry i of group g is the quantised value of
 *          pattern p = 8+i (bit j of p selects +a_j, otherwise -a_j);
 *          patterns p < 8 are recovered as -qlut[7-p]
 *   scales, biases [N][K/32] float, one pair per 32 activations
 *   idx    [bits][K/4] uint8, low nibble = 4-bit pattern of weight bit-plane b
 */
#include <stddef.h>
#include <stdint.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

#define JT_TMAC_G 4
#define JT_TMAC_LUT_HALF 8
#define JT_TMAC_LUT_FULL 16
#define JT_TMAC_ACT_GROUP 32
#define JT_TMAC_ALIGN 64

/* Byte sizes of the table and of one parameter array (scales or biases).
 * Reference: tmac.h:53-54, src/tmac.c:168-228. */
int jt_tmac_qlut_bytes(size_t n, size_t k, size_t *JT_RESTRICT out);
int jt_tmac_param_bytes(size_t n, size_t k, size_t *JT_RESTRICT out);

/* Build the quantised tables for act[N][K]. Reference: tmac.h:59-60,
 * src/tmac.c:230-385. */
int jt_tmac_lut_ctor(const float *JT_RESTRICT act, size_t n, size_t k, int8_t *JT_RESTRICT qlut,
                     float *JT_RESTRICT scales, float *JT_RESTRICT biases);

/* One dot product from one row's tables and one column's bit-planes.
 * Reference: tmac.h:69-72, src/tmac.c:387-506. */
int jt_tmac_lookup_accum(const int8_t *JT_RESTRICT qlut, const uint8_t *JT_RESTRICT idx,
                         const float *JT_RESTRICT scales, const float *JT_RESTRICT biases,
                         size_t ngroups, size_t nblocks, int bits,
                         float w_scale, float *JT_RESTRICT out);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_TMAC_H */
