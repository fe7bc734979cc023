#pragma once
#ifndef JIMOTONO_LOWBIT_H
#define JIMOTONO_LOWBIT_H
/*
 * Low-bit routed-expert weights (INT2 gate/up, INT4 down) on the MI355X.
 * Drop-in for the reference's include/jimotono/lowbit.h.
 *
 * Level grid (same as the reference, src/lowbit.c:42-45, 77-88): an n-level
 * (n = 2^bits) code li in [0, n-1] stands for (2*li - (n-1)) / (n-1) * maxabs,
 * li = clamp(floor(t*(n-1)/2 + (n-1)/2 + 0.5), 0, n-1), t = w / maxabs in fp64.
 *
 * jt_lowbit_gemm_lut keeps the reference's T-MAC arithmetic (int8 activation
 * lookup tables per 32 activations, bit-plane lookups, fp64 aggregation,
 * sign fix) and is bit-identical to it; it runs as HIP kernels. The fast
 * MoE path of this library does not use it (see jimotono/hip_moe.h).
 */
#include <stddef.h>
#include <stdint.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* 0 = fp32, 1 = fake-quant, 2 = true LUT. Reference: lowbit.h:30-31,
 * src/lowbit.c:16-29. */
int jt_lowbit_set_mode(int mode);
int jt_lowbit_get_mode(void);

/* is_down != 0 -> 4, else 2. Reference: lowbit.h:34, src/lowbit.c:31-39. */
int jt_lowbit_bits_for(int is_down, int *JT_RESTRICT out_bits);

/* Quantise-dequantise w[0..n) on the level grid with one max-abs scale.
 * Reference: lowbit.h:38-39, src/lowbit.c:47-91. */
int jt_lowbit_fakequant(const float *JT_RESTRICT w, float *JT_RESTRICT fq, size_t n, int bits);

/* One weight column col[k] -> bit-planes idx[bits][k/4] (low nibble j of
 * idx[b*ngroups+g] = bit b of the code of col[4g+j]) and w_scale = maxabs.
 * Reference: lowbit.h:43-44, src/lowbit.c:93-141. */
int jt_lowbit_col_to_idx(const float *JT_RESTRICT col, size_t k, int bits, uint8_t *JT_RESTRICT idx,
                         float *JT_RESTRICT w_scale);

/* Y[me][h] = X[me][k] * W[k][h] through the T-MAC lookup kernel; k % 32 != 0
 * falls back to an fp64-accumulated GEMM, me == 0 is a no-op.
 * Reference: lowbit.h:52-53, src/lowbit.c:158-267. */
int jt_lowbit_gemm_lut(const float *JT_RESTRICT X, const float *JT_RESTRICT W, float *JT_RESTRICT Y, int me, int h,
                       int k, int bits);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_LOWBIT_H */
