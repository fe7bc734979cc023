#pragma once
#ifndef JIMOTONO_MOE_GEMM_H
#define JIMOTONO_MOE_GEMM_H
/*
 * fp32 dense GEMM and exact transpose on the MI355X. Drop-in for the
 * reference's include/jimotono/moe_gemm.h.
 *
 * jt_gemm_mat_f32 accumulates each C[m][n] in fp32, k in increasing order,
 * one rounded multiply and one rounded add per step (no fused multiply-add),
 * so its result is bit-identical to the reference's scalar and AVX2 kernels
 * (src/moe_gemm.c:47-61, 68-89).
 */
#include <stddef.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Micro-tile sizes of the reference CPU kernel, kept for source
 * compatibility (reference moe_gemm.h:53-54); the GPU kernel ignores them. */
#define JT_GEMM_MR 12
#define JT_GEMM_NR 4

/* C[M][N] = A[M][K] * B[K][N], row-major; M == 0 is a no-op.
 * Rejects a non-finite result with JT_ERR_INVAL/EINVAL, C untouched.
 * Reference: moe_gemm.h:59-60, src/moe_gemm.c:92-170. */
int jt_gemm_mat_f32(const float *JT_RESTRICT A, const float *JT_RESTRICT B, float *JT_RESTRICT C, int M, int N,
                    int K);

/* dst[cols][rows] = src[rows][cols]. Reference: moe_gemm.h:65-66,
 * src/moe_gemm.c:17-42. */
int jt_transpose_f32(const float *JT_RESTRICT src, float *JT_RESTRICT dst, int rows, int cols);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_MOE_GEMM_H */
