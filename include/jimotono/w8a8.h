#pragma once
#ifndef JIMOTONO_W8A8_H
#define JIMOTONO_W8A8_H
/*
 * W8A8 symmetric int8 quantisation and int8 x int8 -> int32 GEMM, computed on
 * an AMD Instinct MI355X (gfx950). Drop-in for the reference's
 * include/jimotono/w8a8.h; every prototype below keeps the reference
 * signature, argument meaning and fail-closed behaviour.
 *
 * Host pointers in, host pointers out: each call stages its inputs into HBM,
 * runs HIP kernels, checks the device-side error flag and copies the result
 * back before returning. Outputs are written only when the whole call
 * succeeded (validation errors and computed-overflow errors alike leave the
 * output untouched). Arithmetic contract (bit-exact with the reference):
 *   scale = (float)(max|x| / 127)  (fp64 divide; all-zero input -> 1.0, q = 0)
 *   q     = clamp(round(x / scale_d), -127, 127), round half away from zero
 *   C     = (float)((double)acc * ((double)sA * (double)sB[n])), acc int32
 */
#include <stddef.h>
#include <stdint.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

#define JT_W8A8_QMAX 127
#define JT_W8A8_QMIN (-127)

/* Process-wide mode flag, 0 = fp32 path (default), 1 = W8A8 path.
 * Reference: include/jimotono/w8a8.h:61-65, src/w8a8.c:53-73. */
int jt_w8a8_set_enabled(int enabled);
int jt_w8a8_get_enabled(int *JT_RESTRICT out_enabled);
int jt_w8a8_is_enabled(void);

/* Whole-array quantisation with one scale.
 * Reference: w8a8.h:71-74, src/w8a8.c:688-747. */
int jt_w8a8_quant_per_tensor(const float *JT_RESTRICT src, size_t n, int8_t *JT_RESTRICT dst,
                             float *JT_RESTRICT out_scale);
/* dst[i] = (float)((double)src[i] * scale). Reference: w8a8.h:76-78,
 * src/w8a8.c:749-785. */
int jt_w8a8_dequant_per_tensor(const int8_t *JT_RESTRICT src, float scale, size_t n,
                               float *JT_RESTRICT dst);
/* One scale per row of src[rows][cols]. Reference: w8a8.h:83-86,
 * src/w8a8.c:787-855. */
int jt_w8a8_quant_per_channel(const float *JT_RESTRICT src, size_t rows, size_t cols,
                              int8_t *JT_RESTRICT dst, float *JT_RESTRICT scales);
/* Reference: w8a8.h:88-91, src/w8a8.c:857-907. */
int jt_w8a8_dequant_per_channel(const int8_t *JT_RESTRICT src, const float *JT_RESTRICT scales,
                                size_t rows, size_t cols, float *JT_RESTRICT dst);

/* C[M][N] = sA * sB * sum_k Aq[m][k] * Bq[k][n]; Aq [M][K], Bq [K][N]
 * (row-major), M == 0 is a no-op. Reference: w8a8.h:101-104,
 * src/w8a8.c:955-1019. */
int jt_w8a8_gemm_per_tensor(const int8_t *JT_RESTRICT Aq, const int8_t *JT_RESTRICT Bq, float sA,
                            float sB, float *JT_RESTRICT C, int M, int N, int K);
/* As above with one scale per output column, sB_col[N].
 * Reference: w8a8.h:108-111, src/w8a8.c:1021-1072. */
int jt_w8a8_gemm_per_channel(const int8_t *JT_RESTRICT Aq, const int8_t *JT_RESTRICT Bq, float sA,
                             const float *JT_RESTRICT sB_col, float *JT_RESTRICT C, int M, int N,
                             int K);

/* dst = dequant(quant(src)). Reference: w8a8.h:117-121,
 * src/w8a8.c:1074-1200. */
int jt_w8a8_fakequant_per_tensor(const float *JT_RESTRICT src, size_t n, float *JT_RESTRICT dst);
int jt_w8a8_fakequant_per_channel(const float *JT_RESTRICT src, size_t rows, size_t cols,
                                  float *JT_RESTRICT dst);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_W8A8_H */
