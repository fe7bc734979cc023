#pragma once
#ifndef JIMOTONO_GDN2_H
#define JIMOTONO_GDN2_H
/*
 * Gated DeltaNet-2 linear attention on the MI355X: the decode step and the
 * WY-form prefill chunk. Drop-in for the reference's include/jimotono/gdn2.h
 * (same names, argument meaning, return codes and errno):
 *
 *   S_t = (I - k_t (b_t*k_t)^T) Diag(alpha_t) S_{t-1} + k_t (w_t*v_t)^T,
 *   o_t = S_t^T q_t,
 *
 * with q, k L2-normalised inside, S [dk][dv] fp32 row-major.
 *
 * The state helpers work on host memory exactly as the reference's do (a
 * 64-byte aligned, zeroed block). jt_gdn2_l2norm, jt_gdn2_decode_step and
 * the prefill chunks are host-pointer calls: the arguments are checked, the
 * vectors and the state go to HBM, a HIP kernel does the update in the
 * reference's fp32 operation order (bit-identical results) and S and the
 * outputs come back only when the inputs passed the checks (non-finite
 * values or alpha outside [0,1]: JT_ERR_INVAL, S and the outputs
 * untouched). A caller that keeps states in HBM uses jt_hip_gdn2_* in
 * jimotono/hip_gdn2.h. The scratch arguments are checked for size as the
 * reference checks them; the device kernels use their own workspace, so the
 * caller's scratch is left as it was (the reference leaves its normalised
 * q and k there; their contents after a call are unspecified here). As in
 * the reference (restrict pointers), S, the outputs and the scratch must
 * not overlap each other or the inputs; overlap is not detected.
 */
#include <stddef.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Reference gdn2.h:32-35. */
#define JT_GDN2_MAX_D 1024
#define JT_GDN2_EPS_DEFAULT 1e-6f

/* dk*dv*4 bytes. Reference gdn2.h:49-50. */
int jt_gdn2_state_bytes(int dk, int dv, size_t *JT_RESTRICT out_bytes);
/* 64-byte aligned, zeroed host state. Reference gdn2.h:52-57. */
int jt_gdn2_state_alloc(float **JT_RESTRICT out_S, int dk, int dv);
void jt_gdn2_state_free(float *S);
/* Zero S (sequence boundary). Reference gdn2.h:59-61. */
int jt_gdn2_state_reset(float *JT_RESTRICT S, int dk, int dv);
/* 2*dk + 2*dv. Reference gdn2.h:63-65. */
int jt_gdn2_scratch_floats(int dk, int dv, size_t *JT_RESTRICT out_n);
/* y = x / ||x||, 0 when ||x|| < eps; eps <= 0 or NaN is JT_ERR_INVAL.
 * Reference gdn2.h:67-69, src/gdn2.c:219-250. */
int jt_gdn2_l2norm(const float *JT_RESTRICT x, float *JT_RESTRICT y, int n,
                   float eps);
/* One decode step. S 64-byte aligned (else JT_ERR_ALIGN); scratch_n >=
 * jt_gdn2_scratch_floats. Reference gdn2.h:71-86, src/gdn2.c:252-405. */
int jt_gdn2_decode_step(float *JT_RESTRICT S, float *JT_RESTRICT out_o,
                        const float *JT_RESTRICT q, const float *JT_RESTRICT k,
                        const float *JT_RESTRICT v, const float *JT_RESTRICT b,
                        const float *JT_RESTRICT w,
                        const float *JT_RESTRICT alpha, int dk, int dv,
                        float *JT_RESTRICT scratch, size_t scratch_n);
/* One chunk of 16 / 32 tokens: Q, K, B, Alpha [C][dk]; V, W, Out [C][dv];
 * scratch_n >= 4*C*dk + 2*C*dv + C*C + dk. Equal to C decode steps up to
 * fp32 rounding. Reference gdn2.h:88-113, src/gdn2.c:474-862. */
int jt_gdn2_prefill_chunk16(float *JT_RESTRICT S, float *JT_RESTRICT Out,
                            const float *JT_RESTRICT Q,
                            const float *JT_RESTRICT K,
                            const float *JT_RESTRICT V,
                            const float *JT_RESTRICT B,
                            const float *JT_RESTRICT W,
                            const float *JT_RESTRICT Alpha, int dk, int dv,
                            float *JT_RESTRICT scratch, size_t scratch_n);
int jt_gdn2_prefill_chunk32(float *JT_RESTRICT S, float *JT_RESTRICT Out,
                            const float *JT_RESTRICT Q,
                            const float *JT_RESTRICT K,
                            const float *JT_RESTRICT V,
                            const float *JT_RESTRICT B,
                            const float *JT_RESTRICT W,
                            const float *JT_RESTRICT Alpha, int dk, int dv,
                            float *JT_RESTRICT scratch, size_t scratch_n);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_GDN2_H */
