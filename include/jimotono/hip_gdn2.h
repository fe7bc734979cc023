#pragma once
#ifndef JIMOTONO_HIP_GDN2_H
#define JIMOTONO_HIP_GDN2_H
/*
 * Device-resident, batched Gated DeltaNet-2 for the MI355X. No single
 * counterpart in the reference: it is jt_gdn2_decode_step and
 * jt_gdn2_prefill_chunk16/32 (reference include/jimotono/gdn2.h:71-113,
 * src/gdn2.c:252-862) for H independent heads (or sequences) whose states
 * stay in HBM, each head's result bit-identical to the reference call on
 * that head. Pointers are device pointers; calls are asynchronous on
 * `stream` (a hipStream_t as void*, NULL = the null stream). A head whose
 * inputs hold a non-finite value or an alpha outside [0,1] keeps its state
 * and outputs and raises JT_HIP_EF_NONFINITE_INPUT (jimotono/hip_moe.h;
 * read with jt_hip_sync_errors).
 */
#include <stddef.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One decode step per head: S [H][dk][dv] updated in place, o [H][dv];
 * q, k, b, alpha [H][dk]; v, w [H][dv]; dk, dv in 1..1024. */
int jt_hip_gdn2_decode(float *dS, float *dO, const float *dq, const float *dk_,
                       const float *dv_, const float *db, const float *dw,
                       const float *dalpha, int H, int dk, int dv, void *stream);

/* Heads per prefill call: the heads are a grid dimension of its launches. */
#define JT_HIP_GDN2_MAX_PREFILL_HEADS 65535

/* Workspace bytes of jt_hip_gdn2_prefill (0 for invalid arguments, H
 * outside 1..JT_HIP_GDN2_MAX_PREFILL_HEADS included):
 * 4*ceil(H/64)*64 + H*(T/C)*(7*C*dk + 2*C*C)*4 -- one record per (head,
 * chunk), since every chunk's state-independent part is prepared at once. */
size_t jt_hip_gdn2_prefill_ws_bytes(int H, int T, int C, int dk);
/* Prefill of T tokens per head in T/C chunks of C = 16 or 32 (T % C == 0),
 * each chunk equal to the reference's jt_gdn2_prefill_chunk{C} on the state
 * the previous chunk left: Q, K, B, Alpha [H][T][dk]; V, W, Out [H][T][dv];
 * S [H][dk][dv] in place. A head with a bad value among its T tokens keeps
 * its S and Out. H in 1..JT_HIP_GDN2_MAX_PREFILL_HEADS (JT_ERR_INVAL,
 * EINVAL otherwise). d_ws: jt_hip_gdn2_prefill_ws_bytes(H, T, C, dk) bytes,
 * 16-byte aligned, not kept between calls. */
int jt_hip_gdn2_prefill(float *dS, float *dOut, const float *dQ,
                        const float *dK, const float *dV, const float *dB,
                        const float *dW, const float *dA, int H, int T, int C,
                        int dk, int dv, void *d_ws, size_t ws_bytes,
                        void *stream);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_HIP_GDN2_H */
