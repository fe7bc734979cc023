#pragma once
#ifndef JIMOTONO_HIP_MOE_H
#define JIMOTONO_HIP_MOE_H
/*
 * Device-resident quantised MoE path for the AMD Instinct MI355X (gfx950).
 *
 * This header has no single counterpart in the reference: it is the
 * prepared-weight, HBM-resident form of the reference's quantised MoE
 * forward (src/moe_layer.c:980-1614 with the W8A8 helpers
 * src/moe_layer.c:164-274 and the low-bit driver src/lowbit.c:158-267).
 * The host-pointer prototypes in w8a8.h / lowbit.h / moe_layer.h are the
 * drop-in; this API is what a caller that keeps activations on the GPU uses.
 *
 * All pointers named d* are device (HBM) pointers; `stream` is a hipStream_t
 * passed as void* (NULL = the HIP null stream, which is also torch's default
 * stream, so work the caller queued there is ordered). Calls are asynchronous
 * on that stream. Arguments are validated on the host before anything is
 * enqueued (JT_ERR_INVAL, nothing written). Data-dependent failures found by
 * the kernels (a non-finite activation, an overflowing epilogue) raise bits in
 * the device error word of the stream the call was made on (each stream has
 * its own word, so one caller never reads another stream's bits; past 63
 * streams in use at once the rest share one word) instead of a partial
 * result being trusted; jt_hip_sync_errors() waits for a stream and returns
 * (and clears) the bits raised so far by calls on that stream. The word is
 * keyed by the stream handle: call jt_hip_stream_forget() before destroying
 * a stream the library has run on, since HIP may hand the same handle to a
 * later stream, which would otherwise inherit unread bits.
 *
 * Formats of a prepared layer (built on the GPU from fp32 weights):
 *  - shared experts: int8 codes, one fp32 scale per output channel (the
 *    reference's jt_w8a8_quant_per_channel formula), gate/up rows interleaved
 *    in blocks of 16 so a SwiGLU pair lands in one wavefront;
 *  - routed experts: gate/up INT2 and down INT4 level codes li (the
 *    reference's odd-symmetric grid, src/lowbit.c:42-45, 77-88) with one
 *    fp16 scale maxabs_g/(2^bits-1) per `group` (64) weights along K;
 *  - weights are stored in 16-channel x 64-K panels whose byte order equals
 *    the operand layout of v_mfma_i32_16x16x64_i8, so a panel is one
 *    coalesced 1 KiB (int8), 512 B (INT4) or 256 B (INT2) wavefront load.
 * Activations are quantised per token (one fp32 scale per row).
 */
#include <stddef.h>
#include <stdint.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ---- */

/* Bind the calling thread's HIP device (idempotent; called implicitly by
 * every other entry point with device 0). */
int jt_hip_init(int device);
/* Wait for `stream` (NULL: for the whole device), then read and clear the
 * device error word of `stream` (NULL: of the null stream).
 * *out_flags gets the raised JT_HIP_EF_* bits (0 = clean). Returns JT_OK, or
 * JT_ERR_IO on a HIP failure. */
int jt_hip_sync_errors(void *stream, uint32_t *out_flags);
/* Release `stream`'s error word: waits for the stream, clears its word
 * (unread bits are dropped) and frees the slot for the next new stream.
 * Call it before destroying a stream the library has launched on. A stream
 * the library has not seen is a no-op. No reference counterpart: the
 * reference has no streams. Returns JT_OK, or JT_ERR_IO on a HIP failure. */
int jt_hip_stream_forget(void *stream);
/* Number of device allocations (hipMalloc) the library has made so far in
 * this process: a diagnostic that lets a caller check that a call allocated
 * nothing. No reference counterpart (the reference allocates host memory
 * only). Returns JT_OK, or JT_ERR_INVAL (EINVAL) for a NULL out. */
int jt_hip_alloc_count(uint64_t *out);

#define JT_HIP_EF_NONFINITE_INPUT 0x1u /* NaN/Inf in an activation row */
#define JT_HIP_EF_RANGE 0x2u           /* epilogue value overflowed fp32 */
#define JT_HIP_EF_NONFINITE_MID 0x4u   /* non-finite SwiGLU / logits / Y */
#define JT_HIP_EF_BAD_ID 0x8u          /* routed expert id out of range */

/* ---- per-token activation quantisation ----
 * dX [rows][cols] fp32 -> dXq [rows][cols] int8, dscale [rows] fp32, same
 * formula as jt_w8a8_quant_per_channel (reference src/w8a8.c:812-851). */
int jt_hip_quant_rows(const float *dX, int rows, int cols, int8_t *dXq,
                      float *dscale, void *stream);

/* ---- W8A8 GEMM with prepared weights ---- */
typedef struct jt_hip_w8a8 jt_hip_w8a8;
/* Quantise dW [N][K] fp32 per output row on the GPU and pack it. */
int jt_hip_w8a8_prepare(const float *dW, int N, int K, jt_hip_w8a8 **out);
/* Pack already-quantised codes given in the reference layout dBq [K][N]
 * with column scales dsB [N] (no requantisation). */
int jt_hip_w8a8_prepare_kn(const int8_t *dBq, const float *dsB, int N, int K,
                           jt_hip_w8a8 **out);
/* dC [M][N] = (float)((double)acc * ((double)dsA[m] * (double)sB[n])),
 * acc = sum_k dAq[m][k] * B[n][k] in int32. M <= 16 uses the streaming GEMV
 * kernel, larger M the MFMA kernel; both give identical bits. */
int jt_hip_w8a8_gemm(const jt_hip_w8a8 *W, const int8_t *dAq,
                     const float *dsA, float *dC, int M, void *stream);
/* Copy out the quantised weights in the reference layout: Bq [K][N] int8
 * and sB [N] fp32 (host pointers; for tests). */
int jt_hip_w8a8_export(const jt_hip_w8a8 *W, int8_t *Bq_kn, float *sB);
/* The per-token INT8 projection of fp32 activations (the mixed-precision
 * design's attention projections, reference AGENTS.MD:43-51): dC [M][N] =
 * the GEMM above of dX [M][K] fp32 quantised per row with
 * jt_w8a8_quant_per_channel's formula inside the call, bit-identical to
 * jt_hip_quant_rows followed by jt_hip_w8a8_gemm. M <= 16 quantises in the
 * GEMM's own blocks (no workspace; K % 4 == 0, K <= 4096, dX 16-byte
 * aligned); larger M uses d_ws of jt_hip_w8a8_gemm_f32_ws_bytes(W, M) bytes. */
size_t jt_hip_w8a8_gemm_f32_ws_bytes(const jt_hip_w8a8 *W, int M);
int jt_hip_w8a8_gemm_f32(const jt_hip_w8a8 *W, const float *dX, float *dC,
                         int M, void *d_ws, size_t ws_bytes, void *stream);
void jt_hip_w8a8_free(jt_hip_w8a8 *W);

/* ---- one W8A8 SwiGLU expert (the shared-expert block) ----
 * dWg, dWu [h][n], dWd [h][n] (reference shared-expert layout,
 * moe_layer.h:59-61): Y = down(silu(X Wg^T) * (X Wu^T)) with per-token
 * int8 activations on both GEMMs. */
typedef struct jt_hip_ffn jt_hip_ffn;
int jt_hip_ffn_prepare(const float *dWg, const float *dWu, const float *dWd,
                       int n, int h, jt_hip_ffn **out);
/* dY [T][n] = the expert output for dX [T][n] (fp32). The expert's own
 * workspace grows to the largest T seen: a call with more rows than reserved
 * waits for the whole device, frees and reallocates before it enqueues
 * anything (jt_hip_ffn_reserve does that ahead of time). */
int jt_hip_ffn_fwd(jt_hip_ffn *F, const float *dX, float *dY, int T,
                   void *stream);
/* Size the expert's own workspace for T rows now (synchronous; T > 0), so
 * that later jt_hip_ffn_fwd calls of at most T rows neither allocate nor
 * synchronise (for serving loops and HIP graph capture). */
int jt_hip_ffn_reserve(jt_hip_ffn *F, int T);
/* jt_hip_ffn_fwd that allocates nothing. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its workspace is a fixed 16 MiB device array per GPU, held until the
 * process ends, instead of the expert's own grow-on-demand buffers.
 * The workspace of T rows is, each part rounded up to 256 bytes:
 *   T*round_up(n,64) + 4T + 4T*h + T*round_up(h,64) + 4T bytes;
 * a larger T returns JT_ERR_NOSUP with errno E2BIG, nothing enqueued
 * (n = 1024, h = 2816: T <= 1110). Every call on one GPU shares the array,
 * so calls that overlap on a GPU (two streams, two threads) race; calls in
 * one stream's order do not. Same outputs as jt_hip_ffn_fwd, bit for bit. */
int jt_hip_ffn_fwd_noalloc(jt_hip_ffn *F, const float *dX, float *dY, int T,
                           void *stream);
void jt_hip_ffn_free(jt_hip_ffn *F);

/* ---- quantised MoE layer ---- */
typedef struct jt_hip_moe_desc {
    int n;          /* model width: K of gate/up, N of down */
    int h;          /* routed expert hidden width */
    int n_experts;  /* routed experts E (1..JT_MOE_MAX_EXPERTS) */
    int topk;       /* k (1..min(E, 64)) */
    int n_shared;   /* shared experts S (0..8) */
    int h_shared;   /* shared expert hidden width (the reference ties it to h) */
    int group;      /* low-bit scale group along K: 64 */
    int max_tokens; /* largest T a forward may be called with */
} jt_hip_moe_desc;

typedef struct jt_hip_moe jt_hip_moe;

/* Build a layer from fp32 device weights in the reference layouts:
 * dWgate [E][n]; dWg, dWu, dWd [E][h][n]; dWg_s, dWu_s, dWd_s
 * [S][h_shared][n] (NULL when S == 0). dWgate may be NULL for a layer that is
 * only driven through jt_hip_moe_fwd_routed. */
int jt_hip_moe_prepare(const jt_hip_moe_desc *desc, const float *dWgate,
                       const float *dWg, const float *dWu, const float *dWd,
                       const float *dWg_s, const float *dWu_s,
                       const float *dWd_s, jt_hip_moe **out);

/* Full forward: fp64 gate logits, top-k softmax, dropless expert sort,
 * routed INT2/INT4 grouped GEMMs, shared W8A8 experts, fp64 combine.
 * dX, dY [T][n] fp32, T <= max_tokens. */
int jt_hip_moe_fwd(jt_hip_moe *L, const float *dX, float *dY, int T,
                   void *stream);

/* Forward with caller-supplied routing: d_ids [T][k] int32 (distinct per
 * token, < E) and d_weights [T][k] fp32 replace the router. */
int jt_hip_moe_fwd_routed(jt_hip_moe *L, const float *dX, const int32_t *d_ids,
                          const float *d_weights, float *dY, int T,
                          void *stream);

/* The forward plus the residual add of the reference's training loop
 * (bench/kernel/train_tinystories.c:1147-1160, after jt_moe_fwd_batch),
 * fused into the combine: dY = (float)((double)dX + (double)m) with
 * m = the layer output as jt_hip_moe_fwd writes it (two roundings, as
 * there; a non-finite sum raises JT_HIP_EF_NONFINITE_MID). d_ids and
 * d_weights as in jt_hip_moe_fwd_routed, or both NULL to run the router.
 * dY may be dX (in place). */
int jt_hip_moe_fwd_residual(jt_hip_moe *L, const float *dX, const int32_t *d_ids,
                            const float *d_weights, float *dY, int T,
                            void *stream);

/* Device buffers of the last forward, for inspection. */
enum jt_hip_moe_buf {
    JT_HIP_BUF_IDS = 0,     /* int32 [T][k] */
    JT_HIP_BUF_WEIGHTS = 1, /* fp32 [T][k] */
    JT_HIP_BUF_PERM = 2,    /* int32 [T*k], flattened q grouped by expert */
    JT_HIP_BUF_OFF = 3,     /* int32 [E+1] */
    JT_HIP_BUF_XQ = 4,      /* int8 [T][n] */
    JT_HIP_BUF_XSCALE = 5,  /* fp32 [T] */
    JT_HIP_BUF_YE = 6,      /* fp32 [T*k][n], routed expert output per pair */
    JT_HIP_BUF_YS = 7,      /* fp32 [S][T][n], shared expert outputs */
    JT_HIP_BUF_LOGITS = 8,  /* fp32 [T][E]: the reference's logit for every expert that
                               could reach the top-k (every selected one); with the
                               int8-bounded router (E <= 256, d % 64 == 0) the others
                               hold the float of their int8 approximation */
    JT_HIP_BUF_HQ = 9,      /* int8 [T*k][h]: routed hidden rows (SwiGLU output) as
                               int8 codes, in sorted row order (row r is pair perm[r]) */
    JT_HIP_BUF_HSCALE = 10, /* fp32 [T*k]: their per-row scales, same order */
};
int jt_hip_moe_buffer(const jt_hip_moe *L, int which, void **dptr,
                      size_t *bytes);

/* Quantised routed weights of expert e in plain layouts (host pointers):
 * gate/up codes li [2][h][n] uint8 and fp16 scales [2][h][n/group] (uint16
 * bits); down codes [n][h] uint8 and scales [n][h/group]. */
int jt_hip_moe_export_routed(const jt_hip_moe *L, int e, uint8_t *gu_codes,
                             uint16_t *gu_scales, uint8_t *d_codes,
                             uint16_t *d_scales);

/* A prepared layer as bytes, in the order the kernels read its weights,
 * so that a model is stored once as its execution plan (the reference's
 * "model format = execution plan", DESIGN.MD:94-104, with quantised
 * artifacts kept out of the repository, ROADMAP.MD:149-157). The buffer
 * holds a 4 KiB header (magic "JTMOEQ1", version 1, the layer's sizes, a
 * section table, a 64-bit checksum of the payload) and the device arrays
 * byte for byte, each section 4 KiB aligned: the router gate (with its
 * int8 code panels when the layer has them), the routed INT2 gate/up and
 * INT4 down panels with their fp16 group scales, and each shared expert's
 * int8 panels with their fp32 channel scales. buf == NULL only sets
 * *bytes (the size needed); a cap below it returns JT_ERR_INVAL. */
int jt_hip_moe_save(const jt_hip_moe *L, void *buf, size_t cap, size_t *bytes);
/* A layer from jt_hip_moe_save's bytes (host memory): the arrays are
 * copied to the GPU as they are, with no quantisation or packing, and the
 * workspace is sized for max_tokens as in jt_hip_moe_desc. A wrong magic,
 * version, size, section table or checksum returns JT_ERR_INVAL (EINVAL)
 * with nothing allocated. The layer's forwards are bit-identical to the
 * saved layer's. */
int jt_hip_moe_load(const void *buf, size_t bytes, int max_tokens,
                    jt_hip_moe **out);

/* Per-stage device time of the most recent forwards, recorded with HIP
 * events on the forward's stream while profiling is on. */
int jt_hip_moe_set_profiling(jt_hip_moe *L, int on);
/* Fills names[i] (static strings) and total milliseconds ms[i] summed over
 * the profiled forwards since the last reset, plus the number of forwards in
 * *count; returns the number of stages in *n (at most cap). */
int jt_hip_moe_stage_times(jt_hip_moe *L, const char **names, double *ms,
                           int cap, int *n, int *count);
void jt_hip_moe_free(jt_hip_moe *L);

/* ---- batched backward on device pointers ----
 * The device form of jt_moe_bwd_batch (moe_layer.h; reference
 * src/moe_layer.c:1684-2502): the same arguments as device pointers
 * (ids, perm, off as size_t), validate = 1 for the checked form, 0 for the
 * unchecked one, and a caller workspace d_ws of at least
 * jt_hip_moe_bwd_batch_ws_bytes() bytes, 256-byte aligned. perm needs
 * off[E] entries. Asynchronous on `stream`; inconsistent ids / off / perm
 * raise JT_HIP_EF_BAD_ID, non-finite inputs (validate) JT_HIP_EF_NONFINITE_INPUT
 * and non-finite intermediates JT_HIP_EF_NONFINITE_MID, and the outputs are
 * then not meaningful (read them with jt_hip_sync_errors). The workspace is
 * not kept between calls. */
size_t jt_hip_moe_bwd_batch_ws_bytes(int T, int n, int h, int n_experts,
                                     int topk, int n_shared);
int jt_hip_moe_bwd_batch(
    const float *dY, const float *X, const float *Wgate, const float *Wg,
    const float *Wu, const float *Wd, const float *Wg_s, const float *Wu_s,
    const float *Wd_s, const size_t *ids, const float *weights,
    const float *Gsel, const float *Usel, const float *Ysel, const float *Gs,
    const float *Us, const size_t *perm, const size_t *off,
    const unsigned char *drop, float *dX, float *dWgate, float *dWg,
    float *dWu, float *dWd, float *dWg_s, float *dWu_s, float *dWd_s,
    float *dLogits, int T, int n, int h, int n_experts, int topk,
    int n_shared, int validate, void *d_ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_HIP_MOE_H */
