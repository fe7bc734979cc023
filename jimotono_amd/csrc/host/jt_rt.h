/*
 * Internal runtime of libjimotono_hip (C11): device binding, the library
 * stream, the device error word, grow-only staging buffers for the
 * host-pointer entry points, and the HIP -> jt_err_t/errno mapping.
 */
#ifndef JT_RT_H
#define JT_RT_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "jimotono/common.h"
#include "../kernels/jt_launch.h"

/* device error bits (same values as the kernels' EF_* flags) */
#define JT_EF_NONFINITE_INPUT 0x1u
#define JT_EF_RANGE 0x2u
#define JT_EF_NONFINITE_MID 0x4u
#define JT_EF_BAD_ID 0x8u
#define JT_EF_QRANGE 0x10u

enum {
    JT_SLOT_A = 0,
    JT_SLOT_B,
    JT_SLOT_C,
    JT_SLOT_D,
    JT_SLOT_E,
    JT_SLOT_F,
    JT_SLOT_G,
    JT_SLOT_H,
    JT_SLOT_I,
    JT_SLOT_J,
    JT_SLOT_K,
    JT_SLOT_L,
    JT_SLOT_M,
    JT_SLOT_N,
    JT_SLOT_O,
    JT_SLOT_P,
    JT_SLOT_LAYER, /* the drop-in layer forward's workspace (host/moe_layer.c) */
    JT_SLOT_BWD,   /* the drop-in batched backward's workspace (host/moe_bwd.c) */
    JT_NSLOTS
};

typedef struct jt_rt {
    int ready;
    int device;
    hipStream_t stream;
    uint32_t *d_err;     /* device error words, one per stream (JT_ERR_WORDS) */
    uint32_t *d_scratch; /* small device scratch (reductions) */
    void *slot[JT_NSLOTS];
    size_t slot_bytes[JT_NSLOTS];
    void *hslot[2]; /* pinned host staging (jt_rt_hbuf) */
    size_t hslot_bytes[2];
} jt_rt;

/* Initialise on first use (device 0 unless jt_hip_init chose another).
 * Returns NULL with errno = ENODEV/EIO when no GPU is usable. */
jt_rt *jt_rt_get(void);
/* hipError_t -> JT_OK / JT_ERR_NOMEM (ENOMEM) / JT_ERR_IO (EIO). */
int jt_rt_err(hipError_t e);
/* Grow-only device buffer of slot `s` with at least `bytes` bytes. */
void *jt_rt_buf(jt_rt *rt, int s, size_t bytes, int *rc);
/* The device error word of `stream`: each stream the library has launched
 * on gets its own word (the null stream included), so callers on different
 * streams never see each other's error bits. Past JT_ERR_WORDS - 1 distinct
 * streams the rest share the last word. */
#define JT_ERR_WORDS 64
#define JT_ERR_STRIDE 16 /* words between two streams' error words (64 B) */
uint32_t *jt_rt_errw(jt_rt *rt, hipStream_t stream);
/* Synchronise `stream`, read and clear that stream's device error word. */
int jt_rt_flags(jt_rt *rt, hipStream_t stream, uint32_t *flags);
/* Map error bits to the reference's return/errno convention
 * (non-finite input or bad code -> EINVAL, computed overflow -> ERANGE). */
int jt_rt_flags_to_rc(uint32_t flags);

/* Grow-only pinned host buffer `s` (0 or 1) of at least `bytes` bytes, for
 * host inputs and outputs staged through one copy or one wait: a grown
 * buffer replaces the old one after the library stream has drained. */
void *jt_rt_hbuf(jt_rt *rt, int s, size_t bytes, int *rc);

/* host<->device copies on the library stream (synchronous) */
int jt_rt_h2d(jt_rt *rt, void *dst, const void *src, size_t bytes);
int jt_rt_d2h(jt_rt *rt, void *dst, const void *src, size_t bytes);

static inline size_t jt_round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

/* Every device allocation of the host layer goes through jt_rt_malloc, which
 * counts the successful ones (jt_hip_alloc_count reads the count), so a test
 * can show that an entry point allocated nothing. */
hipError_t jt_rt_malloc(void **p, size_t bytes);
#ifndef JT_RT_NO_MALLOC_MACRO
#define hipMalloc(p, bytes) jt_rt_malloc((void **)(p), (bytes))
#endif

#endif /* JT_RT_H */
