#pragma once
#ifndef JIMOTONO_COMMON_H
#define JIMOTONO_COMMON_H
/*
 * Shared definitions of the jimotono C ABI, MI355X build.
 *
 * The error codes, their numeric values and the errno convention are part of
 * the drop-in contract and therefore identical to the reference
 * (include/jimotono/common.h:21-28): every entry point returns JT_OK or a
 * JT_ERR_* code and sets errno (EINVAL for bad arguments, ERANGE for a
 * computed non-finite value, ENOMEM for allocation failure). The HIP build
 * adds one mapping of its own: a failed HIP runtime call is reported as
 * JT_ERR_IO with errno = EIO, and a missing GPU as JT_ERR_IO with
 * errno = ENODEV.
 */
#include <stddef.h>
#include <stdint.h>

#if defined(__BYTE_ORDER__) && (__BYTE_ORDER__ == __ORDER_BIG_ENDIAN__)
#error "jimotono is little-endian only"
#endif

#define JT_CACHELINE 64

/* The reference prototypes carry C99 restrict; the same qualifier is spelled
 * __restrict__ when a header is read by a C++ (HIP) translation unit. */
#ifdef __cplusplus
#define JT_RESTRICT __restrict__
#else
#define JT_RESTRICT restrict
#endif

typedef enum jt_err {
    JT_OK = 0,
    JT_ERR_NOMEM = 1,
    JT_ERR_INVAL = 2,
    JT_ERR_IO = 3,
    JT_ERR_ALIGN = 4,
    JT_ERR_NOSUP = 5,
} jt_err_t;

/* Width limit shared by the W8A8 GEMM and the MoE layer
 * (reference include/jimotono/train_bwd.h:35). It bounds |acc| of an int8 dot
 * product at 127*127*4096 < 2^31. */
#ifndef JT_BWD_MAX_WIDE
#define JT_BWD_MAX_WIDE 4096
#endif

#define JT_VERSION_MAJOR 0
#define JT_VERSION_MINOR 0
#define JT_VERSION_PATCH 1

#endif /* JIMOTONO_COMMON_H */
