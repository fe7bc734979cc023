#pragma once
#ifndef JIMOTONO_ROUTING_H
#define JIMOTONO_ROUTING_H
/*
 * MoE top-k selection on the MI355X. Drop-in for jt_routing_topk of the
 * reference's include/jimotono/routing.h. The training-only losses declared
 * next to it in the reference (jt_routing_balance_loss,
 * jt_routing_sticky_loss) are not part of the forward matmul path and are not
 * provided by this library.
 */
#include <stddef.h>

#include "jimotono/common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Select the k largest of logits[0..n) (ties -> lower index, -INF never
 * preferred over a finite value, NaN rejected), then softmax over the
 * selected k: w_p = (float)exp(l_p - max) in fp64, scaled by (float)(1/sum).
 * Reference: routing.h:56-57, src/routing.c:16-76. */
int jt_routing_topk(const float *JT_RESTRICT logits, size_t n, size_t k, size_t *JT_RESTRICT out_ids,
                    float *JT_RESTRICT out_weights);

#ifdef __cplusplus
}
#endif

#endif /* JIMOTONO_ROUTING_H */
