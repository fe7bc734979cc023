// Top-k selection and softmax of one row of logits by one wavefront, with
// the row's keys held in registers (E <= 64 * EPL). Shared by the top-k
// launch (route.hip) and the decode launch that runs top-k beside the
// shared experts' gate/up (gemm_i8.hip).
//
// The reference (src/routing.c:16-76) scans the row k times with a
// strict-greater comparison, treating already selected entries as -INF:
// round p takes the first index of the largest remaining value. Keys make
// that one integer maximum per round: the order-preserving bits of the value
// (-0 folded into +0, which the reference's comparisons do not tell apart)
// above ~index, so that ties go to the lower index. A selected element keys
// as -INF with its index, so once only -INF remains the lowest index wins
// again even if already taken, as in the reference's scan.
#pragma once
#include "jt_dev.h"

#define TOPK_KEY_NEGINF 0x007fffffull  // key bits of -INF

template <int EPL>
__device__ __forceinline__ bool topk_wave_reg(const float *__restrict__ lg, int E, int k,
                                              int lane, int64_t row, int32_t *__restrict__ ids,
                                              int64_t *__restrict__ ids64,
                                              float *__restrict__ w, uint32_t *err) {
    float val[EPL];
    uint64_t key[EPL];
    int nan = 0;
#pragma unroll
    for (int u = 0; u < EPL; u++) {
        const int i = lane + 64 * u;
        val[u] = i < E ? lg[i] : 0.f;
        nan |= i < E && isnan(val[u]);
        uint32_t b = __builtin_bit_cast(uint32_t, val[u] + 0.0f);
        b ^= (b >> 31) ? 0xffffffffu : 0x80000000u;
        key[u] = i < E ? (((uint64_t)b << 32) | (uint32_t)~i) : 0ull;  // 0: below every key
    }
    if (wave_or_i(nan)) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return false;
    }
    int mysel = -1;
    float lv = -__builtin_inff();
    for (int p = 0; p < k; p++) {
        uint64_t best = key[0];
#pragma unroll
        for (int u = 1; u < EPL; u++) best = key[u] > best ? key[u] : best;
        const int bi = (int)~(uint32_t)wave_max_u64(best);  // wave-uniform
        const int bu = bi >> 6, bl = bi & 63;
        float sv = val[0];
#pragma unroll
        for (int u = 0; u < EPL; u++) {
            if (u == bu) sv = val[u];
            if (lane == bl && u == bu) key[u] = (TOPK_KEY_NEGINF << 32) | (uint32_t)~bi;
        }
        // the selected logit itself (not -INF when re-selected)
        sv = __builtin_bit_cast(float,
                                __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), bl));
        if (lane == p) {
            mysel = bi;
            lv = sv;
        }
    }
    // softmax over the selected, in selection order; the first selected is
    // the maximum
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                   __builtin_bit_cast(int, lv), 0));
    const double e = lane < k ? exp((double)lv - (double)mx) : 0.0;
    double sum = 0.0;
    for (int p = 0; p < k; p++) sum += readlane_f64(e, p);
    const bool ok = (sum > 0.0) && isfinite(sum);
    if (!ok) {
        if (lane == 0) raise_err(err, EF_NONFINITE_MID);
        return false;
    }
    const float inv = (float)(1.0 / sum);
    if (lane < k) {
        const float wv = (float)e * inv;
        ids[row * k + lane] = mysel;
        if (ids64) ids64[row * k + lane] = mysel;
        w[row * k + lane] = wv;
        if (!(wv >= 0.0f) || !isfinite(wv)) raise_err(err, EF_NONFINITE_MID);
    }
    return true;
}

// keys per lane for a row of E <= 1024 logits (0: the LDS form is used)
__host__ __device__ constexpr int topk_epl(int E) {
    return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : E <= 1024 ? 16 : 0;
}
