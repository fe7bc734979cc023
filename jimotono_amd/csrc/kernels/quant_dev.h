// The reference's per-row int8 quantiser (src/w8a8.c:787-855) for one row
// per wavefront: fp32 max-abs reduction (exact: the reference takes the max
// of exact fp64 widenings), fp64 divide, round half away from zero. Used by
// k_quant_rows and by launches that quantise token rows beside other work.
#pragma once
#include "jt_dev.h"

// Row r by one wavefront (lane = its lane index). Rows of up to
// 64*4*QR_REG floats (4096) are read once into registers with all loads in
// flight, reduced, and quantised from the registers; longer or unaligned
// rows take the two-pass loop.
#define QR_REG 16

__device__ __forceinline__ void quant_row_wave(const float *__restrict__ X, int64_t r, int cols,
                                               int8_t *__restrict__ Q, int64_t ldq,
                                               float *__restrict__ scale, uint32_t *err,
                                               int lane) {
    const float *x = X + r * cols;
    int8_t *q = Q + r * ldq;
    const bool vec = (cols & 3) == 0 && (((uintptr_t)x | (uintptr_t)q) & 3) == 0 &&
                     ((uintptr_t)x & 15) == 0;
    float m = 0.0f;
    int bad = 0;
    if (vec && cols <= 64 * 4 * QR_REG) {
        const float4 *x4 = (const float4 *)x;
        const int n4 = cols >> 2;
        float4 v[QR_REG];
#pragma unroll
        for (int i = 0; i < QR_REG; i++) {
            const int c = lane + 64 * i;
            v[i] = c < n4 ? x4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // max |x| over the bit patterns with the sign cleared: for
        // non-negative floats integer order is float order, and any inf or
        // NaN lands at or above the bits of +inf
        uint32_t mu = 0;
#pragma unroll
        for (int i = 0; i < QR_REG; i++) {
            if (64 * i < n4) {  // wave-uniform; constant indices keep v[] in registers
                mu = max(mu, max(abs_bits(v[i].x), abs_bits(v[i].y)));
                mu = max(mu, max(abs_bits(v[i].z), abs_bits(v[i].w)));
            }
        }
        mu = wave_max_u(mu);
        bad = mu >= 0x7f800000u;
        m = __builtin_bit_cast(float, mu);
        QuantParams p = quant_params(m);
        if (bad || !p.ok) {
            if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
            return;
        }
        const float inv = quant_inv_f(p.scale_d);
        uint32_t *q4 = (uint32_t *)q;
        uint32_t fmask = 0;  // bit i: a code of v[i] needs the exact quotient
        // every word first, then every store: stores between the steps make
        // the compiler wait for each store before it reuses that store's
        // address registers, one memory round trip per word
        uint32_t wd[QR_REG];
#pragma unroll
        for (int i = 0; i < QR_REG; i++) {
            wd[i] = 0;
            if (64 * i < n4) {  // wave-uniform
                bool f = false;
                const uint32_t b0 = (uint8_t)quant_code_try(v[i].x, inv, f);
                const uint32_t b1 = (uint8_t)quant_code_try(v[i].y, inv, f);
                const uint32_t b2 = (uint8_t)quant_code_try(v[i].z, inv, f);
                const uint32_t b3 = (uint8_t)quant_code_try(v[i].w, inv, f);
                // lanes past the row hold zeros; with inv = inf (max|x| below
                // ~3.7e-37) their codes would fail too, and the exact rewrite
                // below must not store past the row
                fmask |= (uint32_t)(f && lane + 64 * i < n4) << i;
                wd[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
        }
#pragma unroll
        for (int i = 0; i < QR_REG; i++) {
            const int c = lane + 64 * i;
            if (64 * i < n4 && c < n4) q4[c] = wd[i];
        }
        if (lane == 0) scale[r] = p.scale_f;
        // rare: rewrite those words exactly, picking v[j] out of the
        // registers with selects (a dynamic index would spill v[] to scratch)
        while (fmask) {
            const int j = __builtin_ctz(fmask);
            fmask &= fmask - 1;
            float4 u = v[0];
#pragma unroll
            for (int i = 1; i < QR_REG; i++)
                if (i == j) u = v[i];
            const uint32_t b0 = (uint8_t)quant_code(u.x, p.scale_d);
            const uint32_t b1 = (uint8_t)quant_code(u.y, p.scale_d);
            const uint32_t b2 = (uint8_t)quant_code(u.z, p.scale_d);
            const uint32_t b3 = (uint8_t)quant_code(u.w, p.scale_d);
            q4[lane + 64 * j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        return;
    }
    if (vec) {
        const float4 *x4 = (const float4 *)x;
        for (int c = lane; c < (cols >> 2); c += 64) {
            const float4 v = x4[c];
            bad |= (!isfinite(v.x)) || (!isfinite(v.y)) || (!isfinite(v.z)) || (!isfinite(v.w));
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int c = lane; c < cols; c += 64) {
            float v = x[c];
            bad |= !isfinite(v);
            m = fmaxf(m, fabsf(v));
        }
    }
    m = wave_max_f(m);
    bad = wave_or_i(bad);
    QuantParams p = quant_params(m);
    if (bad || !p.ok) {
        if (lane == 0) raise_err(err, bad ? EF_NONFINITE_INPUT : EF_RANGE);
        return;
    }
    if (lane == 0) scale[r] = p.scale_f;
    const float inv = quant_inv_f(p.scale_d);
    if (vec) {
        const float4 *x4 = (const float4 *)x;
        uint32_t *q4 = (uint32_t *)q;
        for (int c = lane; c < (cols >> 2); c += 64) {
            const float4 v = x4[c];
            const uint32_t b0 = (uint8_t)quant_code_fast(v.x, p.scale_d, inv);
            const uint32_t b1 = (uint8_t)quant_code_fast(v.y, p.scale_d, inv);
            const uint32_t b2 = (uint8_t)quant_code_fast(v.z, p.scale_d, inv);
            const uint32_t b3 = (uint8_t)quant_code_fast(v.w, p.scale_d, inv);
            q4[c] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
    } else {
        for (int c = lane; c < cols; c += 64)
            q[c] = (int8_t)quant_code_fast(x[c], p.scale_d, inv);
    }
}

