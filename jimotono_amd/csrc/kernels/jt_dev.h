// Device-side helpers shared by the gfx950 kernels of libjimotono_hip.
//
// Numerics policy: every translation unit is compiled with
// -ffp-contract=off, so a*b+c below is a rounded multiply followed by a
// rounded add, as in the reference build (CMakeLists.txt:14-24). Where a
// fused multiply-add is used on purpose (fma()), the product is exact in
// fp64 and the fused form rounds identically to the separate one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define JT_WAVE 64

typedef int v4i __attribute__((ext_vector_type(4)));

// Error bits raised by kernels into the library's device error word.
#define EF_NONFINITE_INPUT 0x1u
#define EF_RANGE 0x2u
#define EF_NONFINITE_MID 0x4u
#define EF_BAD_ID 0x8u
#define EF_QRANGE 0x10u   // an int8 code of -128 (outside [-127, 127])

__device__ __forceinline__ void raise_err(uint32_t *err, uint32_t bits) {
    if (err) atomicOr(err, bits);
}

// ---- wavefront reductions (64 lanes) ----
// Wave reductions on DPP lane moves (no LDS traffic): row_shr 1, 2, 4, 8
// leaves each 16-lane row's result in its lane 15, row_bcast 15 and 31 carry
// rows into lane 63, which is then read as a scalar. Lanes without a DPP
// source keep their own value (old = v), so no identity element is needed.
#define JT_DPP(v, ctrl, rmask) \
    __builtin_amdgcn_update_dpp((v), (v), (ctrl), (rmask), 0xf, false)
template <typename Op>
__device__ __forceinline__ int wave_reduce_i(int v, Op op) {
    v = op(v, JT_DPP(v, 0x111, 0xf));  // row_shr:1
    v = op(v, JT_DPP(v, 0x112, 0xf));  // row_shr:2
    v = op(v, JT_DPP(v, 0x114, 0xf));  // row_shr:4
    v = op(v, JT_DPP(v, 0x118, 0xf));  // row_shr:8
    v = op(v, JT_DPP(v, 0x142, 0xa));  // row_bcast:15 into rows 1, 3
    v = op(v, JT_DPP(v, 0x143, 0xc));  // row_bcast:31 into rows 2, 3
    return __builtin_amdgcn_readlane(v, 63);
}
#undef JT_DPP
__device__ __forceinline__ float wave_max_f(float v) {
    return __builtin_bit_cast(float, wave_reduce_i(__builtin_bit_cast(int, v), [](int a, int b) {
        return __builtin_bit_cast(int, fmaxf(__builtin_bit_cast(float, a),
                                             __builtin_bit_cast(float, b)));
    }));
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    return (uint32_t)wave_reduce_i((int)v, [](int a, int b) {
        return (int)max((uint32_t)a, (uint32_t)b);
    });
}
// bits of |x|
__device__ __forceinline__ uint32_t abs_bits(float x) {
    return __builtin_bit_cast(uint32_t, x) & 0x7fffffffu;
}
__device__ __forceinline__ int wave_sum_i(int v) {
    return wave_reduce_i(v, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ int wave_or_i(int v) {
    return wave_reduce_i(v, [](int a, int b) { return a | b; });
}

// ---- the reference's int8 quantiser (src/w8a8.c:815-850) ----
// scale_d = maxabs / 127 (fp64 divide), stored scale (float)scale_d,
// q = clamp(round(x / scale_d), -127, 127), round half away from zero.
// maxabs == 0 -> scale 1 and all codes 0.
struct QuantParams {
    double scale_d;  // 0 when the row is all zero
    float scale_f;
    bool ok;
};
__device__ __forceinline__ QuantParams quant_params(float maxabs_f) {
    QuantParams p;
    double maxabs = (double)maxabs_f;
    if (maxabs == 0.0) {
        p.scale_d = 0.0;
        p.scale_f = 1.0f;
        p.ok = true;
        return p;
    }
    p.scale_d = maxabs / 127.0;
    p.scale_f = (float)p.scale_d;
    p.ok = isfinite(p.scale_d) && p.scale_d > 0.0 && isfinite(p.scale_f) &&
           p.scale_f > 0.0f;
    return p;
}
__device__ __forceinline__ int quant_code(float x, double scale_d) {
    if (scale_d == 0.0) return 0;
    double qd = round((double)x / scale_d);
    qd = qd > 127.0 ? 127.0 : (qd < -127.0 ? -127.0 : qd);
    return (int)qd;
}
// Same code as quant_code without fp64 per element: y = x * inv_f with
// inv_f = (float)(1/scale_d) differs from the exact quotient x/scale_d by
// less than 2^-22 relative (two fp32 roundings and the fp64 reciprocal),
// i.e. < 3.1e-5 absolute for |x/scale_d| <= 128. round-half-away of the two
// can differ only if a half-integer lies between them, so whenever y is
// within 1e-4 of a half-integer (|y - rint(y)| > 0.4999) the exact fp64
// quotient is recomputed; otherwise rint(y) is not a tie and equals the
// exact round-half-away code.
__device__ __forceinline__ int quant_code_fast(float x, double scale_d, float inv_f) {
    if (scale_d == 0.0) return 0;
    if (!(inv_f < __builtin_inff())) return quant_code(x, scale_d);  // 1/scale_d > FLT_MAX
    const float y = x * inv_f;
    const float q = rintf(y);  // y - q is exact; no tie outside the guard band
    if (fabsf(y - q) > 0.4999f) return quant_code(x, scale_d);
    return (int)__builtin_amdgcn_fmed3f(q, -127.0f, 127.0f);
}
// inv_f for quant_code_fast: (float)(1/scale_d), 0 for an all-zero row
__device__ __forceinline__ float quant_inv_f(double scale_d) {
    return scale_d != 0.0 ? (float)(1.0 / scale_d) : 0.0f;
}

// ---- IEEE binary16 <-> binary64, round to nearest even ----
__device__ __forceinline__ double f16_to_f64(uint16_t h) {
    int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? __builtin_nan("") : __builtin_inf();
    else v = ldexp((double)(m + 1024), e - 25);
    return s ? -v : v;
}
__device__ __forceinline__ uint16_t f64_to_f16(double x) {
    uint16_t sign = signbit(x) ? 0x8000u : 0u;
    if (isnan(x)) return (uint16_t)(sign | 0x7e00u);
    double a = fabs(x);
    if (a == 0.0) return sign;
    if (isinf(a)) return (uint16_t)(sign | 0x7c00u);
    int e;
    (void)frexp(a, &e);
    int E = e - 1;
    if (E < -14) {
        double q = rint(ldexp(a, 24));
        return (uint16_t)(sign | (uint16_t)q);
    }
    double q = rint(ldexp(a, 10 - E));
    if (q >= 2048.0) {
        q = 1024.0;
        E += 1;
    }
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((E + 15) << 10) |
                      (uint16_t)(q - 1024.0));
}

// ---- odd-symmetric low-bit level (src/lowbit.c:78-86) ----
__device__ __forceinline__ int lowbit_code(double w, double maxabs, int bits) {
    int nl = 1 << bits;
    double t = (maxabs == 0.0) ? 0.0 : w / maxabs;
    double li = floor(t * (double)(nl - 1) / 2.0 + (double)(nl - 1) / 2.0 + 0.5);
    long l = (long)li;
    if (l < 0) l = 0;
    if (l > (long)(nl - 1)) l = nl - 1;
    return (int)l;
}

// ---- SwiGLU of the reference (src/moe_layer.c:139-156) ----
__device__ __forceinline__ bool silu_mul(float g, float u, float *s) {
    double gi = (double)g, ui = (double)u;
    double sig = 1.0 / (1.0 + exp(-gi));
    double silu = gi * sig;
    double v = silu * ui;
    *s = (float)v;
    return isfinite(v) && isfinite(sig) && isfinite(silu);
}

// ---- panel layouts of prepared weights ----
// A weight matrix W[N][K] (N output channels, K reduction) is stored as
// panels of 16 channels x 64 K. Inside a panel, lane l = kc*16 + c
// (kc = k-chunk 0..3, c = channel 0..15) owns the 16 consecutive K values
// k = 64*kb + 16*kc + 0..15 of channel c, which is the per-lane operand
// layout of v_mfma_i32_16x16x64_i8. Panel (p, kb) starts at
// (p * (K/64) + kb) * PANEL_BYTES.
//   int8: 16 bytes per lane, byte b = code of k offset b     (1024 B/panel)
//   INT4: 8 bytes per lane; value of k offset 4o+j is nibble (o%2) of
//         byte j of dword o/2                               (512 B/panel)
//   INT2: 4 bytes per lane; value of k offset 4o+j is bits [8j+2o, 8j+2o+1]
//                                                           (256 B/panel)
// Low-bit codes are the level index li; the signed value is 2*li-(2^bits-1).
// fp16 group scales (group = 64 = one panel K block) are stored as
// [N/16][K/64][16] uint16.

// INT2 codes (li in 0..3, 4 per byte lane layout above) -> 4 dwords of
// signed int8 values {-3,-1,1,3}: one byte-select per dword.
__device__ __forceinline__ v4i unpack_int2(uint32_t w) {
    const uint32_t lut = 0x0301FFFDu;  // bytes: li0=-3, li1=-1, li2=1, li3=3
    v4i r;
    r.x = (int)__builtin_amdgcn_perm(0u, lut, w & 0x03030303u);
    r.y = (int)__builtin_amdgcn_perm(0u, lut, (w >> 2) & 0x03030303u);
    r.z = (int)__builtin_amdgcn_perm(0u, lut, (w >> 4) & 0x03030303u);
    r.w = (int)__builtin_amdgcn_perm(0u, lut, (w >> 6) & 0x03030303u);
    return r;
}
// INT4 codes (li in 0..15) -> signed int8 2*li-15, per byte without
// inter-byte borrow: ((2li+1) | 0x80) - 0x10, then flip bit 7 back.
__device__ __forceinline__ int int4_bytes(uint32_t nib) {
    uint32_t x = (nib << 1) | 0x81818181u;
    return (int)((x - 0x10101010u) ^ 0x80808080u);
}
__device__ __forceinline__ v4i unpack_int4(uint32_t w0, uint32_t w1) {
    v4i r;
    r.x = int4_bytes(w0 & 0x0F0F0F0Fu);
    r.y = int4_bytes((w0 >> 4) & 0x0F0F0F0Fu);
    r.z = int4_bytes(w1 & 0x0F0F0F0Fu);
    r.w = int4_bytes((w1 >> 4) & 0x0F0F0F0Fu);
    return r;
}

__device__ __forceinline__ v4i mfma16x16x64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
