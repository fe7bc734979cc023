// Device-side helpers shared by the gfx950 kernels of libjimotono_hip.
//
// Numerics policy: every translation unit is compiled with
// -ffp-contract=off, so a*b+c below is a rounded multiply followed by a
// rounded add, as in the reference build (CMakeLists.txt:14-24). Where a
// fused multiply-add is used on purpose (fma()), the product is exact in
// fp64 and the fused form rounds identically to the separate one.
#pragma once
#include <hip/hip_runtime.h>
#include <atomic>
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
// the same on 64-bit values (both halves move with the same DPP control);
// the maximum is returned to every lane
template <int CTRL, int RMASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, RMASK, 0xf, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, RMASK, 0xf, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    return o > v ? o : v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_u64<0x111, 0xf>(v);  // row_shr:1
    v = dpp_max_u64<0x112, 0xf>(v);  // row_shr:2
    v = dpp_max_u64<0x114, 0xf>(v);  // row_shr:4
    v = dpp_max_u64<0x118, 0xf>(v);  // row_shr:8
    v = dpp_max_u64<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_max_u64<0x143, 0xc>(v);  // row_bcast:31
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}
// max over the 16 lanes of each DPP row, in every lane of the row (row
// rotations 1, 2, 4, 8)
__device__ __forceinline__ uint32_t row16_allmax_u(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x121, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x122, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x124, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xf, 0xf, false));
    return v;
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
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
// The guard-band test of quant_code_fast without its fallback, for unrolled
// rows: the exact path inlined at each of 64 codes would make a kernel tens
// of KiB long (a decode-sized launch then waits on instruction fetch), so
// the caller recomputes with quant_code the codes whose `fail` came back set.
// inv_f = 0 (all-zero row) gives code 0; inv_f = inf makes y - q NaN and
// so fails, like the explicit test in quant_code_fast.
__device__ __forceinline__ int quant_code_try(float x, float inv_f, bool &fail) {
    const float y = x * inv_f;
    const float q = rintf(y);
    fail |= !(fabsf(y - q) <= 0.4999f);
    return (int)__builtin_amdgcn_fmed3f(q, -127.0f, 127.0f);
}
// quant_code as a real call, for rare fallbacks inside unrolled code
__device__ __attribute__((noinline)) int quant_code_call(float x, double scale_d) {
    return quant_code(x, scale_d);
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

// ---- exp for the SwiGLU, fp64 ----
// Tang's table-driven method (ACM TOMS 15(2), 1989): x = (64m + j) ln2/64 + r
// with |r| <= ln2/128, exp(x) = 2^m * 2^(j/64) * e^r, e^r from its degree-5
// Taylor polynomial (truncation below 2^-54 relative), applied as
// t + t (e^r - 1) with one rounding. ln2/64 is split in two parts
// (Cody-Waite) so the reduction is accurate to a few ulp of r. Within about
// an ulp of exp; x is clamped to [-746, 710], where the double result is 0
// and inf.
__device__ const double jt_exp2_64th[64] = {
    1.0, 1.0108892860517005, 1.0218971486541166, 1.0330248790212284,
    1.0442737824274138, 1.0556451783605572, 1.0671404006768237, 1.0787607977571199,
    1.0905077326652577, 1.102382583307841, 1.1143867425958924, 1.1265216186082418,
    1.1387886347566916, 1.1511892299529827, 1.1637248587775775, 1.1763969916502812,
    1.189207115002721, 1.202156731452703, 1.215247359980469, 1.22848053610687,
    1.241857812073484, 1.255380757024691, 1.2690509571917332, 1.2828700160787783,
    1.2968395546510096, 1.3109612115247644, 1.3252366431597413, 1.339667524053303,
    1.3542555469368927, 1.3690024229745905, 1.383909881963832, 1.3989796725383112,
    1.4142135623730951, 1.42961333839197, 1.4451808069770467, 1.460917794180647,
    1.4768261459394993, 1.4929077282912648, 1.5091644275934228, 1.5255981507445384,
    1.5422108254079407, 1.559004400237837, 1.5759808451078865, 1.593142151342267,
    1.6104903319492543, 1.6280274218573478, 1.645755478153965, 1.6636765803267364,
    1.681792830507429, 1.7001063537185235, 1.718619298122478, 1.7373338352737062,
    1.7562521603732995, 1.7753764925265212, 1.7947090750031072, 1.8142521755003989,
    1.8340080864093424, 1.8539791250833855, 1.8741676341103, 1.8945759815869656,
    1.9152065613971474, 1.9360617934922943, 1.9571441241754002, 1.978456026387951};
template <typename TAB>
__device__ __forceinline__ double exp_tang(double x, const TAB &tab) {
    x = fmin(fmax(x, -746.0), 710.0);
    const double kd = rint(x * 92.33248261689366);  // 64 / ln2
    const int k = (int)kd;
    double r = fma(-kd, 0.010830424696249145, x);  // ln2/64, high part
    r = fma(-kd, 3.623510646634843e-19, r);        // low part
    double q = fma(r, 1.0 / 120.0, 1.0 / 24.0);  // e^r - 1 = r (1 + r/2 + ...)
    q = fma(r, q, 1.0 / 6.0);
    q = fma(r, q, 0.5);
    q = fma(r, q, 1.0);
    q *= r;
    const double t = tab[k & 63];
    return ldexp(fma(t, q, t), k >> 6);  // t (1 + q) with one rounding
}
__device__ __forceinline__ double exp_tang(double x) { return exp_tang(x, jt_exp2_64th); }

// The table in LDS: a kernel declares `__shared__ double tab[64]` and, where
// the whole wavefront is active, each wave stores lane l's entry l
// (exp_tab_stage, the entry loaded with the other epilogue loads by
// exp_tab_load). Every wave writes the same values, so the overlapping
// stores are benign, and a wave's LDS operations are processed in order,
// so the wave's own reads after its stores see the table without a
// barrier. The per-element lookup is then an LDS read: a global load per
// element made each element wait on vmcnt, which also counts the stores
// of the elements before it.
__device__ __forceinline__ double exp_tab_load(int lane) { return jt_exp2_64th[lane & 63]; }
__device__ __forceinline__ void exp_tab_stage(double *tab, int lane, double v) {
    tab[lane & 63] = v;
}
// 1/d for 1 <= d < 2^1000: hardware reciprocal and two Newton steps (within
// an ulp of the correctly rounded quotient)
__device__ __forceinline__ double recip_ge1(double d) {
    double r = __builtin_amdgcn_rcp(d);
    double e = fma(-d, r, 1.0);
    r = fma(r, e, r);
    e = fma(-d, r, 1.0);
    return fma(r, e, r);
}

// ---- SwiGLU of the reference (src/moe_layer.c:139-156) ----
// v = (g * (1 / (1 + exp(-g)))) * u in fp64, rounded to float, with the
// reference's operation order. exp and the reciprocal are each within about
// an ulp of the reference's glibc results, so v differs from the
// reference's only where it lies within a few 1e-16 of a float rounding
// boundary. The reference's finiteness test on sig, silu and v fails
// exactly when g or u is not finite (for finite g, sig is in [0, 1] and v is
// a finite double), which is what is returned.
template <typename TAB>
__device__ __forceinline__ bool silu_mul(float g, float u, float *s, const TAB &tab) {
    const double gi = (double)g, ui = (double)u;
    const double ex = exp_tang(-gi, tab);
    const double sig = ex > 1e300 ? 0.0 : recip_ge1(1.0 + ex);
    const double silu = gi * sig;
    *s = (float)(silu * ui);
    return isfinite(g) && isfinite(u);
}
__device__ __forceinline__ bool silu_mul(float g, float u, float *s) {
    return silu_mul(g, u, s, jt_exp2_64th);
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
