// Gated DeltaNet-2 (the reference's src/gdn2.c) on gfx950: the decode step
// and the WY-form prefill chunk, batched over independent heads.
//
// Every output keeps the reference's fp32 operation order (separate
// multiply and add roundings, the same summation chains), so results are
// bit-identical to src/gdn2.c. Both kernels run the columns j of a head's
// state S [dk][dv] in parallel: the reference's update treats each column
// independently once the per-head vectors (normalised q/k, decay products,
// the WY matrices) are known.
//
//  k_gdn2_decode      : one block per head. Checks the head's inputs (a bad
//                       head raises EF_NONFINITE_INPUT and is left as it
//                       was), the two L2 norms (sequential fp64 sums, as
//                       src/gdn2.c:219-250), then per column: decay and the
//                       erase coefficient (pass 1), erase + write + read-out
//                       (pass 2), src/gdn2.c:333-405.
//  k_gdn2_check       : a prefill's inputs, per head, before any chunk.
//  k_gdn2_prep        : per (chunk, head), all chunks at once: everything
//                       that does not depend on the state -- norms, ke, the
//                       decay products, the strictly lower L and the lower
//                       P (src/gdn2.c:537-714), the row weights of the state
//                       update (:768-788).
//  k_gdn2_cols        : per (head, 256/C columns), every chunk in order in
//                       one launch: B, the forward substitution, Out and the
//                       state update (:614-680, 716-842).
#include "jt_dev.h"
#include "jt_launch.h"

namespace {

constexpr float GDN2_EPS = 1e-6f;

// 1 / ||x|| as the reference rounds it: fp64 sum of squares in index order,
// fp64 sqrt and divide, then float; *zero when the norm is below eps.
// The loads go out 16 at a time ahead of the ordered sum.
__device__ __forceinline__ float inv_norm(const float *x, int n, bool *zero) {
    double ss = 0.0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = x[i + u];
#pragma unroll
        for (int u = 0; u < 16; u++) ss = ss + (double)v[u] * (double)v[u];
    }
    for (; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
    const double nrm = sqrt(ss);
    *zero = nrm < (double)GDN2_EPS;
    return *zero ? 0.0f : (float)(1.0 / nrm);
}

__device__ __forceinline__ bool bad_vec(const float *x, int n, int tid, int nt) {
    bool bad = false;
    for (int i = tid; i < n; i += nt) bad |= !isfinite(x[i]);
    return bad;
}

__device__ __forceinline__ bool bad_alpha(const float *a, int n, int tid, int nt) {
    bool bad = false;
    for (int i = tid; i < n; i += nt) bad |= !(a[i] >= 0.0f && a[i] <= 1.0f);
    return bad;
}

// LDS: qn, kn, ke, al [dk] (dk <= 1024). One thread per column (blockDim
// = dv rounded up to 64, at most 256). Both passes read the column in
// chunks of 64 rows (then 32, then single rows), all of a chunk's loads
// issued before its ordered arithmetic (measured at 512 heads of 128x128:
// 18.3 us against 20.0 us with chunks of 32 and 20.9 us with 128); pass 2 re-reads the column (from cache) and recomputes the
// decayed value, which is the same product as pass 1's.
__global__ __launch_bounds__(256) void k_gdn2_decode(float *__restrict__ S, float *__restrict__ O,
                                                     const float *__restrict__ q,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     const float *__restrict__ b,
                                                     const float *__restrict__ w,
                                                     const float *__restrict__ alpha, int dk,
                                                     int dv, uint32_t *err) {
    __shared__ float qn[1024], kn[1024], ke[1024], al[1024];
    __shared__ float invs[2];
    __shared__ int zeros[2];
    const int h = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
    const float *qh = q + (int64_t)h * dk, *kh = k + (int64_t)h * dk;
    const float *bh = b + (int64_t)h * dk, *ah = alpha + (int64_t)h * dk;
    const float *vh = v + (int64_t)h * dv, *wh = w + (int64_t)h * dv;
    float *Sh = S + (int64_t)h * dk * dv, *Oh = O + (int64_t)h * dv;
    bool bad = bad_vec(qh, dk, tid, nt) || bad_vec(kh, dk, tid, nt) || bad_vec(bh, dk, tid, nt) ||
               bad_vec(ah, dk, tid, nt) || bad_alpha(ah, dk, tid, nt) ||
               bad_vec(vh, dv, tid, nt) || bad_vec(wh, dv, tid, nt);
    if (__syncthreads_or(bad)) {  // fail-closed: this head's S and o untouched
        if (tid == 0) raise_err(err, EF_NONFINITE_INPUT);
        return;
    }
    for (int i = tid; i < dk; i += nt) {  // raw q, k into LDS for the norms
        qn[i] = qh[i];
        kn[i] = kh[i];
        al[i] = ah[i];
    }
    __syncthreads();
    const int kt = nt > 64 ? 64 : 1;  // the k norm on a second wave when there is one
    if (tid == 0 || tid == kt) {
        bool z;
        const float iv = inv_norm(tid ? kn : qn, dk, &z);
        invs[tid ? 1 : 0] = iv;
        zeros[tid ? 1 : 0] = z;
    }
    __syncthreads();
    for (int i = tid; i < dk; i += nt) {
        const float qi = zeros[0] ? 0.0f : qn[i] * invs[0];
        const float ki = zeros[1] ? 0.0f : kn[i] * invs[1];
        qn[i] = qi;
        kn[i] = ki;
        ke[i] = bh[i] * ki;
    }
    __syncthreads();
    for (int j = tid; j < dv; j += nt) {
        const float *col = Sh + j;
        float c = 0.0f, o = 0.0f;
        const float vw = wh[j] * vh[j];
        // rows in chunks of 64, then one of 32, then one at a time; each
        // chunk's loads all issue before its ordered arithmetic
        int i0 = 0;
        for (; i0 + 64 <= dk; i0 += 64) {
            float x[64];
#pragma unroll
            for (int u = 0; u < 64; u++) x[u] = col[(int64_t)(i0 + u) * dv];
#pragma unroll
            for (int u = 0; u < 64; u++) c = c + ke[i0 + u] * (x[u] * al[i0 + u]);
        }
        for (; i0 + 32 <= dk; i0 += 32) {
            float x[32];
#pragma unroll
            for (int u = 0; u < 32; u++) x[u] = col[(int64_t)(i0 + u) * dv];
#pragma unroll
            for (int u = 0; u < 32; u++) c = c + ke[i0 + u] * (x[u] * al[i0 + u]);
        }
        for (; i0 < dk; i0++) c = c + ke[i0] * (col[(int64_t)i0 * dv] * al[i0]);
        auto upd = [&](int i, float xv) {
            float r = xv * al[i] - kn[i] * c;
            r = r + kn[i] * vw;
            Sh[(int64_t)i * dv + j] = r;
            o = o + qn[i] * r;
        };
        i0 = 0;
        for (; i0 + 64 <= dk; i0 += 64) {
            float x[64];
#pragma unroll
            for (int u = 0; u < 64; u++) x[u] = col[(int64_t)(i0 + u) * dv];
#pragma unroll
            for (int u = 0; u < 64; u++) upd(i0 + u, x[u]);
        }
        for (; i0 + 32 <= dk; i0 += 32) {
            float x[32];
#pragma unroll
            for (int u = 0; u < 32; u++) x[u] = col[(int64_t)(i0 + u) * dv];
#pragma unroll
            for (int u = 0; u < 32; u++) upd(i0 + u, x[u]);
        }
        for (; i0 < dk; i0++) upd(i0, col[(int64_t)i0 * dv]);
        Oh[j] = o;
    }
}

// flag[h] |= 1 when head h's inputs (nk values of each dk-wide array from
// h*hk, nv of each dv-wide one from h*hv) hold a non-finite value or an
// alpha outside [0,1]; the later kernels leave such a head as it was.
// blockIdx.y = head, blockIdx.x strides over the values; flag zeroed before.
__global__ __launch_bounds__(256) void k_gdn2_check(const float *__restrict__ Q,
                                                    const float *__restrict__ K,
                                                    const float *__restrict__ B,
                                                    const float *__restrict__ A,
                                                    const float *__restrict__ V,
                                                    const float *__restrict__ W, int64_t hk,
                                                    int64_t hv, int nk, int nv,
                                                    int *__restrict__ flag, uint32_t *err) {
    const int h = blockIdx.y;
    const int i0 = blockIdx.x * 256 + threadIdx.x, st = gridDim.x * 256;
    const float *q = Q + h * hk, *k = K + h * hk, *b = B + h * hk, *a = A + h * hk;
    const float *v = V + h * hv, *w = W + h * hv;
    bool bad = false;
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)b | (uintptr_t)a |
                         (uintptr_t)v | (uintptr_t)w;
    if (((nk | nv) & 3) == 0 && (al & 15) == 0) {
        // 16-byte loads, four element groups of each array per thread in flight
        auto fin = [](float4 x) {
            return isfinite(x.x) && isfinite(x.y) && isfinite(x.z) && isfinite(x.w);
        };
        auto unit = [](float4 x) {
            return x.x >= 0.0f && x.x <= 1.0f && x.y >= 0.0f && x.y <= 1.0f && x.z >= 0.0f &&
                   x.z <= 1.0f && x.w >= 0.0f && x.w <= 1.0f;
        };
        const float4 *q4 = (const float4 *)q, *k4 = (const float4 *)k, *b4 = (const float4 *)b;
        const float4 *a4 = (const float4 *)a, *v4 = (const float4 *)v, *w4 = (const float4 *)w;
#pragma unroll 4
        for (int i = i0; i < nk / 4; i += st)
            bad |= !fin(q4[i]) || !fin(k4[i]) || !fin(b4[i]) || !unit(a4[i]);
#pragma unroll 4
        for (int i = i0; i < nv / 4; i += st) bad |= !fin(v4[i]) || !fin(w4[i]);
    } else {
        for (int i = i0; i < nk; i += st)
            bad |= !isfinite(q[i]) || !isfinite(k[i]) || !isfinite(b[i]) ||
                   !(a[i] >= 0.0f && a[i] <= 1.0f);
        for (int i = i0; i < nv; i += st) bad |= !isfinite(v[i]) || !isfinite(w[i]);
    }
    bad = wave_or_i(bad);
    if (bad && (threadIdx.x & 63) == 0) {
        atomicOr(&flag[h], 1);
        raise_err(err, EF_NONFINITE_INPUT);
    }
}

// Record of one (head, chunk) in the prefill workspace (floats): CF
// (forward decay products alpha_0..t), WI = ke*CF, QI = q*CF, WG (row
// weights of the state update) [C][dk]; L, P [C][C]; and, when the chunk's
// operands do not fit in LDS, Qn, Kn, KE [C][dk].
__host__ __device__ constexpr int64_t chunk_rec_floats(int C, int dk) {
    return 7LL * C * dk + 2LL * C * C;
}

// Everything of a chunk that does not depend on the state: one block per
// (chunk, head), all chunks of a prefill at once. Norms, ke, the decay
// products and the WY matrices: L[t][s] = (ke_t*cum(t,s)).k_s (t > s),
// P[t][s] = (q_t*cum(t,s)).k_s (t >= s), cum(t,s) = alpha_{s+1}*...*alpha_t
// in that order, each a sum in four chains over i % 4 (the tail
// i >= dk & ~3 into chain 0), then (c0+c1)+(c2+c3) (src/gdn2.c:537-714,
// 768-788). CL: the chunk's operands live in LDS (C*dk <= CHUNK_LDS),
// rows at stride dk + 4 so lanes on different rows fall on distinct banks;
// the decay products are formed once per (s, i) in t order. Otherwise
// thread (t, s, chain) forms its own products.
constexpr int CHUNK_LDS = 4096;
template <bool CL>
__global__ __launch_bounds__(256) void k_gdn2_prep(const float *__restrict__ Q,
                                                   const float *__restrict__ K,
                                                   const float *__restrict__ B,
                                                   const float *__restrict__ A, int64_t hk,
                                                   int C, int dk, const int *__restrict__ flag,
                                                   float *__restrict__ rec) {
    __shared__ float invs[64];
    __shared__ int zeros[64];
    __shared__ float part[2][CL ? 2 : 32][32][4];  // [L/P][s (of the pair)][t][chain]
    constexpr int NL = CL ? CHUNK_LDS + 4 * 32 : 1;
    __shared__ float a_l[NL], q_l[NL], k_l[NL], e_l[NL];
    __shared__ float term_l[2][2][CL ? NL : 1];  // [L/P][s of the pair][t][i]
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lk = dk + 4;
    if (flag[h]) return;
    const int64_t Ck = (int64_t)C * dk;
    const int64_t at0 = h * hk + c * Ck;
    const float *Qh = Q + at0, *Kh = K + at0, *Bh = B + at0, *Ah = A + at0;
    float *r = rec + ((int64_t)h * gridDim.x + c) * chunk_rec_floats(C, dk);
    float *CF = r, *WI = CF + Ck, *QI = WI + Ck, *WG = QI + Ck;
    float *L = WG + Ck, *P = L + (int64_t)C * C, *Qn = P + (int64_t)C * C, *Kn = Qn + Ck;
    float *KE = Kn + Ck;
    if (CL) {  // raw rows into LDS for the norms
        for (int64_t n = tid; n < Ck; n += 256) {
            const int t = (int)(n / dk), i = (int)(n % dk);
            q_l[t * lk + i] = Qh[n];
            k_l[t * lk + i] = Kh[n];
            a_l[t * lk + i] = Ah[n];
        }
        __syncthreads();
    }
    if (tid < 2 * C) {  // one row norm per thread
        const int t = tid % C;
        bool z;
        const float *row = CL ? (tid < C ? q_l : k_l) + t * lk : (tid < C ? Qh : Kh) + (int64_t)t * dk;
        invs[tid] = inv_norm(row, dk, &z);
        zeros[tid] = z;
    }
    __syncthreads();
    for (int64_t n = tid; n < Ck; n += 256) {
        const int t = (int)(n / dk), i = (int)(n % dk), l = t * lk + i;
        const float qv = zeros[t] ? 0.0f : (CL ? q_l[l] : Qh[n]) * invs[t];
        const float kv = zeros[C + t] ? 0.0f : (CL ? k_l[l] : Kh[n]) * invs[C + t];
        const float ev = Bh[n] * kv;
        if (CL) {
            q_l[l] = qv;
            k_l[l] = kv;
            e_l[l] = ev;
        } else {
            Qn[n] = qv;
            Kn[n] = kv;
            KE[n] = ev;
        }
    }
    __syncthreads();
    const float *Ab = CL ? a_l : Ah, *Eb = CL ? e_l : KE, *Qb = CL ? q_l : Qn;
    const float *Kb = CL ? k_l : Kn;
    const int ld = CL ? lk : dk;  // row stride of those operands
    for (int i = tid; i < dk; i += 256) {
        float cf = 1.0f;  // alpha_0 * ... * alpha_t, t ascending
        for (int t = 0; t < C; t++) {
            cf = cf * Ab[t * ld + i];
            CF[(int64_t)t * dk + i] = cf;
            WI[(int64_t)t * dk + i] = Eb[t * ld + i] * cf;
            QI[(int64_t)t * dk + i] = Qb[t * ld + i] * cf;
        }
        float sf = 1.0f;  // alpha_{s+1} * ..., accumulated from the end
        for (int s = C - 1; s >= 0; s--) {
            WG[(int64_t)s * dk + i] = Kb[s * ld + i] * sf;
            sf = sf * Ab[s * ld + i];
        }
    }
    const int dk4 = dk & ~3;
    if (CL) {
        // two s at a time: thread (s, i) walks t upward forming cum(t,s)[i]
        // and the two terms of every (t, s) chain element into LDS; then
        // thread (t, s, chain) sums its chain in i order
        for (int s0 = 0; s0 < C; s0 += 2) {
            for (int idx = tid; idx < 2 * dk; idx += 256) {
                const int sl = idx / dk, i = idx % dk, s = s0 + sl;
                const float ks = Kb[s * ld + i];
                float cu = 1.0f;
                for (int t = s; t < C; t++) {
                    if (t > s) cu = cu * Ab[t * ld + i];
                    term_l[0][sl][t * lk + i] = (Eb[t * ld + i] * cu) * ks;
                    term_l[1][sl][t * lk + i] = (Qb[t * ld + i] * cu) * ks;
                }
            }
            __syncthreads();
            for (int job = tid; job < 2 * C * 4; job += 256) {
                const int ch = job & 3, t = (job >> 2) % C, sl = job / (4 * C), s = s0 + sl;
                if (s > t) continue;
                const float *tl = term_l[0][sl] + t * lk, *tp = term_l[1][sl] + t * lk;
                float lsum = 0.0f, psum = 0.0f;
                for (int i = ch; i < dk4; i += 4) {
                    lsum = lsum + tl[i];
                    psum = psum + tp[i];
                }
                if (ch == 0)
                    for (int i = dk4; i < dk; i++) {
                        lsum = lsum + tl[i];
                        psum = psum + tp[i];
                    }
                part[0][sl][t][ch] = lsum;
                part[1][sl][t][ch] = psum;
            }
            __syncthreads();
            for (int pr = tid; pr < 2 * C; pr += 256) {
                const int t = pr % C, sl = pr / C, s = s0 + sl;
                const float *pl = part[0][sl][t], *pp = part[1][sl][t];
                L[t * C + s] = s < t ? (pl[0] + pl[1]) + (pl[2] + pl[3]) : 0.0f;
                P[t * C + s] = s <= t ? (pp[0] + pp[1]) + (pp[2] + pp[3]) : 0.0f;
            }
        }
    } else {
        for (int job = tid; job < 4 * C * C; job += 256) {
            const int ch = job & 3, pr = job >> 2, t = pr / C, s = pr % C;
            if (s > t) continue;
            const float *ks = Kb + s * ld, *qt = Qb + t * ld, *et = Eb + t * ld;
            float lsum = 0.0f, psum = 0.0f;
            auto term = [&](int i) {
                float cu = 1.0f;
                for (int rr = s + 1; rr <= t; rr++) cu = cu * Ab[rr * ld + i];
                lsum = lsum + (et[i] * cu) * ks[i];
                psum = psum + (qt[i] * cu) * ks[i];
            };
            for (int i = ch; i < dk4; i += 4) term(i);
            if (ch == 0)
                for (int i = dk4; i < dk; i++) term(i);
            part[0][s][t][ch] = lsum;
            part[1][s][t][ch] = psum;
        }
        __syncthreads();
        for (int pr = tid; pr < C * C; pr += 256) {
            const int t = pr / C, s = pr % C;
            const float *pl = part[0][s][t], *pp = part[1][s][t];
            L[pr] = s < t ? (pl[0] + pl[1]) + (pl[2] + pl[3]) : 0.0f;
            P[pr] = s <= t ? (pp[0] + pp[1]) + (pp[2] + pp[3]) : 0.0f;
        }
    }
}

// The state recurrence over all chunks, in order, in one launch: one block
// per (head, NC = 256/C columns) -- the columns of S never mix. Per chunk,
// phase 1 thread (t, column) runs the chains over i of
// B_t = vw_t - sum_i WI[t][i] S[i] and Out_t = sum_i QI[t][i] S[i]; phase 2
// the forward substitution (I + L) E = B per column with the column's C
// values in registers; phase 3 Out_t += sum_{s<=t} P[t][s] E_s; phase 4
// thread (i, column) S[i] <- CF[C-1][i] S[i] + sum_s WG[s][i] E_s
// (src/gdn2.c:614-680, 716-842). CL: each chunk's record is staged in LDS
// and the block's S tile stays in LDS from the first chunk to the last.
// (CL with dk % 4 == 0 runs as k_gdn2_cols4 below.)
template <int C, bool CL>
__global__ __launch_bounds__(256) void k_gdn2_cols(float *__restrict__ S, float *__restrict__ Out,
                                                   const float *__restrict__ V,
                                                   const float *__restrict__ W, int64_t hv,
                                                   int nch, int dk, int dv,
                                                   const int *__restrict__ flag,
                                                   const float *__restrict__ rec) {
    constexpr int NC = 256 / C;
    constexpr int NL = CL ? CHUNK_LDS + 4 * 32 : 1;
    __shared__ float G[C][NC], Ob[C][NC];
    // the S tile: dk*NC <= CHUNK_LDS*NC/C values when C*dk <= CHUNK_LDS
    __shared__ __attribute__((aligned(16))) float wi_l[NL], qi_l[NL], wg_l[NL];
    __shared__ float s_l[CL ? CHUNK_LDS * NC / C : 1];
    __shared__ __attribute__((aligned(16))) float lp_l[CL ? 2 * C * C : 1], cf_l[CL ? 1024 : 1];
    const int h = blockIdx.x, j0 = blockIdx.y * NC, tid = threadIdx.x, lk = dk + 4;
    if (flag[h]) return;  // a rejected head keeps its S and Out
    const int64_t Ck = (int64_t)C * dk;
    float *Sh = S + (int64_t)h * dk * dv;
    const int ncol = min(NC, dv - j0);
    const int t = tid / NC, jj = tid % NC, j = j0 + jj;
    const bool live = jj < ncol;
    const int ld = CL ? lk : dk;
    if (CL) {
        for (int n = tid; n < dk * NC; n += 256) {
            const int i = n / NC, cc = n % NC;
            s_l[n] = cc < ncol ? Sh[(int64_t)i * dv + j0 + cc] : 0.0f;
        }
    }
    for (int c = 0; c < nch; c++) {
        const float *r = rec + ((int64_t)h * nch + c) * chunk_rec_floats(C, dk);
        const float *CF = r, *WI = CF + Ck, *QI = WI + Ck, *WG = QI + Ck;
        const float *L = WG + Ck, *P = L + C * C;
        if (CL) {
            for (int64_t n = tid; n < Ck; n += 256) {
                const int tt = (int)(n / dk), i = (int)(n % dk);
                wi_l[tt * lk + i] = WI[n];
                qi_l[tt * lk + i] = QI[n];
                wg_l[tt * lk + i] = WG[n];
            }
            for (int n = tid; n < 2 * C * C; n += 256) lp_l[n] = L[n];  // L then P
            for (int i = tid; i < dk; i += 256) cf_l[i] = CF[(int64_t)(C - 1) * dk + i];
            __syncthreads();
        }
        const float *wi_b = CL ? wi_l : WI, *qi_b = CL ? qi_l : QI, *wg_b = CL ? wg_l : WG;
        const float *L_b = CL ? lp_l : L, *P_b = CL ? lp_l + C * C : P;
        const int64_t vo = h * hv + ((int64_t)c * C + t) * dv + j;
        if (live) {
            float g = W[vo] * V[vo];  // vw_t
            float o = 0.0f;
            const float *wi = wi_b + t * ld, *qi = qi_b + t * ld;
#pragma unroll 8
            for (int i = 0; i < dk; i++) {
                const float sv = CL ? s_l[i * NC + jj] : Sh[(int64_t)i * dv + j];
                g = g - wi[i] * sv;
                o = o + qi[i] * sv;
            }
            G[t][jj] = g;
            Ob[t][jj] = o;
        }
        __syncthreads();
        if (tid < ncol) {
            float g[C];
#pragma unroll
            for (int tt = 0; tt < C; tt++) g[tt] = G[tt][tid];
#pragma unroll
            for (int tt = 1; tt < C; tt++)
#pragma unroll
                for (int s = 0; s < tt; s++) g[tt] = g[tt] - L_b[tt * C + s] * g[s];
#pragma unroll
            for (int tt = 0; tt < C; tt++) G[tt][tid] = g[tt];
        }
        __syncthreads();
        if (live) {
            float o = Ob[t][jj];
            for (int s = 0; s <= t; s++) o = o + P_b[t * C + s] * G[s][jj];
            Out[vo] = o;
        }
        for (int idx = tid; idx < dk * NC; idx += 256) {
            const int i = idx / NC, cc = idx % NC;
            if (cc >= ncol) continue;
            float *sp = Sh + (int64_t)i * dv + j0 + cc;
            float rv = (CL ? s_l[idx] : *sp) * (CL ? cf_l[i] : CF[(int64_t)(C - 1) * dk + i]);
#pragma unroll 8
            for (int s = 0; s < C; s++) rv = rv + wg_b[s * ld + i] * G[s][cc];
            if (CL)
                s_l[idx] = rv;
            else
                *sp = rv;
        }
        __syncthreads();
    }
    if (CL) {
        for (int n = tid; n < dk * NC; n += 256) {
            const int i = n / NC, cc = n % NC;
            if (cc < ncol) Sh[(int64_t)i * dv + j0 + cc] = s_l[n];
        }
    }
}
// Register prefetch of a chunk's record for k_gdn2_cols4 (operands in LDS,
// dk % 4 == 0): thread tid's float4 f = tid + 256u (u < 4) of WI, QI and WG
// [C][dk], of L and P, and of CF's last row; indices past an array are
// clamped to its last element (loaded, never stored), so every register is
// always written. GDN2_PF_PUT stores part u of WI, QI and WG into LDS rows
// of stride lk.
#define GDN2_PF(cc)                                                                           \
    do {                                                                                      \
        const float4 *r4 =                                                                    \
            (const float4 *)(rec + ((int64_t)h * nch + (cc)) * chunk_rec_floats(C, dk));      \
        int f_ = min(tid, n4 - 1);                                                            \
        wi0 = r4[n4 + f_], qi0 = r4[2 * n4 + f_], wg0 = r4[3 * n4 + f_];                      \
        f_ = min(tid + 256, n4 - 1);                                                          \
        wi1 = r4[n4 + f_], qi1 = r4[2 * n4 + f_], wg1 = r4[3 * n4 + f_];                      \
        f_ = min(tid + 512, n4 - 1);                                                          \
        wi2 = r4[n4 + f_], qi2 = r4[2 * n4 + f_], wg2 = r4[3 * n4 + f_];                      \
        f_ = min(tid + 768, n4 - 1);                                                          \
        wi3 = r4[n4 + f_], qi3 = r4[2 * n4 + f_], wg3 = r4[3 * n4 + f_];                      \
        lp0 = r4[4 * n4 + min(tid, nlp - 1)];                                                 \
        lp1 = r4[4 * n4 + min(tid + 256, nlp - 1)];                                           \
        cf4 = r4[(C - 1) * dk / 4 + min(tid, dk / 4 - 1)];                                    \
        if (live) {                                                                           \
            const int64_t vq = h * hv + ((int64_t)(cc) * C + t) * dv + j;                     \
            pvw = W[vq] * V[vq];                                                              \
        }                                                                                     \
    } while (0)
#define GDN2_PF_PUT(u, a, b, g)                                                               \
    do {                                                                                      \
        const int f_ = tid + 256 * (u);                                                       \
        if (f_ < n4) {                                                                        \
            const int at_ = (4 * f_ / dk) * lk + 4 * f_ % dk;                                 \
            *(float4 *)(wi_l + at_) = a;                                                      \
            *(float4 *)(qi_l + at_) = b;                                                      \
            *(float4 *)(wg_l + at_) = g;                                                      \
        }                                                                                     \
    } while (0)

// k_gdn2_cols for operands in LDS with dk % 4 == 0, with
// every LDS operand read 16 bytes at a time: the S tile is held transposed
// (column cc's dk values contiguous, stride dk + 4) and so is G (column
// cc's C values contiguous), so phase 1 reads 4 consecutive i of WI, QI
// and S, phases 2 and 3 4 consecutive s of L, P and G, and phase 4 (thread
// = 4 consecutive i of one column) 4 consecutive i of WG and S per s. Each
// value is still formed by the same operations in the same order as in
// k_gdn2_cols (phase 1's chains in ascending i, the substitution in
// ascending s, and so on), so the results are the same bits; only the
// number of LDS instructions drops, which is what a chunk's phases wait on.
// The output row sum of phase 1 stays in the thread's register until
// phase 3 (same thread). NC = 128 / C columns per block (half the block's
// threads in phases 1, 3 and 4) doubles the blocks when 256 / C columns
// per block would leave CUs idle; each column's arithmetic is unchanged.
template <int C, int NC>
__global__ __launch_bounds__(256) void k_gdn2_cols4(float *__restrict__ S, float *__restrict__ Out,
                                                    const float *__restrict__ V,
                                                    const float *__restrict__ W, int64_t hv,
                                                    int nch, int dk, int dv,
                                                    const int *__restrict__ flag,
                                                    const float *__restrict__ rec) {
    static_assert(C * NC == 256 || C * NC == 128, "256 or 128 (t, column) pairs");
    static_assert(CHUNK_LDS / 4 / 256 == 4 && 2 * C * C / 4 <= 512,
                  "the prefetch holds 4 float4 of each [C][dk] array and 2 of L, P");
    constexpr int NL = CHUNK_LDS + 4 * 32;
    constexpr int SKMAX = CHUNK_LDS / C + 4;  // S column stride bound (dk <= CHUNK_LDS / C)
    constexpr int GS = C + 4;                 // G column stride
    __shared__ __attribute__((aligned(16))) float G[NC * GS];
    __shared__ __attribute__((aligned(16))) float wi_l[NL], qi_l[NL], wg_l[NL];
    __shared__ __attribute__((aligned(16))) float sT[NC * SKMAX];
    __shared__ __attribute__((aligned(16))) float lp_l[2 * C * C], cf_l[1024];
    const int h = blockIdx.x, j0 = blockIdx.y * NC, tid = threadIdx.x, lk = dk + 4;
    if (flag[h]) return;  // a rejected head keeps its S and Out
    const int64_t Ck = (int64_t)C * dk;
    float *Sh = S + (int64_t)h * dk * dv;
    const int ncol = min(NC, dv - j0);
    // with C * NC = 128 the upper 128 threads only copy records and pass
    // the barriers
    const int t = tid / NC, jj = tid % NC, j = j0 + jj;
    const bool live = jj < ncol && tid < C * NC;
    const int sk = dk + 4;  // S column stride (16-byte rows, lanes of nearby columns on distinct banks)
    for (int n = tid; n < dk * NC; n += 256) {
        const int i = n / NC, cc = n % NC;
        sT[cc * sk + i] = cc < ncol ? Sh[(int64_t)i * dv + j0 + cc] : 0.0f;
    }
    const int n4 = (int)(Ck / 4), nlp = C * C / 2;
    float4 wi0, wi1, wi2, wi3, qi0, qi1, qi2, qi3, wg0, wg1, wg2, wg3, lp0, lp1, cf4;
    float pvw = 0.0f;
    GDN2_PF(0);
    const int q4 = dk / 4;
    for (int c = 0; c < nch; c++) {
        GDN2_PF_PUT(0, wi0, qi0, wg0);
        GDN2_PF_PUT(1, wi1, qi1, wg1);
        GDN2_PF_PUT(2, wi2, qi2, wg2);
        GDN2_PF_PUT(3, wi3, qi3, wg3);
        if (tid < nlp) *(float4 *)(lp_l + 4 * tid) = lp0;  // L then P
        if (tid + 256 < nlp) *(float4 *)(lp_l + 4 * (tid + 256)) = lp1;
        if (tid < dk / 4) *(float4 *)(cf_l + 4 * tid) = cf4;
        const float vw0 = pvw;
        __syncthreads();
        if (c + 1 < nch) GDN2_PF(c + 1);  // in flight through this chunk's phases
        const int64_t vo = h * hv + ((int64_t)c * C + t) * dv + j;
        // ---- phase 1: B_t and the first part of Out_t for column jj ----
        float o = 0.0f;
        if (live) {
            float g = vw0;
            const float4 *wi = (const float4 *)(wi_l + t * lk), *qi = (const float4 *)(qi_l + t * lk);
            const float4 *sv = (const float4 *)(sT + jj * sk);
#pragma unroll 4
            for (int u = 0; u < q4; u++) {
                const float4 w4 = wi[u], x4 = qi[u], s4 = sv[u];
                g = g - w4.x * s4.x;
                o = o + x4.x * s4.x;
                g = g - w4.y * s4.y;
                o = o + x4.y * s4.y;
                g = g - w4.z * s4.z;
                o = o + x4.z * s4.z;
                g = g - w4.w * s4.w;
                o = o + x4.w * s4.w;
            }
            G[jj * GS + t] = g;
        }
        __syncthreads();
        // ---- phase 2: (I + L) E = B per column, E over G ----
        if (tid < ncol) {
            float gv[C];
#pragma unroll
            for (int u = 0; u < C / 4; u++) {
                const float4 x = *(const float4 *)(G + tid * GS + 4 * u);
                gv[4 * u] = x.x, gv[4 * u + 1] = x.y, gv[4 * u + 2] = x.z, gv[4 * u + 3] = x.w;
            }
#pragma unroll
            for (int tt = 1; tt < C; tt++) {
                const float *Lr = lp_l + tt * C;
#pragma unroll
                for (int u = 0; u < C / 4; u++) {
                    if (4 * u >= tt) break;
                    const float4 l4 = *(const float4 *)(Lr + 4 * u);
                    gv[tt] = gv[tt] - l4.x * gv[4 * u];
                    if (4 * u + 1 < tt) gv[tt] = gv[tt] - l4.y * gv[4 * u + 1];
                    if (4 * u + 2 < tt) gv[tt] = gv[tt] - l4.z * gv[4 * u + 2];
                    if (4 * u + 3 < tt) gv[tt] = gv[tt] - l4.w * gv[4 * u + 3];
                }
            }
#pragma unroll
            for (int u = 0; u < C / 4; u++)
                *(float4 *)(G + tid * GS + 4 * u) =
                    make_float4(gv[4 * u], gv[4 * u + 1], gv[4 * u + 2], gv[4 * u + 3]);
        }
        __syncthreads();
        // ---- phase 3: Out_t += sum_{s<=t} P[t][s] E_s ----
        if (live) {
            const float *Pr = lp_l + C * C + t * C;
            const float *Gc = G + jj * GS;
            for (int u = 0; 4 * u <= t; u++) {
                const float4 p4 = *(const float4 *)(Pr + 4 * u);
                const float4 e4 = *(const float4 *)(Gc + 4 * u);
                o = o + p4.x * e4.x;
                if (4 * u + 1 <= t) o = o + p4.y * e4.y;
                if (4 * u + 2 <= t) o = o + p4.z * e4.z;
                if (4 * u + 3 <= t) o = o + p4.w * e4.w;
            }
            Out[vo] = o;
        }
        // ---- phase 4: S[i] <- CF[C-1][i] S[i] + sum_s WG[s][i] E_s ----
        for (int u = tid; u < q4 * NC; u += 256) {
            const int cc = u / q4, i4 = u % q4;
            if (cc >= ncol) continue;
            float4 *sp = (float4 *)(sT + cc * sk) + i4;
            const float4 s4 = *sp, f4 = *(const float4 *)(cf_l + 4 * i4);
            float4 rv = make_float4(s4.x * f4.x, s4.y * f4.y, s4.z * f4.z, s4.w * f4.w);
            const float *Gc = G + cc * GS;
#pragma unroll
            for (int v = 0; v < C / 4; v++) {
                const float4 e4 = *(const float4 *)(Gc + 4 * v);
                const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 w4 = *(const float4 *)(wg_l + (4 * v + q) * lk + 4 * i4);
                    rv.x = rv.x + w4.x * ev[q];
                    rv.y = rv.y + w4.y * ev[q];
                    rv.z = rv.z + w4.z * ev[q];
                    rv.w = rv.w + w4.w * ev[q];
                }
            }
            *sp = rv;
        }
        __syncthreads();
    }
    for (int n = tid; n < dk * NC; n += 256) {
        const int i = n / NC, cc = n % NC;
        if (cc < ncol) Sh[(int64_t)i * dv + j0 + cc] = sT[cc * sk + i];
    }
}
#undef GDN2_PF
#undef GDN2_PF_PUT

}  // namespace

// Workspace of jtk_gdn2_prefill: H flag words (padded to 64 floats) and one
// record per (head, chunk).
extern "C" size_t jtk_gdn2_prefill_ws_bytes(int H, int T, int C, int dk) {
    const int64_t flags = ((int64_t)H + 63) / 64 * 64;
    return (size_t)(flags + (int64_t)H * (T / C) * chunk_rec_floats(C, dk)) * sizeof(float);
}

// H heads, one decode step each. dk, dv in 1..1024.
extern "C" int jtk_gdn2_decode(float *S, float *O, const float *q, const float *k,
                               const float *v, const float *b, const float *w,
                               const float *alpha, int H, int dk, int dv, uint32_t *err,
                               hipStream_t s) {
    if (H <= 0 || dk <= 0 || dv <= 0 || dk > 1024 || dv > 1024) return (int)hipErrorInvalidValue;
    const unsigned nt = (unsigned)(dv >= 256 ? 256 : (dv + 63) / 64 * 64);
    hipLaunchKernelGGL(k_gdn2_decode, dim3((unsigned)H), dim3(nt), 0, s, S, O, q, k, v, b, w,
                       alpha, dk, dv, err);
    return (int)hipGetLastError();
}

// H heads, T tokens each in T/C chunks of C (16 or 32): head h's rows of
// the dk-wide inputs start at h*hk, of V, W and Out at h*hv. All of a
// head's T tokens are checked first (a head with a bad value keeps its S
// and Out), every chunk's state-independent part is prepared in one
// launch, then one launch runs the chunks' state updates in order. ws of
// jtk_gdn2_prefill_ws_bytes(H, T, C, dk).
extern "C" int jtk_gdn2_prefill(float *S, float *Out, const float *Q, const float *K,
                                const float *V, const float *B, const float *W,
                                const float *A, int64_t hk, int64_t hv, int H, int T, int C,
                                int dk, int dv, float *ws, uint32_t *err, hipStream_t s) {
    if (H <= 0 || H > 65535 || (C != 16 && C != 32) || T <= 0 || T % C || dk <= 0 || dv <= 0 ||
        dk > 1024 || dv > 1024 || (int64_t)T * (dk > dv ? dk : dv) > INT32_MAX)
        return (int)hipErrorInvalidValue;
    const int nch = T / C;
    int *flag = (int *)ws;
    float *rec = ws + ((int64_t)H + 63) / 64 * 64;
    int le = jtk_zero_u32((uint32_t *)flag, H, s);
    const int64_t most = (int64_t)T * (dk > dv ? dk : dv);
    const unsigned nb = (unsigned)((most + 255) / 256 < 64 ? (most + 255) / 256 : 64);
    hipLaunchKernelGGL(k_gdn2_check, dim3(nb, (unsigned)H), dim3(256), 0, s, Q, K, B, A, V, W,
                       hk, hv, T * dk, T * dv, flag, err);
    const bool cl = (int64_t)C * dk <= CHUNK_LDS;
    if (cl)
        hipLaunchKernelGGL(k_gdn2_prep<true>, dim3((unsigned)nch, (unsigned)H), dim3(256), 0, s,
                           Q, K, B, A, hk, C, dk, flag, rec);
    else
        hipLaunchKernelGGL(k_gdn2_prep<false>, dim3((unsigned)nch, (unsigned)H), dim3(256), 0, s,
                           Q, K, B, A, hk, C, dk, flag, rec);
    const dim3 grid((unsigned)H, (unsigned)((dv + 256 / C - 1) / (256 / C)));
    const bool v4 = dk % 4 == 0;  // the record prefetch with 16-byte loads
    // narrow blocks (128 / C columns) when the wide ones would not fill the
    // GPU's 256 CUs
    const bool narrow = (int64_t)grid.x * grid.y < 256;
    const dim3 grid_n((unsigned)H, (unsigned)((dv + 128 / C - 1) / (128 / C)));
    if (C == 16 && cl && v4 && narrow)
        hipLaunchKernelGGL((k_gdn2_cols4<16, 8>), grid_n, dim3(256), 0, s, S, Out, V, W, hv, nch,
                           dk, dv, flag, rec);
    else if (C == 32 && cl && v4 && narrow)
        hipLaunchKernelGGL((k_gdn2_cols4<32, 4>), grid_n, dim3(256), 0, s, S, Out, V, W, hv, nch,
                           dk, dv, flag, rec);
    else if (C == 16 && cl && v4)
        hipLaunchKernelGGL((k_gdn2_cols4<16, 16>), grid, dim3(256), 0, s, S, Out, V, W, hv, nch,
                           dk, dv, flag, rec);
    else if (C == 32 && cl && v4)
        hipLaunchKernelGGL((k_gdn2_cols4<32, 8>), grid, dim3(256), 0, s, S, Out, V, W, hv, nch,
                           dk, dv, flag, rec);
    else if (C == 16 && cl)
        hipLaunchKernelGGL((k_gdn2_cols<16, true>), grid, dim3(256), 0, s, S, Out, V, W,
                           hv, nch, dk, dv, flag, rec);
    else if (C == 16)
        hipLaunchKernelGGL((k_gdn2_cols<16, false>), grid, dim3(256), 0, s, S, Out, V, W,
                           hv, nch, dk, dv, flag, rec);
    else if (cl)
        hipLaunchKernelGGL((k_gdn2_cols<32, true>), grid, dim3(256), 0, s, S, Out, V, W,
                           hv, nch, dk, dv, flag, rec);
    else
        hipLaunchKernelGGL((k_gdn2_cols<32, false>), grid, dim3(256), 0, s, S, Out, V, W,
                           hv, nch, dk, dv, flag, rec);
    return le | (int)hipGetLastError();
}

// y = x / ||x|| (the reference's l2norm) for R rows of n.
__global__ __launch_bounds__(64) void k_gdn2_l2norm(const float *__restrict__ x,
                                                    float *__restrict__ y, int n, float eps) {
    const int r = blockIdx.x;
    __shared__ float inv;
    __shared__ int zero;
    const float *xr = x + (int64_t)r * n;
    if (threadIdx.x == 0) {
        double ss = 0.0;
        for (int i = 0; i < n; i++) ss = ss + (double)xr[i] * (double)xr[i];
        const double nrm = sqrt(ss);
        zero = nrm < (double)eps;
        inv = zero ? 0.0f : (float)(1.0 / nrm);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 64) y[(int64_t)r * n + i] = zero ? 0.0f : xr[i] * inv;
}

extern "C" int jtk_gdn2_l2norm(const float *x, float *y, int rows, int n, float eps,
                               hipStream_t s) {
    hipLaunchKernelGGL(k_gdn2_l2norm, dim3((unsigned)rows), dim3(64), 0, s, x, y, n, eps);
    return (int)hipGetLastError();
}

extern "C" int jtk_preload_gdn2(void) {
    hipFuncAttributes a;
    return (int)hipFuncGetAttributes(&a, (const void *)(k_gdn2_l2norm));
}
