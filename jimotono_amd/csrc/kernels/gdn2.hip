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
//  k_gdn2_chunk_prep  : per head of a C-token chunk: checks, norms, ke, vw,
//                       forward decay products, the strictly lower L and
//                       the lower P (src/gdn2.c:537-714), the row weights
//                       of the state update (:768-788).
//  k_gdn2_chunk_cols  : per (head, 64 columns): B, the forward substitution,
//                       Out and the state update (:614-680, 716-842) with
//                       the chunk's C rows of a column in registers.
#include "jt_dev.h"
#include "jt_launch.h"

namespace {

constexpr float GDN2_EPS = 1e-6f;

// 1 / ||x|| as the reference rounds it: fp64 sum of squares in index order,
// fp64 sqrt and divide, then float; *zero when the norm is below eps.
__device__ __forceinline__ float inv_norm(const float *x, int n, bool *zero) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
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

// LDS: qn, kn, ke, al [dk] (dk <= 1024). Pass 1 writes the decayed column
// back and pass 2 re-reads it (the same thread, so from cache).
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
    const int h = blockIdx.x, tid = threadIdx.x;
    const float *qh = q + (int64_t)h * dk, *kh = k + (int64_t)h * dk;
    const float *bh = b + (int64_t)h * dk, *ah = alpha + (int64_t)h * dk;
    const float *vh = v + (int64_t)h * dv, *wh = w + (int64_t)h * dv;
    float *Sh = S + (int64_t)h * dk * dv, *Oh = O + (int64_t)h * dv;
    bool bad = bad_vec(qh, dk, tid, 256) || bad_vec(kh, dk, tid, 256) ||
               bad_vec(bh, dk, tid, 256) || bad_vec(ah, dk, tid, 256) ||
               bad_alpha(ah, dk, tid, 256) || bad_vec(vh, dv, tid, 256) ||
               bad_vec(wh, dv, tid, 256);
    if (__syncthreads_or(bad)) {  // fail-closed: this head's S and o untouched
        if (tid == 0) raise_err(err, EF_NONFINITE_INPUT);
        return;
    }
    if (tid == 0 || tid == 64) {  // two waves, one norm each
        bool z;
        const float iv = inv_norm(tid ? kh : qh, dk, &z);
        invs[tid ? 1 : 0] = iv;
        zeros[tid ? 1 : 0] = z;
    }
    __syncthreads();
    for (int i = tid; i < dk; i += 256) {
        const float qi = zeros[0] ? 0.0f : qh[i] * invs[0];
        const float ki = zeros[1] ? 0.0f : kh[i] * invs[1];
        qn[i] = qi;
        kn[i] = ki;
        ke[i] = bh[i] * ki;
        al[i] = ah[i];
    }
    __syncthreads();
    for (int j = tid; j < dv; j += 256) {
        float *col = Sh + j;
        float c = 0.0f;
#pragma unroll 8
        for (int i = 0; i < dk; i++) {
            const float s = col[(int64_t)i * dv] * al[i];
            col[(int64_t)i * dv] = s;
            c = c + ke[i] * s;
        }
        const float vw = wh[j] * vh[j];
        float o = 0.0f;
#pragma unroll 8
        for (int i = 0; i < dk; i++) {
            float r = col[(int64_t)i * dv] - kn[i] * c;
            r = r + kn[i] * vw;
            col[(int64_t)i * dv] = r;
            o = o + qn[i] * r;
        }
        Oh[j] = o;
    }
}

// Per-head chunk workspace (floats): Qn, Kn, KE, CF (forward decay
// products alpha_0..t), WI = KE*CF, QI = Qn*CF, WG (row weights of the
// state update) [C][dk] each; L, P [C][C].
__host__ __device__ constexpr int64_t chunk_ws_floats(int C, int dk) {
    return 7LL * C * dk + 2LL * C * C;
}

// flag[h] = 1 when head h's inputs (nk values of each dk-wide array from
// h*hk, nv of each dv-wide one from h*hv) hold a non-finite value or an
// alpha outside [0,1]; the later kernels leave such a head as it was.
__global__ __launch_bounds__(256) void k_gdn2_check(const float *__restrict__ Q,
                                                    const float *__restrict__ K,
                                                    const float *__restrict__ B,
                                                    const float *__restrict__ A,
                                                    const float *__restrict__ V,
                                                    const float *__restrict__ W, int64_t hk,
                                                    int64_t hv, int nk, int nv,
                                                    int *__restrict__ flag, uint32_t *err) {
    const int h = blockIdx.x, tid = threadIdx.x;
    bool bad = bad_vec(Q + h * hk, nk, tid, 256) || bad_vec(K + h * hk, nk, tid, 256) ||
               bad_vec(B + h * hk, nk, tid, 256) || bad_vec(A + h * hk, nk, tid, 256) ||
               bad_alpha(A + h * hk, nk, tid, 256) || bad_vec(V + h * hv, nv, tid, 256) ||
               bad_vec(W + h * hv, nv, tid, 256);
    bad = __syncthreads_or(bad);
    if (tid == 0) {
        flag[h] = bad ? 1 : 0;
        if (bad) raise_err(err, EF_NONFINITE_INPUT);
    }
}

// (x*cum)*y summed over i in four chains (i % 4 for i < dk & ~3, the tail
// into chain 0), then (s0+s1)+(s2+s3) (src/gdn2.c:584-599, 702-713); cum =
// alpha_{s+1} * ... * alpha_t in that order (1 when t == s).
__device__ __forceinline__ void dots_ts(const float *KEt, const float *Qt, const float *Ks,
                                        const float *A, int dk, int s, int t, bool want_l,
                                        float *l_out, float *p_out) {
    float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int dk4 = dk & ~3;
    for (int i = 0; i < dk; i++) {
        float cum = 1.0f;
        for (int r = s + 1; r <= t; r++) cum = cum * A[(int64_t)r * dk + i];
        const int ch = i < dk4 ? (i & 3) : 0;
        if (want_l) ls[ch] = ls[ch] + (KEt[i] * cum) * Ks[i];
        ps[ch] = ps[ch] + (Qt[i] * cum) * Ks[i];
    }
    *l_out = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    *p_out = (ps[0] + ps[1]) + (ps[2] + ps[3]);
}

// Head h's chunk rows start at X + h*hk (dk-wide arrays) / h*hv (dv-wide).
__global__ __launch_bounds__(256) void k_gdn2_chunk_prep(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ B,
    const float *__restrict__ A, int64_t hk, int C, int dk, const int *__restrict__ flag,
    float *__restrict__ ws) {
    __shared__ float invs[64];
    __shared__ int zeros[64];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int64_t Ck = (int64_t)C * dk;
    if (flag[h]) return;
    const float *Qh = Q + h * hk, *Kh = K + h * hk, *Bh = B + h * hk, *Ah = A + h * hk;
    float *wsh = ws + (int64_t)h * chunk_ws_floats(C, dk);
    float *Qn = wsh, *Kn = Qn + Ck, *KE = Kn + Ck, *CF = KE + Ck, *WI = CF + Ck, *QI = WI + Ck;
    float *WG = QI + Ck, *L = WG + Ck, *P = L + (int64_t)C * C;
    if (tid < 2 * C) {  // one row norm per thread
        const int t = tid % C;
        bool z;
        invs[tid] = inv_norm((tid < C ? Qh : Kh) + (int64_t)t * dk, dk, &z);
        zeros[tid] = z;
    }
    __syncthreads();
    for (int64_t n = tid; n < Ck; n += 256) {
        const int t = (int)(n / dk);
        const float qv = zeros[t] ? 0.0f : Qh[n] * invs[t];
        const float kv = zeros[C + t] ? 0.0f : Kh[n] * invs[C + t];
        Qn[n] = qv;
        Kn[n] = kv;
        KE[n] = Bh[n] * kv;
    }
    __syncthreads();
    for (int i = tid; i < dk; i += 256) {
        float cf = 1.0f;  // alpha_0 * ... * alpha_t, t ascending
        for (int t = 0; t < C; t++) {
            cf = cf * Ah[(int64_t)t * dk + i];
            CF[(int64_t)t * dk + i] = cf;
            WI[(int64_t)t * dk + i] = KE[(int64_t)t * dk + i] * cf;
            QI[(int64_t)t * dk + i] = Qn[(int64_t)t * dk + i] * cf;
        }
        float sf = 1.0f;  // alpha_{s+1} * ..., accumulated from the end
        for (int s = C - 1; s >= 0; s--) {
            WG[(int64_t)s * dk + i] = Kn[(int64_t)s * dk + i] * sf;
            sf = sf * Ah[(int64_t)s * dk + i];
        }
    }
    __syncthreads();
    for (int pr = tid; pr < C * C; pr += 256) {
        const int t = pr / C, s = pr % C;
        if (s > t) continue;
        float l, p;
        dots_ts(KE + (int64_t)t * dk, Qn + (int64_t)t * dk, Kn + (int64_t)s * dk, Ah, dk, s, t,
                s < t, &l, &p);
        L[pr] = s < t ? l : 0.0f;
        P[pr] = p;
    }
}

template <int C>
__global__ __launch_bounds__(64) void k_gdn2_chunk_cols(
    float *__restrict__ S, float *__restrict__ Out, const float *__restrict__ V,
    const float *__restrict__ W, int64_t hv, int dk, int dv, const int *__restrict__ flag,
    const float *__restrict__ ws) {
    const int h = blockIdx.x, j = blockIdx.y * 64 + threadIdx.x;
    const int64_t Ck = (int64_t)C * dk;
    const float *wsh = ws + (int64_t)h * chunk_ws_floats(C, dk);
    const float *CF = wsh + 3 * Ck, *WI = CF + Ck, *QI = WI + Ck, *WG = QI + Ck;
    const float *L = WG + Ck, *P = L + C * C;
    if (flag[h] || j >= dv) return;  // a rejected head keeps its S and Out
    float *col = S + (int64_t)h * dk * dv + j;
    const float *Vh = V + h * hv, *Wh = W + h * hv;
    float g[C], o[C];
#pragma unroll
    for (int t = 0; t < C; t++) {
        g[t] = Wh[(int64_t)t * dv + j] * Vh[(int64_t)t * dv + j];  // vw_t
        o[t] = 0.0f;
    }
    // B_t = vw_t - sum_i WI[t][i] S[i], Out_t = sum_i QI[t][i] S[i] (i ascending)
    for (int i = 0; i < dk; i++) {
        const float sv = col[(int64_t)i * dv];
#pragma unroll
        for (int t = 0; t < C; t++) {
            g[t] = g[t] - WI[(int64_t)t * dk + i] * sv;
            o[t] = o[t] + QI[(int64_t)t * dk + i] * sv;
        }
    }
    // (I + L) E = B
#pragma unroll
    for (int t = 1; t < C; t++)
#pragma unroll
        for (int s = 0; s < t; s++) g[t] = g[t] - L[t * C + s] * g[s];
    float *Oh = Out + h * hv + j;
#pragma unroll
    for (int t = 0; t < C; t++) {
        float ot = o[t];
#pragma unroll
        for (int s = 0; s <= t; s++) ot = ot + P[t * C + s] * g[s];
        Oh[(int64_t)t * dv] = ot;
    }
    // S <- CF[C-1] * S + sum_s WG[s] E_s
    for (int i = 0; i < dk; i++) {
        float r = col[(int64_t)i * dv] * CF[(int64_t)(C - 1) * dk + i];
#pragma unroll
        for (int s = 0; s < C; s++) r = r + WG[(int64_t)s * dk + i] * g[s];
        col[(int64_t)i * dv] = r;
    }
}

}  // namespace

// Workspace of jtk_gdn2_prefill: H flag words (padded to 64 floats) and the
// per-head chunk area.
extern "C" size_t jtk_gdn2_chunk_ws_bytes(int H, int C, int dk) {
    const int64_t flags = ((int64_t)H + 63) / 64 * 64;
    return (size_t)(flags + (int64_t)H * chunk_ws_floats(C, dk)) * sizeof(float);
}

// H heads, one decode step each. dk, dv in 1..1024.
extern "C" int jtk_gdn2_decode(float *S, float *O, const float *q, const float *k,
                               const float *v, const float *b, const float *w,
                               const float *alpha, int H, int dk, int dv, uint32_t *err,
                               hipStream_t s) {
    if (H <= 0 || dk <= 0 || dv <= 0 || dk > 1024 || dv > 1024) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gdn2_decode, dim3((unsigned)H), dim3(256), 0, s, S, O, q, k, v, b, w,
                       alpha, dk, dv, err);
    return (int)hipGetLastError();
}

// H heads, T tokens each in T/C chunks of C (16 or 32), in order: head h's
// rows of the dk-wide inputs start at h*hk, of V, W and Out at h*hv; all
// of a head's T tokens are checked first, and a head with a bad value keeps
// its S and Out. ws of jtk_gdn2_chunk_ws_bytes(H, C, dk).
extern "C" int jtk_gdn2_prefill(float *S, float *Out, const float *Q, const float *K,
                                const float *V, const float *B, const float *W,
                                const float *A, int64_t hk, int64_t hv, int H, int T, int C,
                                int dk, int dv, float *ws, uint32_t *err, hipStream_t s) {
    if (H <= 0 || (C != 16 && C != 32) || T <= 0 || T % C || dk <= 0 || dv <= 0 ||
        dk > 1024 || dv > 1024 || (int64_t)T * (dk > dv ? dk : dv) > INT32_MAX)
        return (int)hipErrorInvalidValue;
    int *flag = (int *)ws;
    float *cw = ws + ((int64_t)H + 63) / 64 * 64;
    hipLaunchKernelGGL(k_gdn2_check, dim3((unsigned)H), dim3(256), 0, s, Q, K, B, A, V, W, hk,
                       hv, T * dk, T * dv, flag, err);
    const dim3 grid((unsigned)H, (unsigned)((dv + 63) / 64));
    for (int c0 = 0; c0 < T; c0 += C) {
        const int64_t ok = (int64_t)c0 * dk, ov = (int64_t)c0 * dv;
        hipLaunchKernelGGL(k_gdn2_chunk_prep, dim3((unsigned)H), dim3(256), 0, s, Q + ok, K + ok,
                           B + ok, A + ok, hk, C, dk, flag, cw);
        if (C == 16)
            hipLaunchKernelGGL(k_gdn2_chunk_cols<16>, grid, dim3(64), 0, s, S, Out + ov, V + ov,
                               W + ov, hv, dk, dv, flag, cw);
        else
            hipLaunchKernelGGL(k_gdn2_chunk_cols<32>, grid, dim3(64), 0, s, S, Out + ov, V + ov,
                               W + ov, hv, dk, dv, flag, cw);
    }
    return (int)hipGetLastError();
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
