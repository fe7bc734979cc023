// Issue-rate calibration of the GPU the kernels run on, for bench.py's
// `--only calib` entry (libjimotono_calib.so, separate from the drop-in
// library): how fast the matrix cores and the vector ALUs retire work alone,
// whether their work overlaps when it comes from different waves or from one
// wave, and how fast the 128x256 int8 tile GEMM's main loop runs when its
// operands are in HBM, aliased into L2, or both. The numbers bound what the
// grouped GEMMs can reach, independently of the peak figures on paper.
#include <hip/hip_runtime.h>

#include "../kernels/gemm_w8a8.h"

namespace {

// Per iteration each wave of a 512-thread block does, by mode:
//   0: 16 int8 MFMAs (16x16x64) on register operands
//   1: 64 fp32 FMAs (16 independent chains of 4)
//   2: waves 0-3 the MFMAs of mode 0, waves 4-7 the FMAs of mode 1
//   3: both in every wave
//   4-6: as 1-3 with 64 fp64 FMAs (8 chains of 8)
//   7: mode 0 with its 8 operand fragments read from LDS each iteration
//   8: mode 7 and a workgroup barrier per iteration
template <int MODE>
__global__ __launch_bounds__(512, 4) void k_issue(int iters, float *out) {
    __shared__ __attribute__((aligned(16))) int8_t lds[24 * 1024];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (MODE >= 7) {
        for (int i = threadIdx.x; i < 24 * 1024 / 4; i += 512)
            ((uint32_t *)lds)[i] = (uint32_t)i * 2654435761u;
        __syncthreads();
    }
    v4i acc[4][4], a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = (v4i){lane, lane * 3, i, 7};
        b[i] = (v4i){lane ^ i, 5, lane, i};
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (v4i){0, 0, 0, 0};
    }
    float f[16];
    double d[8];
#pragma unroll
    for (int i = 0; i < 16; i++) f[i] = lane * 0.001f + i;
#pragma unroll
    for (int i = 0; i < 8; i++) d[i] = lane * 0.001 + i;
    const bool split = MODE == 2 || MODE == 5;
    const bool do_m = MODE == 0 || MODE == 3 || MODE == 6 || MODE >= 7 || (split && wave < 4);
    const bool do_v = (MODE >= 1 && MODE <= 6 && MODE != 2 && MODE != 5) || (split && wave >= 4);
    const bool f64 = MODE >= 4 && MODE <= 6;
    const int wm = (wave >> 2) * 4, wn = (wave & 3) * 4;  // fragment rows of this wave (LDS modes)
    for (int it = 0; it < iters; it++) {
        if (MODE >= 7) {
            // panels wn+8+j (j < 4) and wm+i: at most panel 23 of 24
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = *(const v4i *)(lds + (8 + wn + j) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = *(const v4i *)(lds + (wm + i) * 1024 + lane * 16);
        }
        if (do_m) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = mfma16x16x64(a[i], b[j], acc[i][j]);
        }
        if (do_v) {
            if (f64) {
#pragma unroll
                for (int r = 0; r < 8; r++)
#pragma unroll
                    for (int i = 0; i < 8; i++) d[i] = __builtin_fma(d[i], 0.999, 0.001);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int i = 0; i < 16; i++) f[i] = __builtin_fmaf(f[i], 0.999f, 0.001f);
            }
        }
        if (MODE == 8) __syncthreads();
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) s += (float)(acc[i][j].x + acc[i][j].w);
#pragma unroll
    for (int i = 0; i < 16; i++) s += f[i] + (float)d[i / 2];
    out[blockIdx.x * 512 + threadIdx.x] = s;
}

template <int MODE>
hipError_t launch_issue(int blocks, int iters, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_issue<MODE>, dim3((unsigned)blocks), dim3(512), 0, s, iters, out);
    return hipGetLastError();
}

hipError_t issue_mode(int mode, int blocks, int iters, float *out, hipStream_t s) {
    switch (mode) {
        case 0: return launch_issue<0>(blocks, iters, out, s);
        case 1: return launch_issue<1>(blocks, iters, out, s);
        case 2: return launch_issue<2>(blocks, iters, out, s);
        case 3: return launch_issue<3>(blocks, iters, out, s);
        case 4: return launch_issue<4>(blocks, iters, out, s);
        case 5: return launch_issue<5>(blocks, iters, out, s);
        case 6: return launch_issue<6>(blocks, iters, out, s);
        case 7: return launch_issue<7>(blocks, iters, out, s);
        case 8: return launch_issue<8>(blocks, iters, out, s);
        default: return hipErrorInvalidValue;
    }
}

// Mean duration (ms) of `reps` back-to-back launches of f() after one
// untimed launch, from events on the null stream.
template <typename F>
hipError_t time_launches(F f, int reps, float *ms) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = f();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipEventRecord(e0, nullptr);
    for (int r = 0; r < reps && e == hipSuccess; r++) e = f();
    if (e == hipSuccess) e = hipEventRecord(e1, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    if (e == hipSuccess) *ms = t / reps;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return e;
}

}  // namespace

// Mode `mode` (0-8, above) over `blocks` blocks of 8 waves, `iters`
// iterations per wave: *ms = mean duration of 3 timed launches.
extern "C" int jt_calib_issue(int mode, int blocks, int iters, float *ms) {
    if (mode < 0 || mode > 8 || blocks <= 0 || blocks > 4096 || iters <= 0 || !ms)
        return (int)hipErrorInvalidValue;
    float *out = nullptr;
    hipError_t e = hipMalloc((void **)&out, (size_t)blocks * 512 * sizeof(float));
    if (e != hipSuccess) return (int)e;
    e = time_launches([&] { return issue_mode(mode, blocks, iters, out, nullptr); }, 3, ms);
    const hipError_t ef = hipFree(out);
    return (int)(e != hipSuccess ? e : ef);
}

// The plain-epilogue 128x256 tile GEMM (8 waves, 3-stage LDS ring, the
// configuration of the shared gate/up) at K = 1024 with zero scales, case:
//   0: M 4096, N 11264; A [4096][1024], the weight panels and C [M][N] in
//      their own buffers (the shared gate/up's operand traffic)
//   1: as 0 with every C row aliased onto row 0 (ldc 0: no output traffic)
//   2: as 1 with every A row aliased onto row 0 (lda 0: only W streams)
//   3: M 180224, N 256 (a 256 KB weight, L2-resident), A and C aliased: the
//      same 1408 tiles with no operand leaving L2
// *us = mean duration of 20 timed launches; *tops = 2 M N K / duration.
extern "C" int jt_calib_tile(int which, float *us, double *tops) {
    if (which < 0 || which > 3 || !us || !tops) return (int)hipErrorInvalidValue;
    const int K = 1024, Mbig = 180224, Nbig = 11264;
    const int M = which == 3 ? Mbig : 4096, N = which == 3 ? 256 : Nbig;
    const int lda = which >= 2 ? 0 : K, ldc = which >= 1 ? 0 : N;
    int8_t *A = nullptr, *W = nullptr;
    float *sA = nullptr, *sB = nullptr, *C = nullptr;
    uint32_t *err = nullptr;
    hipError_t e = hipMalloc((void **)&A, (size_t)4096 * K);
    if (e == hipSuccess) e = hipMalloc((void **)&W, (size_t)Nbig * K);
    if (e == hipSuccess) e = hipMalloc((void **)&sA, (size_t)Mbig * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&sB, (size_t)Nbig * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&C, (size_t)4096 * Nbig * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&err, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(A, 1, (size_t)4096 * K);
    if (e == hipSuccess) e = hipMemset(W, 1, (size_t)Nbig * K);
    if (e == hipSuccess) e = hipMemset(sA, 0, (size_t)Mbig * sizeof(float));
    if (e == hipSuccess) e = hipMemset(sB, 0, (size_t)Nbig * sizeof(float));
    if (e == hipSuccess) e = hipMemset(err, 0, sizeof(uint32_t));
    float ms = 0.0f;
    if (e == hipSuccess)
        e = time_launches(
            [&] {
                return launch_w8a8_tile<EPI_PLAIN, 128, 256, 2, 4, 1, 3, 4>(
                    A, lda, sA, W, sB, M, N, N, K, C, ldc, err, nullptr);
            },
            20, &ms);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) {
        *us = ms * 1000.0f;
        *tops = 2.0 * M * N * (double)K / (ms * 1e-3) / 1e12;
    }
    void *bufs[] = {A, W, sA, sB, C, err};
    for (void *p : bufs)
        if (p) {
            const hipError_t ef = hipFree(p);
            if (e == hipSuccess) e = ef;
        }
    return (int)e;
}
