// Fixed device scratch for the entry points that must not allocate
// (jt_hip_ffn_fwd_noalloc): a file-scope __device__ array of JT_SCRATCH_BYTES
// that every GPU the library runs on holds until the process ends.
//
// In host code the array's name is only a stand-in for the symbol: its
// device address, different on each GPU, comes from hipGetSymbolAddress,
// called once per device by jtk_scratch_init (the library's set-up, with
// that device current). Host code uses only that address afterwards.
#include <hip/hip_runtime.h>

#include <atomic>

#include "jt_launch.h"

static __device__ __align__(256) unsigned char scratch[JT_SCRATCH_BYTES];

#define JT_MAX_DEVICES 64
static std::atomic<void *> g_scratch[JT_MAX_DEVICES];

extern "C" int jtk_scratch_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= JT_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (g_scratch[dev].load()) return 0;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch[dev].store(p);
    return 0;
}

__global__ __launch_bounds__(256) void k_scratch_zero(uint32_t *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

extern "C" int jtk_scratch_zero(uint32_t *p, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_scratch_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return (int)hipGetLastError();
}

extern "C" int jtk_preload_gemm_i8(void);
extern "C" int jtk_preload_legacy(void);
extern "C" int jtk_preload_quant(void);
extern "C" int jtk_preload_route(void);
extern "C" int jtk_preload_router(void);
extern "C" int jtk_preload_bwd(void);
extern "C" int jtk_preload_gdn2(void);

extern "C" int jtk_preload(void) {
    int e = jtk_preload_gemm_i8();
    if (!e) e = jtk_preload_legacy();
    if (!e) e = jtk_preload_quant();
    if (!e) e = jtk_preload_route();
    if (!e) e = jtk_preload_router();
    if (!e) e = jtk_preload_bwd();
    if (!e) e = jtk_preload_gdn2();
    if (!e) {
        hipFuncAttributes a;
        e = (int)hipFuncGetAttributes(&a, (const void *)k_scratch_zero);
    }
    return e;
}

extern "C" void *jtk_scratch(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= JT_MAX_DEVICES) return nullptr;
    return g_scratch[dev].load();
}
