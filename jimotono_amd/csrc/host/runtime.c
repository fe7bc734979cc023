/*
 * runtime.c -- device binding, library stream, error word and staging
 * buffers of libjimotono_hip. C11 over the HIP runtime C API.
 *
 * Threading: like the reference (src/w8a8.c:53, src/lowbit.c:16) the
 * host-pointer entry points are not reentrant: they share the staging
 * buffers and the error word of one process-wide runtime.
 */
#define JT_RT_NO_MALLOC_MACRO /* this file defines the counting wrapper */
#include "jt_rt.h"

#include <errno.h>
#include <pthread.h>
#include <stdatomic.h>
#include <string.h>

#include "jimotono/hip_moe.h"

static jt_rt g_rt;
static int g_req_device = 0;

/* stream -> error word: slot i (0 .. JT_ERR_WORDS - 2) belongs to
 * g_err_stream[i] while g_err_live[i]; the last slot is shared by streams
 * past the table. jt_hip_stream_forget frees a slot (its word cleared), and
 * the next new stream takes the lowest free slot. */
static pthread_mutex_t g_err_mu = PTHREAD_MUTEX_INITIALIZER;
static hipStream_t g_err_stream[JT_ERR_WORDS - 1];
static unsigned char g_err_live[JT_ERR_WORDS - 1];
static int g_err_used;

static atomic_ullong g_allocs; /* successful device allocations so far */

hipError_t jt_rt_malloc(void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) atomic_fetch_add(&g_allocs, 1ull);
    return e;
}

int jt_hip_alloc_count(uint64_t *out) {
    if (!out) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    *out = (uint64_t)atomic_load(&g_allocs);
    return JT_OK;
}

int jt_rt_err(hipError_t e) {
    if (e == hipSuccess) return JT_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
        errno = ENOMEM;
        return JT_ERR_NOMEM;
    }
    errno = EIO;
    return JT_ERR_IO;
}

jt_rt *jt_rt_get(void) {
    if (g_rt.ready) return &g_rt;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || g_req_device >= n) {
        errno = ENODEV;
        return NULL;
    }
    if (hipSetDevice(g_req_device) != hipSuccess) {
        errno = EIO;
        return NULL;
    }
    memset(&g_rt, 0, sizeof(g_rt));
    g_rt.device = g_req_device;
    /* a blocking stream: the synchronous host-pointer calls and the weight
     * preparation are ordered after work the caller queued on the null
     * stream (torch's default stream, for one) */
    if (hipStreamCreateWithFlags(&g_rt.stream, hipStreamDefault) != hipSuccess ||
        jt_rt_malloc((void **)&g_rt.d_err, JT_ERR_WORDS * JT_ERR_STRIDE * 4) != hipSuccess ||
        jt_rt_malloc((void **)&g_rt.d_scratch, 4096) != hipSuccess ||
        hipMemset(g_rt.d_err, 0, JT_ERR_WORDS * JT_ERR_STRIDE * 4) != hipSuccess) {
        errno = EIO;
        return NULL;
    }
    /* every code object now, not at the first launch of one of its kernels
     * (a no-allocation entry point must not make the runtime allocate) */
    if (jtk_preload() != 0) {
        errno = EIO;
        return NULL;
    }
    /* the no-allocation entry points' scratch address on this device; if the
     * lookup fails they report JT_ERR_IO and everything else still works */
    (void)jtk_scratch_init();
    g_rt.ready = 1;
    return &g_rt;
}

int jt_hip_init(int device) {
    if (device < 0) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    if (g_rt.ready) {
        if (device != g_rt.device) {
            errno = EINVAL; /* one device per process */
            return JT_ERR_INVAL;
        }
        return hipSetDevice(device) == hipSuccess ? JT_OK : jt_rt_err(hipErrorUnknown);
    }
    g_req_device = device;
    return jt_rt_get() ? JT_OK : JT_ERR_IO;
}

void *jt_rt_buf(jt_rt *rt, int s, size_t bytes, int *rc) {
    if (bytes == 0) bytes = 16;
    if (rt->slot_bytes[s] >= bytes) return rt->slot[s];
    if (rt->slot[s]) {
        (void)hipStreamSynchronize(rt->stream);
        (void)hipFree(rt->slot[s]);
        rt->slot[s] = NULL;
        rt->slot_bytes[s] = 0;
    }
    size_t want = jt_round_up(bytes, 1u << 16);
    hipError_t e = jt_rt_malloc(&rt->slot[s], want);
    if (e != hipSuccess) {
        rt->slot[s] = NULL;
        *rc = jt_rt_err(e);
        return NULL;
    }
    rt->slot_bytes[s] = want;
    return rt->slot[s];
}

void *jt_rt_hbuf(jt_rt *rt, int s, size_t bytes, int *rc) {
    if (bytes == 0) bytes = 16;
    if (rt->hslot_bytes[s] >= bytes) return rt->hslot[s];
    if (rt->hslot[s]) {
        (void)hipStreamSynchronize(rt->stream);
        (void)hipHostFree(rt->hslot[s]);
        rt->hslot[s] = NULL;
        rt->hslot_bytes[s] = 0;
    }
    const size_t want = jt_round_up(bytes, 1u << 16);
    const hipError_t e = hipHostMalloc(&rt->hslot[s], want, hipHostMallocDefault);
    if (e != hipSuccess) {
        rt->hslot[s] = NULL;
        *rc = jt_rt_err(e);
        return NULL;
    }
    rt->hslot_bytes[s] = want;
    return rt->hslot[s];
}

uint32_t *jt_rt_errw(jt_rt *rt, hipStream_t stream) {
    pthread_mutex_lock(&g_err_mu);
    int i = 0, freed = -1;
    while (i < g_err_used && !(g_err_live[i] && g_err_stream[i] == stream)) {
        if (!g_err_live[i] && freed < 0) freed = i;
        i++;
    }
    if (i == g_err_used) { /* a new stream: a freed slot (word already zero) first */
        if (freed >= 0)
            i = freed;
        else if (g_err_used < JT_ERR_WORDS - 1)
            g_err_used++;
        if (i < JT_ERR_WORDS - 1) {
            g_err_stream[i] = stream;
            g_err_live[i] = 1;
        }
    }
    pthread_mutex_unlock(&g_err_mu);
    return rt->d_err + (size_t)i * JT_ERR_STRIDE;
}

int jt_hip_stream_forget(void *stream) {
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    hipStream_t st = (hipStream_t)stream;
    pthread_mutex_lock(&g_err_mu);
    int i = 0;
    while (i < g_err_used && !(g_err_live[i] && g_err_stream[i] == st)) i++;
    int rc = JT_OK;
    if (i < g_err_used) {
        /* the stream's queued work may still raise bits: let it finish,
         * then clear the word so the slot's next owner starts clean */
        const uint32_t zero = 0;
        hipError_t e = hipStreamSynchronize(st);
        if (e == hipSuccess)
            e = hipMemcpy(rt->d_err + (size_t)i * JT_ERR_STRIDE, &zero, sizeof(zero),
                          hipMemcpyHostToDevice);
        if (e == hipSuccess)
            g_err_live[i] = 0;
        else
            rc = jt_rt_err(e);
    }
    pthread_mutex_unlock(&g_err_mu);
    return rc;
}

int jt_rt_flags(jt_rt *rt, hipStream_t stream, uint32_t *flags) {
    uint32_t f = 0, *w = jt_rt_errw(rt, stream);
    hipError_t e = hipStreamSynchronize(stream);
    if (e == hipSuccess) e = hipMemcpy(&f, w, sizeof(f), hipMemcpyDeviceToHost);
    if (e == hipSuccess && f != 0) e = hipMemset(w, 0, sizeof(uint32_t));
    if (e != hipSuccess) return jt_rt_err(e);
    *flags = f;
    return JT_OK;
}

int jt_rt_flags_to_rc(uint32_t flags) {
    if (flags == 0) return JT_OK;
    if (flags & (JT_EF_NONFINITE_INPUT | JT_EF_QRANGE | JT_EF_BAD_ID)) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    if (flags & JT_EF_RANGE) {
        errno = ERANGE;
        return JT_ERR_INVAL;
    }
    errno = EINVAL; /* non-finite intermediate */
    return JT_ERR_INVAL;
}

int jt_rt_h2d(jt_rt *rt, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return JT_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, rt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    return jt_rt_err(e);
}

int jt_rt_d2h(jt_rt *rt, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return JT_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, rt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    return jt_rt_err(e);
}

int jt_hip_sync_errors(void *stream, uint32_t *out_flags) {
    jt_rt *rt = jt_rt_get();
    if (!rt) return JT_ERR_IO;
    if (!out_flags) {
        errno = EINVAL;
        return JT_ERR_INVAL;
    }
    if (!stream) { /* NULL: wait for the whole device, then read the word */
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return jt_rt_err(e);
    }
    return jt_rt_flags(rt, (hipStream_t)stream, out_flags);
}
