// Device code of the one-block stable counting sort of (token, slot) pairs
// by expert and of the grouped GEMMs' tile list, shared by the sort
// launches (route.hip) and the decode launch that sorts in its last
// top-k block (gemm_i8.hip). The sort follows src/moe_layer.c:895-978: pairs
// in index order, each expert's kept pairs (rank < cap) contiguous from its
// offset, stable within an expert.
#pragma once
#include "jt_dev.h"

// tiles[i] = {e, off[e] + j*R, rows, 0} (int4) for the j-th R-row tile of
// expert e, experts in ascending order; *ntiles = total.
__device__ __forceinline__ void put_tiles(int4 *tiles, int start, int e, int base, int cnt,
                                          int R) {
    for (int j = 0; j * R < cnt; j++)
        tiles[start + j] = make_int4(e, base + j * R, min(R, cnt - j * R), 0);
}

#define SORT_SMALL 1024
#define SORT_EMAX 4096

// Exclusive scan of one int per thread over a 1024-thread block: wave scans
// with lane shuffles, then one pass over the 16 wave totals (2 barriers).
__device__ __forceinline__ int block_excl_scan_1024(int v, int *wsum, int *total) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 16; w++) {
        const int c = wsum[w];
        before += w < wave ? c : 0;
        all += c;
    }
    *total = all;
    __syncthreads();  // wsum is reused by the next scan
    return before + x - v;
}

// The body of the one-block sort: thread t holds pair t's expert e (-1:
// none). The LDS arrays are the caller's.
struct SortSmallLds {
    int sid[SORT_SMALL];
    int cnt[SORT_EMAX];
    int eoff[SORT_EMAX + 1];
    int buf[16];
};
static __device__ void sort_small_core(int e, int Tk, int E, int64_t cap, int R,
                                int32_t *__restrict__ off, int64_t *__restrict__ off64,
                                int32_t *__restrict__ perm, int64_t *__restrict__ perm64,
                                uint8_t *__restrict__ drop, int32_t *__restrict__ tiles,
                                int32_t *__restrict__ ntiles, SortSmallLds &sm) {
    int *sid = sm.sid, *cnt = sm.cnt, *eoff = sm.eoff, *buf = sm.buf;
    const int t = threadIdx.x;
    sid[t] = e;
    for (int i = t; i < E; i += 1024) cnt[i] = 0;
    __syncthreads();
    if (e >= 0) atomicAdd(&cnt[e], 1);
    int r = 0;  // stable rank: earlier pairs with the same expert
    if (e >= 0) {
        const int4 *s4 = (const int4 *)sid;
        int i = 0;
        for (; i + 4 <= t; i += 4) {
            const int4 v = s4[i >> 2];
            r += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
        }
        for (; i < t; i++) r += (sid[i] == e);
    }
    __syncthreads();
    // per-thread experts 4t..4t+3: kept counts and tile counts
    int kc[4], nt[4], ks = 0, ts = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int x = 4 * t + u;
        kc[u] = x < E ? (int)min((int64_t)cnt[x], cap) : 0;
        nt[u] = (kc[u] + R - 1) / R;
        ks += kc[u];
        ts += nt[u];
    }
    int ktot, ttot;
    int kbase = block_excl_scan_1024(ks, buf, &ktot);
    int tbase = block_excl_scan_1024(ts, buf, &ttot);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int x = 4 * t + u;
        if (x < E) {
            eoff[x] = kbase;
            off[x] = kbase;
            if (off64) off64[x] = kbase;
            put_tiles((int4 *)tiles, tbase, x, kbase, kc[u], R);
        }
        kbase += kc[u];
        tbase += nt[u];
    }
    if (t == 0) {
        off[E] = ktot;
        if (off64) off64[E] = ktot;
        *ntiles = ttot;
    }
    __syncthreads();
    if (e >= 0) {
        const bool kept = r < cap;
        if (drop) drop[t] = kept ? 0 : 1;
        if (kept) {
            perm[eoff[e] + r] = t;
            if (perm64) perm64[eoff[e] + r] = t;
        }
    }
}

