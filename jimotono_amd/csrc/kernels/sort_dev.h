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


// The same sort for at most SORTF_TK pairs and SORTF_E experts, with the
// same outputs, run by the first Tk / 64 waves of a block of at least
// SORTF_TK threads: a pair's rank within its wave comes from one ballot per
// bit of the expert id (the lanes whose id agrees on every bit), the
// earlier waves' counts of its expert from LDS, and the expert offsets and
// tile bases from one wave's scan over the experts (lane l owns experts
// l*EPL .. l*EPL + EPL - 1). No pass over the earlier pairs and one block
// barrier less than sort_small_core.
#define SORTF_TK 256
#define SORTF_E 1024
struct SortFastLds {
    int wcnt[SORTF_TK / 64][SORTF_E];  // pairs of expert x in wave w
    int eoff[SORTF_E];
};
union SortLds {
    SortSmallLds small;
    SortFastLds fast;
};

__device__ __forceinline__ int wave_incl_scan_i(int x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}

static __device__ void sort_small_fast(int e, int Tk, int E, int64_t cap, int R,
                                       int32_t *__restrict__ off, int64_t *__restrict__ off64,
                                       int32_t *__restrict__ perm, int64_t *__restrict__ perm64,
                                       uint8_t *__restrict__ drop, int32_t *__restrict__ tiles,
                                       int32_t *__restrict__ ntiles, SortFastLds &sm) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int NW = (Tk + 63) >> 6;
    int *flat = &sm.wcnt[0][0];
    for (int i = t; i < NW * SORTF_E; i += blockDim.x) flat[i] = 0;
    __syncthreads();
    int r = 0;  // stable rank: earlier pairs with the same expert
    if (wave < NW) {
        uint64_t m = __ballot(e >= 0);
        for (int b = 0; (1 << b) < E; b++) {
            const int bit = (e >> b) & 1;
            const uint64_t bb = __ballot(bit);
            m &= bit ? bb : ~bb;
        }
        r = __popcll(m & ((1ull << lane) - 1ull));
        if (e >= 0 && r == 0) sm.wcnt[wave][e] = __popcll(m);
    }
    __syncthreads();
    if (e >= 0)
        for (int w = 0; w < wave; w++) r += sm.wcnt[w][e];
    if (wave == 0) {
        // lane l: experts l*EPL .. l*EPL + EPL - 1 (EPL <= 16); their kept
        // counts are summed here and read again from LDS below (no private
        // array, which would live in scratch memory)
        const int EPL = (E + 63) >> 6, x0 = lane * EPL;
        int ks = 0, ts = 0;
        for (int u = 0; u < EPL; u++) {
            const int x = x0 + u;
            int c = 0;
            // every count is read (x <= 63 * 16 + 15 stays in the array) so
            // the reads issue back to back; the unused ones are dropped
#pragma unroll
            for (int w = 0; w < SORTF_TK / 64; w++) {
                const int v = sm.wcnt[w][x];
                c += w < NW ? v : 0;
            }
            const int kc = x < E ? (int)min((int64_t)c, cap) : 0;
            ks += kc;
            ts += (kc + R - 1) / R;
        }
        const int kin = wave_incl_scan_i(ks, lane), tin = wave_incl_scan_i(ts, lane);
        int kbase = kin - ks, tbase = tin - ts;
        for (int u = 0; u < EPL; u++) {
            const int x = x0 + u;
            if (x >= E) break;
            int c = 0;
#pragma unroll
            for (int w = 0; w < SORTF_TK / 64; w++) {
                const int v = sm.wcnt[w][x];
                c += w < NW ? v : 0;
            }
            const int kc = (int)min((int64_t)c, cap);
            sm.eoff[x] = kbase;
            off[x] = kbase;
            if (off64) off64[x] = kbase;
            put_tiles((int4 *)tiles, tbase, x, kbase, kc, R);
            kbase += kc;
            tbase += (kc + R - 1) / R;
        }
        if (lane == 63) {
            off[E] = kin;
            if (off64) off64[E] = kin;
            *ntiles = tin;
        }
    }
    __syncthreads();
    if (e >= 0) {
        const bool kept = r < cap;
        if (drop) drop[t] = kept ? 0 : 1;
        if (kept) {
            perm[sm.eoff[e] + r] = t;
            if (perm64) perm64[sm.eoff[e] + r] = t;
        }
    }
}
