// Device side of the routed-expert router (see route.hip for the algorithm);
// included by route.hip (the routing launch) and gemv.hip (the decode
// pipeline's combined route + rotate launch).
#pragma once

#include "route.h"

namespace exl3 {

constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteBatch = 8;  // 64-route rows whose keys a wave loads at once

// Exclusive prefix sum over the 1024 threads of the block; returns this
// thread's prefix and writes the total to *total.  `tmp` holds 16 ints.
__device__ inline int block_exclusive_scan(int v, int* tmp, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) tmp[w] = incl;
    __syncthreads();
    if (w == 0) {  // scan of the wave totals by one wave (shuffles, no serial loop)
        const int t = lane < kRouteWaves ? tmp[lane] : 0;
        int acc = t;
#pragma unroll
        for (int d = 1; d < kRouteWaves; d <<= 1) {
            const int u = __shfl_up(acc, d, 64);
            if (lane >= d) acc += u;
        }
        if (lane < kRouteWaves) tmp[lane] = acc - t;
        if (lane == kRouteWaves - 1) tmp[kRouteWaves] = acc;
    }
    __syncthreads();
    const int r = tmp[w] + incl - v;
    *total = tmp[kRouteWaves];
    __syncthreads();  // tmp is reused by the next scan
    return r;
}

__device__ __forceinline__ int route_key(const void* ids, int ids_i64, int r, int live_routes,
                                         int n_local) {
    if (r >= live_routes) return n_local;
    const int64_t e = ids_i64 ? reinterpret_cast<const int64_t*>(ids)[r]
                              : (int64_t)reinterpret_cast<const int32_t*>(ids)[r];
    return (e < 0 || e >= n_local) ? n_local : (int)e;
}

// Rank of each lane among the active lanes of the wave holding the same key
// (`nbits` key bits), and the mask of those peers.
__device__ __forceinline__ uint64_t peer_mask(int key, int nbits) {
    uint64_t peers = __ballot(1);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

__device__ inline void route_multisplit_body(const void* ids, int ids_i64, int n_routes, int topk, int n_local,
                                      const int32_t* n_valid, int tile_rows, const RouteOut& o) {
    extern __shared__ int lds_i[];
    int* cnt = lds_i;                                     // [kRouteWaves][n_local + 1]
    int* tmp = lds_i + kRouteWaves * (n_local + 1);       // [kRouteWaves + 1]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int digits = n_local + 1;
    int nbits = 0;
    while ((1 << nbits) < digits) ++nbits;
    const int live_routes = n_valid ? min(n_routes, max(0, n_valid[0]) * topk) : n_routes;
    for (int i = threadIdx.x; i < kRouteWaves * digits; i += kRouteThreads) cnt[i] = 0;
    __syncthreads();

    // Phase 1: per-wave stable ranks; route_pos temporarily holds the rank
    // of each route within its wave's run of the same expert.
    // The keys of kRouteBatch consecutive 64-route rows are loaded before
    // the first is ranked, so a wave waits on one memory round trip per
    // batch instead of one per 64 routes.
    const int per = (n_routes + kRouteWaves - 1) / kRouteWaves;
    const int r0 = w * per, r1 = min(n_routes, r0 + per);
    int* wcnt = cnt + w * digits;
    for (int base = r0; base < r1; base += 64 * kRouteBatch) {
        int key[kRouteBatch];
#pragma unroll
        for (int b = 0; b < kRouteBatch; ++b) {
            const int r = base + 64 * b + lane;
            key[b] = r < r1 ? route_key(ids, ids_i64, r, live_routes, n_local) : n_local;
        }
#pragma unroll
        for (int b = 0; b < kRouteBatch; ++b) {
            const int r = base + 64 * b + lane;
            if (base + 64 * b >= r1) break;  // wave-uniform
            if (r < r1) {
                const uint64_t peers = peer_mask(key[b], nbits);
                const int leader = __ffsll((unsigned long long)peers) - 1;
                const int below = __popcll(peers & ((1ull << lane) - 1ull));
                int old = 0;
                if (lane == leader) {
                    old = wcnt[key[b]];
                    wcnt[key[b]] = old + __popcll(peers);
                }
                old = __shfl(old, leader, 64);
                o.route_pos[r] = old + below;
            }
        }
    }
    __syncthreads();

    // Phase 2: per-expert totals, their exclusive scan, and each wave's base
    // for each expert (digit-major, wave-minor: stable).  Thread d owns digit d
    // (n_local + 1 <= kRouteThreads digits).
    const int d = threadIdx.x;
    int tot = 0;
    if (d < digits)
        for (int i = 0; i < kRouteWaves; ++i) tot += cnt[i * digits + d];
    int unused;
    const int off = block_exclusive_scan(d < digits ? tot : 0, tmp, &unused);
    if (d < digits) {
        int run = off;
        for (int i = 0; i < kRouteWaves; ++i) {
            const int c = cnt[i * digits + d];
            cnt[i * digits + d] = run;
            run += c;
        }
    }
    const int has = (d < n_local && tot > 0) ? 1 : 0;
    int n_active;
    const int slot = block_exclusive_scan(has, tmp, &n_active);
    if (has) {
        o.slot_expert[slot] = d;
        o.slot_start[slot] = off;
        o.slot_rows[slot] = tot;
    }
    if (threadIdx.x == 0) o.n_active[0] = n_active;
    if (o.n_sorted && d == n_local) o.n_sorted[0] = off;  // routes before the sentinel bucket
    if (tile_rows > 0) {
        const int nt = has ? (tot + tile_rows - 1) / tile_rows : 0;
        int n_mt;
        const int mt0 = block_exclusive_scan(nt, tmp, &n_mt);
        for (int k = 0; k < nt; ++k) {
            o.mt_slot[mt0 + k] = slot;
            if (o.mt_expert) o.mt_expert[mt0 + k] = d;
            o.mt_row0[mt0 + k] = k * tile_rows;
        }
        if (threadIdx.x == 0) o.n_mtiles[0] = n_mt;
    }
    __syncthreads();

    // Phase 3: sorted positions.
    for (int base = r0; base < r1; base += 64 * kRouteBatch) {
        int key[kRouteBatch], rank[kRouteBatch];
#pragma unroll
        for (int b = 0; b < kRouteBatch; ++b) {
            const int r = base + 64 * b + lane;
            key[b] = r < r1 ? route_key(ids, ids_i64, r, live_routes, n_local) : n_local;
            rank[b] = r < r1 ? o.route_pos[r] : 0;
        }
#pragma unroll
        for (int b = 0; b < kRouteBatch; ++b) {
            const int r = base + 64 * b + lane;
            if (r >= r1) continue;
            if (key[b] < n_local) {
                const int pos = cnt[w * digits + key[b]] + rank[b];
                o.route_pos[r] = pos;
                o.row_token[pos] = r / topk;
                o.row_expert[pos] = key[b];
                if (o.row_route) o.row_route[pos] = r;
            } else {
                o.route_pos[r] = -1;
            }
        }
    }
}


}  // namespace exl3
