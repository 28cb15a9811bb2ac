// Device-side routing for the routed-expert executors (decode and prefill).
//
// One workgroup of 16 wave64s computes a stable sort of the T*topk routes by
// local expert id (the reference builds the same grouping on the host with
// argsort + scatter_add_, src/vllm_exl3/exl3.py:3275-3332, or in the padded
// kernel's stage 0, csrc/p2b_moe.cu:1380-1412).  The sort is a wave-level
// multisplit: each wave owns a contiguous range of routes and walks it 64 at
// a time; the lanes that carry the same expert find each other with one
// ballot per key bit, the lowest of them bumps the wave's counter for that
// expert in LDS, and every lane's rank is the old counter plus the number of
// its peers below it.  A block scan over (expert, wave) then gives every
// route its sorted position.  No atomics, no host round trip: the result is
// the same run to run and the host never reads it.
//
// Outputs (all in the caller's workspace):
//   n_active, slot_expert/start/rows  one slot per expert with >= 1 route,
//                                     in increasing expert order
//   row_token, row_expert             sorted row -> token, expert
//   route_pos                         route (t*topk + k) -> sorted row, or -1
//   n_mtiles, mt_slot, mt_row0        row tiles of tile_rows rows per slot
//                                     (prefill GEMM work list; optional)
//   n_sorted                          number of routes kept (optional)
#include "route_impl.h"

namespace exl3 {
namespace {

__global__ __launch_bounds__(kRouteThreads) void route_multisplit_kernel(
    const void* ids, int ids_i64, int n_routes, int topk, int n_local, const int32_t* n_valid,
    int tile_rows, RouteOut o) {
    route_multisplit_body(ids, ids_i64, n_routes, topk, n_local, n_valid, tile_rows, o);
}

// ---------------------------------------------------------------------------
// Multi-workgroup form: workgroups of 16 waves, one 64-route row per wave
// (1024 routes per workgroup).
// ---------------------------------------------------------------------------
constexpr int kWideRoutes = kRouteThreads;  // routes per workgroup

// Stable ranks within the workgroup (in route_pos) and the workgroup's
// count per digit (cnt[block][digit]; digit n_local collects the dropped
// routes): per-wave ranks from the peer masks, then each wave's base per
// digit (the counts of the earlier waves).
__global__ __launch_bounds__(kRouteThreads) void route_wide_count(const void* ids, int ids_i64, int n_routes,
                                                                  int topk, int n_local, const int32_t* n_valid,
                                                                  int* cnt, int* rank) {
    extern __shared__ int lc[];  // [kRouteWaves][digits]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int digits = n_local + 1;
    int nbits = 0;
    while ((1 << nbits) < digits) ++nbits;
    const int live_routes = n_valid ? min(n_routes, max(0, n_valid[0]) * topk) : n_routes;
    for (int i = threadIdx.x; i < kRouteWaves * digits; i += kRouteThreads) lc[i] = 0;
    __syncthreads();
    const int r = blockIdx.x * kWideRoutes + threadIdx.x;
    int key = n_local, below = 0;
    if (r < n_routes) {
        key = route_key(ids, ids_i64, r, live_routes, n_local);
        const uint64_t peers = peer_mask(key, nbits);
        const int leader = __ffsll((unsigned long long)peers) - 1;
        if (lane == leader) lc[w * digits + key] = __popcll(peers);
        below = __popcll(peers & ((1ull << lane) - 1ull));
    }
    __syncthreads();
    // thread d: the waves' bases for digit d and the workgroup's total
    for (int d = threadIdx.x; d < digits; d += kRouteThreads) {
        int run = 0;
        for (int i = 0; i < kRouteWaves; ++i) {
            const int c = lc[i * digits + d];
            lc[i * digits + d] = run;
            run += c;
        }
        cnt[(size_t)blockIdx.x * digits + d] = run;
    }
    __syncthreads();
    if (r < n_routes) rank[r] = lc[w * digits + key] + below;
}

// Per-digit totals, their scan, each workgroup's base per digit
// (digit-major, workgroup-minor: stable), the slot and row-tile tables.  One
// workgroup; thread d owns digit d; the counts of 8 workgroups are loaded at
// a time.
__global__ __launch_bounds__(kRouteThreads) void route_wide_scan(int n_blocks, int n_local, int tile_rows,
                                                                 int* cnt, RouteOut o) {
    __shared__ int tmp[kRouteWaves + 1];
    constexpr int kBatch = 8;
    const int d = threadIdx.x, digits = n_local + 1;
    int tot = 0;
    if (d < digits)
        for (int i0 = 0; i0 < n_blocks; i0 += kBatch) {
            int c[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) c[i] = i0 + i < n_blocks ? cnt[(size_t)(i0 + i) * digits + d] : 0;
#pragma unroll
            for (int i = 0; i < kBatch; ++i) tot += c[i];
        }
    int unused;
    const int off = block_exclusive_scan(d < digits ? tot : 0, tmp, &unused);
    if (d < digits) {
        int run = off;
        for (int i0 = 0; i0 < n_blocks; i0 += kBatch) {
            int c[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) c[i] = i0 + i < n_blocks ? cnt[(size_t)(i0 + i) * digits + d] : 0;
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                if (i0 + i < n_blocks) cnt[(size_t)(i0 + i) * digits + d] = run;
                run += c[i];
            }
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
    if (o.n_sorted && d == n_local) o.n_sorted[0] = off;
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
}

// Sorted positions: the workgroup's base for the route's digit plus its rank.
__global__ __launch_bounds__(256) void route_wide_place(const void* ids, int ids_i64, int n_routes, int topk,
                                                        int n_local, const int32_t* n_valid, const int* cnt,
                                                        RouteOut o) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= n_routes) return;
    const int live_routes = n_valid ? min(n_routes, max(0, n_valid[0]) * topk) : n_routes;
    const int key = route_key(ids, ids_i64, r, live_routes, n_local);
    if (key < n_local) {
        const int pos = cnt[(size_t)(r / kWideRoutes) * (n_local + 1) + key] + o.route_pos[r];
        o.route_pos[r] = pos;
        o.row_token[pos] = r / topk;
        o.row_expert[pos] = key;
        if (o.row_route) o.row_route[pos] = r;
    } else {
        o.route_pos[r] = -1;
    }
}

}  // namespace

size_t route_scratch_bytes(int n_routes, int n_local) {
    const size_t n_blocks = ((size_t)n_routes + kWideRoutes - 1) / kWideRoutes;
    return sizeof(int) * n_blocks * (size_t)(n_local + 1);
}

hipError_t launch_route_wide(const void* ids, int ids_i64, int n_routes, int topk, int n_local,
                             const int32_t* n_valid, int tile_rows, const RouteOut& o, int* scratch,
                             hipStream_t st) {
    if (n_routes < 1 || n_routes > kRouteWideMax || n_local < 1 || n_local > kRouteMaxLocal || !scratch)
        return hipErrorInvalidValue;
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)route_wide_count, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(sizeof(int) * kRouteWaves * (kRouteMaxLocal + 1)));
        if (e != hipSuccess) (void)hipGetLastError();
        return e;
    }();
    if (attr != hipSuccess) return attr;
    const int blocks = (n_routes + kWideRoutes - 1) / kWideRoutes;
    const size_t lds = sizeof(int) * kRouteWaves * (size_t)(n_local + 1);
    route_wide_count<<<blocks, kRouteThreads, lds, st>>>(ids, ids_i64, n_routes, topk, n_local, n_valid, scratch,
                                                         o.route_pos);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    route_wide_scan<<<1, kRouteThreads, 0, st>>>(blocks, n_local, tile_rows, scratch, o);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    route_wide_place<<<(n_routes + 255) / 256, 256, 0, st>>>(ids, ids_i64, n_routes, topk, n_local, n_valid,
                                                             scratch, o);
    return hipGetLastError();
}

size_t route_lds_bytes(int n_local) {
    return sizeof(int) * ((size_t)kRouteWaves * (n_local + 1) + kRouteWaves + 1);
}

hipError_t launch_route(const void* ids, int ids_i64, int n_routes, int topk, int n_local,
                        const int32_t* n_valid, int tile_rows, const RouteOut& o, hipStream_t st) {
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)route_multisplit_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)route_lds_bytes(kRouteMaxLocal));
        if (e != hipSuccess) (void)hipGetLastError();
        return e;
    }();
    if (attr != hipSuccess) return attr;
    route_multisplit_kernel<<<1, kRouteThreads, route_lds_bytes(n_local), st>>>(
        ids, ids_i64, n_routes, topk, n_local, n_valid, tile_rows, o);
    return hipGetLastError();
}

}  // namespace exl3
