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

}  // namespace

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
