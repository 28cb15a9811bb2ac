// Device-side routing shared by the decode and prefill routed-expert
// executors (implementation in route.hip).
#pragma once

#include "exl3_common.h"

namespace exl3 {

constexpr int kRouteThreads = 1024;
constexpr int kRouteMaxLocal = 1023;  // experts per layer the router accepts

struct RouteOut {
    int* n_active;     // [1]
    int* slot_expert;  // [max_slots]
    int* slot_start;   // [max_slots]
    int* slot_rows;    // [max_slots]
    int* row_token;    // [n_routes]: sorted row -> token
    int* row_expert;   // [n_routes]: sorted row -> local expert
    int* route_pos;    // [n_routes]: route (t*topk+k) -> sorted row, or -1
    int* n_mtiles;     // [1]          (only when tile_rows > 0)
    int* mt_slot;      // [max_mtiles]
    int* mt_row0;      // [max_mtiles]
    int* n_sorted;     // [1] routes kept (nullable)
    int* mt_expert;    // [max_mtiles] local expert of each row tile (nullable)
    int* row_route;    // [n_routes]: sorted row -> route (nullable)
};

// Upper bound of the row tiles produced for tile_rows-row tiles.
inline int64_t route_max_mtiles(int64_t n_routes, int64_t max_slots, int64_t tile_rows) {
    return (n_routes + tile_rows - 1) / tile_rows + max_slots;
}

size_t route_lds_bytes(int n_local);

// Stable sort of the n_routes = T*topk routes by local expert; ids outside
// [0, n_local) and rows at or beyond *n_valid (when given) are dropped.
// Requires n_local <= kRouteMaxLocal.
hipError_t launch_route(const void* ids, int ids_i64, int n_routes, int topk, int n_local,
                        const int32_t* n_valid, int tile_rows, const RouteOut& o, hipStream_t st);

// The same sort spread over many workgroups, for large route counts (the
// single-workgroup sort walks n_routes / 16 routes per wave): three launches
// (ranks and counts per 1024-route workgroup, one scan over (expert,
// workgroup), placement) with the same outputs bit for bit.  `scratch` holds route_scratch_bytes(n_routes,
// n_local) bytes; n_routes <= kRouteWideMax.
constexpr int kRouteWideMin = 2048;
constexpr int kRouteWideMax = 1 << 16;
size_t route_scratch_bytes(int n_routes, int n_local);
hipError_t launch_route_wide(const void* ids, int ids_i64, int n_routes, int topk, int n_local,
                             const int32_t* n_valid, int tile_rows, const RouteOut& o, int* scratch,
                             hipStream_t st);

}  // namespace exl3
