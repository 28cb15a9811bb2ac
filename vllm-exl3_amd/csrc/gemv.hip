// Decode-path kernels: streaming EXL3 GEMV (plain linear and the two MoE
// projections), device-side routing and the deterministic top-k combine.
//
// Replaces, on one MI355X:
//   * exl3_gemv / exl3_gemm (csrc/exl3_gemv.cu:23-63, csrc/exl3_gemm.cu:8-31,
//     bindings csrc/bindings.cpp:110-147);
//   * the fused decode MoE p2b_fused_moe{,_mk,_padded}
//     (csrc/p2b_moe.cu:643-1071, 1295-2487) as four ordinary launches, no
//     grid barriers, no device-scope fences, no host synchronisation:
//       route    stable sort of the routes by expert (one workgroup);
//       gate/up  raw split-K partial sums of both projections;
//       down     its activation staging finishes gate/up (sum of splits,
//                output rotation x svh, fp16 rounding, SwiGLU, down suh,
//                down input rotation), then raw split-K partial sums;
//       combine  per (token, column block): finish each route's down result
//                (rotation x svh) and sum w * d in slot order
//                (csrc/p2b_moe.cu:1976-2008): deterministic, no atomics.
#include "gemv_core.h"

#include <cmath>

namespace exl3 {
namespace {

constexpr int kMaxMRB = 16;       // activation rows per row group (one MFMA row block)
constexpr int kMaxRoutes = 8192;  // routes sortable by the single-workgroup router
constexpr int kRouteBits = 13;    // log2(kMaxRoutes)
constexpr int kRouteThreads = 1024;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Duplicate each of 4 fp16 values: (h0,h1),(h2,h3) -> h0,h0,h1,h1,h2,h2,h3,h3.
__device__ __forceinline__ half8_t dup4(uint32_t d0, uint32_t d1) {
    v4u r;
    r.x = __builtin_amdgcn_perm(d0, d0, 0x05040504u);
    r.y = __builtin_amdgcn_perm(d0, d0, 0x07060706u);
    r.z = __builtin_amdgcn_perm(d1, d1, 0x05040504u);
    r.w = __builtin_amdgcn_perm(d1, d1, 0x07060706u);
    return __builtin_bit_cast(half8_t, r);
}

// Stream the wave's tile rows of one projection for the current chunk and
// accumulate into acc[8] (one float4 per 16-column tile).
//   tbase:     byte address of tile (first tile row of the chunk, j*8)
//   row_bytes: bytes between consecutive tile rows (tiles_n * 32K)
//   nkt:       tile rows in the chunk; the wave takes rows wave, wave+4, ...
//   A:         this projection's activations [nkt][MRB][16] fp16 (kappa order)
template <int K, int CB>
__device__ __forceinline__ void stream_rows(const uint8_t* __restrict__ tbase, size_t row_bytes,
                                            int nkt, int wave, int lane, uint32_t* stage,
                                            const uint16_t* A, int MRB, int arow,
                                            float4_t (&acc)[8]) {
    constexpr int span = 256 * K;
    constexpr int tile_bytes = 32 * K;
    const bool ld = lane * 16 < span;
    const LaneWords lw = lane_words<K>(lane);
    const int g = lane >> 4;
    const int n = nkt > wave ? (nkt - wave + kWaves - 1) / kWaves : 0;
    const uint8_t* lane_base = tbase + lane * 16;
    v4u buf[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
        if (d < n && ld)
            buf[d] = __builtin_nontemporal_load(
                reinterpret_cast<const v4u*>(lane_base + (size_t)(wave + d * kWaves) * row_bytes));
    const uint8_t* st = reinterpret_cast<const uint8_t*>(stage);
    for (int i0 = 0; i0 < n; i0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int i = i0 + d;
            if (i < n) {
                if (ld) reinterpret_cast<v4u*>(stage)[lane] = buf[d];
                const int inext = i + kDepth;
                if (inext < n && ld)
                    buf[d] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(
                        lane_base + (size_t)(wave + inext * kWaves) * row_bytes));
                const int ktl = wave + i * kWaves;
                const uint32_t* ap =
                    reinterpret_cast<const uint32_t*>(A + ((size_t)ktl * MRB + arow) * 16 + 4 * g);
                const half8_t a = dup4(ap[0], ap[1]);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t hi = *reinterpret_cast<const uint32_t*>(st + t * tile_bytes + lw.off_hi);
                    const uint32_t lo = *reinterpret_cast<const uint32_t*>(st + t * tile_bytes + lw.off_lo);
                    uint32_t b[4];
                    decode4<K, CB>(hi, lo, lw.shift, b);
                    acc[t] = mfma16x16x32(a, b, acc[t]);
                }
            }
        }
    }
}

struct Proj {
    const uint8_t* trellis;
    const uint16_t* suh;
    const uint16_t* svh;
    int K;
};

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// Activation of the routed expert, with the reference's clamp rules
// (src/vllm_exl3/exl3.py:2386-2409): gate clamped from above, up symmetric.
__device__ __forceinline__ float activate(float g, float u, int act, float limit) {
    if (act == kActRelu2) {
        if (limit > 0.0f) u = fminf(fmaxf(u, -limit), limit);
        const float r = fmaxf(u, 0.0f);
        return r * r;
    }
    if (limit > 0.0f) {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
    }
    if (act == kActSwigluOai) return (u + 1.0f) * g * (1.0f / (1.0f + __expf(-1.702f * g)));
    return silu_f(g) * u;
}

// Output side of one 128-column block for one row: v[h] holds the summed,
// not yet rotated result at column lane + 64 h; returns (H v / sqrt(128)) * svh.
__device__ __forceinline__ void finish_block(float& v0, float& v1, const uint16_t* svh, int c0,
                                             int lane) {
    had128(v0, v1, lane);
    v0 = v0 * kHadNorm * (float)bits_to_half(svh[c0]);
    v1 = v1 * kHadNorm * (float)bits_to_half(svh[c0 + 64]);
}

// Finish gate/up for one route row and one 128-block hb of the intermediate
// dimension, and rotate the activation for the down projection.  g and u
// leave the GEMV as fp16 and the activation is stored as fp16
// (src/vllm_exl3/exl3.py:2403-2410, csrc/p2b_moe.cu:755-768).
__device__ __forceinline__ void gateup_finish(const GemvParams& p, const Proj* gu, int nproj,
                                              const uint16_t* down_suh, int64_t row, int hb,
                                              int lane, float& a0, float& a1) {
    const int inter = p.in_features;
    const int c0 = hb * 128 + lane;
    float v[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        if (q < nproj) {
            for (int ss = 0; ss < p.src_S; ++ss) {
                const float* src = p.src_ws + (((int64_t)q * p.src_S + ss) * p.n_rows_ws + row) * inter;
                v[q][0] += src[c0];
                v[q][1] += src[c0 + 64];
            }
            finish_block(v[q][0], v[q][1], gu[q].svh, c0, lane);
        }
    }
    float a[2];
    for (int h = 0; h < 2; ++h) {
        const float u = (float)f32_to_f16_rne(nproj == 2 ? v[1][h] : v[0][h]);
        const float g = nproj == 2 ? (float)f32_to_f16_rne(v[0][h]) : 0.0f;
        a[h] = (float)f32_to_f16_rne(activate(g, u, p.act, p.limit));
    }
    a[0] *= (float)bits_to_half(down_suh[c0]);
    a[1] *= (float)bits_to_half(down_suh[c0 + 64]);
    had128(a[0], a[1], lane);
    a0 = a[0] * kHadNorm;
    a1 = a[1] * kHadNorm;
}

template <int CB, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nJ = p.out_features >> 7;
    const int item = blockIdx.x;
    const int s = item % p.S;
    const int rest = item / p.S;
    const int j = rest % nJ;
    const int slot = rest / nJ;

    int rows, row_base, expert = 0;
    if constexpr (MODE == kModeLinear) {
        rows = p.m_rows;
        row_base = 0;
    } else {
        if (slot >= *p.n_active) return;
        expert = p.slot_expert[slot];
        row_base = p.slot_start[slot];
        rows = p.slot_rows[slot];
    }
    // projections streamed by this kernel
    const int nproj = (MODE == kModeGateUp && !p.gateless) ? 2 : 1;
    Proj pr[2];
    // Down: gate/up projections whose partials are finished while staging
    Proj gu[2];
    const uint16_t* down_suh = nullptr;
    if constexpr (MODE == kModeLinear) {
        pr[0] = {reinterpret_cast<const uint8_t*>(p.w_trellis), p.w_suh, p.w_svh, p.kuni[0]};
        pr[1] = pr[0];
    } else {
        auto load_proj = [&](int pj) {
            Proj q;
            q.trellis = reinterpret_cast<const uint8_t*>(p.tab[3 * pj][expert]);
            q.suh = reinterpret_cast<const uint16_t*>(p.tab[3 * pj + 1][expert]);
            q.svh = reinterpret_cast<const uint16_t*>(p.tab[3 * pj + 2][expert]);
            q.K = p.ktab[pj] ? (int)p.ktab[pj][expert] : p.kuni[pj];
            return q;
        };
        if constexpr (MODE == kModeGateUp) {
            pr[0] = load_proj(p.gateless ? 1 : 0);
            pr[1] = load_proj(1);
        } else {
            pr[0] = load_proj(2);
            pr[1] = pr[0];
            gu[0] = load_proj(p.gateless ? 1 : 0);
            gu[1] = load_proj(1);
            down_suh = pr[0].suh;
        }
    }
    const int gu_nproj = p.gateless ? 1 : 2;

    const int MRB = p.MRB;
    const int tiles_n = p.out_features >> 4;
    const int hb_first = s * p.R_hb;  // first 128-row input block of this split
    uint32_t* stage = reinterpret_cast<uint32_t*>(lds) + wave * (kStageBytes / 4);
    uint16_t* A = reinterpret_cast<uint16_t*>(lds + kWaves * kStageBytes);
    float* red = reinterpret_cast<float*>(lds + kWaves * kStageBytes);
    const int g = lane >> 4, nu = lane & 15;
    const int col_nu = sigma_col(nu);

    for (int rg = 0; rg < rows; rg += MRB) {
        const int nr = min(MRB, rows - rg);
        const int arow = min(lane & 15, nr - 1);
        float4_t acc[2][8];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[q][t] = float4_t{0.f, 0.f, 0.f, 0.f};

        for (int c0 = 0; c0 < p.R_hb; c0 += p.C_hb) {
            const int nb = min(p.C_hb, p.R_hb - c0);
            const int qstride = nb * 8 * MRB * 16;  // fp16 elements per projection block
            __syncthreads();
            // ---- activations of this chunk, rotated, into LDS ----
            const int units = nproj * nr * nb;
            for (int u = wave; u < units; u += kWaves) {
                const int q = u / (nr * nb);
                const int r = (u / nb) % nr;
                const int hb = u % nb;
                const int64_t fb = (int64_t)(hb_first + c0 + hb) * 128;
                float v0, v1;
                if constexpr (MODE == kModeDown) {
                    gateup_finish(p, gu, gu_nproj, down_suh, row_base + rg + r, hb_first + c0 + hb,
                                  lane, v0, v1);
                } else {
                    int64_t tok;
                    if constexpr (MODE == kModeLinear)
                        tok = rg + r;
                    else
                        tok = p.row_token[row_base + rg + r];
                    v0 = load_act(p.x, p.x_dtype, tok * p.x_stride + fb + lane);
                    v1 = load_act(p.x, p.x_dtype, tok * p.x_stride + fb + lane + 64);
                    const uint16_t* su = q ? pr[1].suh : pr[0].suh;
                    v0 *= (float)bits_to_half(su[fb + lane]);
                    v1 *= (float)bits_to_half(su[fb + lane + 64]);
                    had128(v0, v1, lane);
                    v0 *= kHadNorm;
                    v1 *= kHadNorm;
                }
                uint16_t* Aq = A + q * qstride;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int c = lane + 64 * h;
                    const int ktl = hb * 8 + (c >> 4);
                    Aq[(ktl * MRB + r) * 16 + pi_inv(c & 15)] =
                        half_to_bits(f32_to_f16_rne(h ? v1 : v0));
                }
            }
            __syncthreads();
            // ---- stream the packed tiles of each projection ----
            // (projection index kept compile-time so acc stays in registers)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (q < nproj) {
                    const size_t tile_bytes = 32u * (size_t)pr[q].K;
                    const size_t row_bytes = (size_t)tiles_n * tile_bytes;
                    const uint8_t* tb = pr[q].trellis + ((size_t)(hb_first + c0) * 8 * tiles_n +
                                                         (size_t)j * 8) * tile_bytes;
                    const uint16_t* Aq = A + q * qstride;
                    switch (pr[q].K) {
                        case 2: stream_rows<2, CB>(tb, row_bytes, nb * 8, wave, lane, stage, Aq, MRB, arow, acc[q]); break;
                        case 3: stream_rows<3, CB>(tb, row_bytes, nb * 8, wave, lane, stage, Aq, MRB, arow, acc[q]); break;
                        case 4: stream_rows<4, CB>(tb, row_bytes, nb * 8, wave, lane, stage, Aq, MRB, arow, acc[q]); break;
                        default: break;  // rejected on the host
                    }
                }
            }
        }
        // ---- cross-wave reduction into red[q][row][128], fixed wave order ----
        __syncthreads();
        for (int w = 0; w < kWaves; ++w) {
            if (wave == w) {
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    if (q < nproj)
#pragma unroll
                        for (int t = 0; t < 8; ++t)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int row = 4 * g + i;
                                if (row < nr) {
                                    float* dst = red + (q * MRB + row) * 128 + t * 16 + col_nu;
                                    *dst = (w == 0 ? 0.0f : *dst) + acc[q][t][i];
                                }
                            }
            }
            __syncthreads();
        }
        if (MODE == kModeLinear && p.S == 1) {
            // single split: finish in place
            for (int r = wave; r < nr; r += kWaves) {
                float v0 = red[r * 128 + lane], v1 = red[r * 128 + lane + 64];
                finish_block(v0, v1, pr[0].svh, j * 128 + lane, lane);
                const int64_t o = (int64_t)(rg + r) * p.out_stride + j * 128 + lane;
                store_out(p.out, p.out_dtype, o, v0);
                store_out(p.out, p.out_dtype, o + 64, v1);
            }
        } else {
            for (int e = tid; e < nproj * nr * 128; e += kThreads) {
                const int q = e / (nr * 128), r = (e >> 7) % nr, c = e & 127;
                p.ws[(((int64_t)q * p.S + s) * p.n_rows_ws + row_base + rg + r) * p.out_features +
                     j * 128 + c] = red[(q * MRB + r) * 128 + c];
            }
        }
        __syncthreads();
    }
}

// Linear with split-K: out[m] = finish(sum of splits).  One wave per
// (row, 128-column block).
__global__ __launch_bounds__(256) void linear_finish_kernel(const float* __restrict__ ws, int S,
                                                            int m, int out_f,
                                                            const uint16_t* __restrict__ svh,
                                                            void* out, int out_dtype) {
    const int lane = threadIdx.x & 63;
    const int nJ = out_f >> 7;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= m * nJ) return;
    const int r = item / nJ, j = item % nJ;
    float v0 = 0.f, v1 = 0.f;
    for (int ss = 0; ss < S; ++ss) {
        const float* src = ws + ((int64_t)ss * m + r) * out_f + j * 128;
        v0 += src[lane];
        v1 += src[lane + 64];
    }
    finish_block(v0, v1, svh, j * 128 + lane, lane);
    const int64_t o = (int64_t)r * out_f + j * 128 + lane;
    store_out(out, out_dtype, o, v0);
    store_out(out, out_dtype, o + 64, v1);
}

// ---------------------------------------------------------------------------
// Routing: stable sort of the T*topk routes by local expert id (sentinel
// routes last), then slots = runs of one expert.  One workgroup.
// ---------------------------------------------------------------------------
struct RouteOut {
    int* n_active;    // [1]
    int* slot_expert; // [max_slots]
    int* slot_start;  // [max_slots]
    int* slot_rows;   // [max_slots]
    int* row_token;   // [n_routes]: sorted row -> token
    int* row_expert;  // [n_routes]: sorted row -> local expert
    int* route_pos;   // [n_routes]: route (t*topk+k) -> sorted row, or -1
};

__global__ __launch_bounds__(kRouteThreads) void route_kernel(const void* ids, int ids_i64, int n_routes,
                                                              int topk, int n_local,
                                                              const int32_t* n_valid, RouteOut o) {
    __shared__ uint32_t key[kMaxRoutes];
    __shared__ int wave_sum[kRouteThreads / 64];
    const int tid = threadIdx.x;
    int np2 = 1;
    while (np2 < n_routes) np2 <<= 1;
    // rows at or beyond the device-side live-row count are padding: their
    // routes become sentinels (the host never reads n_valid)
    const int live_routes = n_valid ? min(n_routes, max(0, n_valid[0]) * topk) : n_routes;
    for (int i = tid; i < np2; i += kRouteThreads) {
        uint32_t k = 0xFFFFFFFFu;
        if (i < n_routes) {
            const int64_t e = ids_i64 ? reinterpret_cast<const int64_t*>(ids)[i]
                                      : (int64_t)reinterpret_cast<const int32_t*>(ids)[i];
            const bool live = i < live_routes;
            const uint32_t el = (!live || e < 0 || e >= n_local) ? (uint32_t)n_local : (uint32_t)e;
            k = (el << kRouteBits) | (uint32_t)i;
        }
        key[i] = k;
    }
    __syncthreads();
    // bitonic sort, ascending
    for (int k = 2; k <= np2; k <<= 1) {
        for (int jj = k >> 1; jj > 0; jj >>= 1) {
            for (int i = tid; i < np2; i += kRouteThreads) {
                const int ixj = i ^ jj;
                if (ixj > i) {
                    const uint32_t a = key[i], b = key[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        key[i] = b;
                        key[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    // run starts -> slot ids via a block-wide exclusive scan; each thread owns
    // a contiguous range of sorted positions
    const int per = (n_routes + kRouteThreads - 1) / kRouteThreads;
    const int p0 = tid * per, p1 = min(n_routes, p0 + per);
    int cnt = 0;
    for (int q = p0; q < p1; ++q) {
        const uint32_t e = key[q] >> kRouteBits;
        if (e < (uint32_t)n_local && (q == 0 || (key[q - 1] >> kRouteBits) != e)) ++cnt;
    }
    const int lane = tid & 63, w = tid >> 6;
    int incl = cnt;
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) wave_sum[w] = incl;
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int i = 0; i < kRouteThreads / 64; ++i) {
            const int t = wave_sum[i];
            wave_sum[i] = acc;
            acc += t;
        }
        o.n_active[0] = acc;
    }
    __syncthreads();
    int slot = wave_sum[w] + incl - cnt;  // exclusive prefix for this thread's range
    for (int q = p0; q < p1; ++q) {
        const uint32_t kq = key[q];
        const uint32_t e = kq >> kRouteBits;
        const int route = (int)(kq & ((1u << kRouteBits) - 1));
        if (e < (uint32_t)n_local) {
            o.route_pos[route] = q;
            o.row_token[q] = route / topk;
            o.row_expert[q] = (int)e;
            if (q == 0 || (key[q - 1] >> kRouteBits) != e) {
                o.slot_expert[slot] = (int)e;
                o.slot_start[slot] = q;
                int end = q + 1;
                while (end < n_routes && (key[end] >> kRouteBits) == e) ++end;
                o.slot_rows[slot] = end - q;
                ++slot;
            }
        } else {
            o.route_pos[route] = -1;
        }
    }
}

// out[t, block j] = sum_k w[t,k] * finish(sum_s partial_s[pos(t,k)]) in slot
// order; sentinel routes are skipped (their rows are never read, so unwritten
// rows cannot leak NaN).  One wave per (token, 128-column block).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ ws, int S,
                                                     int n_routes, int H, const int* route_pos,
                                                     const int* row_expert,
                                                     const int64_t* down_svh_tab,
                                                     const void* weights, int w_dtype, int T,
                                                     int topk, void* out, int out_dtype) {
    const int lane = threadIdx.x & 63;
    const int nJ = H >> 7;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= T * nJ) return;
    const int t = item / nJ, j = item % nJ;
    const int c0 = j * 128 + lane;
    float acc0 = 0.f, acc1 = 0.f;
    for (int k = 0; k < topk; ++k) {
        const int pos = route_pos[t * topk + k];
        if (pos < 0) continue;
        float v0 = 0.f, v1 = 0.f;
        for (int ss = 0; ss < S; ++ss) {
            const float* src = ws + ((int64_t)ss * n_routes + pos) * H;
            v0 += src[c0];
            v1 += src[c0 + 64];
        }
        finish_block(v0, v1, reinterpret_cast<const uint16_t*>(down_svh_tab[row_expert[pos]]), c0,
                     lane);
        const int64_t wi = (int64_t)t * topk + k;
        float w;
        if (w_dtype == kF32)
            w = reinterpret_cast<const float*>(weights)[wi];
        else if (w_dtype == kF16)
            w = (float)bits_to_half(reinterpret_cast<const uint16_t*>(weights)[wi]);
        else
            w = __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(weights)[wi] << 16);
        acc0 += w * v0;
        acc1 += w * v1;
    }
    const int64_t o = (int64_t)t * H + c0;
    store_out(out, out_dtype, o, acc0);
    store_out(out, out_dtype, o + 64, acc1);
}

// ---------------------------------------------------------------------------
// Host-side planning (shared by the workspace queries and the launches)
// ---------------------------------------------------------------------------
constexpr int kTargetItems = 2048;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Largest divisor of n_hb with base_items * S <= target (at least 1).
inline int pick_splits(int n_hb, int base_items) {
    int best = 1;
    for (int d = 1; d <= n_hb; ++d)
        if (n_hb % d == 0 && (int64_t)base_items * d <= kTargetItems) best = d;
    return best;
}

// Hadamard blocks whose activations fit the LDS budget at once.
inline int pick_chunk(int R_hb, int nproj, int MRB) {
    const int per_hb = nproj * 8 * MRB * 16 * 2;  // bytes
    int c = (40 * 1024) / per_hb;
    if (c < 1) c = 1;
    return c < R_hb ? c : R_hb;
}

inline size_t gemv_lds_bytes(int C_hb, int nproj, int MRB) {
    const size_t a = (size_t)nproj * C_hb * 8 * MRB * 16 * 2;
    const size_t r = (size_t)nproj * MRB * 128 * 4;
    return kWaves * kStageBytes + (a > r ? a : r);
}

struct PhasePlan {
    int S, R_hb, C_hb;
    size_t lds;
};

inline PhasePlan plan_phase(int in_f, int base_items, int nproj, int MRB) {
    PhasePlan pp;
    const int n_hb = in_f / 128;
    pp.S = pick_splits(n_hb, base_items);
    pp.R_hb = n_hb / pp.S;
    pp.C_hb = pick_chunk(pp.R_hb, nproj, MRB);
    pp.lds = gemv_lds_bytes(pp.C_hb, nproj, MRB);
    return pp;
}

struct MoePlan {
    int n_routes, max_slots, MRB, nproj;
    PhasePlan gu, dn;
    size_t off_route, off_wsgu, off_wsd, total;
};

inline MoePlan plan_moe(int64_t T, int64_t topk, int64_t n_local, int64_t hidden, int64_t inter,
                        int gateless) {
    MoePlan m;
    m.n_routes = (int)(T * topk);
    m.max_slots = (int)(m.n_routes < n_local ? m.n_routes : n_local);
    m.MRB = (int)(T < kMaxMRB ? (T < 1 ? 1 : T) : kMaxMRB);
    m.nproj = gateless ? 1 : 2;
    m.gu = plan_phase((int)hidden, m.max_slots * (int)(inter / 128), m.nproj, m.MRB);
    m.dn = plan_phase((int)inter, m.max_slots * (int)(hidden / 128), 1, m.MRB);
    size_t off = 0;
    m.off_route = off;
    off += align256(sizeof(int) * (1 + 3 * (size_t)m.max_slots + 3 * (size_t)m.n_routes));
    m.off_wsgu = off;
    off += align256(4 * (size_t)m.nproj * m.gu.S * m.n_routes * inter);
    m.off_wsd = off;
    off += align256(4 * (size_t)m.dn.S * m.n_routes * hidden);
    m.total = off;
    return m;
}

struct LinPlan {
    int MRB;
    PhasePlan ph;
    size_t total;
};

inline LinPlan plan_linear(int64_t m, int64_t in_f, int64_t out_f) {
    LinPlan lp;
    lp.MRB = (int)(m < kMaxMRB ? m : kMaxMRB);
    lp.ph = plan_phase((int)in_f, (int)(out_f / 128), 1, lp.MRB);
    lp.total = lp.ph.S > 1 ? align256(4 * (size_t)lp.ph.S * m * out_f) : 0;
    return lp;
}

template <int CB, int MODE>
hipError_t set_lds_cap() {
    // well below the 160 KB per workgroup, leaving room for static LDS
    hipError_t e = hipFuncSetAttribute((const void*)gemv_kernel<CB, MODE>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
    if (e != hipSuccess) (void)hipGetLastError();  // do not leave a sticky error behind
    return e;
}

hipError_t init_lds_caps() {
    static const hipError_t st = [] {
        hipError_t e = hipSuccess;
        hipError_t r[] = {set_lds_cap<0, 0>(), set_lds_cap<0, 1>(), set_lds_cap<0, 2>(),
                          set_lds_cap<1, 0>(), set_lds_cap<1, 1>(), set_lds_cap<1, 2>(),
                          set_lds_cap<2, 0>(), set_lds_cap<2, 1>(), set_lds_cap<2, 2>()};
        for (hipError_t x : r)
            if (x != hipSuccess) e = x;
        return e;
    }();
    return st;
}

template <int MODE>
void launch_gemv(int cb, int grid, size_t lds, hipStream_t st, const GemvParams& p) {
    switch (cb) {
        case 0: gemv_kernel<0, MODE><<<grid, kThreads, lds, st>>>(p); break;
        case 1: gemv_kernel<1, MODE><<<grid, kThreads, lds, st>>>(p); break;
        default: gemv_kernel<2, MODE><<<grid, kThreads, lds, st>>>(p); break;
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
EXL3_API int64_t exl3_gemm_workspace_size(int64_t m, int64_t in_features, int64_t out_features) {
    if (m < 1 || in_features < 128 || out_features < 128) return 0;
    return (int64_t)plan_linear(m, in_features, out_features).total;
}

EXL3_API int exl3_gemm(const void* x, int x_dtype, int64_t m, const int16_t* trellis,
                       int64_t tiles_k, int64_t tiles_n, int64_t K, int codebook,
                       const uint16_t* suh, const uint16_t* svh, void* out, int out_dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
    EXL3_CHECK(K == 2 || K == 3 || K == 4, "exl3_gemm supports K in {2, 3, 4}");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(x_dtype >= 0 && x_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
               "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(m >= 1 && m <= 0x7FFFFFFF, "exl3_gemm needs 1 <= m < 2^31");
    EXL3_CHECK(tiles_k > 0 && tiles_n > 0 && (tiles_k * 16) % 128 == 0 && (tiles_n * 16) % 128 == 0,
               "trellis dimensions must reconstruct whole 128-element Hadamard blocks");
    EXL3_CHECK(tiles_k * 16 <= (1 << 24) && tiles_n * 16 <= (1 << 24), "feature dimensions too large");
    EXL3_CHECK(x && trellis && suh && svh && out, "null pointer argument");
    const int64_t in_f = tiles_k * 16, out_f = tiles_n * 16;
    const LinPlan lp = plan_linear(m, in_f, out_f);
    EXL3_CHECK(workspace_bytes >= (int64_t)lp.total && (lp.total == 0 || workspace),
               "workspace too small: need %zu bytes", lp.total);
    EXL3_HIP(init_lds_caps());
    GemvParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride = in_f;
    p.w_trellis = trellis;
    p.w_suh = suh;
    p.w_svh = svh;
    p.kuni[0] = (int)K;
    p.in_features = (int)in_f;
    p.out_features = (int)out_f;
    p.m_rows = (int)m;
    p.out = out;
    p.out_dtype = out_dtype;
    p.out_stride = out_f;
    p.S = lp.ph.S;
    p.R_hb = lp.ph.R_hb;
    p.C_hb = lp.ph.C_hb;
    p.MRB = lp.MRB;
    p.n_rows_ws = (int)m;
    p.ws = reinterpret_cast<float*>(workspace);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    launch_gemv<kModeLinear>(codebook, (int)(out_f / 128) * lp.ph.S, lp.ph.lds, st, p);
    EXL3_LAUNCHED();
    if (lp.ph.S > 1) {
        const int items = (int)(m * (out_f / 128));
        linear_finish_kernel<<<(items + 3) / 4, 256, 0, st>>>(p.ws, lp.ph.S, (int)m, (int)out_f, svh,
                                                              out, out_dtype);
        EXL3_LAUNCHED();
    }
    return kOk;
}

EXL3_API int64_t exl3_moe_workspace_size(int64_t T, int64_t topk, int64_t n_local, int64_t hidden,
                                         int64_t inter, int gateless) {
    if (T < 1 || topk < 1 || n_local < 1 || hidden < 128 || inter < 128) return 0;
    return (int64_t)plan_moe(T, topk, n_local, hidden, inter, gateless).total;
}

EXL3_API int exl3_moe_forward(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
                              const int64_t* gate_trellis, const int64_t* gate_suh,
                              const int64_t* gate_svh, const int64_t* up_trellis,
                              const int64_t* up_suh, const int64_t* up_svh,
                              const int64_t* down_trellis, const int64_t* down_suh,
                              const int64_t* down_svh, int64_t n_local, const int8_t* k_gate,
                              const int8_t* k_up, const int8_t* k_down, int64_t K_gate,
                              int64_t K_up, int64_t K_down, int codebook, int gateless, int act,
                              float swiglu_limit, const void* ids, int ids_dtype,
                              const void* weights, int w_dtype, int64_t topk,
                              const int32_t* n_valid, void* out, int out_dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
    EXL3_CHECK(T >= 1 && topk >= 1 && T * topk <= kMaxRoutes,
               "fused MoE decode supports 1 <= T*topk <= %d routes", kMaxRoutes);
    EXL3_CHECK(hidden > 0 && hidden % 128 == 0,
               "fused MoE hidden width must be a positive multiple of 128");
    EXL3_CHECK(inter > 0 && inter % 128 == 0,
               "fused MoE local intermediate width must be a positive multiple of 128");
    EXL3_CHECK(hidden <= (1 << 20) && inter <= (1 << 20), "fused MoE dimensions too large");
    EXL3_CHECK(n_local >= 1 && n_local < (1 << 18), "fused MoE n_local must be in [1, 2^18)");
    EXL3_CHECK(std::isfinite(swiglu_limit) && swiglu_limit >= 0.0f,
               "fused MoE SwiGLU limit must be finite and nonnegative (0 disables clipping)");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(act == kActSilu || act == kActRelu2 || act == kActSwigluOai,
               "fused MoE activation must be 0 (silu), 2 (relu2, gateless) or 3 (swiglu-oai)");
    EXL3_CHECK(!gateless || act == kActRelu2, "a gateless layer uses the relu2 activation");
    EXL3_CHECK(x_dtype >= 0 && x_dtype <= 2 && w_dtype >= 0 && w_dtype <= 2 && out_dtype >= 0 &&
                   out_dtype <= 2 && (ids_dtype == 0 || ids_dtype == 1),
               "dtype ids: values 0 fp16, 1 bf16, 2 fp32; ids 0 int32, 1 int64");
    const int64_t Ks[3] = {K_gate, K_up, K_down};
    const int8_t* kt[3] = {k_gate, k_up, k_down};
    for (int i = 0; i < 3; ++i)
        EXL3_CHECK(kt[i] || (Ks[i] >= 2 && Ks[i] <= 4),
                   "fused MoE K must be 2, 3 or 4 (or come from a per-expert K table)");
    EXL3_CHECK(x && ids && weights && out && up_trellis && up_suh && up_svh && down_trellis &&
                   down_suh && down_svh && (gateless || (gate_trellis && gate_suh && gate_svh)),
               "fused MoE: null pointer argument");
    const MoePlan mp = plan_moe(T, topk, n_local, hidden, inter, gateless);
    EXL3_CHECK(workspace && workspace_bytes >= (int64_t)mp.total,
               "fused MoE workspace too small: need %zu bytes", mp.total);
    EXL3_HIP(init_lds_caps());
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);

    RouteOut ro;
    int* rbase = reinterpret_cast<int*>(ws + mp.off_route);
    ro.n_active = rbase;
    ro.slot_expert = rbase + 1;
    ro.slot_start = ro.slot_expert + mp.max_slots;
    ro.slot_rows = ro.slot_start + mp.max_slots;
    ro.row_token = ro.slot_rows + mp.max_slots;
    ro.row_expert = ro.row_token + mp.n_routes;
    ro.route_pos = ro.row_expert + mp.n_routes;
    route_kernel<<<1, kRouteThreads, 0, st>>>(ids, ids_dtype, mp.n_routes, (int)topk, (int)n_local,
                                              n_valid, ro);
    EXL3_LAUNCHED();

    GemvParams p = {};
    const int64_t* tabs[9] = {gateless ? up_trellis : gate_trellis, gateless ? up_suh : gate_suh,
                              gateless ? up_svh : gate_svh, up_trellis, up_suh, up_svh,
                              down_trellis, down_suh, down_svh};
    for (int i = 0; i < 9; ++i) p.tab[i] = tabs[i];
    for (int i = 0; i < 3; ++i) {
        p.ktab[i] = kt[i];
        p.kuni[i] = (int)Ks[i];
    }
    p.gateless = gateless;
    p.n_active = ro.n_active;
    p.slot_expert = ro.slot_expert;
    p.slot_start = ro.slot_start;
    p.slot_rows = ro.slot_rows;
    p.row_token = ro.row_token;
    p.max_slots = mp.max_slots;
    p.MRB = mp.MRB;
    p.n_rows_ws = mp.n_routes;
    p.limit = swiglu_limit;
    p.act = act;
    float* ws_gu = reinterpret_cast<float*>(ws + mp.off_wsgu);
    float* ws_d = reinterpret_cast<float*>(ws + mp.off_wsd);

    // gate/up: raw partial sums [nproj][S_gu][routes][inter]
    GemvParams pg = p;
    pg.x = x;
    pg.x_dtype = x_dtype;
    pg.x_stride = hidden;
    pg.in_features = (int)hidden;
    pg.out_features = (int)inter;
    pg.S = mp.gu.S;
    pg.R_hb = mp.gu.R_hb;
    pg.C_hb = mp.gu.C_hb;
    pg.ws = ws_gu;
    launch_gemv<kModeGateUp>(codebook, mp.max_slots * (int)(inter / 128) * mp.gu.S, mp.gu.lds, st, pg);
    EXL3_LAUNCHED();

    // down: finishes gate/up while staging, raw partials [S_d][routes][hidden]
    GemvParams pd = p;
    pd.src_ws = ws_gu;
    pd.src_S = mp.gu.S;
    pd.in_features = (int)inter;
    pd.out_features = (int)hidden;
    pd.S = mp.dn.S;
    pd.R_hb = mp.dn.R_hb;
    pd.C_hb = mp.dn.C_hb;
    pd.ws = ws_d;
    launch_gemv<kModeDown>(codebook, mp.max_slots * (int)(hidden / 128) * mp.dn.S, mp.dn.lds, st, pd);
    EXL3_LAUNCHED();

    const int items = (int)(T * (hidden / 128));
    combine_kernel<<<(items + 3) / 4, 256, 0, st>>>(ws_d, mp.dn.S, mp.n_routes, (int)hidden,
                                                    ro.route_pos, ro.row_expert, down_svh, weights,
                                                    w_dtype, (int)T, (int)topk, out, out_dtype);
    EXL3_LAUNCHED();
    return kOk;
}
