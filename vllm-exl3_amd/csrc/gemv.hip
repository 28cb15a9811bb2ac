// Decode-path kernels: streaming EXL3 GEMV (plain linear and the two MoE
// projections), device-side routing and the deterministic top-k combine.
//
// Replaces, on one MI355X:
//   * exl3_gemv / exl3_gemm (csrc/exl3_gemv.cu:23-63, csrc/exl3_gemm.cu:8-31,
//     bindings csrc/bindings.cpp:110-147);
//   * the fused decode MoE p2b_fused_moe{,_mk,_padded}
//     (csrc/p2b_moe.cu:643-1071, 1295-2487) as six ordinary launches, no
//     grid barriers, no device-scope fences, no host synchronisation:
//       route    stable sort of the routes by expert (one workgroup), with
//                the slots' row groups of MRB rows;
//       rotate   each kept route's gate/up input rows, rotated once (suh,
//                128-Hadamard, fp16) into the GEMV's image order;
//       gate/up  raw split-K partial sums of both projections;
//       act      finishes gate/up per route (sum of splits, output rotation
//                x svh, fp16 rounding, activation, down suh, down input
//                rotation);
//       down     raw split-K partial sums;
//       combine  per (token, column block): finish each route's down result
//                (rotation x svh) and sum w * d in slot order
//                (csrc/p2b_moe.cu:1976-2008): deterministic, no atomics.
// The GEMV phases run one of two kernels chosen by the planner: one unit per
// workgroup (gemv_wg_kernel) when the units fill at most a couple of rounds
// of resident workgroups, else the persistent gemv_kernel, which streams a
// balanced range of units per workgroup with its trellis pipeline kept full
// across them.
#include "gemv_core.h"
#include "linear.h"
#include "profile.h"
#include "route_impl.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace exl3 {
namespace {

constexpr int kMaxMRB = 16;       // activation rows per row group (one MFMA row block)
constexpr int kMoeMRB = 8;        // row-group size of the MoE phases
constexpr int kMaxRoutes = 8192;  // routes sortable by the bitonic router
constexpr int64_t kMaxRoutesMultisplit = 1 << 20;  // routes of the multisplit router
constexpr int kRouteBits = 13;    // log2(kMaxRoutes)

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

typedef __attribute__((address_space(1))) const v4u* gv4p;

// Stream of one chunk's tile rows for one wave.  base: the wave's first row
// (wave-uniform, so loads go through a scalar buffer resource and the row
// advance is the scalar offset: no per-lane 64-bit pointers and no VALU
// address arithmetic per row); step: bytes between the wave's consecutive
// rows (4 tile rows); n: the wave's rows.  The lane's 16 bytes of a row are
// LaneGeo::voff.
struct Stream {
    const uint8_t* base;
    uint32_t step;
    int n;
};

// One 16-byte piece of a tile row: base + voff + soff, streamed (nt).
__device__ __forceinline__ v4u load_row(const uint8_t* base, uint32_t voff, uint32_t soff) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7FFFFFFF, 0x00020000);
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 2));
}

// Consume one chunk of bit width K: per row, stage the 256*K bytes in LDS
// (layout LK, see LaneGeo), refill the pipeline slot, read the sixteen words
// this lane needs, decode and issue eight MFMAs.  buf[d] holds row d (mod
// kDepth) on entry.  Refills of all but the last block of kDepth rows load
// this chunk's later rows; the last block refills slot d with row d of the
// next chunk (ns, lane offset ns_voff; the current chunk's first row again
// when there is none), so the next chunk - another column block, split or
// slot - starts with its pipeline already full.
template <int CB, int LK>
__device__ __forceinline__ void consume_chunk(v4u (&buf)[kDepth], const Stream& cs, const Stream& ns,
                                              bool has_next, int ns_K, const LaneGeo& geo,
                                              uint32_t ns_voff, int K_rt, int lane, int wave,
                                              uint32_t* stage, const uint16_t* A, int MRB, int arow,
                                              float4_t (&acc)[8]) {
    const int K = LK ? LK : K_rt;
    constexpr int ts = stage_tile_stride<LK>();
    const int n = cs.n;
    const uint32_t sh1 = (uint32_t)K, sh2 = 2u * K, sh3 = 3u * K;
    const int g = lane >> 4;
    uint8_t* st = reinterpret_cast<uint8_t*>(stage);
    const uint32_t* arow_p = reinterpret_cast<const uint32_t*>(A + (size_t)arow * 16 + 4 * g) +
                             (size_t)wave * MRB * 8;
    const int a_step = kWaves * MRB * 8;  // uint32 words between this wave's consecutive rows
    auto put_g = [&](int d, const LaneGeo& gg) { *reinterpret_cast<v4u*>(st + gg.wr) = buf[d]; };
    auto put = [&](int d) { put_g(d, geo); };
    auto compute_g = [&](int i, const LaneGeo& gg) {
        const uint32_t* ap = arow_p + (size_t)i * a_step;
        // all sixteen words of the row first: one LDS latency per row
        uint32_t wh[8], wl[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            wh[t] = *reinterpret_cast<const uint32_t*>(st + t * ts + gg.off_hi);
            wl[t] = *reinterpret_cast<const uint32_t*>(st + t * ts + gg.off_lo);
        }
        const half8_t a = dup4(ap[0], ap[1]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t b[4];
            decode4<CB>(wh[t], wl[t], gg.shift, sh3, sh2, sh1, b);
            acc[t] = mfma16x16x32(a, b, acc[t]);
        }
    };
    auto compute = [&](int i) { compute_g(i, geo); };
    if (n % kDepth == 0 && ns.n >= kDepth) {
        // whole blocks, branch-free; a block's refills target the rows of the
        // next block, which for the last block (peeled) is the next chunk's
        // first, at the next chunk's bit width.
        auto block = [&](int i, const uint8_t* bb, uint32_t bs, int kk) {
            // The lane offset is rebuilt from the lane id in every block (a
            // few VALU): kept live across the loop it may be spilled, and the
            // reload - a memory load like the trellis rows - would make every
            // block wait for all rows in flight.
            // (mixed-K launches rebuild all of the lane's geometry the same way)
            uint32_t lid;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lid));
            const uint32_t voff = (int)lid < 16 * kk ? lid * 16 : 0;
            const LaneGeo gg = LK ? geo : lane_geo_padded(K, lid);
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                put_g(d, gg);
                buf[d] = load_row(bb, voff, (uint32_t)d * bs);
                compute_g(i + d, gg);
                // keep each row's refill in its row: refills sunk past later
                // rows leave those rows waiting for almost every load in flight
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        int i = 0;
        for (; i + kDepth < n; i += kDepth) block(i, cs.base + (size_t)(i + kDepth) * cs.step, cs.step, K);
        block(i, ns.base, ns.step, LK ? LK : ns_K);
        return;
    }
    // short or ragged chunks (an input width that is not a multiple of 512):
    // refills clamp to the chunk's last row, and the last block's rows past n
    // only refill
    const int last = (n - 1) & ~(kDepth - 1);  // first row of the last block
    int i = 0;
    for (; i < last; i += kDepth) {
        const uint8_t* bb = cs.base + (size_t)i * cs.step;
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            put(d);
            buf[d] = load_row(bb, geo.voff, (uint32_t)(min(i + d + kDepth, n - 1) - i) * cs.step);
            compute(i + d);
        }
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        if (i + d < n) {
            put(d);
            if (has_next) buf[d] = load_row(ns.base, ns_voff, (uint32_t)min(d, ns.n - 1) * ns.step);
            compute(i + d);
        } else if (has_next) {
            buf[d] = load_row(ns.base, ns_voff, (uint32_t)min(d, ns.n - 1) * ns.step);
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

// Sum of the S split partials at columns c0 and c0 + 64 of one row, in split
// order (deterministic), with the loads of up to 8 splits issued together.
__device__ __forceinline__ void sum_splits(const float* __restrict__ base, int64_t split_stride,
                                           int S, int c0, float& v0, float& v1) {
    int ss = 0;
    for (; ss + 8 <= S; ss += 8) {
        float a[8], b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            a[i] = base[(ss + i) * split_stride + c0];
            b[i] = base[(ss + i) * split_stride + c0 + 64];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v0 += a[i];
            v1 += b[i];
        }
    }
    for (; ss < S; ++ss) {
        v0 += base[ss * split_stride + c0];
        v1 += base[ss * split_stride + c0 + 64];
    }
}

// Output side of one 128-column block for one row: v[h] holds the summed,
// not yet rotated result at column lane + 64 h; returns (H v / sqrt(128)) * svh.
__device__ __forceinline__ void finish_block(float& v0, float& v1, const uint16_t* svh, int c0,
                                             int lane) {
    had128(v0, v1, lane);
    const float hs = kHadNorm * had_sign64(lane);  // with had128's lane sign
    v0 = v0 * hs * (float)bits_to_half(svh[c0]);
    v1 = v1 * hs * (float)bits_to_half(svh[c0 + 64]);
}

// The activation of one route row and 128-block hb of the intermediate
// dimension from the summed raw gate (q 0) and up (q 1) results v[q][h]
// (column hb*128 + lane + 64 h): rotation x svh, fp16, clamp + activation,
// fp16, x down suh, rotation for the down projection.  g and u leave the
// GEMV as fp16 and the activation is stored as fp16
// (src/vllm_exl3/exl3.py:2403-2410, csrc/p2b_moe.cu:755-768).
__device__ __forceinline__ void act_finish(float (&v)[2][2], const Proj* gu, int nproj,
                                           const uint16_t* down_suh, int hb, int lane, int act,
                                           float limit, float& a0, float& a1) {
    const int c0 = hb * 128 + lane;
#pragma unroll
    for (int q = 0; q < 2; ++q)
        if (q < nproj) finish_block(v[q][0], v[q][1], gu[q].svh, c0, lane);
    float a[2];
    for (int h = 0; h < 2; ++h) {
        const float u = (float)f32_to_f16_rne(nproj == 2 ? v[1][h] : v[0][h]);
        const float g = nproj == 2 ? (float)f32_to_f16_rne(v[0][h]) : 0.0f;
        a[h] = (float)f32_to_f16_rne(activate(g, u, act, limit));
    }
    a[0] *= (float)bits_to_half(down_suh[c0]);
    a[1] *= (float)bits_to_half(down_suh[c0 + 64]);
    had128(a[0], a[1], lane);
    const float hs = kHadNorm * had_sign64(lane);  // with had128's lane sign
    a0 = a[0] * hs;
    a1 = a[1] * hs;
}

// Finish gate/up for one route row and 128-block hb from the split partials.
__device__ __forceinline__ void gateup_finish(const GemvParams& p, const Proj* gu, int nproj,
                                              const uint16_t* down_suh, int64_t row, int hb,
                                              int lane, float& a0, float& a1) {
    const int inter = p.in_features;
    const int c0 = hb * 128 + lane;
    float v[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        if (q < nproj) {
            sum_splits(p.src_ws + ((int64_t)q * p.src_S * p.n_rows_ws + row) * inter,
                       (int64_t)p.n_rows_ws * inter, p.src_S, c0, v[q][0], v[q][1]);
        }
    }
    act_finish(v, gu, nproj, down_suh, hb, lane, p.act, p.limit, a0, a1);
}


// Position of input c of a row in the GEMV image: each 16 consecutive inputs
// are stored in the MFMA k order of the GEMV (input c at pi_inv(c & 15)), so
// a workgroup stages a row's tile rows with plain 16-byte copies.
__device__ __forceinline__ int64_t image_pos(int64_t c) { return (c & ~15ll) + pi_inv((int)(c & 15)); }

// Rotated activation rows for the decode GEMV, in image order:
// img_q[row] = fp16(had128(fp16(x[token]) * suh_q) / sqrt(128)).  Linear:
// row = token = the unit's row.  MoE: the unit's row is route r, the image row
// is its sorted position route_pos[r] (dropped routes are skipped), token
// r / topk, suh of the route's expert per projection.  One wave per (row,
// 128-input block); computed once per row instead of once per workgroup.
struct RotateArgs {
    const void* x;
    int x_dtype;
    int64_t x_stride;
    int in_f, n_rows;
    const int* route_pos;   // null: linear
    int topk;
    const int* row_expert;
    const uint16_t* suh;         // linear
    const int64_t* suh_tab[2];   // MoE: per-expert suh of the two projections
    int nproj;
    uint16_t* img[2];
    // batched: row r = (slot r / batch_m, input row r % batch_m), suh of the
    // slot's expert from suh_tab[0]; rows of ids outside the table are skipped
    const int* expert_list;
    int batch_m, n_ptr;
};

// BPW consecutive 128-input blocks of one row per wave: the row's metadata
// loads (route position, expert, suh pointer) are paid once and the blocks'
// activation and suh loads issue together.
template <int BPW>
__global__ __launch_bounds__(256) void rotate_rows_kernel(RotateArgs a) {
    const int lane = threadIdx.x & 63;
    const int nb = a.in_f >> 7, nbw = (nb + BPW - 1) / BPW;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (int64_t)a.n_rows * nbw) return;
    const int r = (int)(unit / nbw), hb0 = (int)(unit % nbw) * BPW;
    int64_t row = r, tok = r;
    int e = 0;
    if (a.route_pos) {
        const int pos = a.route_pos[r];
        if (pos < 0) return;  // wave-uniform
        row = pos;
        tok = r / a.topk;
        e = a.row_expert[pos];
    } else if (a.expert_list) {
        e = a.expert_list[r / a.batch_m];
        if (e < 0 || e >= a.n_ptr) return;  // wave-uniform
        tok = r % a.batch_m;
    }
    float x0[BPW], x1[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int64_t fb = (int64_t)min(hb0 + i, nb - 1) * 128;  // a block past the row is not stored
        x0[i] = load_act(a.x, a.x_dtype, tok * a.x_stride + fb + lane);
        x1[i] = load_act(a.x, a.x_dtype, tok * a.x_stride + fb + lane + 64);
    }
    const float hs = kHadNorm * had_sign64(lane);  // with had128's lane sign
    for (int q = 0; q < a.nproj; ++q) {
        const uint16_t* su = (a.route_pos || a.expert_list)
                                 ? reinterpret_cast<const uint16_t*>(a.suh_tab[q][e])
                                 : a.suh;
        float v0[BPW], v1[BPW];
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            const int64_t fb = (int64_t)min(hb0 + i, nb - 1) * 128;
            v0[i] = x0[i] * (float)bits_to_half(su[fb + lane]);
            v1[i] = x1[i] * (float)bits_to_half(su[fb + lane + 64]);
        }
        uint16_t* dst = a.img[q] + row * a.in_f;
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            if (hb0 + i >= nb) break;  // wave-uniform
            const int64_t fb = (int64_t)(hb0 + i) * 128;
            had128(v0[i], v1[i], lane);
            dst[image_pos(fb + lane)] = half_to_bits(f32_to_f16_rne(v0[i] * hs));
            dst[image_pos(fb + lane + 64)] = half_to_bits(f32_to_f16_rne(v1[i] * hs));
        }
    }
}

// Rotation launch: one wave per 128-input block while the grid fits about
// one round of resident waves (32 per CU), else one wave per four blocks of
// a row (the grid then still fills the chip; the per-wave load chain of the
// row's metadata dominates such launches: C3, 27,648 one-block waves).
inline void launch_rotate(const RotateArgs& ra, hipStream_t st) {
    const int nb = ra.in_f >> 7;
    const int64_t one = (int64_t)ra.n_rows * nb;
    if (nb >= 4 && one > 32 * (int64_t)num_cus()) {
        const int64_t units = (int64_t)ra.n_rows * ((nb + 3) / 4);
        rotate_rows_kernel<4><<<(unsigned)((units + 3) / 4), 256, 0, st>>>(ra);
    } else {
        rotate_rows_kernel<1><<<(unsigned)((one + 3) / 4), 256, 0, st>>>(ra);
    }
}

// Down-projection input rows, in image order: for every sorted row (kept
// route), finish gate/up (sum of the split partials, output rotation x svh,
// fp16 rounding, activation, down suh, input rotation).  One wave per
// (sorted row, 128-block of the intermediate dimension); p carries the
// gate/up partials and tables.
__global__ __launch_bounds__(256) void act_rows_kernel(GemvParams p, int n_rows, const int* n_sorted,
                                                       const int* row_expert, uint16_t* img) {
    const int lane = threadIdx.x & 63;
    const int inter = p.in_features;
    const int nb = inter >> 7;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (int64_t)n_rows * nb) return;
    // sorted rows directly (rows past the kept routes exit): the partials
    // and the row's expert are the first loads, no route lookup before them
    const int pos = (int)(unit / nb), hb = (int)(unit % nb);
    if (pos >= *n_sorted) return;  // wave-uniform
    const int e = row_expert[pos];
    Proj gu[2];
    gu[0].svh = reinterpret_cast<const uint16_t*>(p.tab[p.gateless ? 5 : 2][e]);
    gu[1].svh = reinterpret_cast<const uint16_t*>(p.tab[5][e]);
    const uint16_t* down_suh = reinterpret_cast<const uint16_t*>(p.tab[7][e]);
    float a0, a1;
    gateup_finish(p, gu, p.gateless ? 1 : 2, down_suh, pos, hb, lane, a0, a1);
    uint16_t* dst = img + (int64_t)pos * inter;
    dst[image_pos((int64_t)hb * 128 + lane)] = half_to_bits(f32_to_f16_rne(a0));
    dst[image_pos((int64_t)hb * 128 + lane + 64)] = half_to_bits(f32_to_f16_rne(a1));
}

// Copy the rotated activations of rows [row0, row0 + nr) for tile rows
// [kt0, kt0 + nkt) from their image (row-major fp16 rows, MFMA k order inside
// each 16 inputs) into the LDS operand layout A[kt][MRB][16].  Every load of
// a batch is issued before its stores, so the copy costs about one L2 round
// trip.
__device__ __forceinline__ void stage_rows(const uint16_t* img, int64_t x_stride, int64_t row0, int nr,
                                           int kt0, int nkt, int MRB, uint16_t* A, int tid) {
    typedef __attribute__((address_space(1))) const v4u* gv4c;
    const int pieces = nr * nkt * 2;  // 16-byte pieces, row-major
    constexpr int kBatch = 4;  // loads in flight per thread: the restage runs beside the trellis pipeline
    for (int b0 = 0; b0 < pieces; b0 += kThreads * kBatch) {
        v4u v[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int pc = b0 + b * kThreads + tid;
            if (pc < pieces) {
                const int h = pc & 1, kt = (pc >> 1) % nkt, r = (pc >> 1) / nkt;
                v[b] = *(gv4c)(img + (row0 + r) * x_stride + (int64_t)(kt0 + kt) * 16 + 8 * h);
            }
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int pc = b0 + b * kThreads + tid;
            if (pc < pieces) {
                const int h = pc & 1, kt = (pc >> 1) % nkt, r = (pc >> 1) / nkt;
                *reinterpret_cast<v4u*>(A + (kt * MRB + r) * 16 + 8 * h) = v[b];
            }
        }
    }
}

// A workgroup's position in its sequence of chunks.  A unit is one (row
// group, projection, split, 128-column block) - every unit streams the same
// bytes, so equal unit ranges are equal work - numbered with the column
// block fastest, then the split, the projection and the group, so
// consecutive units of one group, projection and split share the staged
// activations.  A row group is up to MRB rows of one slot; a chunk is one
// staged range (up to C_hb 128-row blocks) of the split's input rows.
struct Cursor {
    int64_t u;  // unit; -1: past the workgroup's range
    int grp, q, s, j, c;
    // of (grp, q): slot, first row of the group within the slot, rows of the
    // slot, its first activation / output row, bit width, trellis
    int slot, rg, rows, row_base, K;
    const uint8_t* trellis;
};

// Tables of the cursor's (group, projection); false when it has nothing to
// stream (a batched expert id outside the table, a per-expert K outside
// {2, 3, 4}).  Table selects are written out so that the kernel-argument
// tables are never indexed with a run-time value.
template <int MODE, int LK>
__device__ __forceinline__ bool load_unit(const GemvParams& p, Cursor& c, int n_groups) {
    if constexpr (MODE == kModeLinear) {
        c.slot = 0;
        c.rg = c.grp * p.MRB;
        c.rows = p.m_rows;
        c.row_base = 0;
        c.trellis = reinterpret_cast<const uint8_t*>(p.w_trellis);
        c.K = LK ? LK : p.kuni[0];
        return true;
    } else if constexpr (MODE == kModeBatched) {
        const int gps = (p.batch_m + p.MRB - 1) / p.MRB;  // groups per slot
        c.slot = c.grp / gps;
        c.rg = (c.grp - c.slot * gps) * p.MRB;
        c.rows = p.batch_m;
        c.row_base = c.slot * p.batch_m;
        c.K = LK ? LK : p.kuni[0];
        const int e = p.expert_list[c.slot];
        if (e < 0 || e >= p.n_ptr) return false;
        c.trellis = reinterpret_cast<const uint8_t*>(p.tab[0][e]);
        return true;
    } else {
        const int e = p.group_expert[c.grp];
        c.slot = p.group_slot[c.grp];
        c.rg = p.group_row0[c.grp];
        if (c.grp >= n_groups) return false;
        const bool up = MODE == kModeGateUp && (p.gateless || c.q);
        const int64_t* tt = MODE == kModeDown ? p.tab[6] : up ? p.tab[3] : p.tab[0];
        c.trellis = reinterpret_cast<const uint8_t*>(tt[e]);
        c.rows = p.slot_rows[c.slot];
        c.row_base = p.slot_start[c.slot];
        if constexpr (LK != 0) {
            c.K = LK;  // the host picks LK only for a uniform K
            return c.rows > 0;
        } else {
            const int8_t* kt = MODE == kModeDown ? p.ktab[2] : up ? p.ktab[1] : p.ktab[0];
            const int ku = MODE == kModeDown ? p.kuni[2] : up ? p.kuni[1] : p.kuni[0];
            // the byte table is read with a vector load: make its value
            // wave-uniform, or every address derived from it (the stream's
            // buffer resource) would be treated as divergent
            c.K = __builtin_amdgcn_readfirstlane(kt ? (int)kt[e] : ku);
            // a per-expert K outside {2, 3, 4} streams nothing here (never
            // misaddresses): gemv_anyk_kernel computes that unit (K 5, 6) or
            // writes its partials as zeros (any other K)
            return c.rows > 0 && c.K >= 2 && c.K <= 4;
        }
    }
}

// Step c to the next unit with something to stream; c.u = -1 past u1.  ok:
// whether c's current (group, projection) has anything to stream.  Tables are
// reloaded only when the group or projection changes.
// (Units below u1 lie in groups below the group count: no check is needed.)
template <int MODE, int LK>
__device__ __forceinline__ void next_unit(const GemvParams& p, int64_t u1, int nq, int n_j, Cursor& c,
                                          bool ok) {
    c.c = 0;
    do {
        if (++c.u >= u1) {
            c.u = -1;
            return;
        }
        if (++c.j == n_j) {
            c.j = 0;
            if (++c.s == p.S) {
                c.s = 0;
                if (++c.q == nq) {
                    c.q = 0;
                    ++c.grp;
                }
                ok = load_unit<MODE, LK>(p, c, 0x7FFFFFFF);
            }
        }
    } while (!ok);
}

// Place c at unit u (the first of the workgroup's range) or the next one with
// something to stream.
template <int MODE, int LK>
__device__ __forceinline__ void seek_unit(const GemvParams& p, int64_t u, int64_t u1, int nq, int n_j,
                                          int n_groups, Cursor& c) {
    if (u >= u1) {
        c.u = -1;
        return;
    }
    const int per_group = nq * p.S * n_j;
    c.grp = (int)(u / per_group);
    int rem = (int)(u - (int64_t)c.grp * per_group);
    c.j = rem % n_j;
    rem /= n_j;
    c.s = rem % p.S;
    c.q = rem / p.S;
    c.u = u;
    c.c = 0;
    if (!load_unit<MODE, LK>(p, c, n_groups)) next_unit<MODE, LK>(p, u1, nq, n_j, c, false);
}

// Step c to the next chunk of the workgroup's range.
template <int MODE, int LK>
__device__ __forceinline__ void advance(const GemvParams& p, int64_t u1, int nq, int n_j, int nc,
                                        Cursor& c) {
    if (++c.c < nc) return;
    next_unit<MODE, LK>(p, u1, nq, n_j, c, true);
}

// The wave's trellis stream over chunk c (see Stream).
__device__ __forceinline__ Stream stream_of(const GemvParams& p, const Cursor& c, int wave) {
    const int tiles_n = p.out_features >> 4;
    const size_t tile_bytes = 32u * (unsigned)c.K;
    const size_t row_bytes = (size_t)tiles_n * tile_bytes;
    const int hb0 = c.s * p.R_hb + c.c * p.C_hb;
    const int nb = min(p.C_hb, p.R_hb - c.c * p.C_hb);
    Stream st;
    st.base = c.trellis + ((size_t)hb0 * 8 * tiles_n + (size_t)c.j * 8) * tile_bytes + (size_t)wave * row_bytes;
    st.step = (uint32_t)(row_bytes * kWaves);
    st.n = nb * 2;  // nb * 8 tile rows shared by the four waves
    return st;
}

template <int MODE>
__device__ __forceinline__ void stage_chunk(const GemvParams& p, const Cursor& c, uint16_t* A, int tid) {
    const int hb0 = c.s * p.R_hb + c.c * p.C_hb;
    const int nb = min(p.C_hb, p.R_hb - c.c * p.C_hb);
    const uint16_t* img = reinterpret_cast<const uint16_t*>((MODE == kModeGateUp && c.q) ? p.x2 : p.x);
    stage_rows(img, p.x_stride, (int64_t)c.row_base + c.rg, min(p.MRB, c.rows - c.rg), hb0 * 8, nb * 8,
               p.MRB, A, tid);
}

// Sum of the four waves' partials at (row, column), in wave order.
__device__ __forceinline__ float red_sum(const float* red, int MRB, int row, int c) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += red[(w * MRB + row) * 128 + c];
    return v;
}

// Persistent decode GEMV.  The grid is at most one wave of resident
// workgroups; workgroup b takes units [b*U/G, (b+1)*U/G) of the U units of
// the launch (U from the device-side slot count for the MoE phases) and
// streams their chunks back to back: the trellis pipeline runs across chunk
// and unit boundaries, activations are restaged only when the slot,
// projection, split, row group or input range changes, and each finished
// (unit, row group) is reduced over the waves in LDS and written as a raw
// split partial (or, for a single split of a plain or batched linear,
// finished in place).
template <int CB, int MODE, int LK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemv_kernel(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar stream bases
    const int n_j = p.out_features >> 7;
    const int nq = (MODE == kModeGateUp && !p.gateless) ? 2 : 1;
    const int nc = (p.R_hb + p.C_hb - 1) / p.C_hb;
    const int MRB = p.MRB;
    int n_groups;
    if constexpr (MODE == kModeLinear || MODE == kModeBatched) {
        n_groups = p.max_groups;  // ceil(m / MRB) (per listed expert)
    } else {
        n_groups = min(*p.n_groups, p.max_groups);
    }
    const int64_t U = (int64_t)n_groups * nq * p.S * n_j;
    const int64_t u0 = (int64_t)blockIdx.x * U / gridDim.x;
    const int64_t u1 = (int64_t)(blockIdx.x + 1) * U / gridDim.x;

    // LDS: [stage 4 x 1 KB][A: C_hb x 8 x MRB x 16 fp16][red: 4 waves x MRB x 128 fp32]
    uint32_t* stage = reinterpret_cast<uint32_t*>(lds) + wave * (kStageBytes / 4);
    uint16_t* A = reinterpret_cast<uint16_t*>(lds + kWaves * kStageBytes);
    float* red = reinterpret_cast<float*>(lds + kWaves * kStageBytes + (size_t)p.C_hb * 8 * MRB * 32);

    if constexpr (MODE == kModeBatched) {
        // ids outside the table give zero outputs (written by the finisher when split)
        if (p.S == 1) {
            const int per_group = p.S * n_j, gps = (p.batch_m + MRB - 1) / MRB;
            for (int64_t u = u0; u < u1; ++u) {
                const int grp = (int)(u / per_group), j = (int)(u % n_j);
                const int slot = grp / gps, rg = (grp - slot * gps) * MRB;
                const int e = p.expert_list[slot];
                if (e >= 0 && e < p.n_ptr) continue;
                const int nr = min(MRB, p.batch_m - rg);
                for (int i = tid; i < nr * 128; i += kThreads)
                    store_out(p.out, p.out_dtype,
                              (int64_t)(slot * p.batch_m + rg + (i >> 7)) * p.out_stride + j * 128 + (i & 127),
                              0.0f);
            }
        }
    }
    Cursor cur;
    seek_unit<MODE, LK>(p, u0, u1, nq, n_j, n_groups, cur);
    if (cur.u < 0) return;

    v4u buf[kDepth];
    LaneGeo geo = lane_geo<LK>(cur.K, lane);
    Stream cs = stream_of(p, cur, wave);
#pragma unroll
    for (int d = 0; d < kDepth; ++d) buf[d] = load_row(cs.base, geo.voff, (uint32_t)min(d, cs.n - 1) * cs.step);
    Cursor nxt = cur;
    advance<MODE, LK>(p, u1, nq, n_j, nc, nxt);
    stage_chunk<MODE>(p, cur, A, tid);
    __syncthreads();

    float4_t acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int g = lane >> 4;
    const int col_nu = sigma_col(lane & 15);
    while (true) {
        const bool has_next = nxt.u >= 0;
        const bool same_k = !has_next || nxt.K == cur.K;
        // with no next chunk the last refills re-read the current one's first row
        const Stream ns = has_next ? stream_of(p, nxt, wave) : Stream{cs.base, 0u, cs.n};
        const uint32_t ns_voff = same_k ? geo.voff : (lane < 16 * nxt.K ? lane * 16 : 0);
        const int nr = min(MRB, cur.rows - cur.rg);
        const int arow = min(lane & 15, nr - 1);
        consume_chunk<CB, LK>(buf, cs, ns, has_next, has_next ? nxt.K : cur.K, geo, ns_voff, cur.K, lane, wave,
                              stage, A, MRB, arow, acc);
        const bool flush = !has_next || nxt.u != cur.u;
        const bool restage =
            has_next && (nxt.grp != cur.grp || nxt.q != cur.q || nxt.s != cur.s || nxt.c != cur.c);
        if (flush) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 4 * g + i;
                    if (row < nr) red[(wave * MRB + row) * 128 + t * 16 + col_nu] = acc[t][i];
                }
                acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (flush || restage) __syncthreads();
        if (restage) stage_chunk<MODE>(p, nxt, A, tid);
        if (flush) {
            if ((MODE == kModeLinear || MODE == kModeBatched) && p.S == 1) {
                // single split: finish in place
                const uint16_t* svh = p.w_svh;
                if constexpr (MODE == kModeBatched)
                    svh = reinterpret_cast<const uint16_t*>(p.tab[2][p.expert_list[cur.slot]]);
                for (int r = wave; r < nr; r += kWaves) {
                    float v0 = red_sum(red, MRB, r, lane), v1 = red_sum(red, MRB, r, lane + 64);
                    finish_block(v0, v1, svh, cur.j * 128 + lane, lane);
                    v0 += load_bias(p.bias, p.bias_dtype, cur.j * 128 + lane);
                    v1 += load_bias(p.bias, p.bias_dtype, cur.j * 128 + lane + 64);
                    const int64_t o = (int64_t)(cur.row_base + cur.rg + r) * p.out_stride + cur.j * 128 + lane;
                    store_out(p.out, p.out_dtype, o, v0);
                    store_out(p.out, p.out_dtype, o + 64, v1);
                }
            } else {
                float* dst = p.ws + (((int64_t)cur.q * p.S + cur.s) * p.n_rows_ws + cur.row_base + cur.rg) *
                                        p.out_features +
                             cur.j * 128;
                for (int e = tid; e < nr * 128; e += kThreads)
                    dst[(int64_t)(e >> 7) * p.out_features + (e & 127)] = red_sum(red, MRB, e >> 7, e & 127);
            }
        }
        if (!has_next) break;
        if (flush || restage) __syncthreads();
        cur = nxt;
        cs = ns;
        advance<MODE, LK>(p, u1, nq, n_j, nc, nxt);
        if (!same_k) geo = lane_geo<LK>(cur.K, lane);
    }
}

// ---------------------------------------------------------------------------
// One-unit-per-workgroup GEMV, for launches whose units fill at most about two
// rounds of resident workgroups (decode at small batch): workgroup = (slot,
// projection, split, 128-column block), all row groups of the slot in turn.
// Each workgroup starts its trellis stream cold, but the launch needs no unit
// count and no group tables, and keeps the fewest registers live.
// ---------------------------------------------------------------------------
// Stream the wave's tile rows of one projection for the current chunk and
// accumulate into acc[8] (one float4 per 16-column tile).
//   tbase:     byte address of tile (first tile row of the chunk, j*8)
//   row_bytes: bytes between consecutive tile rows (tiles_n * 32K)
//   nkt:       tile rows in the chunk; the wave takes rows wave, wave+4, ...
//   A:         this projection's activations [nkt][MRB][16] fp16 (kappa order)
// The pipeline keeps kWgDepth rows in flight.  Its steady state has no
// branches: lanes past the 256*K-byte row span reload the span's first 16
// bytes, prefetches past the last row reload the last row (all in bounds),
// and every lane stores into the 1 KB stage (bytes past the span are never
// read).
template <int K>
struct WgStream {
    const uint8_t* base;  // the wave's first row (wave-uniform: a scalar buffer resource)
    uint32_t voff;        // this lane's 16 bytes of a row
    uint32_t step;        // bytes between the wave's consecutive rows (the scalar offset)
    int n;                // rows of this wave in the chunk
    v4u buf[kWgDepth];
};

// Issue the loads of the wave's first kWgDepth rows (clamped, in bounds) so
// they are in flight while the activations are staged.
template <int K>
__device__ __forceinline__ void wg_prefetch(WgStream<K>& rs, const uint8_t* tbase,
                                                size_t row_bytes, int nkt, int wave, int lane) {
    constexpr int span = 256 * K;
    rs.n = nkt > wave ? (nkt - wave + kWaves - 1) / kWaves : 0;
    rs.base = tbase + (size_t)wave * row_bytes;
    rs.voff = lane * 16 < span ? lane * 16 : 0;
    rs.step = (uint32_t)(row_bytes * kWaves);  // a chunk lies within one projection (< 2 GiB)
    if (rs.n == 0) return;
#pragma unroll
    for (int d = 0; d < kWgDepth; ++d) rs.buf[d] = load_row(rs.base, rs.voff, (uint32_t)min(d, rs.n - 1) * rs.step);
}

// Consume the wave's rows: per row, stage 256*K bytes in LDS, refill the
// pipeline, read the sixteen words this lane needs, decode and issue eight
// MFMAs.  The steady state has no branches: lanes past the row span reload
// its first 16 bytes, prefetches past the last row reload the last row (all
// in bounds), and every lane stores into the 1 KB stage (bytes past the span
// are never read).
template <int K, int CB>
__device__ __forceinline__ void wg_consume(WgStream<K>& rs, int wave, int lane, uint32_t* stage,
                                               const uint16_t* A, int MRB, int arow,
                                               float4_t (&acc)[8]) {
    constexpr int tile_bytes = 32 * K;
    const int n = rs.n;
    if (n == 0) return;
    const LaneGeo lw = lane_geo<K>(K, lane);
    const int g = lane >> 4;
    const uint8_t* st = reinterpret_cast<const uint8_t*>(stage);
    const uint32_t* arow_p = reinterpret_cast<const uint32_t*>(A + (size_t)arow * 16 + 4 * g) +
                             (size_t)wave * MRB * 8;
    const int a_step = kWaves * MRB * 8;  // uint32 words between this wave's consecutive rows
    auto consume = [&](int d, int i) {
        reinterpret_cast<v4u*>(stage)[lane] = rs.buf[d];
        rs.buf[d] = load_row(rs.base, rs.voff, (uint32_t)min(i + kWgDepth, n - 1) * rs.step);
        const uint32_t* ap = arow_p + (size_t)i * a_step;
        // all sixteen words of the row first: one LDS latency per row
        uint32_t wh[8], wl[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            wh[t] = *reinterpret_cast<const uint32_t*>(st + t * tile_bytes + lw.off_hi);
            wl[t] = *reinterpret_cast<const uint32_t*>(st + t * tile_bytes + lw.off_lo);
        }
        const half8_t a = dup4(ap[0], ap[1]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t b[4];
            decode4<CB>(wh[t], wl[t], lw.shift, 3 * K, 2 * K, K, b);
            acc[t] = mfma16x16x32(a, b, acc[t]);
        }
    };
    int i = 0;
    for (; i + kWgDepth <= n; i += kWgDepth) {
#pragma unroll
        for (int d = 0; d < kWgDepth; ++d) consume(d, i + d);
    }
#pragma unroll
    for (int d = 0; d < kWgDepth; ++d)
        if (i + d < n) consume(d, i + d);
}

// Everything one projection of one row group needs, shared by all waves.
struct WgGroup {
    int rg, nr, arow, row_base, hb_first, nhb, j, tiles_n, expert;
    const void* img;      // rotated activation rows of the streamed projection
    const int* row_map;   // sorted row -> image row (null: the same row)
    int rpos;             // inline routing: sorted row of this lane's route (-1: dropped)
};

// Routing of a decode step with at most 64 routes by one wave, lane r
// holding route r = t * topk + k: the router's stable order by local expert
// (route_impl.h; dropped routes: ids outside [0, n_local) and rows at or past
// *n_valid), computed with shuffles instead of a sort.
struct WaveRoute {
    int key;       // local expert; n_local when dropped
    int pos;       // sorted row; -1 when dropped
    int cnt;       // routes of this lane's expert
    int slot;      // slot of this lane's expert (experts ascending)
    int tiles;     // row tiles of the slot (first route of an expert), else 0
    int mt0;       // first row tile of the slot (first route of an expert)
    bool first;    // first route of its expert in route order
    int n_active;  // slots
    int n_tiles;   // row tiles
};

__device__ __forceinline__ WaveRoute wave_route(const GemvParams& p, int lane) {
    WaveRoute w;
    const int n = p.r_n_routes, nl = p.r_n_local;
    const int live = p.r_n_valid ? min(n, max(0, p.r_n_valid[0]) * p.r_topk) : n;
    w.key = lane < n ? route_key(p.r_ids, p.r_ids_i64, lane, live, nl) : nl;
    const bool valid = w.key < nl;
    int lt = 0, eqb = 0, cnt = 0;
    for (int j = 0; j < n; ++j) {
        const int kj = __shfl(w.key, j, 64);
        lt += kj < w.key;
        eqb += (kj == w.key) && (j < lane);
        cnt += kj == w.key;
    }
    w.first = valid && eqb == 0;
    w.pos = valid ? lt + eqb : -1;
    w.cnt = cnt;
    w.tiles = w.first ? (cnt + p.MRB - 1) / p.MRB : 0;
    const uint64_t fm = __ballot(w.first);
    int slot = 0, mt0 = 0;
    for (int j = 0; j < n; ++j) {
        const int kj = __shfl(w.key, j, 64), tj = __shfl(w.tiles, j, 64);
        const bool before = ((fm >> j) & 1ull) && kj < w.key;
        slot += before;
        mt0 += before ? tj : 0;
    }
    w.slot = slot;
    w.mt0 = mt0;
    w.n_active = __popcll(fm);
    int tot = w.tiles;
    for (int d = 32; d; d >>= 1) tot += __shfl_xor(tot, d, 64);
    w.n_tiles = tot;
    return w;
}

// The router's tables (RouteOut, row tiles of MRB rows) from one wave's
// routing, for the kernels after the gate/up GEMV.
__device__ __forceinline__ void write_route_tables(const GemvParams& p, const WaveRoute& w, int lane) {
    const RouteOut& o = p.ro;
    if (lane < p.r_n_routes) {
        o.route_pos[lane] = w.pos;
        if (w.pos >= 0) {
            o.row_token[w.pos] = lane / p.r_topk;
            o.row_expert[w.pos] = w.key;
            if (o.row_route) o.row_route[w.pos] = lane;
        }
    }
    if (w.first) {
        o.slot_expert[w.slot] = w.key;
        o.slot_start[w.slot] = w.pos;
        o.slot_rows[w.slot] = w.cnt;
        if (o.n_mtiles) {
            for (int k = 0; k < w.tiles; ++k) {
                o.mt_slot[w.mt0 + k] = w.slot;
                if (o.mt_expert) o.mt_expert[w.mt0 + k] = w.key;
                o.mt_row0[w.mt0 + k] = k * p.MRB;
            }
        }
    }
    const int kept = __popcll(__ballot(w.pos >= 0));
    if (lane == 0) {
        o.n_active[0] = w.n_active;
        if (o.n_mtiles) o.n_mtiles[0] = w.n_tiles;
        if (o.n_sorted) o.n_sorted[0] = kept;
    }
}

// Copy the rotated activations of a row group for tile rows [kt0, kt0 + nkt)
// from their image (row-major fp16 rows, MFMA k order inside each 16 inputs)
// into the LDS operand layout A[kt][MRB][16].  The image row of each of the
// group's rows is looked up once per batch of rows; each thread then owns
// 16-byte pieces (tile row, half) and issues the loads of the batch's rows
// before its stores, so a batch costs about two round trips and no integer
// division.
__device__ __forceinline__ void wg_stage_rows(const GemvParams& p, const WgGroup& G, int kt0, int nkt,
                                           uint16_t* A, int tid) {
    typedef __attribute__((address_space(1))) const v4u* gv4c;
    constexpr int kRowBatch = 4;
    const int MRB = p.MRB;
    const uint16_t* img = reinterpret_cast<const uint16_t*>(G.img);
    const int npc = nkt * 2;  // 16-byte pieces per row
    // a zero the compiler cannot see through: the row map is read with vector
    // loads (one request per wave, no scalar registers held across the copy)
    int vzero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
    for (int r0 = 0; r0 < G.nr; r0 += kRowBatch) {
        int64_t src[kRowBatch];
        const int64_t srow0 = G.row_base + G.rg;
        if (G.row_map) {
#pragma unroll
            for (int b = 0; b < kRowBatch; ++b)
                src[b] = (int64_t)G.row_map[srow0 + min(r0 + b, G.nr - 1) + vzero];
        } else {
#pragma unroll
            for (int b = 0; b < kRowBatch; ++b) src[b] = srow0 + min(r0 + b, G.nr - 1);
        }
#pragma unroll
        for (int b = 0; b < kRowBatch; ++b) src[b] = src[b] * p.x_stride + (int64_t)kt0 * 16;
        for (int c = tid; c < npc; c += kThreads) {
            const int64_t off = (int64_t)(c >> 1) * 16 + 8 * (c & 1);
            v4u v[kRowBatch];
#pragma unroll
            for (int b = 0; b < kRowBatch; ++b)
                if (r0 + b < G.nr) v[b] = *(gv4c)(img + src[b] + off);
#pragma unroll
            for (int b = 0; b < kRowBatch; ++b)
                if (r0 + b < G.nr)
                    *reinterpret_cast<v4u*>(A + ((c >> 1) * MRB + r0 + b) * 16 + 8 * (c & 1)) = v[b];
        }
    }
}

// Rotated activations of a plain linear's rows for tile rows [kt0, kt0 + nkt)
// (whole 128-input blocks), computed from the raw input rows: each wave takes
// (row, block) units in turn, four at a time with all their loads issued
// first, and computes fp16(had128(x * suh) / sqrt(128)) as the rotation
// kernel does, stored in the LDS operand layout A[kt][MRB][16] (the 16
// inputs of a tile row in MFMA k order).  Used for a few rows, where
// rotating in every workgroup costs less than a separate launch.
// Input row of the group's row r: the sorted row itself for a linear; with
// inline routing, the token of the route at that sorted row.
__device__ __forceinline__ int64_t raw_row(const GemvParams& p, const WgGroup& G, int r) {
    const int srow = G.row_base + G.rg + r;
    if (!p.inline_route) return srow;
    const uint64_t m = __ballot(G.rpos == srow);
    return (int64_t)((__ffsll((unsigned long long)m) - 1) / p.r_topk);
}

__device__ __forceinline__ void wg_stage_rotate(const GemvParams& p, const WgGroup& G, int kt0, int nkt,
                                             uint16_t* A, const uint16_t* suh, int wave, int lane) {
    constexpr int kBatch = 4;
    const int MRB = p.MRB;
    const int nb = nkt >> 3, hb0 = kt0 >> 3, nu = G.nr * nb;
    for (int u0 = wave; u0 < nu; u0 += kWaves * kBatch) {
        float v[kBatch][2], su[kBatch][2];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int u = min(u0 + i * kWaves, nu - 1);
            const int r = u / nb, blk = hb0 + u - (u / nb) * nb;
            const int64_t base = raw_row(p, G, r) * p.x_stride + (int64_t)blk * 128;
            v[i][0] = load_act(p.x, p.x_dtype, base + lane);
            v[i][1] = load_act(p.x, p.x_dtype, base + lane + 64);
            su[i][0] = (float)bits_to_half(suh[blk * 128 + lane]);
            su[i][1] = (float)bits_to_half(suh[blk * 128 + lane + 64]);
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int u = u0 + i * kWaves;
            if (u >= nu) break;  // wave-uniform
            const int r = u / nb, b = u - r * nb;
            float v0 = v[i][0] * su[i][0], v1 = v[i][1] * su[i][1];
            had128(v0, v1, lane);
            const float hs = kHadNorm * had_sign64(lane);  // with had128's lane sign
            const int c0 = lane, c1 = lane + 64;
            A[((b * 8 + (c0 >> 4)) * MRB + r) * 16 + pi_inv(c0 & 15)] = half_to_bits(f32_to_f16_rne(v0 * hs));
            A[((b * 8 + (c1 >> 4)) * MRB + r) * 16 + pi_inv(c1 & 15)] = half_to_bits(f32_to_f16_rne(v1 * hs));
        }
    }
}

// Stage the activations of one projection for chunk [c0, c0 + nb) of
// 128-row blocks, stream its tiles, and leave each wave's partial sums in
// red[wave][row][128].  acc lives only inside this K-specialised routine.
template <int K, int CB>
__device__ __forceinline__ void wg_projection(const GemvParams& p, const WgGroup& G, const Proj& pq,
                                               uint32_t* stage, uint16_t* A, float* red, bool restage,
                                               int wave, int lane) {
    float4_t acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int MRB = p.MRB;
    constexpr size_t tile_bytes = 32u * K;
    const size_t row_bytes = (size_t)G.tiles_n * tile_bytes;
    for (int c0 = 0; c0 < G.nhb; c0 += p.C_hb) {
        const int nb = min(p.C_hb, G.nhb - c0);
        // trellis bytes of this chunk start moving before the staging below
        WgStream<K> rs;
        const uint8_t* tb = pq.trellis +
                            ((size_t)(G.hb_first + c0) * 8 * G.tiles_n + (size_t)G.j * 8) * tile_bytes;
        wg_prefetch<K>(rs, tb, row_bytes, nb * 8, wave, lane);
        if (restage) {
            __syncthreads();
            if (p.x_raw)
                wg_stage_rotate(p, G, (G.hb_first + c0) * 8, nb * 8, A, pq.suh, wave, lane);
            else
                wg_stage_rows(p, G, (G.hb_first + c0) * 8, nb * 8, A, threadIdx.x);
            __syncthreads();
        }
        wg_consume<K, CB>(rs, wave, lane, stage, A, MRB, G.arow, acc);
    }
    // when red overlays A, every wave must be done reading A first
    __syncthreads();
    const int g = lane >> 4;
    const int col_nu = sigma_col(lane & 15);
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * g + i;
            if (row < G.nr) red[(wave * MRB + row) * 128 + t * 16 + col_nu] = acc[t][i];
        }
    __syncthreads();
}

template <int CB, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemv_wg_kernel(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar stream bases
    const int nJB = p.out_features >> 7;
    // gate/up: each workgroup streams one of the two projections
    const int nsplit_proj = (MODE == kModeGateUp && !p.gateless) ? 2 : 1;
    int item = blockIdx.x, s, half = -1;
    if ((MODE == kModeGateUp || MODE == kModeDown) && p.tail_halves > 0) {
        // units below tail_halves whole, later ones in S parts
        if (item >= p.tail_halves) {
            half = (item - p.tail_halves) % p.S;
            item = p.tail_halves + (item - p.tail_halves) / p.S;
        }
        s = half < 0 ? 0 : half;
    } else {
        s = (item / nsplit_proj) % p.S;
        item = item % nsplit_proj + item / nsplit_proj / p.S * nsplit_proj;
    }
    const int qsel = item % nsplit_proj;
    const int rest = item / nsplit_proj;
    WgGroup G;
    G.row_map = MODE == kModeGateUp ? p.row_map : nullptr;
    const int jb = rest % nJB;
    const int slot = rest / nJB;

    int rows;
    G.expert = 0;
    if constexpr (MODE == kModeLinear) {
        rows = p.m_rows;
        G.row_base = 0;
    } else if constexpr (MODE == kModeBatched) {
        if (slot >= p.max_slots) return;
        G.expert = p.expert_list[slot];
        G.row_base = slot * p.batch_m;
        rows = p.batch_m;
        if (G.expert < 0 || G.expert >= p.n_ptr) {
            // not a table entry: zero outputs (written by the finisher when split)
            if (p.S == 1)
                for (int e = tid; e < rows * 128; e += kThreads)
                    store_out(p.out, p.out_dtype,
                              (int64_t)(G.row_base + (e >> 7)) * p.out_stride + jb * 128 + (e & 127), 0.0f);
            return;
        }
    } else if (MODE == kModeGateUp && p.inline_route) {
        // route the step in every wave; workgroup 0 publishes the tables
        const WaveRoute wr = wave_route(p, lane);
        if (blockIdx.x == 0 && wave == 0) write_route_tables(p, wr, lane);
        if (slot >= wr.n_active) return;  // workgroup-uniform, before any barrier
        const uint64_t m = __ballot(wr.first && wr.slot == slot);
        const int L = __ffsll((unsigned long long)m) - 1;
        G.expert = __builtin_amdgcn_readfirstlane(__shfl(wr.key, L, 64));
        G.row_base = __builtin_amdgcn_readfirstlane(__shfl(wr.pos, L, 64));
        rows = __builtin_amdgcn_readfirstlane(__shfl(wr.cnt, L, 64));
        G.rpos = wr.pos;
    } else {
        if (slot >= *p.n_active) return;
        G.expert = p.slot_expert[slot];
        G.row_base = p.slot_start[slot];
        rows = p.slot_rows[slot];
    }
    Proj pr;
    if constexpr (MODE == kModeLinear) {
        pr = {reinterpret_cast<const uint8_t*>(p.w_trellis), p.w_suh, p.w_svh, p.kuni[0]};
    } else if constexpr (MODE == kModeBatched) {
        pr = {reinterpret_cast<const uint8_t*>(p.tab[0][G.expert]),
              reinterpret_cast<const uint16_t*>(p.tab[1][G.expert]),
              reinterpret_cast<const uint16_t*>(p.tab[2][G.expert]), p.kuni[0]};
    } else {
        auto load_proj = [&](int pj) {
            Proj q;
            q.trellis = reinterpret_cast<const uint8_t*>(p.tab[3 * pj][G.expert]);
            q.suh = reinterpret_cast<const uint16_t*>(p.tab[3 * pj + 1][G.expert]);
            q.svh = reinterpret_cast<const uint16_t*>(p.tab[3 * pj + 2][G.expert]);
            q.K = p.ktab[pj] ? (int)p.ktab[pj][G.expert] : p.kuni[pj];
            return q;
        };
        pr = MODE == kModeGateUp ? load_proj(p.gateless ? 1 : qsel) : load_proj(2);
    }

    // a per-expert K outside {2, 3, 4} is gemv_anyk_kernel's unit: nothing
    // is streamed or written here (workgroup-uniform, before any barrier)
    if (pr.K < 2 || pr.K > 4) return;
    const int MRB = p.MRB;
    G.img = (MODE == kModeGateUp && qsel) ? p.x2 : p.x;
    G.tiles_n = p.out_features >> 4;
    // input blocks of this unit: the split's, or a half of the whole range
    G.nhb = half < 0 ? p.R_hb : (half == p.S - 1 ? p.R_hb - half * (p.R_hb / p.S) : p.R_hb / p.S);
    G.hb_first = half < 0 ? s * p.R_hb : half * (p.R_hb / p.S);
    // LDS: [stage 4 x 1 KB][A: C_hb x 8 x MRB x 16 fp16 | red: 4 waves x MRB
    // x 128 fp32] (red overlays A: the column block's reduction follows its
    // last read of A)
    uint32_t* stage = reinterpret_cast<uint32_t*>(lds) + wave * (kStageBytes / 4);
    uint16_t* A = reinterpret_cast<uint16_t*>(lds + kWaves * kStageBytes);
    float* red = reinterpret_cast<float*>(lds + kWaves * kStageBytes);

    for (G.rg = 0; G.rg < rows; G.rg += MRB) {
      G.nr = min(MRB, rows - G.rg);
      G.arow = min(lane & 15, G.nr - 1);
      {
        G.j = jb;
        const bool restage = true;
        switch (pr.K) {
            case 2: wg_projection<2, CB>(p, G, pr, stage, A, red, restage, wave, lane); break;
            case 3: wg_projection<3, CB>(p, G, pr, stage, A, red, restage, wave, lane); break;
            default: wg_projection<4, CB>(p, G, pr, stage, A, red, restage, wave, lane); break;
        }
        if ((MODE == kModeLinear || MODE == kModeBatched) && p.S == 1) {
            // single split: finish in place
            for (int r = wave; r < G.nr; r += kWaves) {
                float v0 = red_sum(red, MRB, r, lane), v1 = red_sum(red, MRB, r, lane + 64);
                finish_block(v0, v1, pr.svh, G.j * 128 + lane, lane);
                v0 += load_bias(p.bias, p.bias_dtype, G.j * 128 + lane);
                v1 += load_bias(p.bias, p.bias_dtype, G.j * 128 + lane + 64);
                const int64_t o = (int64_t)(G.row_base + G.rg + r) * p.out_stride + G.j * 128 + lane;
                store_out(p.out, p.out_dtype, o, v0);
                store_out(p.out, p.out_dtype, o + 64, v1);
            }
        } else {
            for (int e = tid; e < G.nr * 128; e += kThreads) {
                const int r = e >> 7, c = e & 127;
                const int64_t o = ((int64_t)qsel * p.S * p.n_rows_ws + G.row_base + G.rg + r) * p.out_features +
                                  G.j * 128 + c;
                p.ws[o + (int64_t)s * p.n_rows_ws * p.out_features] = red_sum(red, MRB, r, c);
                // a whole unit of a split-tail launch: its other slots are zero
                if ((MODE == kModeGateUp || MODE == kModeDown) && p.tail_halves > 0 && half < 0)
                    for (int z = 1; z < p.S; ++z) p.ws[o + (int64_t)z * p.n_rows_ws * p.out_features] = 0.0f;
            }
        }
        __syncthreads();
      }
    }
}

// ---------------------------------------------------------------------------
// Mixed-K MoE units whose per-expert K (from the int8 K tables) is outside the
// streaming kernels' {2, 3, 4}.  The reference's mixed-K tile switch computes
// K 5 and 6 with a generic dequantising tile and zero-fills the tile for any
// other value (csrc/p2b_moe.cu:295-324); this kernel does the same for the
// units the streaming kernels skip, writing the same raw split partials, so
// the consumer kernels need no change.  Workgroup = (slot, projection,
// kAnyKBlocks 128-column blocks); it exits at once for an expert of K 2..4
// (the launch costs a few microseconds when no such expert is routed) and
// otherwise walks its column blocks, the splits and the slot's rows in
// groups of 16.  Per wave and tile
// row: the 256*K bytes are staged in the wave's LDS slot, each lane decodes
// its four tile indices per tile with a general window read (any K), and
// one v_mfma_f32_16x16x32_f16 per tile accumulates, in the operand order of
// the streaming kernels (same image rows, same permuted tile positions).
// ---------------------------------------------------------------------------
constexpr int kAnyKMaxBytes = 256 * 8;  // one tile row at K <= 8
// 128-column blocks per workgroup: in a phase with no K 5/6 expert every
// workgroup only reads its slot's K and exits, so fewer, wider workgroups
// cost less (C3: 8,224 -> 2,056 workgroups per gate/up launch).
constexpr int kAnyKBlocks = 4;

template <int CB, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_anyk_kernel(GemvParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t stage_all[kWaves][kAnyKMaxBytes];
    __shared__ float red[kWaves][16][128];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nJB = p.out_features >> 7;
    const int nq = (MODE == kModeGateUp && !p.gateless) ? 2 : 1;
    const int nJG = (nJB + kAnyKBlocks - 1) / kAnyKBlocks;
    const int item = blockIdx.x;
    const int qsel = item % nq;
    const int jg = (item / nq) % nJG;
    const int slot = item / nq / nJG;
    if (slot >= *p.n_active) return;
    const int e = p.slot_expert[slot];
    const bool up = MODE == kModeGateUp && (p.gateless || qsel);
    const int8_t* ktab = MODE == kModeDown ? p.ktab[2] : up ? p.ktab[1] : p.ktab[0];
    if (!ktab) return;
    const int K = ktab[e];
    if (K >= 2 && K <= 4) return;  // the streaming kernels' unit
    const int64_t* ttab = MODE == kModeDown ? p.tab[6] : up ? p.tab[3] : p.tab[0];
    const uint8_t* trellis = reinterpret_cast<const uint8_t*>(ttab[e]);
    const uint16_t* img = reinterpret_cast<const uint16_t*>((MODE == kModeGateUp && qsel) ? p.x2 : p.x);
    const int rows = p.slot_rows[slot], row_base = p.slot_start[slot];
    const bool compute = K == 5 || K == 6;
    const int tiles_n = p.out_features >> 4;
    const int g = lane >> 4;
    const int col_nu = sigma_col(lane & 15);
    const int q4 = 4 * lane_q(lane);
    uint8_t* st = stage_all[wave];
    const int jb1 = min(nJB, (jg + 1) * kAnyKBlocks);
    for (int jb = jg * kAnyKBlocks; jb < jb1; ++jb)
    for (int s = 0; s < p.S; ++s) {
        float* dst = p.ws + (((int64_t)qsel * p.S + s) * p.n_rows_ws + row_base) * p.out_features + jb * 128;
        // a halved-tail launch: slot 0 holds the whole input range, slot 1 zeros
        if (!compute || (p.tail_halves > 0 && s > 0)) {
            for (int i = tid; i < rows * 128; i += kThreads) dst[(int64_t)(i >> 7) * p.out_features + (i & 127)] = 0.0f;
            continue;
        }
        const int kt0 = s * p.R_hb * 8, nkt = p.R_hb * 8;
        const uint32_t nbits = 256u * K, n32 = 8u * K, tile_bytes = 32u * K;
        for (int rg = 0; rg < rows; rg += 16) {
            const int nr = min(16, rows - rg);
            const int64_t arow = row_base + rg + min(lane & 15, nr - 1);
            float4_t acc[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
            for (int kl = wave; kl < nkt; kl += kWaves) {
                const int kt = kt0 + kl;
                const uint8_t* src = trellis + ((size_t)kt * tiles_n + (size_t)jb * 8) * tile_bytes;
                for (uint32_t off = lane * 16u; off < 8u * tile_bytes; off += 1024u)
                    *reinterpret_cast<v4u*>(st + off) = *reinterpret_cast<const v4u*>(src + off);
                __builtin_amdgcn_wave_barrier();
                const uint32_t* ap = reinterpret_cast<const uint32_t*>(img + arow * p.x_stride + (int64_t)kt * 16 + 4 * g);
                const half8_t a = dup4(ap[0], ap[1]);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t* tw = reinterpret_cast<const uint32_t*>(st + t * tile_bytes);
                    uint32_t b[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // window of tile index q4 + i: stream bits
                        // [(idx + 257) K - 16, (idx + 257) K) mod 256 K, MSB first
                        const uint32_t bit = ((uint32_t)(q4 + i + 1) * K + nbits - 16u) % nbits;
                        const uint32_t i0 = bit >> 5, i1 = i0 + 1 == n32 ? 0 : i0 + 1;
                        const uint32_t win = funnel(tw[i0], tw[i1], 48u - (bit & 31u)) & 0xFFFFu;
                        if constexpr (CB == kCbMul1)
                            b[i] = (uint32_t)half_to_bits(decode_weight<kCbMul1>(win));
                        else
                            b[i] = cb_pair<CB>(win);
                    }
                    acc[t] = mfma16x16x32(a, b, acc[t]);
                }
                __builtin_amdgcn_wave_barrier();  // the stage is rewritten by the next tile row
            }
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][4 * g + i][t * 16 + col_nu] = acc[t][i];
            __syncthreads();
            for (int i = tid; i < nr * 128; i += kThreads) {
                const int r = i >> 7, c = i & 127;
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v += red[w][r][c];
                dst[(int64_t)(rg + r) * p.out_features + c] = v;
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// Routing and input rotation in one launch (decode steps whose gate/up phase
// runs one unit per workgroup): block 0 routes (the stable multisplit sort
// of route_impl.h) while the other blocks rotate every kept route's gate/up
// input rows in route order; the GEMV stages a sorted row through the
// router's sorted row -> route map.  Saves the rotation launch; the two
// halves of the work never wait on each other.
// ---------------------------------------------------------------------------
struct RouteRotateArgs {
    const void* ids;
    int ids_i64, n_routes, topk, n_local, T, tile_rows;
    const int32_t* n_valid;
    const void* x;
    int x_dtype, hidden;
    const int64_t* suh_tab0;  // per-expert suh of the gate (or, gateless, up) projection
    const int64_t* suh_tab1;  // per-expert suh of the up projection
    int nproj;
    uint16_t* img0;           // [n_routes][hidden] rotated rows, route order
    uint16_t* img1;
    RouteOut ro;
};

__global__ __launch_bounds__(kRouteThreads) void route_rotate_kernel(RouteRotateArgs f) {
    if (blockIdx.x == 0) {
        route_multisplit_body(f.ids, f.ids_i64, f.n_routes, f.topk, f.n_local, f.n_valid, f.tile_rows, f.ro);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t nb = blockIdx.x - 1, nblk = gridDim.x - 1;
    const int live = f.n_valid ? min(f.T, max(0, f.n_valid[0])) : f.T;
    const int64_t gw = nb * (kRouteThreads / 64) + (tid >> 6);
    const int64_t nw = nblk * (kRouteThreads / 64);
    const int nhb = f.hidden >> 7;
    for (int64_t u = gw; u < (int64_t)f.n_routes * nhb; u += nw) {
        const int64_t r = u / nhb;
        const int hb = (int)(u % nhb);
        const int64_t t = r / f.topk;
        const int64_t e = f.ids_i64 ? reinterpret_cast<const int64_t*>(f.ids)[r]
                                    : (int64_t)reinterpret_cast<const int32_t*>(f.ids)[r];
        if (t >= live || e < 0 || e >= f.n_local) continue;  // wave-uniform: a dropped route
        const int64_t fb = (int64_t)hb * 128;
        const float x0 = load_act(f.x, f.x_dtype, t * f.hidden + fb + lane);
        const float x1 = load_act(f.x, f.x_dtype, t * f.hidden + fb + lane + 64);
        for (int q = 0; q < f.nproj; ++q) {
            const uint16_t* su = reinterpret_cast<const uint16_t*>(q ? f.suh_tab1[e] : f.suh_tab0[e]);
            float v0 = x0 * (float)bits_to_half(su[fb + lane]);
            float v1 = x1 * (float)bits_to_half(su[fb + lane + 64]);
            had128(v0, v1, lane);
            const float hs = kHadNorm * had_sign64(lane);  // with had128's lane sign
            uint16_t* dst = (q ? f.img1 : f.img0) + r * f.hidden;
            dst[image_pos(fb + lane)] = half_to_bits(f32_to_f16_rne(v0 * hs));
            dst[image_pos(fb + lane + 64)] = half_to_bits(f32_to_f16_rne(v1 * hs));
        }
    }
}

// Linear with split-K: out[m] = finish(sum of splits).  One wave per
// (row, 128-column block).  Batched: row r belongs to slot r / batch_m, whose
// expert's svh comes from svh_tab (ids outside the table give zeros).
struct FinishBatch {
    const int64_t* svh_tab;  // null: single linear
    const int* expert_list;
    int batch_m, n_ptr;
    const void* bias;        // single linear: optional bias [out_f]
    int bias_dtype;
};

__global__ __launch_bounds__(256) void linear_finish_kernel(const float* __restrict__ ws, int S,
                                                            int m, int out_f,
                                                            const uint16_t* __restrict__ svh,
                                                            void* out, int out_dtype, FinishBatch fb) {
    const int lane = threadIdx.x & 63;
    const int nJ = out_f >> 7;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= m * nJ) return;
    const int r = item / nJ, j = item % nJ;
    float v0 = 0.f, v1 = 0.f;
    bool zero = false;
    if (fb.svh_tab) {
        const int e = fb.expert_list[r / fb.batch_m];
        zero = e < 0 || e >= fb.n_ptr;  // wave-uniform
        if (!zero) svh = reinterpret_cast<const uint16_t*>(fb.svh_tab[e]);
    }
    if (!zero) {
        sum_splits(ws + (int64_t)r * out_f, (int64_t)m * out_f, S, j * 128 + lane, v0, v1);
        finish_block(v0, v1, svh, j * 128 + lane, lane);
        v0 += load_bias(fb.bias, fb.bias_dtype, j * 128 + lane);
        v1 += load_bias(fb.bias, fb.bias_dtype, j * 128 + lane + 64);
    }
    const int64_t o = (int64_t)r * out_f + j * 128 + lane;
    store_out(out, out_dtype, o, v0);
    store_out(out, out_dtype, o + 64, v1);
}

// ---------------------------------------------------------------------------
// Routing for layers with more than kRouteMaxLocal local experts: bitonic
// sort of the T*topk routes by local expert id (sentinel routes last) in one
// workgroup, then slots = runs of one expert and, for tile_rows > 0, each
// slot's row tiles of tile_rows rows.  Same outputs as the multisplit router
// of route.hip (which handles every layer up to kRouteMaxLocal experts); at
// most kMaxRoutes routes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRouteThreads) void route_bitonic_kernel(const void* ids, int ids_i64,
                                                                     int n_routes, int topk,
                                                                     int n_local,
                                                                     const int32_t* n_valid,
                                                                     int tile_rows, RouteOut o) {
    __shared__ uint32_t key[kMaxRoutes];
    __shared__ int wave_sum[kRouteThreads / 64];
    __shared__ int wave_tiles[kRouteThreads / 64];
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
    // slots (runs) starting in this thread's range, and their row tiles
    auto run_end = [&](int q, uint32_t e) {
        int end = q + 1;
        while (end < n_routes && (key[end] >> kRouteBits) == e) ++end;
        return end;
    };
    int cnt = 0, tcnt = 0;
    for (int q = p0; q < p1; ++q) {
        const uint32_t e = key[q] >> kRouteBits;
        if (e < (uint32_t)n_local && (q == 0 || (key[q - 1] >> kRouteBits) != e)) {
            ++cnt;
            if (tile_rows > 0) tcnt += (run_end(q, e) - q + tile_rows - 1) / tile_rows;
        }
    }
    const int lane = tid & 63, w = tid >> 6;
    int incl = cnt, tincl = tcnt;
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        const int tt = __shfl_up(tincl, d, 64);
        if (lane >= d) {
            incl += t;
            tincl += tt;
        }
    }
    if (lane == 63) {
        wave_sum[w] = incl;
        wave_tiles[w] = tincl;
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, tacc = 0;
        for (int i = 0; i < kRouteThreads / 64; ++i) {
            const int t = wave_sum[i], tt = wave_tiles[i];
            wave_sum[i] = acc;
            wave_tiles[i] = tacc;
            acc += t;
            tacc += tt;
        }
        o.n_active[0] = acc;
        if (tile_rows > 0) o.n_mtiles[0] = tacc;
    }
    __syncthreads();
    int slot = wave_sum[w] + incl - cnt;      // exclusive prefixes for this thread's range
    int tile = wave_tiles[w] + tincl - tcnt;
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
                const int rows = run_end(q, e) - q;
                o.slot_rows[slot] = rows;
                if (tile_rows > 0)
                    for (int k = 0; k * tile_rows < rows; ++k, ++tile) {
                        o.mt_slot[tile] = slot;
                        if (o.mt_expert) o.mt_expert[tile] = (int)e;
                        o.mt_row0[tile] = k * tile_rows;
                    }
                ++slot;
            }
        } else {
            o.route_pos[route] = -1;
        }
    }
}

// out[t, block j] = sum_k w[t,k] * finish(sum_s partial_s[pos(t,k)]) in slot
// order; sentinel routes are skipped (their rows are never read, so unwritten
// rows cannot leak NaN).  One workgroup per (token, 128-column block); wave k
// finishes routes k, k + waves, ...; the weighted results meet in LDS and are
// summed in slot order.
constexpr int kCombineWaves = 8;
constexpr int kMaxTopk = 64;

__global__ __launch_bounds__(kCombineWaves * 64) void combine_kernel(
    const float* __restrict__ ws, int S, int n_routes, int H, const int* route_pos,
    const int* row_expert, const int64_t* down_svh_tab, const void* weights, int w_dtype, int topk,
    void* out, int out_dtype) {
    __shared__ float part[kMaxTopk][128];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nJ = H >> 7;
    const int t = blockIdx.x / nJ, j = blockIdx.x % nJ;
    const int c0 = j * 128 + lane;
    for (int k = wave; k < topk; k += kCombineWaves) {
        const int pos = route_pos[t * topk + k];
        float v0 = 0.f, v1 = 0.f;
        if (pos >= 0) {
            sum_splits(ws + (int64_t)pos * H, (int64_t)n_routes * H, S, c0, v0, v1);
            finish_block(v0, v1, reinterpret_cast<const uint16_t*>(down_svh_tab[row_expert[pos]]),
                         c0, lane);
            const int64_t wi = (int64_t)t * topk + k;
            float w;
            if (w_dtype == kF32)
                w = reinterpret_cast<const float*>(weights)[wi];
            else if (w_dtype == kF16)
                w = (float)bits_to_half(reinterpret_cast<const uint16_t*>(weights)[wi]);
            else
                w = __builtin_bit_cast(float,
                                       (uint32_t)reinterpret_cast<const uint16_t*>(weights)[wi] << 16);
            v0 *= w;
            v1 *= w;
        }
        part[k][lane] = v0;
        part[k][lane + 64] = v1;
    }
    __syncthreads();
    if (threadIdx.x < 128) {
        float acc = 0.f;
        for (int k = 0; k < topk; ++k) acc += part[k][threadIdx.x];
        store_out(out, out_dtype, (int64_t)t * H + j * 128 + threadIdx.x, acc);
    }
}

// ---------------------------------------------------------------------------
// Host-side planning (shared by the workspace queries and the launches)
// ---------------------------------------------------------------------------
constexpr int kMaxSplits = 16;
// Launch cost model (microseconds, measured on MI355X under a full decode
// load): a workgroup's fixed latency before its first tile row (argument,
// group, table and activation loads, cold trellis stream), a wave's time per
// tile row with three workgroups per CU, the cost of one unit's wave
// reduction and partial write, of one activation restage, and the
// consumer's cost per split.
constexpr double kWgFixedUs = 8.0;
constexpr double kRowUs = 0.9;
constexpr double kUnitUs = 2.0;
constexpr double kStageUs = 1.0;
constexpr double kSplitUs = 0.15;
// LDS per workgroup that keeps three workgroups resident on a 160 KB CU.
constexpr size_t kLdsBudget = 53 * 1024;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workgroups resident at once: three per CU (the GEMV's register budget).
inline int resident_workgroups() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) {
            (void)hipGetLastError();
            cus = 256;
        }
        return 3 * cus;
    }();
    return n;
}

inline size_t gemv_red_bytes(int MRB) { return (size_t)kWaves * MRB * 128 * 4; }

// Hadamard blocks whose activations are staged at once: what the LDS budget
// leaves after the stage slots and the reduction buffer.  For a split of a
// multiple of 4 blocks the chunk is a multiple of 4 dividing it, so every
// chunk gives each wave a whole number of kDepth-row blocks.
inline int pick_chunk(int R_hb, int MRB) {
    const size_t fixed = kWaves * kStageBytes + gemv_red_bytes(MRB);
    const size_t per_hb = (size_t)8 * MRB * 16 * 2;  // staged activations per 128-row block
    int cmax = fixed < kLdsBudget ? (int)((kLdsBudget - fixed) / per_hb) : 1;
    if (cmax < 1) cmax = 1;
    if (R_hb % 4 == 0 && cmax >= 4) {
        for (int c = cmax - cmax % 4; c >= 4; c -= 4)
            if (R_hb % c == 0) return c;
    }
    return cmax < R_hb ? cmax : R_hb;
}

inline size_t gemv_lds_bytes(int C_hb, int MRB) {
    return kWaves * kStageBytes + (size_t)C_hb * 8 * MRB * 16 * 2 + gemv_red_bytes(MRB);
}

struct PhasePlan {
    int S, R_hb, C_hb, grid;
    int wg;  // 1: one unit per workgroup (gemv_wg_kernel); 0: persistent (gemv_kernel)
    size_t lds;
    int halves;  // one-unit MoE phase with a halved tail: the whole units (GemvParams::tail_halves)
};

// One-unit-per-workgroup plan: activation chunk within a 40 KB budget (the
// reduction buffer overlays it), cost = rounds of resident workgroups x
// (fixed latency + rows x row time) + the consumer's per-split cost.
constexpr double kWgRowUs = 0.6;  // a wave's time per tile row, cold-started workgroups
constexpr int kMinUnitsPerWg = 6;

inline int pick_chunk_wg(int R_hb, int MRB) {
    const int per_hb = 8 * MRB * 16 * 2;
    int c = (40 * 1024) / per_hb;
    if (c < 1) c = 1;
    return c < R_hb ? c : R_hb;
}

// EXL3_GEMV_SPLITS=S restricts the planners to that split count when it is
// valid for the phase (tuning; read on every plan, workspace queries included).
inline int gemv_forced_splits() {
    const char* v = std::getenv("EXL3_GEMV_SPLITS");
    return v ? std::atoi(v) : 0;
}

// EXL3_GEMV_TAIL_HALVES=0 keeps whole units past the first round of a
// one-unit MoE phase (tuning; read on every plan, workspace queries included).
inline int gemv_tail_parts() {
    const char* v = std::getenv("EXL3_GEMV_TAIL_HALVES");
    if (v && std::strcmp(v, "0") == 0) return 0;
    const char* n = std::getenv("EXL3_GEMV_TAIL_PARTS");
    return n ? std::atoi(n) : 2;
}

// One-unit-per-workgroup plan.  For a MoE phase whose whole units need a
// second round of resident workgroups, the units past the first round run as
// two halves of the input range each (the first-round units write a zero
// second slot): the SIMD issues from its oldest wave first, so first-round
// workgroups finish in dispatch order over a wide spread of times, and short
// late workgroups end the launch sooner than whole ones.
inline PhasePlan plan_phase_wg(int in_f, int out_f, int wg_items, int MRB, bool moe = false) {
    const int n_hb = in_f / 128, n_j = out_f / 128;
    const int cap = resident_workgroups();
    PhasePlan best = {1, n_hb, pick_chunk_wg(n_hb, MRB), 1, 1, 0};
    double best_t = 1e30;
    const int forced = gemv_forced_splits();
    for (int S = 1; S <= kMaxSplits && S <= n_hb; ++S) {
        if (n_hb % S) continue;
        if (forced > 0 && S != forced && n_hb % forced == 0) continue;
        const int R_hb = n_hb / S;
        const int64_t items = (int64_t)wg_items * n_j * S;
        const int64_t rounds = (items + cap - 1) / cap;
        const double t = rounds * (kWgFixedUs + R_hb * 8.0 / kWaves * kWgRowUs) + S * kSplitUs;
        if (t < best_t) {
            best_t = t;
            best = {S, R_hb, pick_chunk_wg(R_hb, MRB), (int)items, 1, 0};
        }
    }
    const int64_t units = (int64_t)wg_items * n_j;
    const int parts = gemv_tail_parts();
    if (moe && best.S == 1 && units > cap && parts >= 2 && n_hb >= parts && forced <= 0) {
        best.S = parts;
        best.grid = (int)(cap + parts * (units - cap));
        best.halves = cap;
    }
    const size_t a = (size_t)best.C_hb * 8 * MRB * 16 * 2, r = gemv_red_bytes(MRB);
    best.lds = kWaves * kStageBytes + (a > r ? a : r);
    return best;
}

// Split count S (a divisor of the input's 128-blocks; for an input of a
// multiple of 4 blocks, one leaving a multiple of 4 per split, so that every
// chunk streams whole kDepth-row blocks) of the persistent launch minimising
// the modelled time: one fixed latency, then the most loaded workgroup's
// units (ceil(units / resident)) at rows x row time plus the unit's
// reduction and restages, plus the consumer's per-split cost.  Items are row
// groups x streamed projections: est_items the expected count, max_items
// the bound the grid is sized for (they differ for the MoE phases).  The
// persistent kernel pays off once a workgroup holds many units (it balances
// the load and keeps the pipeline warm across them; a unit switch still
// costs about a memory round trip); below kMinUnitsPerWg the
// one-unit-per-workgroup plan (wg_items = slots x streamed projections) is
// used.
// Kernel choice override for testing and tuning: EXL3_GEMV_KERNEL=wg or
// =persistent forces that kernel for every GEMV phase; unset or any other
// value selects by the cost model.  Read on every plan (host side, once per
// call), so a process can compare both kernels on the same inputs.
inline int gemv_kernel_policy() {
    const char* v = std::getenv("EXL3_GEMV_KERNEL");
    if (!v) return 0;
    if (std::strcmp(v, "wg") == 0) return 1;
    if (std::strcmp(v, "persistent") == 0) return 2;
    return 0;
}

inline PhasePlan plan_phase(int in_f, int out_f, int est_items, int max_items, int wg_items, int MRB,
                            bool moe = false) {
    const int policy = gemv_kernel_policy();
    if (policy == 1) return plan_phase_wg(in_f, out_f, wg_items, MRB, moe);
    const int n_hb = in_f / 128, n_j = out_f / 128;
    const int cap = resident_workgroups();
    PhasePlan best = {1, n_hb, pick_chunk(n_hb, MRB), 1, 0, 0};
    double best_t = 1e30;
    int64_t best_per_wg = 0;
    const int forced = gemv_forced_splits();
    for (int S = 1; S <= kMaxSplits && S <= n_hb; ++S) {
        if (n_hb % S) continue;
        const int R_hb = n_hb / S;
        if (n_hb % 4 == 0 && R_hb % 4 != 0) continue;
        if (forced > 0 && S != forced && n_hb % forced == 0 && (n_hb % 4 != 0 || (n_hb / forced) % 4 == 0))
            continue;
        const int C_hb = pick_chunk(R_hb, MRB);
        const int nc = (R_hb + C_hb - 1) / C_hb;
        const int64_t units = (int64_t)est_items * n_j * S;
        const int64_t units_max = (int64_t)max_items * n_j * S;
        const int grid = (int)(units_max < cap ? units_max : cap);
        const int64_t per_wg = (units + grid - 1) / grid;
        const double t = kWgFixedUs +
                         per_wg * (R_hb * 8.0 / kWaves * kRowUs + kUnitUs + (nc > 1 ? nc * kStageUs : 0.0)) +
                         S * kSplitUs;
        if (t < best_t) {
            best_t = t;
            best_per_wg = per_wg;
            best = {S, R_hb, C_hb, grid, 0, 0};
        }
    }
    if (policy != 2 && best_per_wg < kMinUnitsPerWg) return plan_phase_wg(in_f, out_f, wg_items, MRB, moe);
    best.lds = gemv_lds_bytes(best.C_hb, MRB);
    return best;
}

// EXL3_MOE_ROUTE_ROTATE=0 keeps routing and the input rotation in separate
// launches (for comparisons; read on every call).
// EXL3_MOE_INLINE_ROUTE=0 keeps the routing launch for decode steps of at
// most 64 routes (whose gate/up GEMV otherwise routes the step itself).
inline bool moe_inline_route_allowed() {
    const char* v = std::getenv("EXL3_MOE_INLINE_ROUTE");
    return !(v && std::strcmp(v, "0") == 0);
}
constexpr int kInlineRouteMax = 64;     // routes one wave holds
constexpr int kInlineRouteBlocks = 4;   // input blocks per gate/up workgroup

inline bool moe_route_rotate_allowed() {
    const char* v = std::getenv("EXL3_MOE_ROUTE_ROTATE");
    return !(v && v[0] == '0');
}

struct MoePlan {
    int n_routes, max_slots, max_groups, MRB, nproj;
    PhasePlan gu, dn;
    size_t off_route, off_aux, off_wsgu, off_wsd, off_img, off_imgd, total;
};

inline MoePlan plan_moe(int64_t T, int64_t topk, int64_t n_local, int64_t hidden, int64_t inter,
                        int gateless) {
    MoePlan m;
    m.n_routes = (int)(T * topk);
    m.max_slots = (int)(m.n_routes < n_local ? m.n_routes : n_local);
    // a routing slot rarely holds more than 8 of the T rows at decode; larger
    // slots run extra row groups (the weights are streamed once per group)
    m.MRB = (int)(T < kMoeMRB ? (T < 1 ? 1 : T) : kMoeMRB);
    m.nproj = gateless ? 1 : 2;
    // row groups: sum over slots of ceil(rows / MRB) <= routes, and
    // <= (routes + slots * (MRB - 1)) / MRB
    {
        const int64_t a = m.n_routes, b = (m.n_routes + (int64_t)m.max_slots * (m.MRB - 1)) / m.MRB;
        m.max_groups = (int)(a < b ? a : b);
    }
    // the planner's work estimate: about one group per routed slot at decode
    const int64_t est = m.n_routes / m.MRB > m.max_slots ? m.n_routes / m.MRB : m.max_slots;
    const int est_groups = (int)(est < m.max_groups ? est : m.max_groups);
    m.gu = plan_phase((int)hidden, (int)inter, est_groups * m.nproj, m.max_groups * m.nproj,
                      m.max_slots * m.nproj, m.MRB, true);
    m.dn = plan_phase((int)inter, (int)hidden, est_groups, m.max_groups, m.max_slots, m.MRB, true);
    size_t off = 0;
    m.off_route = off;
    off += align256(sizeof(int) * (3 + 3 * (size_t)m.max_slots + 3 * (size_t)m.n_routes +
                                   3 * (size_t)m.max_groups));
    m.off_aux = off;  // sorted row -> route [routes]
    off += align256(sizeof(int) * (size_t)m.n_routes);
    m.off_wsgu = off;
    off += align256(4 * (size_t)m.nproj * m.gu.S * m.n_routes * inter);
    m.off_wsd = off;
    off += align256(4 * (size_t)m.dn.S * m.n_routes * hidden);
    m.off_img = off;  // rotated gate/up input rows [nproj][routes][hidden] fp16
    off += align256(2 * (size_t)m.nproj * m.n_routes * hidden);
    m.off_imgd = off;  // down input rows [routes][inter] fp16
    off += align256(2 * (size_t)m.n_routes * inter);
    m.total = off;
    return m;
}

struct LinPlan {
    int MRB;
    PhasePlan ph;
    size_t off_img, total;
};

// Up to kRawRows rows the linear GEMV's workgroups rotate their own input
// blocks while staging them (no rotation launch, no image in HBM); more rows
// are rotated once by rotate_rows_kernel, since every column block would
// repeat the rotation.  EXL3_LINEAR_RAW=0 keeps the rotation launch
// (tuning and tests; read on every call).
constexpr int64_t kRawRows = 4;

inline bool linear_raw_rows(int64_t m) {
    const char* v = std::getenv("EXL3_LINEAR_RAW");
    if (v && std::strcmp(v, "0") == 0) return false;
    return m <= kRawRows;
}

inline LinPlan plan_linear(int64_t m, int64_t in_f, int64_t out_f) {
    LinPlan lp;
    lp.MRB = (int)(m < kMaxMRB ? m : kMaxMRB);
    const int groups = (int)((m + lp.MRB - 1) / lp.MRB);
    lp.ph = plan_phase((int)in_f, (int)out_f, groups, groups, 1, lp.MRB);
    // [split partials (S > 1)][rotated input rows, fp16]
    lp.off_img = lp.ph.S > 1 ? align256(4 * (size_t)lp.ph.S * m * out_f) : 0;
    lp.total = lp.off_img + align256(2 * (size_t)m * in_f);
    return lp;
}

template <int CB, int MODE>
hipError_t launch_wg(int grid, size_t lds, hipStream_t st, const GemvParams& p) {
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)gemv_wg_kernel<CB, MODE>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e != hipSuccess) (void)hipGetLastError();
        return e;
    }();
    if (attr != hipSuccess) return attr;
    gemv_wg_kernel<CB, MODE><<<grid, kThreads, lds, st>>>(p);
    return hipGetLastError();
}

// One GEMV instance: its dynamic-LDS cap is raised once (well below the
// 160 KB per workgroup; the launches stay under 54 KB), then it is launched.
template <int CB, int MODE, int LK>
hipError_t launch_one(int grid, size_t lds, hipStream_t st, const GemvParams& p) {
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)gemv_kernel<CB, MODE, LK>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e != hipSuccess) (void)hipGetLastError();  // do not leave a sticky error behind
        return e;
    }();
    if (attr != hipSuccess) return attr;
    gemv_kernel<CB, MODE, LK><<<grid, kThreads, lds, st>>>(p);
    return hipGetLastError();
}

// lk: the launch's uniform bit width (lane-linear stage layout), or 0 for a
// mixed-K MoE phase (per-expert K, padded stage layout).
template <int MODE, int CB>
hipError_t launch_lk(int lk, int grid, size_t lds, hipStream_t st, const GemvParams& p) {
    switch (lk) {
        case 2: return launch_one<CB, MODE, 2>(grid, lds, st, p);
        case 3: return launch_one<CB, MODE, 3>(grid, lds, st, p);
        case 4: return launch_one<CB, MODE, 4>(grid, lds, st, p);
        default:
            if constexpr (MODE == kModeGateUp || MODE == kModeDown) return launch_one<CB, MODE, 0>(grid, lds, st, p);
            return hipErrorInvalidValue;
    }
}

template <int MODE>
hipError_t launch_gemv(int cb, int lk, const PhasePlan& ph, hipStream_t st, const GemvParams& p) {
    const int grid = ph.grid;
    const size_t lds = ph.lds;
    if (ph.wg) {
        switch (cb) {
            case 0: return launch_wg<0, MODE>(grid, lds, st, p);
            case 1: return launch_wg<1, MODE>(grid, lds, st, p);
            default: return launch_wg<2, MODE>(grid, lds, st, p);
        }
    }
    switch (cb) {
        case 0: return launch_lk<MODE, 0>(lk, grid, lds, st, p);
        case 1: return launch_lk<MODE, 1>(lk, grid, lds, st, p);
        default: return launch_lk<MODE, 2>(lk, grid, lds, st, p);
    }
}

// The units of a mixed-K MoE phase whose K is outside {2, 3, 4}: one
// workgroup per (slot, streamed projection, kAnyKBlocks 128-column blocks).
template <int MODE>
hipError_t launch_anyk(int cb, int max_slots, int nq, hipStream_t st, const GemvParams& p) {
    const int64_t grid = (int64_t)max_slots * nq * (((p.out_features >> 7) + kAnyKBlocks - 1) / kAnyKBlocks);
    if (grid < 1 || grid > 0x7FFFFFFF) return hipErrorInvalidValue;
    switch (cb) {
        case 0: gemv_anyk_kernel<0, MODE><<<(unsigned)grid, kThreads, 0, st>>>(p); break;
        case 1: gemv_anyk_kernel<1, MODE><<<(unsigned)grid, kThreads, 0, st>>>(p); break;
        default: gemv_anyk_kernel<2, MODE><<<(unsigned)grid, kThreads, 0, st>>>(p); break;
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace exl3

using namespace exl3;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
// Rows from which the dense linear takes the fat path; EXL3_LINEAR_FAT_MIN_ROWS
// overrides the measured default (for testing and tuning; read on every call,
// by the workspace query and the launch alike).
static int64_t linear_fat_min_rows() {
    const char* v = std::getenv("EXL3_LINEAR_FAT_MIN_ROWS");
    if (v && *v) {
        const long long r = std::atoll(v);
        if (r >= 1) return r;
    }
    return kLinearFatMinRows;
}

EXL3_API int64_t exl3_gemm_workspace_size(int64_t m, int64_t in_features, int64_t out_features) {
    if (m < 1 || in_features < 128 || out_features < 128) return 0;
    if (m >= linear_fat_min_rows()) return (int64_t)linear_fat_workspace_bytes(m, in_features, out_features);
    return (int64_t)plan_linear(m, in_features, out_features).total;
}

EXL3_API int exl3_linear(const void* x, int x_dtype, int64_t m, const int16_t* trellis,
                         int64_t tiles_k, int64_t tiles_n, int64_t K, int codebook,
                         const uint16_t* suh, const uint16_t* svh, const void* bias, int bias_dtype,
                         void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                         void* stream) {
    EXL3_CHECK(K == 2 || K == 3 || K == 4, "exl3_gemm supports K in {2, 3, 4}");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(x_dtype >= 0 && x_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2 &&
                   (!bias || (bias_dtype >= 0 && bias_dtype <= 2)),
               "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(m >= 1 && m <= (1 << 26), "exl3_gemm needs 1 <= m <= 2^26");
    EXL3_CHECK(tiles_k > 0 && tiles_n > 0 && (tiles_k * 16) % 128 == 0 && (tiles_n * 16) % 128 == 0,
               "trellis dimensions must reconstruct whole 128-element Hadamard blocks");
    EXL3_CHECK(tiles_k * 16 <= (1 << 20) && tiles_n * 16 <= (1 << 20), "feature dimensions too large");
    EXL3_CHECK(x && trellis && suh && svh && out, "null pointer argument");
    EXL3_CHECK(tiles_k * tiles_n * 32 * K < (1ll << 31), "packed trellis must be smaller than 2 GiB");
    const int64_t in_f = tiles_k * 16, out_f = tiles_n * 16;
    const int64_t need = exl3_gemm_workspace_size(m, in_f, out_f);
    EXL3_CHECK(workspace_bytes >= need && workspace, "workspace too small: need %lld bytes",
               (long long)need);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (m >= linear_fat_min_rows())
        return linear_fat(x, x_dtype, m, trellis, tiles_k, tiles_n, K, codebook, suh, svh, bias, bias_dtype,
                          out, out_dtype, workspace, st);
    const LinPlan lp = plan_linear(m, in_f, out_f);
    uint16_t* img = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(workspace) + lp.off_img);
    RotateArgs ra = {};
    ra.x = x;
    ra.x_dtype = x_dtype;
    ra.x_stride = in_f;
    ra.in_f = (int)in_f;
    ra.n_rows = (int)m;
    ra.suh = suh;
    ra.nproj = 1;
    ra.img[0] = img;
    GemvParams p = {};
    p.x = img;
    p.x_dtype = kF16;
    p.x_stride = in_f;
    p.w_trellis = trellis;
    p.w_suh = suh;
    p.w_svh = svh;
    p.kuni[0] = (int)K;
    p.in_features = (int)in_f;
    p.out_features = (int)out_f;
    p.m_rows = (int)m;
    p.max_groups = (int)((m + lp.MRB - 1) / lp.MRB);
    p.out = out;
    p.out_dtype = out_dtype;
    p.out_stride = out_f;
    p.bias = bias;
    p.bias_dtype = bias_dtype;
    p.S = lp.ph.S;
    p.R_hb = lp.ph.R_hb;
    p.C_hb = lp.ph.C_hb;
    p.MRB = lp.MRB;
    p.n_rows_ws = (int)m;
    p.ws = reinterpret_cast<float*>(workspace);
    profile_begin_call();
    profile_mark(0, st);
    const bool raw = linear_raw_rows(m) && lp.ph.wg;  // the one-unit kernel stages raw rows
    if (raw) {
        p.x = x;
        p.x_dtype = x_dtype;
        p.x_raw = 1;
    } else {
        launch_rotate(ra, st);
        EXL3_LAUNCHED();
    }
    profile_mark(1, st);
    EXL3_HIP(launch_gemv<kModeLinear>(codebook, (int)K, lp.ph, st, p));
    profile_mark(2, st);
    if (lp.ph.S > 1) {
        const int items = (int)(m * (out_f / 128));
        FinishBatch fb = {};
        fb.bias = bias;
        fb.bias_dtype = bias_dtype;
        linear_finish_kernel<<<(items + 3) / 4, 256, 0, st>>>(p.ws, lp.ph.S, (int)m, (int)out_f, svh,
                                                              out, out_dtype, fb);
        EXL3_LAUNCHED();
        profile_mark(3, st);
    }
    return kOk;
}

EXL3_API int exl3_gemm(const void* x, int x_dtype, int64_t m, const int16_t* trellis,
                       int64_t tiles_k, int64_t tiles_n, int64_t K, int codebook,
                       const uint16_t* suh, const uint16_t* svh, void* out, int out_dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
    return exl3_linear(x, x_dtype, m, trellis, tiles_k, tiles_n, K, codebook, suh, svh, nullptr, 0, out,
                       out_dtype, workspace, workspace_bytes, stream);
}

struct BatchPlan {
    int MRB;
    PhasePlan ph;
    size_t off_img, total;
};

inline BatchPlan plan_batched(int64_t m, int64_t n_sel, int64_t in_f, int64_t out_f) {
    BatchPlan bp;
    bp.MRB = (int)(m < kMaxMRB ? m : kMaxMRB);
    const int groups = (int)(n_sel * ((m + bp.MRB - 1) / bp.MRB));
    bp.ph = plan_phase((int)in_f, (int)out_f, groups, groups, (int)n_sel, bp.MRB);
    // [split partials (S > 1)][rotated input rows per slot, fp16]
    bp.off_img = bp.ph.S > 1 ? align256(4 * (size_t)bp.ph.S * n_sel * m * out_f) : 0;
    bp.total = bp.off_img + align256(2 * (size_t)n_sel * m * in_f);
    return bp;
}

EXL3_API int64_t exl3_gemv_batched_workspace_size(int64_t m, int64_t n_sel, int64_t in_features,
                                                  int64_t out_features) {
    if (m < 1 || n_sel < 1 || in_features < 128 || out_features < 128) return 0;
    return (int64_t)plan_batched(m, n_sel, in_features, out_features).total;
}

EXL3_API int exl3_gemv_batched(const void* x, int x_dtype, int64_t m, int64_t in_features,
                               int64_t out_features, const int64_t* trellis_tab,
                               const int64_t* suh_tab, const int64_t* svh_tab, int64_t n_ptr,
                               const int32_t* expert_indices, int64_t n_sel, int64_t K, int codebook,
                               void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                               void* stream) {
    EXL3_CHECK(K == 2 || K == 3 || K == 4, "batched GEMV supports K=2,3,4");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(x_dtype >= 0 && x_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
               "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(m >= 1 && n_sel >= 1 && n_ptr >= 1 && n_sel * m <= (1 << 24),
               "batched GEMV needs m >= 1, at least one expert index and one table entry");
    EXL3_CHECK(in_features % 128 == 0 && out_features % 128 == 0 && in_features > 0 && out_features > 0 &&
                   in_features <= (1 << 20) && out_features <= (1 << 20),
               "batched GEMV feature dimensions must be positive multiples of 128");
    EXL3_CHECK(in_features * out_features / 16 * K / 8 * 16 < (1ll << 31),
               "packed trellis must be smaller than 2 GiB");
    EXL3_CHECK(x && trellis_tab && suh_tab && svh_tab && expert_indices && out,
               "null pointer argument");
    const BatchPlan bp = plan_batched(m, n_sel, in_features, out_features);
    EXL3_CHECK(workspace && workspace_bytes >= (int64_t)bp.total,
               "workspace too small: need %zu bytes", bp.total);
    uint16_t* img = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(workspace) + bp.off_img);
    RotateArgs ra = {};
    ra.x = x;
    ra.x_dtype = x_dtype;
    ra.x_stride = in_features;
    ra.in_f = (int)in_features;
    ra.n_rows = (int)(n_sel * m);
    ra.suh_tab[0] = suh_tab;
    ra.nproj = 1;
    ra.img[0] = img;
    ra.expert_list = expert_indices;
    ra.batch_m = (int)m;
    ra.n_ptr = (int)n_ptr;
    GemvParams p = {};
    p.x = img;
    p.x_dtype = kF16;
    p.x_stride = in_features;
    p.tab[0] = trellis_tab;
    p.tab[1] = suh_tab;
    p.tab[2] = svh_tab;
    p.kuni[0] = (int)K;
    p.in_features = (int)in_features;
    p.out_features = (int)out_features;
    p.max_slots = (int)n_sel;
    p.max_groups = (int)(n_sel * ((m + bp.MRB - 1) / bp.MRB));
    p.expert_list = expert_indices;
    p.n_ptr = (int)n_ptr;
    p.batch_m = (int)m;
    p.out = out;
    p.out_dtype = out_dtype;
    p.out_stride = out_features;
    p.S = bp.ph.S;
    p.R_hb = bp.ph.R_hb;
    p.C_hb = bp.ph.C_hb;
    p.MRB = bp.MRB;
    p.n_rows_ws = (int)(n_sel * m);
    p.ws = reinterpret_cast<float*>(workspace);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    launch_rotate(ra, st);
    EXL3_LAUNCHED();
    EXL3_HIP(launch_gemv<kModeBatched>(codebook, (int)K, bp.ph, st, p));
    if (bp.ph.S > 1) {
        const int64_t items = n_sel * m * (out_features / 128);
        FinishBatch fb{svh_tab, expert_indices, (int)m, (int)n_ptr};
        linear_finish_kernel<<<(unsigned)((items + 3) / 4), 256, 0, st>>>(
            p.ws, bp.ph.S, (int)(n_sel * m), (int)out_features, nullptr, out, out_dtype, fb);
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
    EXL3_CHECK(n_local >= 1 && n_local < (1 << 18), "fused MoE n_local must be in [1, 2^18)");
    const int64_t max_routes = n_local <= kRouteMaxLocal ? kMaxRoutesMultisplit : kMaxRoutes;
    EXL3_CHECK(T >= 1 && topk >= 1 && T * topk <= max_routes,
               "fused MoE decode supports 1 <= T*topk <= %lld routes with %lld local experts",
               (long long)max_routes, (long long)n_local);
    EXL3_CHECK(topk <= kMaxTopk, "fused MoE supports topk <= %d", kMaxTopk);
    EXL3_CHECK(hidden > 0 && hidden % 128 == 0,
               "fused MoE hidden width must be a positive multiple of 128");
    EXL3_CHECK(inter > 0 && inter % 128 == 0,
               "fused MoE local intermediate width must be a positive multiple of 128");
    EXL3_CHECK(hidden <= (1 << 20) && inter <= (1 << 20), "fused MoE dimensions too large");
    EXL3_CHECK(hidden * inter / 2 < (1ll << 31), "fused MoE expert projections must pack below 2 GiB");
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
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);

    profile_begin_call();
    profile_mark(0, st);
    RouteOut ro = {};
    int* rbase = reinterpret_cast<int*>(ws + mp.off_route);
    ro.n_active = rbase;
    ro.slot_expert = rbase + 1;
    ro.slot_start = ro.slot_expert + mp.max_slots;
    ro.slot_rows = ro.slot_start + mp.max_slots;
    ro.row_token = ro.slot_rows + mp.max_slots;
    ro.row_expert = ro.row_token + mp.n_routes;
    ro.route_pos = ro.row_expert + mp.n_routes;
    ro.n_mtiles = ro.route_pos + mp.n_routes;  // row groups of MRB rows
    ro.mt_slot = ro.n_mtiles + 1;
    ro.mt_row0 = ro.mt_slot + mp.max_groups;
    ro.mt_expert = ro.mt_row0 + mp.max_groups;
    ro.n_sorted = ro.mt_expert + mp.max_groups;  // kept routes: the sorted rows act_rows_kernel walks
    const int64_t* tabs[9] = {gateless ? up_trellis : gate_trellis, gateless ? up_suh : gate_suh,
                              gateless ? up_svh : gate_svh, up_trellis, up_suh, up_svh,
                              down_trellis, down_suh, down_svh};
    uint16_t* img_gu = reinterpret_cast<uint16_t*>(ws + mp.off_img);
    uint16_t* img_gu1 = img_gu + (size_t)mp.n_routes * hidden;
    // Route and rotate in one launch when the gate/up GEMV stages its rows
    // through the sorted row -> route map (one unit per workgroup, uniform K).
    // Decode steps of at most 64 routes whose gate/up workgroups stream at
    // most kInlineRouteBlocks input blocks each: the gate/up GEMV routes the
    // step in every workgroup and rotates its rows from x (no routing
    // launch; with longer splits every column block repeating the rotation
    // costs more than the launch, C1 T = 4 +1.5 µs against T = 1 -3 µs).
    const bool inline_route = moe_inline_route_allowed() && mp.gu.wg && mp.n_routes <= kInlineRouteMax &&
                              mp.gu.R_hb <= kInlineRouteBlocks && n_local <= kRouteMaxLocal && !kt[0] &&
                              !kt[1];
    const bool route_rotate = !inline_route && moe_route_rotate_allowed() && mp.gu.wg &&
                              n_local <= kRouteMaxLocal && !kt[0] && !kt[1];
    if (inline_route) {
        ro.row_route = reinterpret_cast<int*>(ws + mp.off_aux);
    } else if (route_rotate) {
        static const hipError_t attr = [] {
            hipError_t e = hipFuncSetAttribute((const void*)route_rotate_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)route_lds_bytes(kRouteMaxLocal));
            if (e != hipSuccess) (void)hipGetLastError();
            return e;
        }();
        EXL3_HIP(attr);
        ro.row_route = reinterpret_cast<int*>(ws + mp.off_aux);
        RouteRotateArgs f = {};
        f.ids = ids;
        f.ids_i64 = (int)ids_dtype;
        f.n_routes = mp.n_routes;
        f.topk = (int)topk;
        f.n_local = (int)n_local;
        f.T = (int)T;
        f.tile_rows = mp.MRB;
        f.n_valid = n_valid;
        f.x = x;
        f.x_dtype = (int)x_dtype;
        f.hidden = (int)hidden;
        f.suh_tab0 = tabs[1];
        f.suh_tab1 = tabs[4];
        f.nproj = mp.nproj;
        f.img0 = img_gu;
        f.img1 = img_gu1;
        f.ro = ro;
        const int64_t units = (int64_t)mp.n_routes * (hidden / 128);
        const int64_t rot_blocks = std::min<int64_t>((units + kRouteThreads / 64 - 1) / (kRouteThreads / 64), 1024);
        route_rotate_kernel<<<(unsigned)(1 + rot_blocks), kRouteThreads, route_lds_bytes((int)n_local), st>>>(f);
        EXL3_LAUNCHED();
    } else if (n_local <= kRouteMaxLocal) {
        EXL3_HIP(launch_route(ids, ids_dtype, mp.n_routes, (int)topk, (int)n_local, n_valid, mp.MRB, ro,
                              st));
    } else {
        route_bitonic_kernel<<<1, kRouteThreads, 0, st>>>(ids, ids_dtype, mp.n_routes, (int)topk,
                                                          (int)n_local, n_valid, mp.MRB, ro);
        EXL3_LAUNCHED();
    }

    GemvParams p = {};
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
    p.n_groups = ro.n_mtiles;
    p.group_slot = ro.mt_slot;
    p.group_row0 = ro.mt_row0;
    p.group_expert = ro.mt_expert;
    p.max_groups = mp.max_groups;
    p.max_slots = mp.max_slots;
    p.MRB = mp.MRB;
    p.n_rows_ws = mp.n_routes;
    p.limit = swiglu_limit;
    p.act = act;
    float* ws_gu = reinterpret_cast<float*>(ws + mp.off_wsgu);
    float* ws_d = reinterpret_cast<float*>(ws + mp.off_wsd);
    uint16_t* img_d = reinterpret_cast<uint16_t*>(ws + mp.off_imgd);

    // gate/up input rows, rotated once per route and projection
    profile_mark(1, st);
    if (!route_rotate && !inline_route) {
        RotateArgs ra = {};
        ra.x = x;
        ra.x_dtype = x_dtype;
        ra.x_stride = hidden;
        ra.in_f = (int)hidden;
        ra.n_rows = mp.n_routes;
        ra.route_pos = ro.route_pos;
        ra.topk = (int)topk;
        ra.row_expert = ro.row_expert;
        ra.suh_tab[0] = tabs[1];
        ra.suh_tab[1] = tabs[4];
        ra.nproj = mp.nproj;
        ra.img[0] = img_gu;
        ra.img[1] = img_gu1;
        launch_rotate(ra, st);
        EXL3_LAUNCHED();
    }

    // gate/up: raw partial sums [nproj][S_gu][routes][inter]
    GemvParams pg = p;
    pg.x = img_gu;
    pg.x2 = img_gu1;
    pg.row_map = route_rotate ? ro.row_route : nullptr;
    pg.x_dtype = kF16;
    pg.x_stride = hidden;
    if (inline_route) {
        pg.x = x;
        pg.x2 = x;
        pg.x_dtype = x_dtype;
        pg.x_raw = 1;
        pg.inline_route = 1;
        pg.r_ids = ids;
        pg.r_ids_i64 = (int)ids_dtype;
        pg.r_n_routes = mp.n_routes;
        pg.r_topk = (int)topk;
        pg.r_n_local = (int)n_local;
        pg.r_n_valid = n_valid;
        pg.ro = ro;
    }
    pg.in_features = (int)hidden;
    pg.out_features = (int)inter;
    pg.S = mp.gu.S;
    pg.R_hb = mp.gu.R_hb;
    pg.C_hb = mp.gu.C_hb;
    pg.tail_halves = mp.gu.halves;
    pg.ws = ws_gu;
    profile_mark(2, st);
    // uniform K over the streamed projections: the lane-linear stage layout
    const int lk_gu = gateless ? (kt[1] ? 0 : (int)Ks[1])
                               : ((!kt[0] && !kt[1] && Ks[0] == Ks[1]) ? (int)Ks[0] : 0);
    EXL3_HIP(launch_gemv<kModeGateUp>(codebook, lk_gu, mp.gu, st, pg));
    if ((!gateless && kt[0]) || kt[1]) EXL3_HIP(launch_anyk<kModeGateUp>(codebook, mp.max_slots, mp.nproj, st, pg));

    // down input rows: gate/up finished once per route
    GemvParams pd = p;
    pd.src_ws = ws_gu;
    pd.src_S = mp.gu.S;
    pd.in_features = (int)inter;
    pd.out_features = (int)hidden;
    pd.S = mp.dn.S;
    pd.R_hb = mp.dn.R_hb;
    pd.C_hb = mp.dn.C_hb;
    pd.tail_halves = mp.dn.halves;
    pd.ws = ws_d;
    pd.x = img_d;
    pd.x_dtype = kF16;
    pd.x_stride = inter;
    profile_mark(3, st);
    const int64_t act_units = (int64_t)mp.n_routes * (inter / 128);
    act_rows_kernel<<<(unsigned)((act_units + 3) / 4), 256, 0, st>>>(pd, mp.n_routes, ro.n_sorted,
                                                                     ro.row_expert, img_d);
    EXL3_LAUNCHED();

    // down: raw partials [S_d][routes][hidden]
    profile_mark(4, st);
    EXL3_HIP(launch_gemv<kModeDown>(codebook, kt[2] ? 0 : (int)Ks[2], mp.dn, st, pd));
    if (kt[2]) EXL3_HIP(launch_anyk<kModeDown>(codebook, mp.max_slots, 1, st, pd));

    profile_mark(5, st);
    combine_kernel<<<(int)(T * (hidden / 128)), kCombineWaves * 64, 0, st>>>(
        ws_d, mp.dn.S, mp.n_routes, (int)hidden, ro.route_pos, ro.row_expert, down_svh, weights,
        w_dtype, (int)topk, out, out_dtype);
    EXL3_LAUNCHED();
    profile_mark(6, st);
    return kOk;
}

// ---------------------------------------------------------------------------
// Decode MoE step without a caller workspace, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  The workspace of exl3_moe_forward comes from `scratch`,
// a file-scope device array that every GPU the library runs on holds until
// the process ends.  In host code the array's name is only a stand-in: its
// device address, one per device, comes from hipGetSymbolAddress at the
// first call on that device and is the only handle passed to kernels.  The
// workspace needs no clearing (every element a kernel reads was written
// earlier in the same call, in stream order), so calls that follow each other
// on one stream may reuse it; calls that overlap on one GPU (other streams,
// other threads) race on it.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on the current device.
int scratch_ptr(void** out) {
    int dev = -1;
    EXL3_HIP(hipGetDevice(&dev));
    EXL3_CHECK(dev >= 0 && dev < kMaxScratchDevices, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        EXL3_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        EXL3_CHECK(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}
}  // namespace

EXL3_API int exl3_moe_forward_noalloc(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
                                      const int64_t* gate_trellis, const int64_t* gate_suh,
                                      const int64_t* gate_svh, const int64_t* up_trellis,
                                      const int64_t* up_suh, const int64_t* up_svh,
                                      const int64_t* down_trellis, const int64_t* down_suh,
                                      const int64_t* down_svh, int64_t n_local, const int8_t* k_gate,
                                      const int8_t* k_up, const int8_t* k_down, int64_t K_gate,
                                      int64_t K_up, int64_t K_down, int codebook, int gateless, int act,
                                      float swiglu_limit, const void* ids, int ids_dtype,
                                      const void* weights, int w_dtype, int64_t topk,
                                      const int32_t* n_valid, void* out, int out_dtype, void* stream) {
    const int64_t need = exl3_moe_workspace_size(T, topk, n_local, hidden, inter, gateless);
    EXL3_CHECK(need <= (int64_t)kNoAllocScratchBytes,
               "fused MoE without a workspace: this call needs %lld bytes of scratch, the library's "
               "scratch array holds %zu (call exl3_moe_forward with a workspace)",
               (long long)need, kNoAllocScratchBytes);
    void* ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc != kOk) return rc;
    // exl3_moe_forward validates every argument (need == 0 for a rejected geometry)
    return exl3_moe_forward(x, x_dtype, T, hidden, inter, gate_trellis, gate_suh, gate_svh, up_trellis,
                            up_suh, up_svh, down_trellis, down_suh, down_svh, n_local, k_gate, k_up,
                            k_down, K_gate, K_up, K_down, codebook, gateless, act, swiglu_limit, ids,
                            ids_dtype, weights, w_dtype, topk, n_valid, out, out_dtype, ws,
                            (int64_t)kNoAllocScratchBytes, stream);
}
