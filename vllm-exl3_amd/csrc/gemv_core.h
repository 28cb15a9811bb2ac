// Streaming EXL3 decode-GEMV core for gfx950 (small row counts: decode).
//
// A unit of work is one 128-column block of one projection over a K-split
// range of input rows for one row group (up to MRB activation rows of one
// routing slot, or of the plain linear).  Two kernels stream units (gemv.hip):
// one unit per workgroup for launches that fill at most a couple of rounds
// of resident workgroups, and a persistent kernel that streams a contiguous
// range of units per workgroup with the trellis pipeline kept full across
// them.  Per wave, per tile row (8 packed 16x16 tiles = 256*K contiguous
// bytes):
//   * one coalesced 128-bit load per lane (a scalar buffer resource for the
//     wave's rows, the row advance as the scalar offset) into registers,
//     software pipelined kDepth rows ahead, then one ds_write_b128 into the
//     wave's LDS slot (no workgroup barrier in the main loop);
//   * each lane reads the two uint32 words that cover the windows of its four
//     consecutive tile indices, funnel-shifts them once, and decodes four
//     weights with bfe / one full-rate 32-bit multiply / bitop3 each;
//   * the codebook's (lo, hi) half pair is fed to MFMA as-is: the K dimension
//     is doubled (each activation duplicated), so the hardware sums the two
//     halves in fp32 and no fp16 add, pack or permute is spent per weight;
//   * one v_mfma_f32_16x16x32_f16 per tile accumulates 16 rows x 16 columns.
// The MFMA row/column order inside a tile is a permutation of the reference's
// tile layout chosen so that every lane's four weights are consecutive tile
// indices (one word pair per lane per tile); activations are staged in LDS in
// the matching permuted, duplicated order, and results are un-permuted when
// they leave the accumulators.
//
// Split-K partials go to a workspace and the consumer kernel sums them in
// split order and runs the epilogue: output 128-Hadamard x svh, and after the
// MoE gate/up phase the activation plus the down projection's input rotation.
// Activations arrive pre-rotated (one rotation per row, not per workgroup).
#pragma once

#include "exl3_common.h"
#include "route.h"

namespace exl3 {

enum GemvMode : int { kModeLinear = 0, kModeGateUp = 1, kModeDown = 2, kModeBatched = 3 };
// Activation ids follow the reference (src/vllm_exl3/exl3.py MOE_ACT_*):
enum ActId : int { kActSilu = 0, kActRelu2 = 2, kActSwigluOai = 3 };
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
// Tile rows in flight per wave: kDepth in the persistent kernel, kWgDepth in
// the one-unit kernel.  Both kernels are VALU-bound while their waves are
// resident, so fewer rows in flight cost nothing there and shorten every
// workgroup's cold start: at a launch's first round all workgroups request
// their first rows at once (C1 T = 16 gate/up 58.4 -> 57.2 µs with 8 -> 4
// and 2, T = 1 step about -2 µs at 2; C3's persistent kernel is 2% faster at
// 4 and 8% slower at 2).
constexpr int kDepth = 4;
constexpr int kWgDepth = 2;
constexpr int kStageBytes = 1024;  // one tile row of 8 tiles at K <= 4

struct GemvParams {
    // Activations: rotated fp16 rows in the GEMV image order (see
    // rotate_rows_kernel), [rows][x_stride]; linear rows are the input rows,
    // MoE rows the sorted routes.  x2: the up projection's rows (gate/up).
    const void* x;
    const void* x2;
    int x_dtype;
    int64_t x_stride;
    // Weights.  Linear: direct pointers.  MoE: device pointer tables indexed
    // by expert id (gate t/su/sv, up t/su/sv, down t/su/sv).
    const int16_t* w_trellis;
    const uint16_t* w_suh;
    const uint16_t* w_svh;
    const int64_t* tab[9];
    const int8_t* ktab[3];  // per-expert K per projection (nullable)
    int kuni[3];            // uniform K per projection (when ktab is null)
    int gateless;
    int in_features, out_features;
    // Routing (MoE): filled on device by the route kernel.
    const int* n_active;
    const int* slot_expert;
    const int* slot_start;
    const int* slot_rows;
    const int* row_token;
    // Row groups of the slots (MRB rows each; the router's row tiles): the
    // persistent GEMV's units are (group, projection, split, column block).
    const int* n_groups;
    const int* group_slot;
    const int* group_row0;
    const int* group_expert;
    int max_groups;
    int max_slots;
    int m_rows;  // linear: number of rows
    // Batched (one linear per listed expert, same input rows): the expert of
    // each slot, the table size (ids outside [0, n_ptr) give zero outputs)
    // and the rows per slot.
    const int* expert_list;
    int n_ptr;
    int batch_m;
    // Output.  Linear: out_dtype rows [m, out]; GateUp: fp16 act_h rows
    // [route_rows, inter] (already rotated for the down projection); Down:
    // fp32 rows [route_rows, hidden].
    void* out;
    int out_dtype;
    int64_t out_stride;
    // Split-K: raw partial sums go to ws[q][s][row][out_features]; they are
    // finished by the consumer kernel (the down kernel's activation staging,
    // the combine kernel, or the linear finish kernel), so no workgroup ever
    // waits on another and no device-scope fence is needed.
    int S;         // splits of the input dimension
    int R_hb;      // 128-row Hadamard blocks per split
    int C_hb;      // Hadamard blocks whose activations are staged at once
    int MRB;       // rows per row group (<= 16)
    int n_rows_ws; // rows addressed in the workspace (route rows or m)
    float* ws;
    // Linear mode: optional bias [out_features] (bias_dtype as x_dtype ids),
    // added after the output rotation.
    const void* bias;
    int bias_dtype;
    // GateUp mode, one unit per workgroup: sorted row -> activation image row
    // (images written in route order by the combined route + rotate launch);
    // null: the image rows are the sorted rows.
    const int* row_map;
    // Down mode: gate/up raw partials to finish while staging activations.
    const float* src_ws;
    int src_S;
    float limit;
    int act;
    // Linear mode, one unit per workgroup and one split: x holds the raw
    // input rows (x_dtype) and each workgroup rotates the blocks it streams
    // into LDS itself (one launch: no image, no split partials).
    int x_raw;
    // One-unit-per-workgroup MoE phases whose units outnumber the resident
    // workgroups: the first tail_halves units run whole (workgroups 0 ..
    // tail_halves - 1, writing split slot 0 and zeros into slot 1), every
    // later unit as two halves of its input range (slots 0 and 1), so the
    // workgroups that start last are short.  S is 2; 0: plain splits.
    int tail_halves;
    // Gate/up of a decode step with at most 64 routes, one unit per
    // workgroup: every wave routes the step itself (ids -> stable order by
    // expert, as the router does) and rotates its rows from the raw input
    // (x_raw); workgroup 0 writes the router's tables (ro) for the kernels
    // that follow.  No routing launch.
    int inline_route;
    const void* r_ids;
    int r_ids_i64, r_n_routes, r_topk, r_n_local;
    const int32_t* r_n_valid;
    RouteOut ro;
};

// ---------------------------------------------------------------------------
// Lane geometry
// ---------------------------------------------------------------------------
// MFMA 16x16x32 f16 operands: lane l = nu + 16 g holds B'[8g..8g+7][nu] and
// A'[m = l % 16][8g..8g+7]; D[4g + i][nu] comes back in component i.
// Tile index bits b0..b7 map to (row, col) as row = b0|b3<<1|b4<<2|b1<<3,
// col = b5|b6<<1|b7<<2|b2<<3.  Lane l decodes tile indices 4q(l)+i, i=0..3,
// which land at MFMA row kappa = 4g + i (tile row pi(kappa)) and MFMA column
// nu (tile column sigma(nu)).
__device__ __forceinline__ int lane_q(int l) {
    return (l & 1) | (((l >> 4) & 1) << 1) | (((l >> 5) & 1) << 2) | (((l >> 1) & 1) << 3) |
           (((l >> 2) & 1) << 4) | (((l >> 3) & 1) << 5);
}
// MFMA k-row kappa (0..15) -> tile row.
__device__ __forceinline__ int pi_row(int k) {
    return (k & 1) | (((k >> 2) & 1) << 1) | (((k >> 3) & 1) << 2) | (((k >> 1) & 1) << 3);
}
// tile row -> MFMA k-row kappa (inverse of pi_row).
__device__ __forceinline__ int pi_inv(int r) {
    return (r & 1) | (((r >> 3) & 1) << 1) | (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 3);
}
// MFMA column nu -> tile column.
__device__ __forceinline__ int sigma_col(int n) { return (n >> 1) | ((n & 1) << 3); }

// Per-lane geometry of a tile row at bit width K (computed when K changes).
// Stage layout LK: for a launch whose K is uniform (LK = K) the staged tile
// row is lane-linear, tile t at t*32K bytes (conflict-free writes, K-specific
// immediate read offsets); for mixed-K launches (LK = 0) each tile sits at a
// 128-byte slot of the 1 KB stage (a 32K-byte tile is a whole number of
// 16-byte pieces, so every lane's piece lies in one tile), so one loop serves
// every K.
struct LaneGeo {
    uint32_t voff;    // the lane's 16 bytes of the row (lanes past the 256K-byte span: 0)
    uint32_t wr;      // LDS offset of that piece in the stage (lanes past the span: 0, same bytes)
    uint32_t off_hi;  // byte offset (in a tile) of the word holding the earlier bits
    uint32_t off_lo;  // byte offset of the word holding the last bit
    uint32_t shift;   // funnel shift that puts the last window at bit 0
};

// Bytes between consecutive tiles of a staged tile row.
template <int LK>
__device__ __forceinline__ constexpr int stage_tile_stride() { return LK ? 32 * LK : 128; }

// The padded (LK = 0) layout's geometry from the lane id with no division
// (K uniform, 2..4): lane / 2K as a reciprocal multiply (exact for lane < 64),
// the modulo of the word index as a select.
__device__ __forceinline__ LaneGeo lane_geo_padded(int K, uint32_t lane) {
    LaneGeo g;
    const uint32_t pieces = 16u * K, per_tile = 2u * K;
    const uint32_t magic = K == 2 ? 64u : (K == 3 ? 43u : 32u);
    const uint32_t tl = (lane * magic) >> 8;
    const bool in = lane < pieces;
    g.voff = in ? lane * 16u : 0u;
    g.wr = in ? tl * 128u + (lane - tl * per_tile) * 16u : 0u;
    const int q = lane_q((int)lane);
    const int E = (4 * q + 4) * K;
    const int wb = (E - 1) >> 5;
    g.off_lo = 4u * wb;
    g.off_hi = 4u * (wb == 0 ? 8 * K - 1 : wb - 1);
    g.shift = 32u * (wb + 1) - E;
    return g;
}

template <int LK>
__device__ __forceinline__ LaneGeo lane_geo(int K, int lane) {
    LaneGeo g;
    const int pieces = 16 * K;  // 16-byte pieces per tile row (8 tiles of 32K bytes)
    g.voff = lane < pieces ? lane * 16 : 0;
    if constexpr (LK != 0) {
        g.wr = g.voff;
    } else {
        const int per_tile = 2 * K;
        g.wr = lane < pieces ? (lane / per_tile) * 128 + (lane % per_tile) * 16 : 0;
    }
    const int n32 = 8 * K;
    const int q = lane_q(lane);
    const int E = (4 * q + 4) * K;  // end (exclusive) of the lane's last window
    const int wb = (E - 1) >> 5;
    g.off_lo = 4u * wb;
    g.off_hi = 4u * ((wb + n32 - 1) % n32);
    g.shift = 32u * (wb + 1) - E;
    return g;
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// The codebook hash x = w*C (+ add for 3INST) mod 2^32 of one 16-bit window
// w (clean: bits above 15 zero).  On gfx950 the 32-bit multiply
// (v_mul_lo_u32) and the 64-bit multiply-add (v_mad_u64_u32, low half kept)
// issue at the full VALU rate, so the whole 32-bit product is one op.
// (The compiler splits a 64-bit multiply-add whose high half is unused into
// a multiply and an add, so the 3INST form is written as the instruction:
// the multiplier in an SGPR, the addend in a VGPR pair - one constant-bus
// read - and its result only feeds ordinary VALU ops.)
template <int CB>
__device__ __forceinline__ uint32_t hash32(uint32_t w) {
    if constexpr (CB == kCb3Inst) {
        const uint64_t r = (uint64_t)w * 89226354u + 64248484u;
        asm volatile("" ::"v"((uint32_t)(r >> 32)));  // keep the full product: one v_mad_u64_u32
        return (uint32_t)r;
    } else {
        return w * 0xCBAC1FEDu;
    }
}

// Decode the lane's four weights of one tile into MFMA B registers (each a
// (lo, hi) fp16 pair whose sum is the weight).  sh1/sh2/sh3 = 3K/2K/K are the
// wave-uniform shifts of the earlier windows.  Per weight, for the two "sum
// of halves" codebooks: one bit-field extract of the window, one full-rate
// multiply for the hash and one v_bitop3 for the mask/xor: three VALU ops per
// weight (plus one funnel shift per four weights).
template <int CB>
__device__ __forceinline__ void decode4(uint32_t hi, uint32_t lo, uint32_t shift, uint32_t sh3,
                                        uint32_t sh2, uint32_t sh1, uint32_t b[4]) {
    const uint32_t s = __builtin_amdgcn_alignbit(hi, lo, shift);
    const uint32_t w[4] = {(s >> sh3) & 0xFFFFu, (s >> sh2) & 0xFFFFu, (s >> sh1) & 0xFFFFu, s & 0xFFFFu};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (CB == kCbMul1) {
            b[i] = (uint32_t)half_to_bits(decode_weight<kCbMul1>(w[i]));  // (value, +0)
        } else {
            b[i] = (hash32<CB>(w[i]) & 0x8FFF8FFFu) ^ 0x3B603B60u;
        }
    }
}

__device__ __forceinline__ float4_t mfma16x16x32(const half8_t& a, const uint32_t b[4], float4_t c) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 bv = {b[0], b[1], b[2], b[3]};
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8_t, bv), c, 0, 0, 0);
}

// Butterfly over 128 values held as (lane, lane + 64), strides 1..64.  A
// lane stage (strides 1..32) is w + c * partner with c = -1 on the lanes
// whose stage bit is set: the butterfly's difference with its operands
// swapped (x_i - x_j for x_j - x_i, the same rounding mirrored).  A stage's
// partner agrees with the lane in every bit already processed, so both carry
// the same sign, and the outputs come out multiplied by had_sign64(lane) =
// (-1)^popcount(lane); the callers fold that sign into their scale, exactly.
// Strides 1, 2, 4, 8 read the partner through DPP row shuffles inside
// v_fmac_f32_dpp (4 takes a quad_perm move first); 16 and 32 through the
// gfx950 permlane swaps of two copies, which leave (own, partner) on the
// lanes whose bit is clear and (partner, own) on the others, so one
// fma(first, c, second) finishes the stage.  No LDS.  Wait states: two
// after a VALU write before a DPP or permlane read of it (five after an EXEC
// write), written out because inline assembly is opaque to the compiler's
// hazard checks.
__device__ __forceinline__ float had_sign64(int lane) { return (__builtin_popcount(lane & 63) & 1) ? -1.0f : 1.0f; }

__device__ __forceinline__ void had128(float& v0, float& v1, int lane) {
    const float c1 = (lane & 1) ? -1.0f : 1.0f, c2 = (lane & 2) ? -1.0f : 1.0f;
    const float c4 = (lane & 4) ? -1.0f : 1.0f, c8 = (lane & 8) ? -1.0f : 1.0f;
    const float c16 = (lane & 16) ? -1.0f : 1.0f, c32 = (lane & 32) ? -1.0f : 1.0f;
    float t0, t1;
    asm volatile(
        "s_nop 4\n\t"
        "v_fmac_f32_dpp %0, %0, %4 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %4 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %0, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_mov_b32_dpp %2, %0 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32_dpp %3, %1 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %2, %6 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %3, %6 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %0, %7 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %7 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : "+v"(v0), "+v"(v1), "=&v"(t0), "=&v"(t1)
        : "v"(c1), "v"(c2), "v"(c4), "v"(c8));
    float a0 = v0, b0 = v0, a1 = v1, b1 = v1;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_permlane16_swap_b32 %2, %3\n\ts_nop 1"
                 : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1));
    v0 = __builtin_fmaf(a0, c16, b0);
    v1 = __builtin_fmaf(a1, c16, b1);
    a0 = v0, b0 = v0, a1 = v1, b1 = v1;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_permlane32_swap_b32 %2, %3\n\ts_nop 1"
                 : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1));
    v0 = __builtin_fmaf(a0, c32, b0);
    v1 = __builtin_fmaf(a1, c32, b1);
    const float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
}

__device__ __forceinline__ float load_act(const void* x, int dtype, int64_t idx) {
    // The reference casts activations to fp16 at the boundary
    // (src/vllm_exl3/exl3.py:2856); mirror that rounding for every dtype.
    if (dtype == kF16) return (float)bits_to_half(reinterpret_cast<const uint16_t*>(x)[idx]);
    float f;
    if (dtype == kBF16) {
        uint32_t b = (uint32_t)reinterpret_cast<const uint16_t*>(x)[idx] << 16;
        f = __builtin_bit_cast(float, b);
    } else {
        f = reinterpret_cast<const float*>(x)[idx];
    }
    return (float)f32_to_f16_rne(f);
}

// Element c of a bias vector (fp16 / bf16 / fp32); 0 without one.
__device__ __forceinline__ float load_bias(const void* b, int dtype, int64_t c) {
    if (!b) return 0.0f;
    if (dtype == kF32) return reinterpret_cast<const float*>(b)[c];
    const uint32_t h = reinterpret_cast<const uint16_t*>(b)[c];
    if (dtype == kF16) return (float)bits_to_half(h);
    return __builtin_bit_cast(float, h << 16);
}

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t idx, float v) {
    if (dtype == kF32) {
        reinterpret_cast<float*>(out)[idx] = v;
    } else if (dtype == kF16) {
        reinterpret_cast<uint16_t*>(out)[idx] = half_to_bits((half_t)v);
    } else {
        uint32_t b = __builtin_bit_cast(uint32_t, v);
        b += 0x7FFFu + ((b >> 16) & 1u);  // RNE to bf16 (finite values)
        reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)(b >> 16);
    }
}

}  // namespace exl3
