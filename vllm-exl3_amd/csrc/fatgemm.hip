// Prefill ("fat") EXL3 GEMM and the routed-expert prefill executor on gfx950.
//
// Replaces the reference's exl3_fat_gemm / exl3_fat_gemm_scatter
// (csrc/exl3_fat_gemm.cu:65-305, K4 MCG only there) and the prefill side of
// the routed-expert dispatch (apply_exl3_fused_moe + apply_exl3_batched_fat,
// src/vllm_exl3/exl3.py:2981-3599, which sort on the host and loop over fat
// experts in Python).
//
// GEMM tile: one 768-thread workgroup (12 wave64s, three per SIMD) owns 256
// rows x 256 output columns of one expert.  Four producer waves (one per
// SIMD) load, stage and decode; eight MFMA waves (2 row halves x 4 column
// quarters) accumulate 128x64 each with v_mfma_f32_16x16x32_f16, so a
// SIMD's VALU decodes the next stage while its matrix core runs the current
// one.  Per 32-deep k-step, the packed trellis of the step (2 tile rows x 16
// tiles) is decoded ONCE into an LDS B tile of real fp16 weights (the
// codebook's two halves summed with one packed fp16 add, which rounds the
// exact sum once like the reference's decoder) and reused by every row of
// the tile.  A producer thread decodes one 8-index group of one tile (32
// weights, both column halves): the window offsets inside the group's K+1
// words are compile-time constants, so the decode needs no dynamic register
// indexing; each 16-byte unit produced is eight consecutive k of one column,
// exactly one MFMA B-operand lane fragment, stored with one ds_write_b128.
//
// Pipeline (one barrier per k-step, three LDS stages): the producers' global
// loads of A rows and packed bits run two k-steps ahead of their staging;
// iteration t: the MFMA waves read and multiply step t while the producers
// decode and stage step t + 2 and issue the loads of step t + 4.  An MFMA
// wave covers only the row fragments of its half that hold rows.
//
// The output rotation is not done in the GEMM epilogue: the GEMM stores
// Z / sqrt(128) (Z = A x Wq) and the consumer kernel - the activation kernel,
// the combine, or the drop-in's output pass - applies the 128-point Hadamard
// and svh where it is otherwise memory-bound.
#include "exl3_common.h"
#include "gemv_core.h"
#include "linear.h"
#include "profile.h"
#include "route.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace exl3 {
namespace {

constexpr int kTM = 256;          // rows per tile
constexpr int kTN = 256;          // output columns per tile
constexpr int kTK = 32;           // k per step (two tile rows)
constexpr int kABytes = kTM * kTK * 2;  // A stage: [256 rows][32 k] fp16, 64 B per row
constexpr int kBBytes = kTN * kTK * 2;  // B stage: [256 cols][32 k] fp16, 64 B per column

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const v4u* gv4p;
typedef __attribute__((address_space(1))) const uint32_t* gu32p;

struct FatParams {
    // A: fp16 rows; row r of the tile is a + (a_row) * lda
    const uint16_t* a;
    int64_t lda;
    // weights
    const uint8_t* trellis;       // single problem
    const int64_t* trellis_tab;   // grouped: per expert
    const int8_t* ktab;           // grouped: per-expert K (nullable)
    int kuni;
    int K_in, N;
    // output: Z * out_scale, fp16 or fp32, row stride ldo
    void* out;
    int out_f32;
    int64_t ldo;
    float out_scale;
    // tiles
    int grouped;
    int M;                        // single problem rows
    const int* n_mtiles;
    const int* mt_slot;
    const int* mt_row0;
    const int* slot_expert;
    const int* slot_start;
    const int* slot_rows;
    int n_ntiles;
    int n_tiles;                  // nproj * max_mtiles * n_ntiles (grid before XCD rounding)
    // Grouped launches may cover two projections of the same shape (the MoE
    // gate and up): tiles [n_tiles / 2, n_tiles) use these operands.  One
    // launch for both fills the workgroup rounds that two launches would
    // each leave part-empty.
    int nproj;
    const uint16_t* a2;
    const int64_t* trellis_tab2;
    const int8_t* ktab2;
    int kuni2;
    void* out2;
    // tiles of at most 128 rows let their idle MFMA waves decode half of B
    // (set by the launch; EXL3_FAT_HELPERS=0 turns it off)
    int helpers;
};

// Decoded (lo, hi) half pair of one window for the sum-of-halves codebooks,
// masked; the weight is half(lo) + half(hi).
template <int CB>
__device__ __forceinline__ uint32_t fat_pair(uint32_t w) {
    constexpr uint32_t C = (CB == kCb3Inst) ? 89226354u : 0xCBAC1FEDu;
    const uint32_t c_lo = C & 0xFFFFu;
    uint32_t lo_prod;
    if constexpr (CB == kCb3Inst) {
        const uint32_t add = 64248484u;
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(lo_prod) : "v"(w), "s"(c_lo), "v"(add));
    } else {
        asm("v_mad_u32_u16 %0, %1, %2, 0" : "=v"(lo_prod) : "v"(w), "s"(c_lo));
    }
    const unsigned short w16 = (unsigned short)w;
    const u16x2_t xv = {w16, w16};
    const u16x2_t cv = {(unsigned short)0, (unsigned short)(C >> 16)};
    const u16x2_t r = xv * cv + __builtin_bit_cast(u16x2_t, lo_prod);
    return (__builtin_bit_cast(uint32_t, r) & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Two weights (index i, index i+1 of a tile) as a packed fp16 pair from the
// 32 stream bits ending at the end of window i+1.
template <int K, int CB>
__device__ __forceinline__ uint32_t decode_pair(uint32_t s) {
    const uint32_t wa = s >> K;  // window of index i
    const uint32_t wb = s;       // window of index i + 1 (low 16 bits)
    if constexpr (CB == kCbMul1) {
        const uint32_t ha = half_to_bits(decode_weight<kCbMul1>(wa & 0xFFFFu));
        const uint32_t hb = half_to_bits(decode_weight<kCbMul1>(wb & 0xFFFFu));
        return ha | (hb << 16);
    } else {
        const uint32_t xa = fat_pair<CB>(wa);
        const uint32_t xb = fat_pair<CB>(wb);
        // lows = (xa.lo, xb.lo), highs = (xa.hi, xb.hi); weights = lows + highs
        const uint32_t lows = __builtin_amdgcn_perm(xb, xa, 0x05040100u);
        const uint32_t highs = __builtin_amdgcn_perm(xb, xa, 0x07060302u);
        const half2_t w = __builtin_bit_cast(half2_t, lows) + __builtin_bit_cast(half2_t, highs);
        return __builtin_bit_cast(uint32_t, w);
    }
}

// Word offset (relative to the group's first word) and funnel shift of pair
// p of unit (b1, b2): the pair's 32 stream bits end at
// E = (2 b1 + 4 b2 + 2 + 8 p) K + 32 bits after the group's first word.
template <int K>
struct PairGeom {
    static constexpr int end(int b1, int b2, int p) { return (2 * b1 + 4 * b2 + 2 + 8 * p) * K + 32; }
    static constexpr int rel(int b1, int b2, int p) { return (end(b1, b2, p) - 1) >> 5; }
    static constexpr int shift(int b1, int b2, int p) { return 32 * (rel(b1, b2, p) + 1) - end(b1, b2, p); }
};

// Byte offset of 16-byte chunk c (8 k values) of row (or column) r in an A or
// B stage: rows of 64 bytes, chunk index xor-ed with bits 2..3 of r and bits
// 3..4 of r.  Any 16 rows starting at a multiple of 16 then cover all 64
// banks at one chunk (the MFMA operand reads), and so do the stage writes
// (four rows x four chunks for A; columns 16 tc + g (+ 8), tc in {0, 1},
// g in 0..7 for the decoded B units).
__device__ __forceinline__ int swz(int r, int c) { return r * 64 + (((c ^ (r >> 2) ^ (r >> 3)) & 3) << 4); }

// LDS-only barrier: the stage buffers are handed over through LDS, and the
// global prefetches must stay in flight across it.  The scheduling barriers
// keep the compiler from hoisting the next k-step's decode arithmetic above
// it: that arithmetic reads the registers loaded last, so hoisting it turns
// the two-step prefetch into a wait for the newest loads (vmcnt(0)).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

struct FatTile {
    int64_t a_row0, out_row0;
    int rows_valid, nt;
    const uint8_t* trellis;
};

// The tile of this workgroup (false: none).  XCD-aware order: consecutive
// logical tiles (the N tiles of one row tile, which share their A rows) land
// on the same XCD and its L2.  pq: the projection's operands.
__device__ __forceinline__ bool fat_tile_of(const FatParams& p, FatParams& pq, FatTile& ft, int& K) {
    const int G = p.n_tiles;
    const int per = (G + 7) >> 3;
    int logical = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (logical >= G) return false;
    if (p.nproj > 1) {
        const int per_q = G / p.nproj;
        if (logical >= per_q) {
            logical -= per_q;
            pq.a = p.a2;
            pq.trellis_tab = p.trellis_tab2;
            pq.ktab = p.ktab2;
            pq.kuni = p.kuni2;
            pq.out = p.out2;
        }
    }
    const int mt = logical / p.n_ntiles;
    ft.nt = logical % p.n_ntiles;
    if (p.grouped) {
        if (mt >= *p.n_mtiles) return false;
        const int slot = p.mt_slot[mt];
        const int row0 = p.mt_row0[mt];
        const int e = p.slot_expert[slot];
        ft.a_row0 = (int64_t)p.slot_start[slot] + row0;
        ft.out_row0 = ft.a_row0;
        ft.rows_valid = min(kTM, p.slot_rows[slot] - row0);
        ft.trellis = reinterpret_cast<const uint8_t*>(pq.trellis_tab[e]);
        K = pq.ktab ? (int)pq.ktab[e] : pq.kuni;
    } else {
        ft.a_row0 = (int64_t)mt * kTM;
        ft.out_row0 = ft.a_row0;
        ft.rows_valid = min(kTM, p.M - mt * kTM);
        ft.trellis = p.trellis;
        K = p.kuni;
    }
    return true;
}

// ---------------------------------------------------------------------------
// 128-point butterfly over values held as adjacent pairs: lane l holds
// elements 2l and 2l+1.  Unnormalised.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void had128_pair(float& a, float& b, int lane) {
    const float s = a + b, d = a - b;
    a = s;
    b = d;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float pa = __shfl_xor(a, m, 64);
        const float pb = __shfl_xor(b, m, 64);
        if (lane & m) {
            a = pa - a;
            b = pb - b;
        } else {
            a = a + pa;
            b = b + pb;
        }
    }
}

__device__ __forceinline__ float h2f(const uint16_t* p, int64_t i) { return (float)bits_to_half(p[i]); }

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return (uint32_t)half_to_bits(f32_to_f16_rne(a)) | ((uint32_t)half_to_bits(f32_to_f16_rne(b)) << 16);
}

// The row kernels below work on 128-blocks held as 16 lanes x 8 consecutive
// elements: every global access is one 16-byte load or store per lane (fp32
// data: two), the butterfly runs over the 8 in-register elements and then
// over 4 lane bits, and a wave covers 4 blocks at a time.  Each wave takes
// kRowGroups such four-block groups of one row (8 consecutive blocks) and
// issues every load of them before the first butterfly; block indices past
// the row clamp to its last block (loads stay in bounds, those lanes' stores
// are dropped).
constexpr int kRowGroups = 2;
constexpr int kRowSpan = 4 * kRowGroups;  // 128-blocks per wave

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Sign of the lane's outputs of had128_x8: (-1)^popcount(lane % 16), as a
// float and as the xor mask of a packed fp16 pair.
__device__ __forceinline__ float had_sign(int lane) { return (__builtin_popcount(lane & 15) & 1) ? -1.0f : 1.0f; }
__device__ __forceinline__ uint32_t had_flip(int lane) {
    return (__builtin_popcount(lane & 15) & 1) ? 0x80008000u : 0u;
}

// 128-point butterfly (unnormalised, natural order) over the block held by
// the lane's 16-lane group: element 8 * (lane % 16) + i is v[i].  A
// cross-lane stage is one v_fmac_f32_dpp per value, w + c * partner with the
// partner's value read through a DPP row shuffle (xor 4 takes a quad_perm
// move first) and c = +1 / -1 on the lanes whose stage bit is clear / set:
// the butterfly's sum, or its difference with the operands swapped
// (x_i - x_j for x_j - x_i: the same rounding, mirrored).  The partner of a
// stage agrees with the lane in every bit already processed, so both carry
// the same sign, and the outputs come out multiplied by had_sign(lane); the
// callers fold that sign into a scale or an operand, exactly.
// Wait states: a DPP read of a VGPR needs two after the VALU write of it
// (five after an EXEC write), hence the s_nop 4 ahead of the first stage;
// inside the sequence every DPP read is at least seven instructions after
// the write it depends on (the eight values of a stage in turn, the xor-4
// moves all before their multiply-adds).
#define EXL3_FMAC_DPP(w, t, c, ctl) asm volatile("v_fmac_f32_dpp %0, %1, %2 " ctl " row_mask:0xf bank_mask:0xf" \
                                                 : "+v"(w) : "v"(t), "v"(c))
__device__ __forceinline__ void had128_x8(float v[8], int lane) {
#pragma unroll
    for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i & b) continue;
            const float a = v[i], c = v[i | b];
            v[i] = a + c;
            v[i | b] = a - c;
        }
    }
    const float c1 = (lane & 1) ? -1.0f : 1.0f, c2 = (lane & 2) ? -1.0f : 1.0f;
    const float c4 = (lane & 4) ? -1.0f : 1.0f, c8 = (lane & 8) ? -1.0f : 1.0f;
    float t[8];
    asm volatile("s_nop 4" ::);
#pragma unroll
    for (int i = 0; i < 8; ++i) EXL3_FMAC_DPP(v[i], v[i], c1, "quad_perm:[1,0,3,2]");
#pragma unroll
    for (int i = 0; i < 8; ++i) EXL3_FMAC_DPP(v[i], v[i], c2, "quad_perm:[2,3,0,1]");
#pragma unroll
    for (int i = 0; i < 8; ++i)
        asm volatile("v_mov_b32_dpp %0, %1 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf" : "=v"(t[i]) : "v"(v[i]));
#pragma unroll
    for (int i = 0; i < 8; ++i) EXL3_FMAC_DPP(v[i], t[i], c4, "row_half_mirror");
#pragma unroll
    for (int i = 0; i < 8; ++i) EXL3_FMAC_DPP(v[i], v[i], c8, "row_ror:8");
}
#undef EXL3_FMAC_DPP

// Elements i..i+7 (i % 8 == 0) of an fp16 array; `flip` (0 or 0x80008000)
// negates them.
__device__ __forceinline__ void ld_f16x8(const uint16_t* p, int64_t i, float v[8], uint32_t flip = 0) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t x = w[k] ^ flip;
        v[2 * k] = (float)bits_to_half(x & 0xFFFFu);
        v[2 * k + 1] = (float)bits_to_half(x >> 16);
    }
}

// Elements i..i+7 of an activation array as fp16 values: fp16 as is, bf16
// and fp32 rounded to fp16 (the reference casts activations to fp16).
__device__ __forceinline__ void ld_act8(const void* x, int dtype, int64_t i, float v[8]) {
    if (dtype == kF32) {
        const float4_t* p = reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(x) + i);
        const float4_t a = p[0], b = p[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = (float)f32_to_f16_rne(a[k]);
            v[4 + k] = (float)f32_to_f16_rne(b[k]);
        }
    } else if (dtype == kBF16) {
        const u32x4_t w = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(x) + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = (float)f32_to_f16_rne(__builtin_bit_cast(float, w[k] << 16));
            v[2 * k + 1] = (float)f32_to_f16_rne(__builtin_bit_cast(float, w[k] & 0xFFFF0000u));
        }
    } else {
        ld_f16x8(reinterpret_cast<const uint16_t*>(x), i, v);
    }
}

// fp16(v[k] * scale) for k = 0..7 stored at p + i with one 16-byte store.
__device__ __forceinline__ void st_f16x8(uint16_t* p, int64_t i, const float v[8], float scale) {
    u32x4_t w;
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = pack_f16(v[2 * k] * scale, v[2 * k + 1] * scale);
    *reinterpret_cast<u32x4_t*>(p + i) = w;
}

// v[0..7] stored at element i of an fp32 / fp16 / bf16 (RNE) array.
__device__ __forceinline__ void st_out8(void* out, int dtype, int64_t i, const float v[8]) {
    if (dtype == kF32) {
        float4_t* p = reinterpret_cast<float4_t*>(reinterpret_cast<float*>(out) + i);
        p[0] = float4_t{v[0], v[1], v[2], v[3]};
        p[1] = float4_t{v[4], v[5], v[6], v[7]};
    } else if (dtype == kF16) {
        st_f16x8(reinterpret_cast<uint16_t*>(out), i, v, 1.0f);
    } else {
        u32x4_t w;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t h[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t b = __builtin_bit_cast(uint32_t, v[2 * k + j]);
                b += 0x7FFFu + ((b >> 16) & 1u);  // RNE to bf16 (finite values)
                h[j] = b >> 16;
            }
            w[k] = h[0] | (h[1] << 16);
        }
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out) + i) = w;
    }
}

// The lane's columns in the wave's kRowSpan blocks starting at block j0 of
// a row of nb blocks: col[g] (clamped into the row) and whether it is real.
struct RowCols {
    int col[kRowGroups];
    bool ok[kRowGroups];
};
__device__ __forceinline__ RowCols row_cols(int j0, int nb, int lane) {
    RowCols rc;
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) {
        const int j = j0 + (lane >> 4) + 4 * g;
        rc.ok[g] = j < nb;
        rc.col[g] = min(j, nb - 1) * 128 + (lane & 15) * 8;
    }
    return rc;
}

// Gate/up input rotation of every sorted route row: A_q[row] =
// fp16(had128(fp16(x[token]) * suh_q[expert]) / sqrt(128)) for q in gate, up.
// One wave per (row, kRowSpan 128-column blocks).
__global__ __launch_bounds__(256) void rotate_in_kernel(const void* x, int x_dtype, int64_t x_stride,
                                                        int H, const int* n_sorted,
                                                        const int* row_token, const int* row_expert,
                                                        const int64_t* suh_g, const int64_t* suh_u,
                                                        int nproj, uint16_t* a_g, uint16_t* a_u,
                                                        int64_t n_units) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= n_units) return;
    const int nb = H >> 7, ng = (nb + kRowSpan - 1) / kRowSpan;
    const int row = (int)(unit / ng), j0 = (int)(unit % ng) * kRowSpan;
    if (row >= *n_sorted) return;
    const RowCols rc = row_cols(j0, nb, lane);
    const int64_t tok = row_token[row];
    const int e = row_expert[row];
    const uint16_t* su[2] = {reinterpret_cast<const uint16_t*>(suh_g[e]),
                             reinterpret_cast<const uint16_t*>(suh_u[e])};
    float xv[kRowGroups][8], sv[2][kRowGroups][8];
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) ld_act8(x, x_dtype, tok * x_stride + rc.col[g], xv[g]);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        if (q >= nproj) break;  // wave-uniform
#pragma unroll
        for (int g = 0; g < kRowGroups; ++g) ld_f16x8(su[q], rc.col[g], sv[q][g]);
    }
    const float scale = kHadNorm * had_sign(lane);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        if (q >= nproj) break;
        uint16_t* dst = (q ? a_u : a_g) + (int64_t)row * H;
#pragma unroll
        for (int g = 0; g < kRowGroups; ++g) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = xv[g][i] * sv[q][g][i];
            had128_x8(v, lane);
            if (rc.ok[g]) st_f16x8(dst, rc.col[g], v, scale);
        }
    }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

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

// Finish gate/up and build the down input: for each sorted row and 128-block
// Finish gate/up and build the down input: for each sorted row and 128-block
// of the intermediate dimension, g = fp16(had(Yg) * svh_g), u likewise,
// a = fp16(act(g, u)), A_d = fp16(had(a * suh_d) / sqrt(128)).  Y holds
// Z / sqrt(128) from the GEMM.  A_d is written over Y_g (same positions).
// One wave per (row, kRowSpan blocks).
__global__ __launch_bounds__(256) void act_kernel(const int* n_sorted, const int* row_expert, int I,
                                                  const int64_t* svh_g, const int64_t* svh_u,
                                                  const int64_t* suh_d, int gateless, int act,
                                                  float limit, uint16_t* y_g, const uint16_t* y_u,
                                                  int64_t n_units) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= n_units) return;
    const int nb = I >> 7, ng = (nb + kRowSpan - 1) / kRowSpan;
    const int row = (int)(unit / ng), j0 = (int)(unit % ng) * kRowSpan;
    if (row >= *n_sorted) return;
    const RowCols rc = row_cols(j0, nb, lane);
    const int e = row_expert[row];
    const uint16_t* svu = reinterpret_cast<const uint16_t*>(svh_u[e]);
    const uint16_t* svg = reinterpret_cast<const uint16_t*>(svh_g[e]);
    const uint16_t* sud = reinterpret_cast<const uint16_t*>(suh_d[e]);
    const int64_t ro = (int64_t)row * I;
    // the output scales carry had128_x8's lane sign
    const uint32_t flip = had_flip(lane);
    const float scale = kHadNorm * had_sign(lane);
    float u[kRowGroups][8], g[kRowGroups][8], vu[kRowGroups][8], vg[kRowGroups][8], d[kRowGroups][8];
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q) {
        ld_f16x8(y_u, ro + rc.col[q], u[q]);
        ld_f16x8(svu, rc.col[q], vu[q], flip);
        ld_f16x8(sud, rc.col[q], d[q]);
        if (!gateless) {
            ld_f16x8(y_g, ro + rc.col[q], g[q]);
            ld_f16x8(svg, rc.col[q], vg[q], flip);
        }
    }
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q) {
        had128_x8(u[q], lane);
        if (!gateless) had128_x8(g[q], lane);
        float r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float uu = (float)f32_to_f16_rne(u[q][i] * vu[q][i]);
            const float gg = gateless ? 0.f : (float)f32_to_f16_rne(g[q][i] * vg[q][i]);
            r[i] = (float)f32_to_f16_rne(activate(gg, uu, act, limit)) * d[q][i];
        }
        had128_x8(r, lane);
        if (rc.ok[q]) st_f16x8(y_g, ro + rc.col[q], r, scale);
    }
}

// out[t, block] = sum over the token's routes, in slot order, of
// w * had(Y_d[pos]) * svh_d (Y_d = Z / sqrt(128)); sentinel routes skipped.
// One wave per (token, kRowSpan 128-column blocks): deterministic, no
// atomics; per route, the loads of all the wave's blocks are issued first.
__global__ __launch_bounds__(256) void prefill_combine_kernel(const uint16_t* y_d, int H, int T,
                                                              int topk, const int* route_pos,
                                                              const int* row_expert,
                                                              const int64_t* svh_d, const void* weights,
                                                              int w_dtype, void* out, int out_dtype) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = H >> 7, ng = (nb + kRowSpan - 1) / kRowSpan;
    if (unit >= (int64_t)T * ng) return;
    const int t = (int)(unit / ng), j0 = (int)(unit % ng) * kRowSpan;
    const RowCols rc = row_cols(j0, nb, lane);
    float s[kRowGroups][8];
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) s[q][i] = 0.f;
    // the token's routes 64 at a time: lane k reads route k0 + k's sorted
    // row, weight, expert and scale row (three dependent loads once per
    // chunk, not per route); the routes then run in pairs, both rows' loads
    // issued before the first butterfly, summed in route order
    for (int k0 = 0; k0 < topk; k0 += 64) {
        const int nk = min(64, topk - k0);
        const int64_t wl = (int64_t)t * topk + k0 + min(lane, nk - 1);
        const int my_pos = route_pos[wl];
        float my_w;
        if (w_dtype == kF32)
            my_w = reinterpret_cast<const float*>(weights)[wl];
        else if (w_dtype == kF16)
            my_w = (float)bits_to_half(reinterpret_cast<const uint16_t*>(weights)[wl]);
        else
            my_w = __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(weights)[wl] << 16);
        const int64_t my_sv = my_pos >= 0 ? svh_d[row_expert[my_pos]] : 0;
        for (int k = 0; k < nk; k += 2) {
            int pos[2];
            const uint16_t* sv[2];
            float w[2], v[2][kRowGroups][8], h[2][kRowGroups][8];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int ku = min(k + u, nk - 1);
                pos[u] = k + u < nk ? __builtin_amdgcn_readlane(my_pos, ku) : -1;
                sv[u] = reinterpret_cast<const uint16_t*>(
                    ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(my_sv >> 32), ku) << 32) |
                    (uint32_t)__builtin_amdgcn_readlane((int)my_sv, ku));
                w[u] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), ku)) *
                       had_sign(lane);  // had128_x8's lane sign
                if (pos[u] < 0) continue;  // wave-uniform
#pragma unroll
                for (int q = 0; q < kRowGroups; ++q) {
                    ld_f16x8(y_d, (int64_t)pos[u] * H + rc.col[q], v[u][q]);
                    ld_f16x8(sv[u], rc.col[q], h[u][q]);
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if (pos[u] < 0) continue;
#pragma unroll
                for (int q = 0; q < kRowGroups; ++q) {
                    had128_x8(v[u][q], lane);
#pragma unroll
                    for (int i = 0; i < 8; ++i) s[q][i] += w[u] * (v[u][q][i] * h[u][q][i]);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q)
        if (rc.ok[q]) st_out8(out, out_dtype, (int64_t)t * H + rc.col[q], s[q]);
}

// Drop-in output pass: rows of Z / sqrt(128) (fp32, in `src`) ->
// had(.) * svh, written to out (scatter == 0) or added as
// out[token_idx[r]] += route_weight[r] * value (scatter == 1).
__global__ __launch_bounds__(256) void fat_out_kernel(const float* src, int M, int N,
                                                      const uint16_t* svh, int scatter,
                                                      const int64_t* token_idx,
                                                      const uint16_t* route_weight, float* out,
                                                      int64_t out_rows) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = N >> 7;
    if (unit >= (int64_t)M * nb) return;
    const int r = (int)(unit / nb), j = (int)(unit % nb);
    const int c = j * 128 + 2 * lane;
    float v0 = src[(int64_t)r * N + c], v1 = src[(int64_t)r * N + c + 1];
    had128_pair(v0, v1, lane);
    v0 *= h2f(svh, c);
    v1 *= h2f(svh, c + 1);
    if (!scatter) {
        out[(int64_t)r * N + c] = v0;
        out[(int64_t)r * N + c + 1] = v1;
    } else {
        const float w = (float)bits_to_half(route_weight[r]);
        const int64_t d = token_idx[r];
        if (d < 0 || d >= out_rows) return;  // wave-uniform: rows outside out are dropped
        atomicAdd(out + d * N + c, w * v0);
        atomicAdd(out + d * N + c + 1, w * v1);
    }
}

// Dense linear, large m: A[row] = fp16(had128(fp16(x[row]) * suh) / sqrt(128)).
// One wave per (row, kRowSpan 128-column blocks).
__global__ __launch_bounds__(256) void linear_rotate_kernel(const void* x, int x_dtype, int H,
                                                            const uint16_t* suh, uint16_t* a,
                                                            int64_t n_units) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= n_units) return;
    const int nb = H >> 7, ng = (nb + kRowSpan - 1) / kRowSpan;
    const int64_t row = unit / ng;
    const int j0 = (int)(unit % ng) * kRowSpan;
    const RowCols rc = row_cols(j0, nb, lane);
    float xv[kRowGroups][8], sv[kRowGroups][8];
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) {
        ld_act8(x, x_dtype, row * H + rc.col[g], xv[g]);
        ld_f16x8(suh, rc.col[g], sv[g]);
    }
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[g][i] *= sv[g][i];
        had128_x8(xv[g], lane);
        if (rc.ok[g]) st_f16x8(a, row * H + rc.col[g], xv[g], kHadNorm * had_sign(lane));
    }
}

// Dense linear, large m: out[row] = had128(Z[row]) * svh (+ bias), Z = A Wq /
// sqrt(128) in fp32 from the GEMM.  One wave per (row, kRowSpan blocks).
__global__ __launch_bounds__(256) void linear_out_kernel(const float* z, int N, const uint16_t* svh,
                                                         const void* bias, int bias_dtype, void* out,
                                                         int out_dtype, int64_t n_units) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= n_units) return;
    const int nb = N >> 7, ng = (nb + kRowSpan - 1) / kRowSpan;
    const int64_t row = unit / ng;
    const int j0 = (int)(unit % ng) * kRowSpan;
    const RowCols rc = row_cols(j0, nb, lane);
    float v[kRowGroups][8], h[kRowGroups][8];
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) {
        const float4_t* p = reinterpret_cast<const float4_t*>(z + row * N + rc.col[g]);
        const float4_t a = p[0], b = p[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[g][k] = a[k];
            v[g][4 + k] = b[k];
        }
        ld_f16x8(svh, rc.col[g], h[g], had_flip(lane));  // with had128_x8's lane sign
    }
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) {
        had128_x8(v[g], lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[g][i] = v[g][i] * h[g][i] + load_bias(bias, bias_dtype, rc.col[g] + i);
        if (rc.ok[g]) st_out8(out, out_dtype, row * N + rc.col[g], v[g]);
    }
}

// ---------------------------------------------------------------------------
// The GEMM tile (see the top of this file): 256 x 256 outputs, four producer
// waves and eight MFMA waves (128 x 64 outputs, 128 accumulator registers
// each); three LDS stages keep one barrier per k-step: step t lives in stage
// t % 3; iteration t multiplies step t, stages step t + 2 (into the stage step
// t - 1 used, whose reads all waves finished before the previous barrier) and
// loads step t + 4.
constexpr int kFatThreads = 768;
constexpr int kFatProducers = 4;  // waves that load, decode and stage; the other eight run the MFMAs
static_assert(kFatThreads / 64 == 3 * kFatProducers, "every third wave is a producer");
constexpr int kStages = 3;
constexpr int kFatLds = kStages * (kABytes + kBBytes);  // 96 KB

template <int K, int CB, int B2>
__device__ __forceinline__ void decode_group_half(const uint32_t (&w)[K + 1], uint8_t* B, int col0, int c0) {
#pragma unroll
    for (int b1 = 0; b1 < 2; ++b1) {
        v4u u;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int rel = PairGeom<K>::rel(b1, B2, p);
            const uint32_t s = __builtin_amdgcn_alignbit(w[rel - 1], w[rel], PairGeom<K>::shift(b1, B2, p));
            u[p] = decode_pair<K, CB>(s);
        }
        *reinterpret_cast<v4u*>(B + swz(col0 + 8 * B2, c0 + b1)) = u;
    }
}

// The K + 1 packed words a thread decodes: the K words of its group (word
// offsets g K .. g K + K - 1 of the tile, contiguous) in one wide load, and
// the word before (the tile's last word for group 0, where the bitstream
// wraps) in one more.  Per k-step the load count, not the bytes, weighs on
// few-row tiles: K + 1 four-byte loads made 32 x 4096 x 65536 take 103 µs,
// these two (three for K 5, 6) 85 µs.
template <int K>
__device__ __forceinline__ void load_group_words(uint32_t (&w)[K + 1], __amdgpu_buffer_rsrc_t trs, int wprev,
                                                 int wfirst, int soff) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(trs, wprev, soff, 0);
    if constexpr (K == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(trs, wfirst, soff, 0);
        w[1] = v[0];
        w[2] = v[1];
    } else if constexpr (K == 3) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(trs, wfirst, soff, 0);
        w[1] = v[0];
        w[2] = v[1];
        w[3] = v[2];
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(trs, wfirst, soff, 0);
        w[1] = v[0];
        w[2] = v[1];
        w[3] = v[2];
        w[4] = v[3];
        if constexpr (K == 5) w[5] = __builtin_amdgcn_raw_buffer_load_b32(trs, wfirst + 16, soff, 0);
        if constexpr (K == 6) {
            const auto u = __builtin_amdgcn_raw_buffer_load_b64(trs, wfirst + 16, soff, 0);
            w[5] = u[0];
            w[6] = u[1];
        }
    }
}

// Producer waves (0..3, one per SIMD): global loads of A rows and packed
// bits two k-steps ahead of their staging; per k-step each thread stages 64
// bytes of A and decodes one 32-weight group (both column halves) into the
// B stage.  One barrier per k-step, three stages, as the consumers.
template <int CB, int K, int NA>
__device__ __forceinline__ void fat_producer(const FatParams& p, const FatTile& ft, uint8_t* lds, int nsteps,
                                             bool helped) {
    constexpr int tile_bytes = 32 * K;
    const int pt = (threadIdx.x >> 6) / 3 * 64 + (threadIdx.x & 63);  // 0..255
    const int tiles_n = p.N >> 4;
    const int ac = pt & 3, ar0 = pt >> 2;  // A: chunk ac of rows ar0 + 64 jj
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.a + ft.a_row0 * p.lda), (short)0, 0x7FFFFFFF, 0x00020000);
    // NA of the four 64-row groups of A hold the tile's rows (a compile-time
    // count, so every load is unconditional and the wait counts exact): the
    // others are neither loaded nor staged, the MFMA rows they would feed
    // are never read
    int a_voff[NA];
#pragma unroll
    for (int jj = 0; jj < NA; ++jj)
        a_voff[jj] = (int)((min(ar0 + 64 * jj, ft.rows_valid - 1) * p.lda + 8 * ac) * 2);
    const int t_idx = pt >> 3, g = pt & 7;  // decode: group g of tile t_idx
    const int tr = t_idx >> 4, tc = t_idx & 15;
    const int tcols = min(16, tiles_n - ft.nt * 16);
    const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(ft.trellis + (size_t)ft.nt * 16 * tile_bytes), (short)0, 0x7FFFFFFF, 0x00020000);
    const int t_voff = (tr * tiles_n + min(tc, tcols - 1)) * tile_bytes;
    const int step_bytes = 2 * tiles_n * tile_bytes;
    // the group's first word, and the word before it (wrapping to the
    // tile's last word for group 0)
    const int w_first = t_voff + 4 * g * K;
    const int w_prev = t_voff + 4 * (g == 0 ? 8 * K - 1 : g * K - 1);
    const int col0 = tc * 16 + g;

    v4u ga[2][NA];
    uint32_t gw[2][K + 1];
    auto load = [&](int t, int r) {
        const int so = min(t, nsteps - 1);
#pragma unroll
        for (int jj = 0; jj < NA; ++jj)
            ga[r][jj] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(ars, a_voff[jj], so * (kTK * 2), 0));
        load_group_words<K>(gw[r], trs, w_prev, w_first, so * step_bytes);
    };
    auto stage = [&](int st, int r) {
        uint8_t* A = lds + st * kABytes;
        uint8_t* B = lds + kStages * kABytes + st * kBBytes;
#pragma unroll
        for (int jj = 0; jj < NA; ++jj) *reinterpret_cast<v4u*>(A + swz(ar0 + 64 * jj, ac)) = ga[r][jj];
        decode_group_half<K, CB, 0>(gw[r], B, col0, 2 * tr);
        if (!helped) decode_group_half<K, CB, 1>(gw[r], B, col0, 2 * tr);
    };
    // prologue: stages 0, 1 hold steps 0, 1; the registers hold steps 2, 3,
    // issued in the loop's order (register set 0 before set 1) so that the
    // loop's first wait is for set 0 only
    load(0, 0);
    load(1, 1);
    stage(0, 0);
    stage(1, 1);
    __builtin_amdgcn_sched_barrier(0);
    load(2, 0);
    __builtin_amdgcn_sched_barrier(0);
    load(3, 1);
    lds_barrier();
    int st_cur = 0;  // stage of step t
    for (int t = 0; t < nsteps; t += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            stage(st_cur == 0 ? 2 : st_cur - 1, u);  // step t + u + 2 into stage (t + u + 2) % 3
            load(t + u + 4, u);
            lds_barrier();
            st_cur = st_cur == 2 ? 0 : st_cur + 1;
        }
    }
}

// Helper waves: in a tile of at most 128 rows the four MFMA waves of the
// second row half have no rows; they decode the second column half of every
// 32-weight group instead (the producers decode the first), with the
// producers' loads, stages and barriers (one per k-step, the same count).
// pt: the thread's group, as the producers number them (0..255).
template <int CB, int K>
__device__ __forceinline__ void fat_helper(const FatParams& p, const FatTile& ft, uint8_t* lds, int nsteps,
                                           int pt) {
    constexpr int tile_bytes = 32 * K;
    const int tiles_n = p.N >> 4;
    const int t_idx = pt >> 3, g = pt & 7;
    const int tr = t_idx >> 4, tc = t_idx & 15;
    const int tcols = min(16, tiles_n - ft.nt * 16);
    const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(ft.trellis + (size_t)ft.nt * 16 * tile_bytes), (short)0, 0x7FFFFFFF, 0x00020000);
    const int t_voff = (tr * tiles_n + min(tc, tcols - 1)) * tile_bytes;
    const int step_bytes = 2 * tiles_n * tile_bytes;
    // the group's first word, and the word before it (wrapping to the
    // tile's last word for group 0)
    const int w_first = t_voff + 4 * g * K;
    const int w_prev = t_voff + 4 * (g == 0 ? 8 * K - 1 : g * K - 1);
    const int col0 = tc * 16 + g;
    uint32_t gw[2][K + 1];
    auto load = [&](int t, int r) {
        const int so = min(t, nsteps - 1);
        load_group_words<K>(gw[r], trs, w_prev, w_first, so * step_bytes);
    };
    auto stage = [&](int st, int r) {
        uint8_t* B = lds + kStages * kABytes + st * kBBytes;
        decode_group_half<K, CB, 1>(gw[r], B, col0, 2 * tr);
    };
    load(0, 0);
    load(1, 1);
    stage(0, 0);
    stage(1, 1);
    __builtin_amdgcn_sched_barrier(0);
    load(2, 0);
    __builtin_amdgcn_sched_barrier(0);
    load(3, 1);
    lds_barrier();
    int st_cur = 0;
    for (int t = 0; t < nsteps; t += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            stage(st_cur == 0 ? 2 : st_cur - 1, u);
            load(t + u + 4, u);
            lds_barrier();
            st_cur = st_cur == 2 ? 0 : st_cur + 1;
        }
    }
}

// Consumer waves (eight): wave c owns row half h = c / 4 (row fragments
// 8 h + i, i < MF: the fragments of its half that hold rows, rounded up) and
// the 64 columns 64 (c % 4) of the tile; per k-step it reads its fragments
// from the stage the producers finished one barrier earlier and issues 4
// MFMAs per row fragment.  No branch sits between the reads and the MFMAs,
// so that all of a step's reads are in flight before the first MFMA waits.
template <int MF>
__device__ __forceinline__ void fat_consumer(const FatParams& p, const FatTile& ft, uint8_t* lds, int nsteps,
                                             int c, bool mma_on) {
    const int lane = threadIdx.x & 63;
    const int h = (c >> 2) & 1, cn = c & 3;
    float4_t acc[MF][4];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int off_ev = swz(lane & 15, lane >> 4), off_od = swz(16 + (lane & 15), lane >> 4) - 16 * 64;
    auto consume = [&](int st) {
        const uint8_t* A = lds + st * kABytes;
        const uint8_t* B = lds + kStages * kABytes + st * kBBytes;
        half8_t fb[4];
#pragma unroll
        for (int nf = 0; nf < 4; ++nf) {
            const int f = 4 * cn + nf;
            fb[nf] = *reinterpret_cast<const half8_t*>(B + f * 1024 + ((f & 1) ? off_od : off_ev));
        }
#pragma unroll
        for (int i = 0; i < MF; ++i) {
            const int f = 8 * h + i;
            const half8_t fa = *reinterpret_cast<const half8_t*>(A + f * 1024 + ((f & 1) ? off_od : off_ev));
#pragma unroll
            for (int nf = 0; nf < 4; ++nf)
                acc[i][nf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa, fb[nf], acc[i][nf], 0, 0, 0);
        }
    };
    lds_barrier();  // the producers' prologue
    int st_cur = 0;
    for (int t = 0; t < nsteps; t += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (mma_on) consume(st_cur);
            lds_barrier();
            st_cur = st_cur == 2 ? 0 : st_cur + 1;
        }
    }
    // epilogue: Z * out_scale for the valid rows
    if (mma_on) {
        const int colw = ft.nt * kTN + 64 * cn + (lane & 15);
#pragma unroll
        for (int i = 0; i < MF; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 16 * (8 * h + i) + 4 * (lane >> 4) + e;
                if (r < ft.rows_valid) {
                    const int64_t o = (ft.out_row0 + r) * p.ldo + colw;
#pragma unroll
                    for (int nf = 0; nf < 4; ++nf) {
                        const float v = acc[i][nf][e] * p.out_scale;
                        if (p.out_f32)
                            reinterpret_cast<float*>(p.out)[o + nf * 16] = v;
                        else
                            reinterpret_cast<uint16_t*>(p.out)[o + nf * 16] = half_to_bits((half_t)v);
                    }
                }
            }
        }
    }
}

__device__ __forceinline__ bool fat_helpers_on(const FatParams& p) { return p.helpers != 0; }

template <int CB, int K>
__device__ __forceinline__ void fat_tile_k(const FatParams& p, const FatTile& ft, uint8_t* lds) {
    const int nsteps = p.K_in / kTK;  // a multiple of 4 (K_in is a multiple of 128)
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // at most 128 rows: the second row half's MFMA waves help decode B
    const bool helped = ft.rows_valid <= 128 && fat_helpers_on(p);
    if (w % 3 == 0) {  // waves 0, 3, 6, 9: one per SIMD
        // the 64-row groups of A the consumers read: their fragments of
        // rows, rounded up to 1, 2, 4, 6 or 8 per row half
        if (ft.rows_valid <= 64)
            fat_producer<CB, K, 1>(p, ft, lds, nsteps, helped);
        else if (ft.rows_valid <= 128)
            fat_producer<CB, K, 2>(p, ft, lds, nsteps, helped);
        else
            fat_producer<CB, K, 4>(p, ft, lds, nsteps, helped);
        return;
    }
    // consumers: c = 0..3 row half 0, 4..7 row half 1 (the helpers of a tile
    // of at most 128 rows).  The dispatcher puts waves w, w + 4 and w + 8 on
    // one SIMD (measured: the SIMD of wave w is a fixed permutation of w % 4,
    // rotated per workgroup), so each SIMD holds one producer (0, 3, 6, 9),
    // one half-0 wave (1, 2, 4, 7) and one half-1 wave (5, 8, 10, 11): the
    // decode and the MFMAs spread evenly whatever the tile's row count.
    // Nibble w of the constant is c (F: producer).
    const int c = (int)((0x76F53F42F10Full >> (4 * w)) & 15);
    if (helped && c >= 4) {
        fat_helper<CB, K>(p, ft, lds, nsteps, (c - 4) * 64 + (int)(threadIdx.x & 63));
        return;
    }
    // the wave's 16-row fragments holding rows (at most 8 in its row half),
    // rounded up to 1, 2, 4, 6 or 8 (wave-uniform)
    const int nfr = min(8, max(0, ((ft.rows_valid + 15) >> 4) - 8 * ((c >> 2) & 1)));
    const bool mma_on = nfr > 0 && 64 * (c & 3) < p.N - ft.nt * kTN;  // a last tile may be narrower
    if (nfr <= 1)
        fat_consumer<1>(p, ft, lds, nsteps, c, mma_on);
    else if (nfr <= 2)
        fat_consumer<2>(p, ft, lds, nsteps, c, mma_on);
    else if (nfr <= 4)
        fat_consumer<4>(p, ft, lds, nsteps, c, mma_on);
    else if (nfr <= 6)
        fat_consumer<6>(p, ft, lds, nsteps, c, mma_on);
    else
        fat_consumer<8>(p, ft, lds, nsteps, c, mma_on);
}

// KSET 0: tiles of K 2..4 (every uniform-K launch and most of a mixed-K
// one); tiles of any other per-expert K are left to the KSET 1 launch, which
// a grouped launch with K tables adds: it computes K 5 and 6 and writes
// zeros for any other K, as the reference's mixed-K tile switch does
// (csrc/p2b_moe.cu:295-324).  Two kernels, so that the K 5/6 decode's
// registers never weigh on the common kernel's allocation.
template <int CB, int KSET>
__global__ __launch_bounds__(kFatThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void fat_gemm_kernel(
    FatParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    FatTile ft;
    int K;
    FatParams pq = p;
    if (!fat_tile_of(p, pq, ft, K)) return;
    if constexpr (KSET == 0) {
        switch (K) {
            case 2: fat_tile_k<CB, 2>(pq, ft, lds); break;
            case 3: fat_tile_k<CB, 3>(pq, ft, lds); break;
            case 4: fat_tile_k<CB, 4>(pq, ft, lds); break;
            default: break;  // the KSET 1 launch's tile
        }
    } else {
        switch (K) {
            case 2: case 3: case 4: break;  // the KSET 0 launch's tile
            case 5: fat_tile_k<CB, 5>(pq, ft, lds); break;
            case 6: fat_tile_k<CB, 6>(pq, ft, lds); break;
            default: {
                // unsupported K: the tile's outputs are zeros
                const int ncols = min(kTN, p.N - ft.nt * kTN);
                for (int i = threadIdx.x; i < ft.rows_valid * ncols; i += kFatThreads) {
                    const int64_t o = (ft.out_row0 + i / ncols) * pq.ldo + (int64_t)ft.nt * kTN + i % ncols;
                    if (pq.out_f32)
                        reinterpret_cast<float*>(pq.out)[o] = 0.0f;
                    else
                        reinterpret_cast<uint16_t*>(pq.out)[o] = 0;
                }
                break;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host planning
// ---------------------------------------------------------------------------
inline size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

hipError_t init_fat_caps() {
    static const hipError_t st = [] {
        hipError_t e = hipSuccess;
        const void* fns[] = {(const void*)fat_gemm_kernel<0, 0>, (const void*)fat_gemm_kernel<1, 0>,
                             (const void*)fat_gemm_kernel<2, 0>, (const void*)fat_gemm_kernel<0, 1>,
                             (const void*)fat_gemm_kernel<1, 1>, (const void*)fat_gemm_kernel<2, 1>};
        for (const void* f : fns) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kFatLds);
            if (r != hipSuccess) {
                (void)hipGetLastError();
                e = r;
            }
        }
        return e;
    }();
    return st;
}

template <int KSET>
void launch_fat_set(int cb, const FatParams& p, hipStream_t st) {
    const int grid = ((p.n_tiles + 7) / 8) * 8;
    switch (cb) {
        case 0: fat_gemm_kernel<0, KSET><<<grid, kFatThreads, kFatLds, st>>>(p); break;
        case 1: fat_gemm_kernel<1, KSET><<<grid, kFatThreads, kFatLds, st>>>(p); break;
        default: fat_gemm_kernel<2, KSET><<<grid, kFatThreads, kFatLds, st>>>(p); break;
    }
}

// The GEMM of one launch: the K 2..4 kernel, then, when the launch reads
// per-expert K tables, the kernel for the other K values.
inline bool fat_helpers_allowed() {
    const char* v = std::getenv("EXL3_FAT_HELPERS");
    return !(v && std::strcmp(v, "0") == 0);
}

hipError_t launch_fat(int cb, const FatParams& p_in, hipStream_t st) {
    FatParams p = p_in;
    p.helpers = fat_helpers_allowed() ? 1 : 0;
    launch_fat_set<0>(cb, p, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.grouped && (p.ktab || (p.nproj > 1 && p.ktab2))) {
        launch_fat_set<1>(cb, p, st);
        e = hipGetLastError();
    }
    return e;
}

struct PrefillPlan {
    int n_routes, max_slots, max_mtiles;
    bool wide_route;  // the multi-workgroup router (large route counts)
    size_t off_route, off_rscr, off_agu, off_ygu, total;
};

// EXL3_ROUTE_WIDE=0 keeps the single-workgroup router for every route count
// (tuning and tests; read on every plan, workspace queries included).
inline bool route_wide_allowed() {
    const char* v = std::getenv("EXL3_ROUTE_WIDE");
    return !(v && std::strcmp(v, "0") == 0);
}

PrefillPlan plan_prefill(int64_t T, int64_t topk, int64_t n_local, int64_t H, int64_t I, int gateless) {
    PrefillPlan pp;
    pp.n_routes = (int)(T * topk);
    pp.max_slots = (int)std::min<int64_t>(pp.n_routes, n_local);
    pp.max_mtiles = (int)route_max_mtiles(pp.n_routes, pp.max_slots, kTM);
    const int nproj = gateless ? 1 : 2;
    pp.wide_route = route_wide_allowed() && pp.n_routes >= kRouteWideMin && pp.n_routes <= kRouteWideMax &&
                    n_local <= kRouteMaxLocal;
    size_t off = 0;
    pp.off_route = off;
    off += a256(sizeof(int) * (3 + 3 * (size_t)pp.max_slots + 3 * (size_t)pp.n_routes +
                               2 * (size_t)pp.max_mtiles));
    pp.off_rscr = off;  // the wide router's counts per 1024-route workgroup
    if (pp.wide_route) off += a256(route_scratch_bytes(pp.n_routes, (int)n_local));
    pp.off_agu = off;  // A_g, A_u [n_routes][H] fp16; later Y_d [n_routes][H] fp16
    off += a256(2 * (size_t)nproj * pp.n_routes * H);
    pp.off_ygu = off;  // Y_g, Y_u [n_routes][I] fp16; A_d over Y_g
    off += a256(2 * (size_t)nproj * pp.n_routes * I);
    pp.total = off;
    return pp;
}

}  // namespace

size_t linear_fat_workspace_bytes(int64_t m, int64_t in_f, int64_t out_f) {
    return a256(2 * (size_t)m * in_f) + a256(4 * (size_t)m * out_f);
}

int linear_fat(const void* x, int x_dtype, int64_t m, const int16_t* trellis, int64_t tiles_k,
               int64_t tiles_n, int64_t K, int codebook, const uint16_t* suh, const uint16_t* svh,
               const void* bias, int bias_dtype, void* out, int out_dtype, void* workspace,
               hipStream_t st) {
    EXL3_HIP(init_fat_caps());
    const int64_t in_f = tiles_k * 16, out_f = tiles_n * 16;
    uint16_t* a = reinterpret_cast<uint16_t*>(workspace);
    float* z = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + a256(2 * (size_t)m * in_f));
    profile_begin_call();
    profile_mark(0, st);
    {
        const int64_t units = m * ((in_f / 128 + kRowSpan - 1) / kRowSpan);
        linear_rotate_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(x, x_dtype, (int)in_f, suh, a,
                                                                          units);
        EXL3_LAUNCHED();
    }
    profile_mark(1, st);
    FatParams p = {};
    p.a = a;
    p.lda = in_f;
    p.trellis = reinterpret_cast<const uint8_t*>(trellis);
    p.kuni = (int)K;
    p.K_in = (int)in_f;
    p.N = (int)out_f;
    p.out = z;
    p.out_f32 = 1;
    p.ldo = out_f;
    p.out_scale = kHadNorm;
    p.grouped = 0;
    p.M = (int)m;
    p.n_ntiles = (int)((out_f + kTN - 1) / kTN);
    p.n_tiles = (int)(((m + kTM - 1) / kTM) * p.n_ntiles);
    EXL3_HIP(launch_fat(codebook, p, st));
    profile_mark(2, st);
    {
        const int64_t units = m * ((out_f / 128 + kRowSpan - 1) / kRowSpan);
        linear_out_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(z, (int)out_f, svh, bias, bias_dtype,
                                                                       out, out_dtype, units);
        EXL3_LAUNCHED();
    }
    profile_mark(3, st);
    return kOk;
}

}  // namespace exl3

using namespace exl3;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static int fat_common_checks(int64_t M, int64_t tiles_k, int64_t tiles_n, int64_t K, int codebook) {
    EXL3_CHECK(K == 2 || K == 3 || K == 4, "exl3_fat_gemm supports K in {2, 3, 4}");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(M >= 1 && M <= (1 << 26), "exl3_fat_gemm needs 1 <= M <= 2^26 rows");
    EXL3_CHECK(tiles_k > 0 && tiles_n > 0 && (tiles_k * 16) % 128 == 0 && (tiles_n * 16) % 128 == 0,
               "output dimension must be divisible by 128");
    EXL3_CHECK(tiles_k * 16 <= (1 << 20) && tiles_n * 16 <= (1 << 20), "exl3_fat_gemm dimensions too large");
    return kOk;
}

EXL3_API int64_t exl3_fat_gemm_workspace_size(int64_t M, int64_t out_features, int scatter) {
    if (M < 1 || out_features < 128) return 0;
    return scatter ? (int64_t)a256(4 * (size_t)M * out_features) : 0;
}

static int fat_gemm_impl(const uint16_t* a, int64_t M, const int16_t* trellis, int64_t tiles_k,
                         int64_t tiles_n, int64_t K, int codebook, const uint16_t* svh,
                         const int64_t* token_idx, const uint16_t* route_weight, float* out,
                         int64_t out_rows, void* workspace, int64_t workspace_bytes, void* stream,
                         int scatter) {
    const int rc = fat_common_checks(M, tiles_k, tiles_n, K, codebook);
    if (rc) return rc;
    EXL3_CHECK(a && trellis && svh && out && (!scatter || (token_idx && route_weight)),
               "exl3_fat_gemm: null pointer argument");
    const int64_t N = tiles_n * 16, K_in = tiles_k * 16;
    const size_t need = (size_t)exl3_fat_gemm_workspace_size(M, N, scatter);
    EXL3_CHECK(workspace_bytes >= (int64_t)need && (need == 0 || workspace),
               "exl3_fat_gemm workspace too small: need %zu bytes", need);
    EXL3_HIP(init_fat_caps());
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    FatParams p = {};
    p.a = a;
    p.lda = K_in;
    p.trellis = reinterpret_cast<const uint8_t*>(trellis);
    p.kuni = (int)K;
    p.K_in = (int)K_in;
    p.N = (int)N;
    float* z = scatter ? reinterpret_cast<float*>(workspace) : out;
    p.out = z;
    p.out_f32 = 1;
    p.ldo = N;
    p.out_scale = kHadNorm;
    p.grouped = 0;
    p.M = (int)M;
    p.n_ntiles = (int)((N + kTN - 1) / kTN);
    const int64_t mtiles = (M + kTM - 1) / kTM;
    EXL3_CHECK(mtiles * p.n_ntiles < (1 << 30), "exl3_fat_gemm problem too large");
    p.n_tiles = (int)(mtiles * p.n_ntiles);
    profile_begin_call();
    profile_mark(0, st);
    EXL3_HIP(launch_fat(codebook, p, st));
    profile_mark(1, st);
    const int64_t units = M * (N / 128);
    fat_out_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(z, (int)M, (int)N, svh, scatter,
                                                                 token_idx, route_weight, out,
                                                                 out_rows);
    EXL3_LAUNCHED();
    profile_mark(2, st);
    return kOk;
}

EXL3_API int exl3_fat_gemm(const uint16_t* a, int64_t M, const int16_t* trellis, int64_t tiles_k,
                           int64_t tiles_n, int64_t K, int codebook, const uint16_t* svh, float* out,
                           void* stream) {
    return fat_gemm_impl(a, M, trellis, tiles_k, tiles_n, K, codebook, svh, nullptr, nullptr, out,
                         M, nullptr, 0, stream, 0);
}

EXL3_API int exl3_fat_gemm_scatter(const uint16_t* a, int64_t M, const int16_t* trellis,
                                   int64_t tiles_k, int64_t tiles_n, int64_t K, int codebook,
                                   const uint16_t* svh, const int64_t* token_idx,
                                   const uint16_t* route_weight, float* out, int64_t out_rows,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
    EXL3_CHECK(out_rows >= 1, "exl3_fat_gemm_scatter needs a non-empty output");
    return fat_gemm_impl(a, M, trellis, tiles_k, tiles_n, K, codebook, svh, token_idx, route_weight,
                         out, out_rows, workspace, workspace_bytes, stream, 1);
}

EXL3_API int64_t exl3_moe_prefill_workspace_size(int64_t T, int64_t topk, int64_t n_local,
                                                 int64_t hidden, int64_t inter, int gateless) {
    if (T < 1 || topk < 1 || n_local < 1 || hidden < 128 || inter < 128) return 0;
    return (int64_t)plan_prefill(T, topk, n_local, hidden, inter, gateless).total;
}

EXL3_API int exl3_moe_prefill(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
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
    EXL3_CHECK(n_local >= 1 && n_local <= kRouteMaxLocal,
               "fused MoE prefill supports 1 <= n_local <= %d local experts", kRouteMaxLocal);
    EXL3_CHECK(T >= 1 && topk >= 1 && T * topk <= (1 << 22),
               "fused MoE prefill supports 1 <= T*topk <= 2^22 routes");
    EXL3_CHECK(hidden > 0 && hidden % 128 == 0,
               "fused MoE hidden width must be a positive multiple of 128");
    EXL3_CHECK(inter > 0 && inter % 128 == 0,
               "fused MoE local intermediate width must be a positive multiple of 128");
    EXL3_CHECK(hidden <= (1 << 20) && inter <= (1 << 20), "fused MoE dimensions too large");
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
    const PrefillPlan pp = plan_prefill(T, topk, n_local, hidden, inter, gateless);
    EXL3_CHECK(workspace && workspace_bytes >= (int64_t)pp.total,
               "fused MoE prefill workspace too small: need %zu bytes", pp.total);
    EXL3_HIP(init_fat_caps());
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    const int nproj = gateless ? 1 : 2;

    profile_begin_call();
    profile_mark(0, st);
    RouteOut ro = {};
    int* rb = reinterpret_cast<int*>(ws + pp.off_route);
    ro.n_active = rb;
    ro.n_mtiles = rb + 1;
    int* n_sorted = rb + 2;
    ro.slot_expert = rb + 3;
    ro.slot_start = ro.slot_expert + pp.max_slots;
    ro.slot_rows = ro.slot_start + pp.max_slots;
    ro.row_token = ro.slot_rows + pp.max_slots;
    ro.row_expert = ro.row_token + pp.n_routes;
    ro.route_pos = ro.row_expert + pp.n_routes;
    ro.mt_slot = ro.route_pos + pp.n_routes;
    ro.mt_row0 = ro.mt_slot + pp.max_mtiles;
    ro.n_sorted = n_sorted;
    if (pp.wide_route)
        EXL3_HIP(launch_route_wide(ids, ids_dtype, pp.n_routes, (int)topk, (int)n_local, n_valid, kTM, ro,
                                   reinterpret_cast<int*>(ws + pp.off_rscr), st));
    else
        EXL3_HIP(launch_route(ids, ids_dtype, pp.n_routes, (int)topk, (int)n_local, n_valid, kTM, ro, st));

    uint16_t* a_g = reinterpret_cast<uint16_t*>(ws + pp.off_agu);
    uint16_t* a_u = a_g + (size_t)(nproj - 1) * pp.n_routes * hidden;
    uint16_t* y_g = reinterpret_cast<uint16_t*>(ws + pp.off_ygu);
    uint16_t* y_u = y_g + (size_t)(nproj - 1) * pp.n_routes * inter;
    const int64_t* gtab_t = gateless ? up_trellis : gate_trellis;
    const int64_t* gtab_su = gateless ? up_suh : gate_suh;
    const int64_t* gtab_sv = gateless ? up_svh : gate_svh;

    profile_mark(1, st);
    {
        const int64_t units = (int64_t)pp.n_routes * ((hidden / 128 + kRowSpan - 1) / kRowSpan);
        rotate_in_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(
            x, x_dtype, hidden, (int)hidden, n_sorted, ro.row_token, ro.row_expert,
            gateless ? up_suh : gate_suh, up_suh, nproj, gateless ? a_u : a_g, a_u, units);
        EXL3_LAUNCHED();
    }
    profile_mark(2, st);
    FatParams p = {};
    p.lda = hidden;
    p.K_in = (int)hidden;
    p.N = (int)inter;
    p.out_f32 = 0;
    p.ldo = inter;
    p.out_scale = kHadNorm;
    p.grouped = 1;
    p.n_mtiles = ro.n_mtiles;
    p.mt_slot = ro.mt_slot;
    p.mt_row0 = ro.mt_row0;
    p.slot_expert = ro.slot_expert;
    p.slot_start = ro.slot_start;
    p.slot_rows = ro.slot_rows;
    p.n_ntiles = (int)((inter + kTN - 1) / kTN);
    // gate and up in one launch (tiles of the second half use the up operands)
    p.nproj = nproj;
    p.n_tiles = nproj * pp.max_mtiles * p.n_ntiles;
    p.a = gateless ? a_u : a_g;
    p.trellis_tab = gateless ? up_trellis : gtab_t;
    p.ktab = gateless ? k_up : k_gate;
    p.kuni = (int)(gateless ? K_up : K_gate);
    p.out = gateless ? y_u : y_g;
    p.a2 = a_u;
    p.trellis_tab2 = up_trellis;
    p.ktab2 = k_up;
    p.kuni2 = (int)K_up;
    p.out2 = y_u;
    EXL3_HIP(launch_fat(codebook, p, st));
    (void)gtab_su;
    profile_mark(3, st);
    {
        const int64_t units = (int64_t)pp.n_routes * ((inter / 128 + kRowSpan - 1) / kRowSpan);
        act_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(
            n_sorted, ro.row_expert, (int)inter, gtab_sv, up_svh, down_suh, gateless, act,
            swiglu_limit, gateless ? y_u : y_g, y_u, units);
        EXL3_LAUNCHED();
    }
    profile_mark(4, st);
    uint16_t* y_d = a_g;  // A_g/A_u are dead: Y_d [n_routes][hidden] fp16
    p.a = gateless ? y_u : y_g;
    p.lda = inter;
    p.K_in = (int)inter;
    p.N = (int)hidden;
    p.trellis_tab = down_trellis;
    p.ktab = k_down;
    p.kuni = (int)K_down;
    p.out = y_d;
    p.ldo = hidden;
    p.n_ntiles = (int)((hidden + kTN - 1) / kTN);
    p.nproj = 1;
    p.n_tiles = pp.max_mtiles * p.n_ntiles;
    EXL3_HIP(launch_fat(codebook, p, st));
    profile_mark(5, st);
    {
        const int64_t units = T * ((hidden / 128 + kRowSpan - 1) / kRowSpan);
        prefill_combine_kernel<<<(unsigned)((units + 3) / 4), 256, 0, st>>>(
            y_d, (int)hidden, (int)T, (int)topk, ro.route_pos, ro.row_expert, down_svh, weights,
            w_dtype, out, out_dtype);
        EXL3_LAUNCHED();
    }
    profile_mark(6, st);
    return kOk;
}
