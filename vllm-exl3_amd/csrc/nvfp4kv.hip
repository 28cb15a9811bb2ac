// The reference's NVFP4 ("q4") paged KV cache on gfx950: page pack, pool
// dequant and the block-sparse split decode attention with its merge.
//
// Replaces src/vllm_exl3/minimax_q4kv_reference.py (pack_q4_row :297-326,
// pack_slot_region_side :352-366, dequant_pool_pages :735-776) and the decode
// overlay q4_sparse_decode + _q4_decode_kernel
// (src/vllm_exl3/minimax_q4kv_kernels.py:385-506, 772-877).  Format (kept
// byte for byte, it is the pool the model writes): 128-token pages, slot
// 2h + side (K 0, V 1) of a page is a flat 9216-byte region, data
// [128 tokens][64 B] (byte j of a token = e2m1 nibbles of dims 2j, 2j+1, low
// nibble even) then 1024 scale bytes (e4m3 per 16 dims; K linear t*8+g, V
// the 4x4 token-quad swizzle).
//
// Pack: one wave per (token, KV head, side) row, lane l owns dims 2l, 2l+1
// (one data byte).  bf16 rounding, group max over 8 lanes, s = max(amax/6,
// 2^-9) as saturating RNE e4m3, q = RZ(x * RN(1/s)) (the RN product, stepped
// toward zero when fma shows it rounded away), RNE e2m1 codes with the
// reference's tie rules.  Bit-exact with the reference packer.
//
// Decode: one 256-thread workgroup per (query token, KV head, chunk of the
// top-k list).  Per listed block: the K and V slots are dequantised into LDS
// as fp16 (e2m1 x e4m3 is exact in fp16) with v_cvt_scalef32_pk_f16_fp4 and
// one packed multiply per pair; scores, the online softmax (log2 domain) and
// P.V run in fp32.  The chunk's normalised output and its log2-sum-exp go
// to a workspace; the merge kernel combines the chunks.
#include "exl3_common.h"
#include "profile.h"

#include <cmath>

namespace exl3 {
namespace {

constexpr int kQ4Page = 128;
constexpr int kQ4Dim = 128;
constexpr int kQ4Slot = 9216;
constexpr int kQ4Data = 8192;
constexpr int kQ4MaxGroup = 16;   // query heads per KV head
constexpr int kQ4Threads = 256;

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float q4_load(const void* x, int dtype, int64_t idx) {
    if (dtype == 2) return reinterpret_cast<const float*>(x)[idx];
    const uint16_t b = reinterpret_cast<const uint16_t*>(x)[idx];
    if (dtype == 0) return (float)bits_to_half(b);
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// fp32 -> bf16 (RNE) -> fp32; NaN becomes the canonical +NaN, as torch's
// float -> bfloat16 cast does (a bf16 input is not converted at all).
__device__ __forceinline__ float bf16_round(float x) {
    if (x != x) return __builtin_bit_cast(float, 0x7FC00000u);
    uint32_t b = __builtin_bit_cast(uint32_t, x);
    b = (b + 0x7FFFu + ((b >> 16) & 1u)) & 0xFFFF0000u;
    return __builtin_bit_cast(float, b);
}

// Saturating RNE fp32 -> e4m3fn byte; NaN -> 0x7F with its sign.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t sign = __builtin_bit_cast(uint32_t, x) >> 31;
    if (x != x) return 0x7Fu | (sign << 7);
    const float ax = fabsf(x);
    const uint32_t bits = __builtin_bit_cast(uint32_t, ax);
    int e8 = (int)((bits >> 23) & 0xFF) - 120;
    uint32_t man = bits & 0x7FFFFFu;
    uint32_t code;
    if (e8 <= 0) {
        // subnormal: round(ax * 512) to nearest even; 8 becomes code 0x08
        const float t = ax * 512.0f;  // exact scaling
        const float fl = floorf(t);
        const float frac = t - fl;
        const uint32_t fi = (uint32_t)fl;
        const uint32_t inc = (frac > 0.5f || (frac == 0.5f && (fi & 1u))) ? 1u : 0u;
        code = fi + inc;
    } else {
        uint32_t m3 = man >> 20;
        const uint32_t rest = man & 0xFFFFFu;
        if (rest > 0x80000u || (rest == 0x80000u && (m3 & 1u))) ++m3;
        if (m3 == 8) {
            m3 = 0;
            ++e8;
        }
        code = (e8 >= 1 && e8 <= 15 && !(e8 == 15 && m3 == 7)) ? (((uint32_t)e8 << 3) | m3) : 0x7Eu;
    }
    return (code | (sign << 7)) & 0xFFu;
}

__device__ __forceinline__ float e4m3_value(uint32_t b) {
    return __builtin_amdgcn_cvt_f32_fp8((int)b, 0);  // OCP e4m3fn (checked on gfx950)
}

// e2m1 code 0..7 of |q| (RNE with the reference's ties); NaN -> 7
__device__ __forceinline__ uint32_t e2m1_code(float a) {
    if (a != a) return 7;
    return (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.0f);
}

// RZ at fp32 of the exact product x * r
__device__ __forceinline__ float rz_mul(float x, float r) {
    const float p = x * r;
    const float e = __builtin_fmaf(x, r, -p);  // exact remainder
    if (p != 0.0f && e != 0.0f && (__builtin_bit_cast(uint32_t, e) ^ __builtin_bit_cast(uint32_t, p)) >> 31 &&
        __builtin_isfinite(p))
        return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, p) - 1u);  // one step toward 0
    return p;
}

__device__ __forceinline__ int scale_offset(int side, int t, int g) {
    if (side == 0) return t * 8 + g;
    return ((t >> 2) * 4 + (g >> 1)) * 8 + (g & 1) * 4 + (t & 3);
}

// One 128-dim row held as dims 2 lane, 2 lane + 1 (bf16 values) packed into
// token t of a slot region: data byte `lane` and, from every 8th lane, the
// e4m3 scale of its 16-dim group.  Group max over 8 lanes, s = max(amax/6,
// 2^-9) as saturating RNE e4m3, q = RZ(x * RN(1/s)), RNE e2m1 codes.
__device__ __forceinline__ void pack_row_lane(float x0, float x1, uint8_t* region, int t, int side,
                                              int lane) {
    // amax ignores NaN (hardware fmax)
    float am = fmaxf(x0 != x0 ? 0.0f : fabsf(x0), x1 != x1 ? 0.0f : fabsf(x1));
    am = fmaxf(am, __shfl_xor(am, 1, 64));
    am = fmaxf(am, __shfl_xor(am, 2, 64));
    am = fmaxf(am, __shfl_xor(am, 4, 64));
    const float s = fmaxf(am / 6.0f, 0.001953125f);  // 2^-9
    const uint32_t sb = e4m3_encode(s);
    const float recip = 1.0f / e4m3_value(sb);
    uint32_t nib[2];
    const float xs[2] = {x0, x1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float q = rz_mul(xs[i], recip);
        const uint32_t c = e2m1_code(fabsf(q));
        nib[i] = c == 0 ? 0u : (c | ((__builtin_bit_cast(uint32_t, q) >> 31) << 3));
    }
    region[t * 64 + lane] = (uint8_t)(nib[0] | (nib[1] << 4));
    if ((lane & 7) == 0) region[kQ4Data + scale_offset(side, t, lane >> 3)] = (uint8_t)sb;
}

struct Q4PackParams {
    const void* k;
    const void* v;
    int dtype;
    int B, H;
    int64_t sb, sh, st;        // element strides of k/v [B, H, L, 128]
    const int* seq_lens;
    const int* block_table;
    int64_t bt_stride;
    int max_blocks;
    int max_len;
    uint8_t* pool;             // [pages][2H][9216]
    int64_t num_pages;
};

__global__ __launch_bounds__(256) void q4_pack_kernel(Q4PackParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    // unit = ((b * max_len + pos) * H + h) * 2 + side
    const int side = (int)(unit & 1);
    const int64_t r = unit >> 1;
    const int h = (int)(r % p.H);
    const int64_t bp = r / p.H;
    const int pos = (int)(bp % p.max_len);
    const int b = (int)(bp / p.max_len);
    if (b >= p.B || pos >= p.seq_lens[b]) return;  // wave-uniform
    const int blk = pos / kQ4Page, t = pos % kQ4Page;
    if (blk >= p.max_blocks) return;
    const int64_t page = p.block_table[(int64_t)b * p.bt_stride + blk];
    if (page < 0 || page >= p.num_pages) return;
    const void* x = side ? p.v : p.k;
    const int64_t base = (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)pos * p.st + 2 * lane;
    float x0 = q4_load(x, p.dtype, base), x1 = q4_load(x, p.dtype, base + 1);
    if (p.dtype != 1) {  // bf16 inputs are already bf16 values
        x0 = bf16_round(x0);
        x1 = bf16_round(x1);
    }
    uint8_t* region = p.pool + (page * (2 * p.H) + 2 * h + side) * (int64_t)kQ4Slot;
    pack_row_lane(x0, x1, region, t, side, lane);
}

// ---------------------------------------------------------------------------
// W1 write side: Gemma QK-norm + partial NeoX RoPE + q4 pack-insert
// (q4_w1_insert / _q4_w1_kernel, src/vllm_exl3/minimax_q4kv_kernels.py:
// 216-348, 661-758; reference reference_w1_write,
// src/vllm_exl3/minimax_q4kv_reference.py:422-612).  One wave per (token,
// branch head) of the fused bf16 row [q | k | v | index_q | index_k], lane l
// holding dims 2l, 2l+1.  fp32 arithmetic with each operation rounded once
// (no contraction): sum of squares as a butterfly over the lanes (pair sums,
// then a balanced tree in lane order), r = 1/sqrt(ss/128 + eps) correctly
// rounded, xn = (x r)(1 + w); RoPE pairs (d, d +- half) read their partner's
// normed value from the owning lane.
// ---------------------------------------------------------------------------
struct Q4W1Params {
    uint16_t* qkv;               // bf16 [T][row]; K and index-K rows rewritten in place
    int64_t row;
    uint16_t* q_out;             // bf16 [T][nq][128]
    uint8_t* index_q_out;        // e4m3 bytes [T][niq][128]
    const void* norm_w[4];       // q, k, index_q, index_k norm weights [128]
    int w_dtype;
    const void* cos_sin;         // [max_pos][rotary_dim] (cos | sin)
    int cs_dtype;
    int64_t max_pos;
    const int64_t* positions;
    const int64_t* slot_mapping;
    const int64_t* index_slot_mapping;
    uint8_t* pool;               // [pages][2 nkv][9216]
    int64_t num_pages;
    uint8_t* index_cache;        // e4m3 bytes [index_rows][128]
    int64_t index_rows;
    float eps;
    int rotary_dim;
    int T, nq, nkv, niq;
};

// fp32 product rounded on its own: the register barrier keeps the backend
// from fusing it into a following add (one rounding, as a scalar CPU does).
__device__ __forceinline__ float mul_rn(float a, float b) {
    float p = a * b;
    asm volatile("" : "+v"(p));
    return p;
}

__device__ __forceinline__ float w1_norm_rope(float& x0, float& x1, const void* w, int w_dtype,
                                              const void* cs, int cs_dtype, int64_t pos,
                                              int rotary_dim, float eps, int lane) {
    float ss = mul_rn(x0, x0) + mul_rn(x1, x1);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) ss = ss + __shfl_xor(ss, m, 64);
    // r = 1 / sqrt(ss / 128 + eps), the square root and the quotient each
    // correctly rounded to fp32: both are taken in fp64 and rounded once to
    // fp32, which gives the correctly rounded fp32 result (53 >= 2 * 24 + 2).
    const float den = ss * 0.0078125f + eps;  // ss / 128 is exact
    const float sq = (float)__builtin_sqrt((double)den);
    const float r = (float)(1.0 / (double)sq);
    const float n0 = mul_rn(mul_rn(x0, r), 1.0f + q4_load(w, w_dtype, 2 * lane));
    const float n1 = mul_rn(mul_rn(x1, r), 1.0f + q4_load(w, w_dtype, 2 * lane + 1));
    const int half = rotary_dim >> 1;
    float y[2] = {n0, n1};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int d = 2 * lane + j;
        const int pd = d < half ? d + half : (d < rotary_dim ? d - half : d);
        const float a = __shfl(n0, pd >> 1, 64), b = __shfl(n1, pd >> 1, 64);  // every lane takes part
        if (d < rotary_dim) {
            const float pv = (pd & 1) ? b : a;
            const int ci = d < half ? d : d - half;
            const float c = q4_load(cs, cs_dtype, pos * rotary_dim + ci);
            const float s = q4_load(cs, cs_dtype, pos * rotary_dim + half + ci);
            const float t1 = mul_rn(y[j], c), t2 = mul_rn(pv, s);
            y[j] = d < half ? t1 - t2 : t1 + t2;
        }
    }
    x0 = y[0];
    x1 = y[1];
    return r;
}

__device__ __forceinline__ uint32_t bf16_bits(float v) { return __builtin_bit_cast(uint32_t, bf16_round(v)) >> 16; }

__global__ __launch_bounds__(256) void q4_w1_kernel(Q4W1Params p) {
    const int lane = threadIdx.x & 63;
    const int per = p.nq + 2 * p.nkv + (p.niq > 0 ? p.niq + 1 : 0);
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (int64_t)p.T * per) return;
    const int64_t token = unit / per;
    const int slot = (int)(unit % per);
    const int64_t pos = p.positions[token];
    if (pos < 0 || pos >= p.max_pos) return;  // wave-uniform; the host rejects these first
    uint32_t* rowp = reinterpret_cast<uint32_t*>(p.qkv + token * p.row + (int64_t)slot * 128) + lane;
    const uint32_t xw = *rowp;
    float x0 = __builtin_bit_cast(float, xw << 16), x1 = __builtin_bit_cast(float, xw & 0xFFFF0000u);
    const int iq_lo = p.nq + 2 * p.nkv;
    if (slot < p.nq) {
        w1_norm_rope(x0, x1, p.norm_w[0], p.w_dtype, p.cos_sin, p.cs_dtype, pos, p.rotary_dim, p.eps, lane);
        reinterpret_cast<uint32_t*>(p.q_out + (token * p.nq + slot) * 128)[lane] =
            bf16_bits(x0) | (bf16_bits(x1) << 16);
    } else if (slot < p.nq + p.nkv) {
        w1_norm_rope(x0, x1, p.norm_w[1], p.w_dtype, p.cos_sin, p.cs_dtype, pos, p.rotary_dim, p.eps, lane);
        const float b0 = bf16_round(x0), b1 = bf16_round(x1);
        *rowp = bf16_bits(x0) | (bf16_bits(x1) << 16);  // processed row back into qkv
        const int64_t sm = p.slot_mapping[token];
        if (sm >= 0 && sm < p.num_pages * kQ4Page) {
            uint8_t* region = p.pool + ((sm / kQ4Page) * (2 * p.nkv) + 2 * (slot - p.nq)) * (int64_t)kQ4Slot;
            pack_row_lane(b0, b1, region, (int)(sm % kQ4Page), 0, lane);
        }
    } else if (slot < iq_lo) {
        const int64_t sm = p.slot_mapping[token];
        if (sm >= 0 && sm < p.num_pages * kQ4Page) {
            uint8_t* region =
                p.pool + ((sm / kQ4Page) * (2 * p.nkv) + 2 * (slot - p.nq - p.nkv) + 1) * (int64_t)kQ4Slot;
            pack_row_lane(x0, x1, region, (int)(sm % kQ4Page), 1, lane);  // bf16 inputs: values as is
        }
    } else if (slot < iq_lo + p.niq) {
        w1_norm_rope(x0, x1, p.norm_w[2], p.w_dtype, p.cos_sin, p.cs_dtype, pos, p.rotary_dim, p.eps, lane);
        const uint32_t e0 = e4m3_encode(bf16_round(x0)), e1 = e4m3_encode(bf16_round(x1));
        reinterpret_cast<uint16_t*>(p.index_q_out + (token * p.niq + (slot - iq_lo)) * 128)[lane] =
            (uint16_t)(e0 | (e1 << 8));
    } else {
        w1_norm_rope(x0, x1, p.norm_w[3], p.w_dtype, p.cos_sin, p.cs_dtype, pos, p.rotary_dim, p.eps, lane);
        *rowp = bf16_bits(x0) | (bf16_bits(x1) << 16);
        const int64_t ism = p.index_slot_mapping[token];
        if (ism >= 0 && ism < p.index_rows) {
            // e4m3(clamp(v, +-448)), NaN -> -448
            const float c0 = x0 != x0 ? -448.0f : fminf(fmaxf(x0, -448.0f), 448.0f);
            const float c1 = x1 != x1 ? -448.0f : fminf(fmaxf(x1, -448.0f), 448.0f);
            reinterpret_cast<uint16_t*>(p.index_cache + ism * 128)[lane] =
                (uint16_t)(e4m3_encode(c0) | (e4m3_encode(c1) << 8));
        }
    }
}

// Pool -> fp32 values [pages][2H][128][128]; one thread per data byte.
__global__ __launch_bounds__(256) void q4_dequant_kernel(const uint8_t* pool, int64_t n_slots,
                                                         float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // byte index over all slots
    if (i >= n_slots * kQ4Data) return;
    const int64_t slot = i / kQ4Data;
    const int j = (int)(i % kQ4Data);
    const int t = j >> 6, byte = j & 63;
    const uint8_t* region = pool + slot * kQ4Slot;
    const int side = (int)(slot & 1);
    const float sc = e4m3_value(region[kQ4Data + scale_offset(side, t, byte >> 3)]);
    const h2v v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4((uint32_t)region[j], 1.0f, 0);
    float* o = out + slot * (kQ4Page * kQ4Dim) + t * kQ4Dim + 2 * byte;
    o[0] = (float)v[0] * sc;
    o[1] = (float)v[1] * sc;
}

// Prefill staging (q4_stage_pages / _q4_stage_kernel,
// src/vllm_exl3/minimax_q4kv_kernels.py:509-566, 880-951): staged row r of
// the bf16 buffer [rows][H][128 tokens][256] holds page pages[r] of the pool,
// K values in columns 0..127 and V values in 128..255 (e2m1 x e4m3 in fp32,
// then bf16; the product has at most 7 significant bits and lies inside
// bf16's normal range, so the bf16 value is exact; a NaN scale code gives
// 0x7FC0).  Row n (one past the last page) is written as zeros, and so is a
// row whose page id is outside [0, num_pages).
//
// One thread per 8 consecutive output columns of one token: one 4-byte data
// load, one scale byte, one 16-byte store; a workgroup covers 8 tokens x 256
// columns of one (row, head), so each store instruction of a wave writes
// 1 KiB of consecutive bytes.  Grid (rows, H, 16).
constexpr int kStageTokPerBlock = 8;

__global__ __launch_bounds__(256) void q4_stage_kernel(const uint8_t* pool, int64_t num_pages, int H,
                                                       const void* pages, int pages_i64, int n,
                                                       uint16_t* stage) {
    const int row = blockIdx.x, head = blockIdx.y;
    const int tid = threadIdx.x;
    const int t = blockIdx.z * kStageTokPerBlock + (tid >> 5);
    const int col = (tid & 31) * 8;  // 0..248
    const int side = col >> 7, d0 = col & 127;
    int64_t page = -1;
    if (row < n)
        page = pages_i64 ? reinterpret_cast<const int64_t*>(pages)[row]
                         : (int64_t)reinterpret_cast<const int32_t*>(pages)[row];
    u32x4 o = {0u, 0u, 0u, 0u};
    if (page >= 0 && page < num_pages) {
        const uint8_t* region = pool + (page * 2 * H + 2 * head + side) * (int64_t)kQ4Slot;
        const uint32_t d = *reinterpret_cast<const uint32_t*>(region + t * 64 + (d0 >> 1));
        const float sc = e4m3_value(region[kQ4Data + scale_offset(side, t, d0 >> 4)]);
        if (sc != sc) {
            o = u32x4{0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u};
        } else {
            const h2v v[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 0),
                              __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 1),
                              __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 2),
                              __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 3)};
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t lo = __builtin_bit_cast(uint32_t, bf16_round((float)v[b][0] * sc)) >> 16;
                const uint32_t hi = __builtin_bit_cast(uint32_t, bf16_round((float)v[b][1] * sc)) >> 16;
                o[b] = lo | (hi << 16);
            }
        }
    }
    *reinterpret_cast<u32x4*>(stage + (((int64_t)row * H + head) * kQ4Page + t) * 256 + col) = o;
}

struct Q4DecodeParams {
    const void* q;
    int q_dtype;
    int total_q, Hq, Hkv, G;
    int64_t q_sn, q_sh;
    const uint8_t* pool;
    int64_t num_pages;
    const int* topk;           // [Hkv][total_q][max_topk] (strides below)
    int64_t tk_sh, tk_sn;
    int max_topk;
    const int* block_table;
    int64_t bt_stride;
    int max_blocks;
    const int* seq_lens;
    int dql;                   // decode_query_len
    float scale_log2;          // sm_scale * log2(e)
    int n_chunks;
    float* o_part;             // [chunks][total_q][Hq][128]
    float* lse_part;           // [chunks][total_q][Hq]
};

// ---------------------------------------------------------------------------
// Block-sparse decode on the matrix cores.  Workgroup = (query token, KV head,
// chunk of the top-k list), four waves.  Per listed block (128 tokens):
//   * staging: every thread converts 64 K and 64 V values of one token with
//     v_cvt_scalef32_pk_f16_fp4 and one packed multiply per pair (e2m1 x its
//     group's e4m3 scale, exact in fp16) into LDS: K as [token][dim], V
//     transposed as [dim][token]; the packed bytes are loaded one block
//     ahead;
//   * scores S[head][token] = q . k on v_mfma_f32_16x16x32_f16 (A = the G
//     query heads of the KV head, padded to 16 rows, fp16 from registers;
//     B = K), wave w takes tokens 32w..32w+31; scaled to the log2 domain in
//     fp32, tokens past the query's position masked;
//   * online softmax in fp32: block maxima across the waves through LDS,
//     P = 2^(S - m) rounded to fp16 into LDS as [head][token];
//   * O[head][dim] += P V on the same MFMA (A = P, B = V), wave w takes dims
//     32w..32w+31; O and each wave's share of the denominator are rescaled
//     by 2^(m_old - m_new).
// The chunk's normalised output and its log2-sum-exp go to the workspace.
// ---------------------------------------------------------------------------
constexpr int kQ4Pitch = kQ4Dim + 8;  // fp16 LDS row pitch: 272 bytes, 16-byte aligned, banks spread

struct Q4Lds {
    uint16_t K[kQ4Page * kQ4Pitch];      // [token][dim]
    uint16_t Vt[kQ4Dim * kQ4Pitch];      // [dim][token]
    uint16_t P[kQ4MaxGroup * kQ4Pitch];  // [head][token]
    float red[4][kQ4MaxGroup];           // per-wave block maxima
    float lsum[4][kQ4MaxGroup];          // per-wave denominators
    int lpage[64], lblk[64];             // the valid blocks of a 64-entry window of the list
    int lcount;
};

// The packed bytes one thread stages: token t = tid / 2, dims 64 h .. 64 h + 63
// (h = tid & 1) of the K and of the V slot, and the four group scales of each.
struct Q4Piece {
    u32x4 k0, k1, v0, v1;
    uint32_t ks, vs;  // scale bytes of groups 4h .. 4h + 3, one per byte
};

__device__ __forceinline__ void q4_load_piece(const uint8_t* base, int tid, Q4Piece& pc) {
    const int t = tid >> 1, h = tid & 1;
    const u32x4* ksrc = reinterpret_cast<const u32x4*>(base + t * 64 + 32 * h);
    const u32x4* vsrc = reinterpret_cast<const u32x4*>(base + kQ4Slot + t * 64 + 32 * h);
    pc.k0 = ksrc[0];
    pc.k1 = ksrc[1];
    pc.v0 = vsrc[0];
    pc.v1 = vsrc[1];
    // scale bytes of groups 4h .. 4h + 3 (scale_offset): K's are four
    // consecutive bytes; V's are byte t % 4 of four consecutive words of one
    // 16-byte block (two loads in place of eight byte loads; the same time,
    // 41 µs on the bench's workload)
    pc.ks = *reinterpret_cast<const uint32_t*>(base + kQ4Data + t * 8 + 4 * h);
    const u32x4 vw = *reinterpret_cast<const u32x4*>(base + kQ4Slot + kQ4Data + (t >> 2) * 32 + 16 * h);
    const uint32_t q = (uint32_t)(t & 3);
    const uint32_t sel = q | ((q + 4) << 8) | 0x0C0C0000u;  // bytes (lo.q, hi.q, 0, 0)
    pc.vs = __builtin_amdgcn_perm(vw.y, vw.x, sel) | (__builtin_amdgcn_perm(vw.w, vw.z, sel) << 16);
}

// The eight fp16 values of one packed word (dims 2b, 2b + 1 in byte b, low
// nibble first), each e2m1 code times the group scale sc.  The conversion's
// own scale operand acts as a power of two (the exponent of an MX block
// scale), so the e4m3 scale is applied by one packed fp16 multiply per pair,
// which is exact: an e2m1 x e4m3 product has at most 7 significant bits.
__device__ __forceinline__ u32x4 q4_cvt_word(uint32_t w, float sc) {
    const h2v s2 = {(_Float16)sc, (_Float16)sc};
    const h2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * s2;
    const h2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * s2;
    const h2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * s2;
    const h2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * s2;
    return u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, c),
                 __builtin_bit_cast(uint32_t, d)};
}

__device__ __forceinline__ void q4_stage_piece(const Q4Piece& pc, int tid, Q4Lds& L) {
    const int t = tid >> 1, h = tid & 1;
    const uint32_t kw[8] = {pc.k0.x, pc.k0.y, pc.k0.z, pc.k0.w, pc.k1.x, pc.k1.y, pc.k1.z, pc.k1.w};
    const uint32_t vw[8] = {pc.v0.x, pc.v0.y, pc.v0.z, pc.v0.w, pc.v1.x, pc.v1.y, pc.v1.z, pc.v1.w};
    u32x4* krow = reinterpret_cast<u32x4*>(L.K + t * kQ4Pitch + 64 * h);
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // word j: dims 64 h + 8 j .. + 7, group 4 h + j / 2
        const float ksc = e4m3_value((pc.ks >> (8 * (j >> 1))) & 0xFFu);
        krow[j] = q4_cvt_word(kw[j], ksc);
        const float vsc = e4m3_value((pc.vs >> (8 * (j >> 1))) & 0xFFu);
        const u32x4 v = q4_cvt_word(vw[j], vsc);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = 64 * h + 8 * j + e;
            L.Vt[d * kQ4Pitch + t] = (uint16_t)(vv[e >> 1] >> (16 * (e & 1)));
        }
    }
}

__global__ __launch_bounds__(kQ4Threads) void q4_decode_kernel(Q4DecodeParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t q4_lds[];
    Q4Lds& L = *reinterpret_cast<Q4Lds*>(q4_lds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const int i = blockIdx.x % p.total_q;
    const int c = blockIdx.x / p.total_q;
    const int h = blockIdx.y;
    const int G = p.G;
    const int req = i / p.dql;
    const int qpos = p.seq_lens[req] - p.dql + (i - req * p.dql);
    const int kv_len = max(qpos + 1, 0);
    const int n_blocks = (kv_len + kQ4Page - 1) / kQ4Page;
    const int real_topk = min(p.max_topk, n_blocks);
    const int chunk = (p.max_topk + p.n_chunks - 1) / p.n_chunks;
    const int c0 = c * chunk, c1 = min(c0 + chunk, real_topk);
    const int* tk = p.topk + (int64_t)h * p.tk_sh + (int64_t)i * p.tk_sn;
    const int* bt = p.block_table + (int64_t)req * p.bt_stride;

    // query fragments (A operand): head m16 (zero past G), dims 32 s + 8 g .. + 7
    half8_t qa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = m16 < G ? q4_load(p.q, p.q_dtype, (int64_t)i * p.q_sn + (int64_t)(h * G + m16) * p.q_sh +
                                                                  32 * s + 8 * g + e)
                                    : 0.0f;
            qa[s][e] = (_Float16)v;
        }
    }
    float4_t o[2];  // O[heads 4 g .. 4 g + 3][dims 32 wave + 16 j + m16]
    o[0] = float4_t{0.f, 0.f, 0.f, 0.f};
    o[1] = float4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[4], l_run[4];  // per head 4 g + r: running max, this lane's share of the denominator
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }

    // The list is walked in windows of 64 entries: wave 0 reads a window's
    // entries and block-table pages with vector loads and compacts the valid
    // ones into LDS, so no dependent scalar load sits in front of a block.
    for (int w0 = c0; w0 < c1; w0 += 64) {
        __syncthreads();  // every wave is done with the previous window
        if (wave == 0) {
            const int e = w0 + lane;
            int pg = -1, bk = 0;
            if (e < c1) {
                bk = tk[e];
                if (bk >= 0 && bk < n_blocks) {
                    const int64_t pp = bt[bk];
                    if (pp >= 0 && pp < p.num_pages) pg = (int)pp;
                }
            }
            const uint64_t vm = __ballot(pg >= 0);
            const int pos = __popcll(vm & ((1ull << lane) - 1ull));
            if (pg >= 0) {
                L.lpage[pos] = pg;
                L.lblk[pos] = bk;
            }
            if (lane == 0) L.lcount = __popcll(vm);
        }
        __syncthreads();
        const int n_list = L.lcount;
        Q4Piece pc;
        if (n_list > 0) q4_load_piece(p.pool + ((int64_t)L.lpage[0] * (2 * p.Hkv) + 2 * h) * kQ4Slot, tid, pc);
        for (int k = 0; k < n_list; ++k) {
            const int cur_blk = L.lblk[k];
            __syncthreads();  // the previous block's LDS reads are done
            q4_stage_piece(pc, tid, L);
            if (k + 1 < n_list)
                q4_load_piece(p.pool + ((int64_t)L.lpage[k + 1] * (2 * p.Hkv) + 2 * h) * kQ4Slot, tid, pc);
            __syncthreads();
            const int n_tok = min(kQ4Page, kv_len - cur_blk * kQ4Page);

            // scores: tokens 32 wave + 16 j + m16 (j = 0, 1), heads 4 g + r
            float4_t sc[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                sc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
                const uint16_t* krow = L.K + (32 * wave + 16 * j + m16) * kQ4Pitch + 8 * g;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const half8_t kb = *reinterpret_cast<const half8_t*>(krow + 32 * s);
                    sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], kb, sc[j], 0, 0, 0);
                }
            }
            float bmax[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float mx = -INFINITY;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int t = 32 * wave + 16 * j + m16;
                    const float v = t < n_tok ? sc[j][r] * p.scale_log2 : -INFINITY;
                    sc[j][r] = v;
                    mx = fmaxf(mx, v);
                }
#pragma unroll
                for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
                bmax[r] = mx;
            }
            if (m16 == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) L.red[wave][4 * g + r] = bmax[r];
            }
            __syncthreads();
            float alpha[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int hh = 4 * g + r;
                const float mb = fmaxf(fmaxf(L.red[0][hh], L.red[1][hh]), fmaxf(L.red[2][hh], L.red[3][hh]));
                const float mn = fmaxf(m_run[r], mb);
                alpha[r] = exp2f(m_run[r] - mn);  // 0 while the old max is -inf
                m_run[r] = mn;
                float ls = 0.0f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float pv = sc[j][r] == -INFINITY ? 0.0f : exp2f(sc[j][r] - mn);
                    const _Float16 ph = (_Float16)pv;
                    ls += (float)ph;
                    L.P[hh * kQ4Pitch + 32 * wave + 16 * j + m16] = __builtin_bit_cast(uint16_t, ph);
                }
                l_run[r] = l_run[r] * alpha[r] + ls;
            }
            __syncthreads();
            // O[heads][dims 32 wave + 16 j + m16] = alpha O + P V
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) o[j][r] *= alpha[r];
                const uint16_t* vrow = L.Vt + (32 * wave + 16 * j + m16) * kQ4Pitch + 8 * g;
                const uint16_t* prow = L.P + m16 * kQ4Pitch + 8 * g;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const half8_t pa = *reinterpret_cast<const half8_t*>(prow + 32 * s);
                    const half8_t vb = *reinterpret_cast<const half8_t*>(vrow + 32 * s);
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[j], 0, 0, 0);
                }
            }
        }
    }
    // denominators: this lane's shares over the 16 lanes of its head group,
    // then over the four waves
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v = l_run[r];
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 16);
        l_run[r] = v;
    }
    __syncthreads();
    if (m16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) L.lsum[wave][4 * g + r] = l_run[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int hh = 4 * g + r;
        if (hh >= G) continue;
        const float l = L.lsum[0][hh] + L.lsum[1][hh] + L.lsum[2][hh] + L.lsum[3][hh];
        const int64_t oi = ((int64_t)c * p.total_q + i) * p.Hq + h * G + hh;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            p.o_part[oi * kQ4Dim + 32 * wave + 16 * j + m16] = l > 0.0f ? o[j][r] / l : 0.0f;
        if (wave == 0 && m16 == 0) p.lse_part[oi] = l > 0.0f ? m_run[r] + log2f(l) : -INFINITY;
    }
}

// out[i][head][d] = sum_c o_c * 2^(lse_c - M) / sum_c 2^(lse_c - M); zero
// when no chunk saw a token.  One thread per (i, head, d).
__global__ __launch_bounds__(256) void q4_merge_kernel(const float* o_part, const float* lse_part,
                                                       int n_chunks, int total_q, int Hq, void* out,
                                                       int out_dtype, int64_t o_sn, int64_t o_sh) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)total_q * Hq * kQ4Dim) return;
    const int d = (int)(idx % kQ4Dim);
    const int64_t ih = idx / kQ4Dim;
    const int head = (int)(ih % Hq), i = (int)(ih / Hq);
    const int64_t stride = (int64_t)total_q * Hq;
    float M = -INFINITY;
    for (int c = 0; c < n_chunks; ++c) M = fmaxf(M, lse_part[c * stride + ih]);
    float num = 0.0f, den = 0.0f;
    if (M > -INFINITY) {
        for (int c = 0; c < n_chunks; ++c) {
            const float w = exp2f(lse_part[c * stride + ih] - M);
            num += w * o_part[(c * stride + ih) * kQ4Dim + d];
            den += w;
        }
    }
    const float v = den > 0.0f ? num / den : 0.0f;
    const int64_t o = (int64_t)i * o_sn + (int64_t)head * o_sh + d;
    if (out_dtype == 2)
        reinterpret_cast<float*>(out)[o] = v;
    else if (out_dtype == 0)
        reinterpret_cast<uint16_t*>(out)[o] = half_to_bits((half_t)v);
    else {
        uint32_t b = __builtin_bit_cast(uint32_t, v);
        b += 0x7FFFu + ((b >> 16) & 1u);
        reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)(b >> 16);
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

EXL3_API int64_t exl3_nvfp4_page_bytes(int64_t num_kv_heads) {
    return num_kv_heads > 0 ? 2 * num_kv_heads * (int64_t)kQ4Slot : 0;
}

EXL3_API int exl3_nvfp4_pack_pages(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_t,
                                   int64_t max_len, const int32_t* seq_lens,
                                   const int32_t* block_table, int64_t bt_stride,
                                   int64_t max_blocks, void* pool, int64_t num_pages, void* stream) {
    EXL3_CHECK(dtype >= 0 && dtype <= 2, "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(B >= 1 && H >= 1 && max_len >= 1 && max_blocks >= 1 && num_pages >= 1,
               "q4 pack: empty geometry");
    EXL3_CHECK(B * max_len * H * 2 < (1ll << 40), "q4 pack: too many rows");
    EXL3_CHECK(k && v && seq_lens && block_table && pool, "null pointer argument");
    Q4PackParams p = {k, v, dtype, (int)B, (int)H, stride_b, stride_h, stride_t,
                      seq_lens, block_table, bt_stride, (int)max_blocks, (int)max_len,
                      reinterpret_cast<uint8_t*>(pool), num_pages};
    const int64_t units = B * max_len * H * 2;
    q4_pack_kernel<<<(unsigned)((units + 3) / 4), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(p);
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int exl3_nvfp4_dequant_pages(const void* pool, int64_t num_pages, int64_t H, float* out,
                                      void* stream) {
    EXL3_CHECK(num_pages >= 1 && H >= 1 && pool && out, "q4 dequant: bad arguments");
    const int64_t n_slots = num_pages * 2 * H;
    const int64_t bytes = n_slots * kQ4Data;
    q4_dequant_kernel<<<(unsigned)((bytes + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        reinterpret_cast<const uint8_t*>(pool), n_slots, out);
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int exl3_nvfp4_stage_pages(const void* pool, int64_t num_pages, int64_t H, const void* pages,
                                    int pages_dtype, int64_t n, void* stage, int64_t capacity,
                                    void* stream) {
    EXL3_CHECK(num_pages >= 1 && H >= 1 && H <= 65535 && pool && stage, "q4 staging: bad arguments");
    EXL3_CHECK(pages_dtype == 0 || pages_dtype == 1, "q4 staging: page ids are int32 (0) or int64 (1)");
    EXL3_CHECK(n >= 0 && (n == 0 || pages), "q4 staging: bad page list");
    EXL3_CHECK(n + 1 <= capacity, "staging buffer holds %lld pages, need %lld", (long long)(capacity - 1),
               (long long)n);
    EXL3_CHECK(n < (1ll << 31) - 1, "q4 staging: too many pages");
    const dim3 grid((unsigned)(n + 1), (unsigned)H, kQ4Page / kStageTokPerBlock);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    profile_begin_call();
    profile_mark(0, st);
    q4_stage_kernel<<<grid, 256, 0, st>>>(reinterpret_cast<const uint8_t*>(pool), num_pages, (int)H, pages,
                                          pages_dtype, (int)n, reinterpret_cast<uint16_t*>(stage));
    EXL3_LAUNCHED();
    profile_mark(1, st);
    return kOk;
}

EXL3_API int64_t exl3_nvfp4_decode_workspace_size(int64_t total_q, int64_t Hq, int64_t n_chunks) {
    if (total_q < 1 || Hq < 1 || n_chunks < 1) return 0;
    return (int64_t)(((size_t)n_chunks * total_q * Hq * (kQ4Dim + 1) * 4 + 255) & ~(size_t)255);
}

EXL3_API int exl3_nvfp4_sparse_decode(const void* q, int q_dtype, int64_t total_q, int64_t Hq,
                                      int64_t Hkv, int64_t q_stride_n, int64_t q_stride_h,
                                      const void* pool, int64_t num_pages, const int32_t* topk_idx,
                                      int64_t topk_stride_h, int64_t topk_stride_n,
                                      int64_t max_topk, const int32_t* block_table,
                                      int64_t bt_stride, int64_t max_blocks,
                                      const int32_t* seq_lens, int64_t decode_query_len,
                                      float sm_scale, void* out, int out_dtype,
                                      int64_t out_stride_n, int64_t out_stride_h, int64_t n_chunks,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
    EXL3_CHECK(q_dtype >= 0 && q_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
               "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(total_q >= 1 && Hkv >= 1 && Hq % Hkv == 0 && Hq / Hkv <= kQ4MaxGroup,
               "q4 decode: Hq must be a multiple of num_kv_heads, at most 16 per KV head");
    EXL3_CHECK(max_topk >= 1 && decode_query_len >= 1 && total_q % decode_query_len == 0 &&
                   n_chunks >= 1 && max_blocks >= 1 && num_pages >= 1,
               "q4 decode: bad geometry");
    EXL3_CHECK(std::isfinite(sm_scale), "q4 decode: sm_scale must be finite");
    EXL3_CHECK(q && pool && topk_idx && block_table && seq_lens && out, "null pointer argument");
    const int64_t need = exl3_nvfp4_decode_workspace_size(total_q, Hq, n_chunks);
    EXL3_CHECK(workspace && workspace_bytes >= need, "workspace too small: need %lld bytes",
               (long long)need);
    Q4DecodeParams p;
    p.q = q;
    p.q_dtype = q_dtype;
    p.total_q = (int)total_q;
    p.Hq = (int)Hq;
    p.Hkv = (int)Hkv;
    p.G = (int)(Hq / Hkv);
    p.q_sn = q_stride_n;
    p.q_sh = q_stride_h;
    p.pool = reinterpret_cast<const uint8_t*>(pool);
    p.num_pages = num_pages;
    p.topk = topk_idx;
    p.tk_sh = topk_stride_h;
    p.tk_sn = topk_stride_n;
    p.max_topk = (int)max_topk;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.max_blocks = (int)max_blocks;
    p.seq_lens = seq_lens;
    p.dql = (int)decode_query_len;
    p.scale_log2 = sm_scale * 1.4426950408889634f;
    p.n_chunks = (int)n_chunks;
    p.o_part = reinterpret_cast<float*>(workspace);
    p.lse_part = p.o_part + (size_t)n_chunks * total_q * Hq * kQ4Dim;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    static const hipError_t lds_ok = [] {
        hipError_t e = hipFuncSetAttribute((const void*)q4_decode_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Q4Lds));
        if (e != hipSuccess) (void)hipGetLastError();
        return e;
    }();
    EXL3_HIP(lds_ok);
    profile_begin_call();
    profile_mark(0, st);
    q4_decode_kernel<<<dim3((unsigned)(total_q * n_chunks), (unsigned)Hkv), kQ4Threads, sizeof(Q4Lds),
                       st>>>(p);
    EXL3_LAUNCHED();
    profile_mark(1, st);
    const int64_t n = total_q * Hq * kQ4Dim;
    q4_merge_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(p.o_part, p.lse_part, (int)n_chunks,
                                                               (int)total_q, (int)Hq, out, out_dtype,
                                                               out_stride_n, out_stride_h);
    EXL3_LAUNCHED();
    profile_mark(2, st);
    return kOk;
}

EXL3_API int exl3_nvfp4_w1_insert(void* qkv, int64_t num_tokens, int64_t row_width,
                                  const void* q_norm_w, const void* k_norm_w,
                                  const void* index_q_norm_w, const void* index_k_norm_w,
                                  int w_dtype, const void* cos_sin_cache, int cs_dtype,
                                  int64_t max_positions, const int64_t* positions,
                                  int64_t num_heads, int64_t num_kv_heads, int64_t num_index_heads,
                                  int64_t rotary_dim, float eps, const int64_t* slot_mapping,
                                  const int64_t* index_slot_mapping, void* pool, int64_t num_pages,
                                  void* index_cache, int64_t index_rows, void* q_out,
                                  void* index_q_out, void* stream) {
    EXL3_CHECK(num_tokens >= 1, "q4 W1 requires a positive token count");
    EXL3_CHECK(num_heads >= 1 && num_kv_heads >= 1 && num_index_heads >= 0,
               "q4 W1 requires num_heads, num_kv_heads >= 1 and num_index_heads >= 0");
    const int64_t per = num_heads + 2 * num_kv_heads + (num_index_heads > 0 ? num_index_heads + 1 : 0);
    EXL3_CHECK(row_width == per * kQ4Dim, "q4 W1 qkv width %lld does not match the branch layout %lld",
               (long long)row_width, (long long)(per * kQ4Dim));
    EXL3_CHECK(rotary_dim > 0 && rotary_dim <= kQ4Dim && rotary_dim % 8 == 0,
               "q4 W1 requires 0 < rotary_dim <= 128 and rotary_dim %% 8 == 0, got %lld",
               (long long)rotary_dim);
    EXL3_CHECK(w_dtype >= 0 && w_dtype <= 2 && cs_dtype >= 0 && cs_dtype <= 2,
               "dtype ids: 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(max_positions >= 1 && num_pages >= 1 && num_tokens * per < (1ll << 40),
               "q4 W1: empty or oversized geometry");
    EXL3_CHECK(qkv && q_norm_w && k_norm_w && cos_sin_cache && positions && slot_mapping && pool && q_out,
               "null pointer argument");
    EXL3_CHECK(num_index_heads == 0 ||
                   (index_q_norm_w && index_k_norm_w && index_slot_mapping && index_cache &&
                    index_q_out && index_rows >= 1),
               "q4 W1 with index heads needs the index norm weights, slot mapping, cache and "
               "index_q buffer");
    Q4W1Params p = {};
    p.qkv = reinterpret_cast<uint16_t*>(qkv);
    p.row = row_width;
    p.q_out = reinterpret_cast<uint16_t*>(q_out);
    p.index_q_out = reinterpret_cast<uint8_t*>(index_q_out);
    p.norm_w[0] = q_norm_w;
    p.norm_w[1] = k_norm_w;
    p.norm_w[2] = index_q_norm_w;
    p.norm_w[3] = index_k_norm_w;
    p.w_dtype = w_dtype;
    p.cos_sin = cos_sin_cache;
    p.cs_dtype = cs_dtype;
    p.max_pos = max_positions;
    p.positions = positions;
    p.slot_mapping = slot_mapping;
    p.index_slot_mapping = index_slot_mapping;
    p.pool = reinterpret_cast<uint8_t*>(pool);
    p.num_pages = num_pages;
    p.index_cache = reinterpret_cast<uint8_t*>(index_cache);
    p.index_rows = index_rows;
    p.eps = eps;
    p.rotary_dim = (int)rotary_dim;
    p.T = (int)num_tokens;
    p.nq = (int)num_heads;
    p.nkv = (int)num_kv_heads;
    p.niq = (int)num_index_heads;
    const int64_t units = num_tokens * per;
    q4_w1_kernel<<<(unsigned)((units + 3) / 4), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(p);
    EXL3_LAUNCHED();
    return kOk;
}
