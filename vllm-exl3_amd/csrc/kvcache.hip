// Paged int4 KV cache on gfx950: page pack / unpack and the split-K decode
// attention kernel with its log-sum-exp merge.
//
// Replaces the reference's 4-bit KV decode overlay (the Triton
// _q4_decode_kernel + vLLM's split merge, src/vllm_exl3/minimax_q4kv_kernels.py:
// 385-506 and 772-877) for the int4-asymmetric format this build defines:
// per (token, KV head, 32-dim group) an fp16 scale and zero, codes 0..15,
// 16-token pages.  A page of one KV head is 2560 bytes:
//   [   0, 1024)  K codes, token-major, in QK matrix-core operand order
//   [1024, 2048)  V codes, dim-major, in PV matrix-core operand order
//   [2048, 2560)  K scale, K zero, V scale, V zero (128 B each): the zeros
//                 fp16 [4 groups][16 tokens], the scales fp16 [4 token
//                 quads][4 groups][4 tokens]
// so that every lane of a decode wave fetches its K and V codes of a page
// with one 16-byte load each and feeds them to MFMA without any shuffle, and
// its tokens' scales with two 16-byte loads per side (nine loads per page;
// the load count, not the bytes, bounded this kernel: scales as [group]
// [token], eight 8-byte loads, took 171 µs on C4 against 131-143 µs).
//
// Decode (one wave per (sequence, KV head, split of the pages)):
//   QK   S^T[t][h] = sum_g s[t,g] * D_g[t][h] + corr[t][h], where D_g is one
//        v_mfma_f32_16x16x32_f16 of the raw codes (fp16 1024 + n, or
//        1024 + 16 n for the upper nibble of each byte) against the query
//        rows of group g (pre-scaled by sm_scale*log2(e), and by 1/16 on the
//        upper-nibble dims), and corr = sum_g z*Qsum_g - s*1024*Qsum'_g is a
//        16x16x16 MFMA with hi/lo-split fp16 sums, so K is never dequantised
//        element by element;
//   softmax  online in the log2 domain with lazy rescaling (threshold 2^8);
//   PV   O^T[d][h] += V_raw^T . (s * P^T) - 1024 * (s * P^T) per 16-dim block
//        (the offset correction is issued into the same accumulator right
//        after the product, so the running sum never carries the offset),
//        plus one MFMA of [zero rows | ones row] . P^T that yields the
//        zero-point term of every group and the softmax denominator.
// Partials (O normalised by the split's own sum, and its log2-sum-exp) are
// combined by the merge kernel.
#include "exl3_common.h"
#include "profile.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace exl3 {
namespace {

constexpr int kKvF16Id = 0, kKvF32Id = 2;  // dtype ids of the C ABI (1 = bf16)
constexpr int kKvPage = 16;
constexpr int kKvDim = 128;
constexpr int kKvPageBytes = 2560;
constexpr int kOffVQ = 1024, kOffKS = 2048, kOffKZ = 2176, kOffVS = 2304, kOffVZ = 2432;
constexpr int kKvMaxGroup = 16;      // query heads per KV head (one MFMA column block)
constexpr int kKvWaves = 8;          // waves per decode workgroup
constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4* gu4p;

// Exact widening of one activation element (no fp16 rounding).
__device__ __forceinline__ float load_f32(const void* x, int dtype, int64_t idx) {
    if (dtype == kKvF32Id) return reinterpret_cast<const float*>(x)[idx];
    const uint16_t b = reinterpret_cast<const uint16_t*>(x)[idx];
    if (dtype == kKvF16Id) return (float)bits_to_half(b);
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__device__ __forceinline__ void store_f(void* out, int dtype, int64_t idx, float v) {
    if (dtype == kKvF32Id) {
        reinterpret_cast<float*>(out)[idx] = v;
    } else if (dtype == kKvF16Id) {
        reinterpret_cast<uint16_t*>(out)[idx] = half_to_bits((half_t)v);
    } else {
        uint32_t b = __builtin_bit_cast(uint32_t, v);
        b += 0x7FFFu + ((b >> 16) & 1u);
        reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)(b >> 16);
    }
}

// Bit offset of a code inside the page (K: token-major operand order; V:
// dim-major operand order).  The same rules as the CPU oracle's
// kv_k_nibble_bit / kv_v_nibble_bit.
__device__ __forceinline__ int k_code_bit(int t, int d) {
    const int g = d >> 5, r = d & 31, j = r >> 3, p = r & 7;
    return (16 * (t + 16 * j) + 4 * g) * 8 + 4 * p;
}
__device__ __forceinline__ int v_code_bit(int t, int d) {
    const int b = d >> 4, m = d & 15, j = t >> 2, i = t & 3;
    const int ib = (i == 0) ? 0 : (i == 1) ? 16 : (i == 2) ? 4 : 20;
    return (kOffVQ + 16 * (m + 16 * j) + 4 * (b >> 1)) * 8 + 8 * (b & 1) + ib;
}

// Index (fp16 element) of the scale of token t, group g inside a page's scale
// array: [token quad][group][token % 4], so that a decode lane's 16 scales
// (its four tokens in every group) are 32 contiguous bytes, two 16-byte
// loads.  Zeros keep [group][token].
__device__ __forceinline__ int kv_scale_index(int t, int g) { return 16 * (t >> 2) + 4 * g + (t & 3); }

// ---------------------------------------------------------------------------
// Pack: one wave per (sequence, logical page, KV head).
// ---------------------------------------------------------------------------
struct KvPackParams {
    const void* k;
    const void* v;
    int dtype;
    int64_t sb, sh, st;  // element strides of sequence, head, token (dim stride 1)
    const int* seq_lens;
    const int* block_table;
    int64_t bt_stride;
    int max_pages;
    uint8_t* pool;
    int64_t page_stride;  // bytes between physical pages
    int num_pages;
    int B, Hkv;
};

__global__ __launch_bounds__(256) void kv_pack_kernel(KvPackParams p) {
    __shared__ uint8_t codes[4][kKvPage * kKvDim];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = lane & 15, j = lane >> 4;
    const int64_t unit = (int64_t)blockIdx.x * 4 + wv;
    const int64_t units = (int64_t)p.B * p.max_pages * p.Hkv;
    bool active = unit < units;
    int b = 0, lp = 0, h = 0, seq = 0, pg = 0;
    if (active) {
        h = (int)(unit % p.Hkv);
        const int64_t r = unit / p.Hkv;
        lp = (int)(r % p.max_pages);
        b = (int)(r / p.max_pages);
        seq = p.seq_lens[b];
        pg = p.block_table[(int64_t)b * p.bt_stride + lp];
        active = lp * kKvPage < seq && pg >= 0 && pg < p.num_pages;
    }
    uint8_t* base = p.pool + (int64_t)pg * p.page_stride + (int64_t)h * kKvPageBytes;
    const int pos = lp * kKvPage + t;
    const bool tok_ok = active && pos < seq;
    for (int side = 0; side < 2; ++side) {
        const void* src = side ? p.v : p.k;
        uint32_t q[4][8];
        uint16_t s16[4], z16[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                x[e] = tok_ok ? load_f32(src, p.dtype,
                                         (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)pos * p.st +
                                             32 * g + 8 * j + e)
                              : 0.0f;
            float mn = x[0], mx = x[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) {
                mn = fminf(mn, x[e]);
                mx = fmaxf(mx, x[e]);
            }
            mn = fminf(mn, __shfl_xor(mn, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mn = fminf(mn, __shfl_xor(mn, 32, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            // zero = fp16(min); scale = fp16((max - min) / 15) in fp32; codes
            // = clamp(rint((x - zero) / scale), 0, 15) with the fp16 values.
            const half_t zh = f32_to_f16_rne(mn);
            const half_t sh = f32_to_f16_rne((mx - mn) / 15.0f);
            const float zf = (float)zh, sf = (float)sh;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float c = sf > 0.0f ? rintf((x[e] - zf) / sf) : 0.0f;
                c = fminf(fmaxf(c, 0.0f), 15.0f);
                q[g][e] = tok_ok ? (uint32_t)c : 0u;
            }
            s16[g] = tok_ok ? half_to_bits(sh) : 0;
            z16[g] = tok_ok ? half_to_bits(zh) : 0;
        }
        if (side == 0) {
            if (active) {
                u32x4 w;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) word |= q[g][e] << (4 * e);
                    w[g] = word;
                }
                *reinterpret_cast<u32x4*>(base + 16 * lane) = w;
            }
        } else {
            uint8_t* cw = codes[wv];
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) cw[t * kKvDim + 32 * g + 8 * j + e] = (uint8_t)q[g][e];
        }
        if (active && j == 0) {
            const int offs = side ? kOffVS : kOffKS, offz = side ? kOffVZ : kOffKZ;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                *reinterpret_cast<uint16_t*>(base + offs + 2 * kv_scale_index(t, g)) = s16[g];
                *reinterpret_cast<uint16_t*>(base + offz + 2 * (16 * g + t)) = z16[g];
            }
        }
    }
    __syncthreads();
    if (active) {
        // V codes: lane l' = m + 16 j' holds dims 16 b + m, tokens 4 j' + i.
        const uint8_t* cw = codes[wv];
        const int m = lane & 15, jj = lane >> 4;
        u32x4 w;
#pragma unroll
        for (int jw = 0; jw < 4; ++jw) {
            uint32_t word = 0;
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const int d = 16 * (2 * jw + hb) + m;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int ib = (i == 0) ? 0 : (i == 1) ? 16 : (i == 2) ? 4 : 20;
                    word |= (uint32_t)cw[(4 * jj + i) * kKvDim + d] << (8 * hb + ib);
                }
            }
            w[jw] = word;
        }
        *reinterpret_cast<u32x4*>(base + kOffVQ + 16 * lane) = w;
    }
}

// ---------------------------------------------------------------------------
// Unpack (test and staging path): codes * scale + zero in fp32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kv_unpack_kernel(const uint8_t* pool, int64_t page_stride,
                                                        int num_pages, int Hkv, const int* seq_lens,
                                                        const int* block_table, int64_t bt_stride,
                                                        int B, int max_pages, float* k_out,
                                                        float* v_out, int64_t L) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (int64_t)B * max_pages * Hkv) return;
    const int h = (int)(unit % Hkv);
    const int64_t r = unit / Hkv;
    const int lp = (int)(r % max_pages), b = (int)(r / max_pages);
    const int seq = seq_lens[b];
    const int pg = block_table[(int64_t)b * bt_stride + lp];
    if (lp * kKvPage >= seq || pg < 0 || pg >= num_pages) return;
    const uint8_t* base = pool + (int64_t)pg * page_stride + (int64_t)h * kKvPageBytes;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + kOffKS);
    for (int idx = lane; idx < 2 * kKvPage * kKvDim; idx += 64) {
        const int side = idx >= kKvPage * kKvDim;
        const int e = idx - side * kKvPage * kKvDim;
        const int t = e / kKvDim, d = e % kKvDim;
        const int pos = lp * kKvPage + t;
        if (pos >= seq || pos >= L) continue;
        const int bit = side ? v_code_bit(t, d) : k_code_bit(t, d);
        const uint32_t c = (base[bit >> 3] >> (bit & 7)) & 0xFu;
        const int gi = 16 * (d >> 5) + t;
        const float s = (float)bits_to_half(sc[(side ? 128 : 0) + kv_scale_index(t, d >> 5)]);
        const float z = (float)bits_to_half(sc[(side ? 192 : 64) + gi]);
        float* o = side ? v_out : k_out;
        o[(((int64_t)b * Hkv + h) * L + pos) * kKvDim + d] = (float)c * s + z;
    }
}

// ---------------------------------------------------------------------------
// Decode attention
// ---------------------------------------------------------------------------
struct CodeMasks {
    uint32_t lo, hi, magic;
};

struct KvDecodeParams {
    const void* q;
    int q_dtype;
    int64_t q_sb, q_sh;  // element strides of sequence and query head (dim stride 1)
    const uint8_t* pool;
    int64_t page_stride;
    int num_pages;
    const int* block_table;
    int64_t bt_stride;
    int max_pages;
    const int* seq_lens;
    int B, Hq, Hkv, G, S, pps;
    float scale_log2;  // sm_scale * log2(e)
    CodeMasks masks;   // 0x000F000F, 0x00F000F0, 0x64006400
    float* o_part;     // [S][B][Hq][128], normalised by the split's own sum
    float* lse_part;   // [S][B][Hq], log2 domain
};

struct PageRegs {
    u32x4 kq, vq;
    u32x2 ks[4], vs[4];
    uint32_t zk, sk;  // K zero and K scale of (group j, token n), low 16 bits
    u32x2 vz;     // V zeros of group n (n < 4), tokens 4 j .. 4 j + 3
};

// Per-lane byte offsets inside a page (constant over the page loop).
struct PageOffsets {
    int codes;  // 16 lane: K codes at +0, V codes at +1024
    int scl;    // 32 j: the lane's tokens' K scales at +2048, V scales at +2304 (32 B each)
    int kzs;    // 32 j + 2 n: K zero of (group j, token n) at +2176
    int ksn;    // K scale of (group j, token n) at +2048
    int vz;     // 32 min(n, 3) + 8 j: V zeros at +2432
};

// One page through a buffer resource whose base is the page: the address
// arithmetic is scalar and out-of-page offsets would read 0.
__device__ __forceinline__ void load_page(PageRegs& r, const uint8_t* base, const PageOffsets& o) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, kKvPageBytes, 0x00020000);
    r.kq = __builtin_amdgcn_raw_buffer_load_b128(rs, o.codes, 0, 0);
    r.vq = __builtin_amdgcn_raw_buffer_load_b128(rs, o.codes + kOffVQ, 0, 0);
    {
        // the lane's four tokens in all four groups: 32 contiguous bytes per side
        const u32x4 k0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o.scl + kOffKS, 0, 0));
        const u32x4 k1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o.scl + kOffKS + 16, 0, 0));
        const u32x4 v0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o.scl + kOffVS, 0, 0));
        const u32x4 v1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o.scl + kOffVS + 16, 0, 0));
        r.ks[0] = u32x2{k0.x, k0.y};
        r.ks[1] = u32x2{k0.z, k0.w};
        r.ks[2] = u32x2{k1.x, k1.y};
        r.ks[3] = u32x2{k1.z, k1.w};
        r.vs[0] = u32x2{v0.x, v0.y};
        r.vs[1] = u32x2{v0.z, v0.w};
        r.vs[2] = u32x2{v1.x, v1.y};
        r.vs[3] = u32x2{v1.z, v1.w};
    }
    // kept apart until use: combining them here would wait on the loads
    r.zk = __builtin_amdgcn_raw_buffer_load_b16(rs, o.kzs + kOffKZ, 0, 0);
    r.sk = __builtin_amdgcn_raw_buffer_load_b16(rs, o.ksn + kOffKS, 0, 0);
    r.vz = __builtin_amdgcn_raw_buffer_load_b64(rs, o.vz + kOffVZ, 0, 0);
}

// Raw codes as fp16 pairs 1024 + n (or 1024 + 16 n for the upper nibble of a
// byte): one v_bitop3_b32 (w & m) | (magic & ~m) per pair (truth table 0xE2
// for operands a = w, b = m, c = magic).

__device__ __forceinline__ half8_t raw8(uint32_t w, const CodeMasks& m) {
    const uint32_t w8 = w >> 8;
    u32x4 r;
    r.x = __builtin_amdgcn_bitop3_b32(w, m.lo, m.magic, 0xE2);
    r.y = __builtin_amdgcn_bitop3_b32(w, m.hi, m.magic, 0xE2);
    r.z = __builtin_amdgcn_bitop3_b32(w8, m.lo, m.magic, 0xE2);
    r.w = __builtin_amdgcn_bitop3_b32(w8, m.hi, m.magic, 0xE2);
    return __builtin_bit_cast(half8_t, r);
}

__device__ __forceinline__ half4_t raw4(uint32_t w, const CodeMasks& m) {
    u32x2 r;
    r.x = __builtin_amdgcn_bitop3_b32(w, m.lo, m.magic, 0xE2);
    r.y = __builtin_amdgcn_bitop3_b32(w, m.hi, m.magic, 0xE2);
    return __builtin_bit_cast(half4_t, r);
}

__device__ __forceinline__ float half_lo(uint32_t w) { return (float)bits_to_half(w & 0xFFFFu); }
__device__ __forceinline__ float half_hi(uint32_t w) { return (float)bits_to_half(w >> 16); }

__device__ __forceinline__ half2_t as_h2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ void split_hi_lo(float x, half_t& hi, half_t& lo) {
    hi = f32_to_f16_rne(x);
    lo = f32_to_f16_rne(x - (float)hi);
}

// Cross-lane max over the four lane rows that share a lane index mod 16
// (lanes n, n + 16, n + 32, n + 48): two gfx950 permlane swaps, no LDS.  The
// swaps are written as instructions (the optimiser merges the builtins' two
// results into one), each fenced by two wait states on both sides because the
// hazard recogniser does not look inside inline assembly.
__device__ __forceinline__ float rows_max(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    float c = fmaxf(a, b), d = c;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(c), "+v"(d));
    return fmaxf(c, d);
}
__device__ __forceinline__ float rows_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// Eight consecutive query elements (dims d0 .. d0 + 7) widened exactly.
__device__ __forceinline__ void load_q8(const void* q, int dtype, int64_t off, float v[8]) {
    if (dtype == kKvF32Id) {
        const float4_t a = *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(q) + off);
        const float4_t b = *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(q) + off + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
        return;
    }
    const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(q) + off);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t hb = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        v[e] = dtype == kKvF16Id ? (float)bits_to_half(hb) : __builtin_bit_cast(float, hb << 16);
    }
}

template <int DEPTH>
__global__ __launch_bounds__(64 * kKvWaves, 2) void kv_decode_kernel(KvDecodeParams p) {
    const int lane = threadIdx.x & 63, j = lane >> 4, n = lane & 15;
    // wave-uniform control: everything below the unit index lives in SGPRs
    // KV head fastest: the waves of one workgroup read the heads of the same
    // physical pages (contiguous in the pool) at about the same time
    const int unit = __builtin_amdgcn_readfirstlane((int)blockIdx.x * kKvWaves + (int)(threadIdx.x >> 6));
    if (unit >= p.B * p.Hkv * p.S) return;
    const int h = unit % p.Hkv;
    const int bs = unit / p.Hkv;
    const int split = bs % p.S, b = bs / p.S;
    const int seq = p.seq_lens[b];
    const int npg = seq > 0 ? min((seq + kKvPage - 1) / kKvPage, p.max_pages) : 0;
    const int p0 = split * p.pps;
    const int p1 = min(p0 + p.pps, npg);
    const int hq = h * p.G + n;
    const bool qvalid = n < p.G;

    // ---- query operands: group g, lane row j holds dims 32 g + 8 j + perm[s]
    half8_t qb[4];
    float qs[4], qc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        float v[8];
        if (qvalid) {
            load_q8(p.q, p.q_dtype, (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + 32 * g + 8 * j, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
        constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        float s_eff = 0.0f, s_raw = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float f = (s & 2) ? 0.0625f : 1.0f;
            const half_t hv = f32_to_f16_rne(v[perm[s]] * p.scale_log2 * f);
            qb[g][s] = hv;
            s_raw += (float)hv;          // coefficient of the 1024 offset
            s_eff += (float)hv / f;      // coefficient of the code value
        }
        qs[g] = rows_sum(s_eff);
        qc[g] = 1024.0f * rows_sum(s_raw);
    }
    // correction operand: k-slots 4 g .. 4 g + 3 = (Qs_hi, Qs_lo, -C_hi, -C_lo) of group g = j
    half4_t cb;
    {
        const float Qs = j == 0 ? qs[0] : j == 1 ? qs[1] : j == 2 ? qs[2] : qs[3];
        const float Cc = j == 0 ? qc[0] : j == 1 ? qc[1] : j == 2 ? qc[2] : qc[3];
        half_t a, c;
        split_hi_lo(Qs, a, c);
        cb[0] = a;
        cb[1] = c;
        split_hi_lo(-Cc, a, c);
        cb[2] = a;
        cb[3] = c;
    }

    float4_t acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    float4_t accz = float4_t{0.f, 0.f, 0.f, 0.f};
    float m_used = -INFINITY;
    const float4_t zero4 = float4_t{0.f, 0.f, 0.f, 0.f};
    const half8_t neg1024 =
        __builtin_bit_cast(half8_t, u32x4{0xE400E400u, 0xE400E400u, 0xE400E400u, 0xE400E400u});
    const half2_t sixteenth = half2_t{(half_t)0.0625f, (half_t)0.0625f};
    const int* bt = p.block_table + (int64_t)b * p.bt_stride;
    const uint8_t* hbase = p.pool + (int64_t)h * kKvPageBytes;
    PageOffsets offs;
    offs.codes = 16 * lane;
    offs.scl = 32 * j;
    offs.kzs = 32 * j + 2 * n;
    offs.ksn = 2 * kv_scale_index(n, j);
    offs.vz = 32 * min(n, 3) + 8 * j;

    // QK^T of one page, the scale fold and the zero/offset correction; with
    // MASK, tokens at or past seq get -inf.
    auto scores = [&](const PageRegs& r, int lp, float (&sv)[4], auto mask_tag) {
        float4_t d[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(raw8(r.kq[g], p.masks), qb[g], zero4, 0, 0, 0);
        u32x2 cav;
        cav.x = __builtin_amdgcn_perm(r.zk, r.zk, 0x01000100u);  // (zero, zero)
        cav.y = __builtin_amdgcn_perm(r.sk, r.sk, 0x01000100u);  // (scale, scale)
        float4_t sc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, cav), cb, zero4, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = sc[i];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t w = (i < 2) ? r.ks[g].x : r.ks[g].y;
                x += ((i & 1) ? half_hi(w) : half_lo(w)) * d[g][i];
            }
            sv[i] = x;
        }
        if constexpr (decltype(mask_tag)::value) {
            const int tok0 = lp * kKvPage + 4 * j;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (tok0 + i >= seq) sv[i] = -INFINITY;
        }
    };
    // online softmax (log2 domain): rescale only when the running maximum has
    // grown by more than 2^8 (one wave-uniform branch per group of pages)
    auto rescale_to = [&](float mx) {
        if (__builtin_amdgcn_ballot_w64(mx > m_used + 8.0f)) {
            const float m_new = fmaxf(m_used, mx);
            const float alpha = m_used == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_used - m_new);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] *= alpha;
            accz *= alpha;
            m_used = m_new;
        }
    };
    // P V of two pages with 16x16x32 MFMAs (k = 8 j + 4 page + i).  Per group
    // the B operand is s * P (upper-nibble tokens / 16); the offset
    // correction -1024 * (s * P) goes into the same accumulators right after
    // the product; one more MFMA of [zero rows | ones row] . P gives the
    // zero-point term of every group and the softmax denominator.
    auto pv2 = [&](const PageRegs& r0, const PageRegs& r1, const float (&s0)[4],
                   const float (&s1)[4]) {
        half2_t pp[2][2];
        {
            float pr[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[i] = __builtin_amdgcn_exp2f(s0[i] - m_used);
                pr[4 + i] = __builtin_amdgcn_exp2f(s1[i] - m_used);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                pp[q][0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(pr[4 * q], pr[4 * q + 1]));
                pp[q][1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(pr[4 * q + 2], pr[4 * q + 3]));
            }
        }
        const half2_t p0s = pp[0][1] * sixteenth, p1s = pp[1][1] * sixteenth;
        half8_t bp[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            u32x4 u;
            u.x = as_u32(pp[0][0] * as_h2(r0.vs[g].x));
            u.y = as_u32(p0s * as_h2(r0.vs[g].y));
            u.z = as_u32(pp[1][0] * as_h2(r1.vs[g].x));
            u.w = as_u32(p1s * as_h2(r1.vs[g].y));
            bp[g] = __builtin_bit_cast(half8_t, u);
        }
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
            const int sh = 8 * (blk & 1);
            const half4_t a0 = raw4(r0.vq[blk >> 1] >> sh, p.masks);
            const half4_t a1 = raw4(r1.vq[blk >> 1] >> sh, p.masks);
            const half8_t a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
            acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bp[blk >> 1], acc[blk], 0, 0, 0);
        }
#pragma unroll
        for (int blk = 0; blk < 8; ++blk)
            acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg1024, bp[blk >> 1], acc[blk], 0, 0, 0);
        u32x4 za = u32x4{r0.vz.x, r0.vz.y, r1.vz.x, r1.vz.y};
        if (n >= 4) za = (n == 4) ? u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u}
                                  : u32x4{0u, 0u, 0u, 0u};
        const half8_t pb = __builtin_bit_cast(
            half8_t, u32x4{as_u32(pp[0][0]), as_u32(pp[0][1]), as_u32(pp[1][0]), as_u32(pp[1][1])});
        accz = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, za), pb, accz, 0, 0, 0);
    };
    using NoMask = std::integral_constant<bool, false>;
    using Mask = std::integral_constant<bool, true>;

    // ---- page loop.  The block-table entries of up to 256 pages sit one per
    // lane in four registers and are read with readlane; DEPTH pages are in
    // flight and are consumed in pairs.  Loads are unconditional (prefetches
    // past the chunk reload its last page), so the wait counts stay exact and
    // the pipeline never drains inside a chunk.  Each pair of full pages
    // shares one maximum and one rescale decision; the remaining (at most
    // DEPTH) pages, including a partial last page, are masked, and a page past
    // the chunk contributes nothing (all its scores are -inf).
    static_assert(DEPTH % 2 == 0, "pages are consumed in pairs");
    const int nfull = seq >> 4;
    PageRegs ring[DEPTH];
    for (int c0 = p0; c0 < p1; c0 += 256) {
        const int c1 = min(c0 + 256, p1);
        const int cf = min(c1, nfull);
        int btv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = c0 + 64 * k + lane;
            const int v = e < c1 ? bt[e] : 0;
            btv[k] = min(max(v, 0), p.num_pages - 1);
        }
        auto base_of = [&](int lp) {
            const int k = min(lp, c1 - 1) - c0;
            const int v = k < 64 ? btv[0] : k < 128 ? btv[1] : k < 192 ? btv[2] : btv[3];
            const int pg = __builtin_amdgcn_readlane(v, k & 63);
            return hbase + (int64_t)pg * p.page_stride;
        };
#pragma unroll
        for (int dd = 0; dd < DEPTH; ++dd) load_page(ring[dd], base_of(c0 + dd), offs);
        int lp = c0;
        for (; lp + DEPTH <= cf; lp += DEPTH) {
#pragma unroll
            for (int dd = 0; dd < DEPTH; dd += 2) {
                float s0[4], s1[4];
                scores(ring[dd], lp + dd, s0, NoMask{});
                scores(ring[dd + 1], lp + dd + 1, s1, NoMask{});
                const float mx = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                       fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
                rescale_to(rows_max(mx));
                pv2(ring[dd], ring[dd + 1], s0, s1);
                load_page(ring[dd], base_of(lp + dd + DEPTH), offs);
                load_page(ring[dd + 1], base_of(lp + dd + 1 + DEPTH), offs);
            }
        }
#pragma unroll
        for (int dd = 0; dd < DEPTH; dd += 2) {
            if (lp + dd < c1) {
                float s0[4], s1[4];
                scores(ring[dd], lp + dd, s0, Mask{});
                scores(ring[dd + 1], lp + dd + 1, s1, Mask{});
                if (lp + dd + 1 >= c1) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) s1[i] = -INFINITY;
                }
                const float mx = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                       fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
                rescale_to(rows_max(mx));
                pv2(ring[dd], ring[dd + 1], s0, s1);
            }
        }
    }

    // ---- epilogue: zero-point term and denominator from the rows of accz
    float zt[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) zt[g] = __shfl(accz[g], n, 64);
    const float lsum = __shfl(accz[0], 16 + n, 64);
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    if (!qvalid) return;
    const int64_t row = ((int64_t)split * p.B + b) * p.Hq + hq;
    float* o = p.o_part + row * kKvDim;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
        float4_t v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (acc[blk][i] + zt[blk >> 1]) * inv;
        *reinterpret_cast<float4_t*>(o + 16 * blk + 4 * j) = v;
    }
    if (j == 0) p.lse_part[row] = lsum > 0.0f ? m_used + __log2f(lsum) : -INFINITY;
}

// out = sum_s 2^(lse_s - M) O_s / sum_s 2^(lse_s - M), one wave per
// (sequence, query head): lane s holds split s's log-sum-exp (S <= 64), lane
// l accumulates dims 2 l, 2 l + 1; the partial rows are loaded 16 splits at a
// time before they are weighted.
constexpr int kKvMaxSplits = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__global__ __launch_bounds__(256) void kv_merge_kernel(const float* o_part, const float* lse_part,
                                                       int S, int B, int Hq, void* out,
                                                       int out_dtype, int64_t o_sb, int64_t o_sh) {
    const int lane = threadIdx.x & 63;
    const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
    if (row >= B * Hq) return;
    const int hq = row % Hq, b = row / Hq;
    const int64_t stride = (int64_t)B * Hq;
    const float l = lane < S ? lse_part[lane * stride + row] : -INFINITY;
    const float M = wave_max(l);
    const float w = (M == -INFINITY || l == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(l - M);
    const float wsum = wave_sum(w);
    typedef float f2 __attribute__((ext_vector_type(2)));
    f2 acc = f2{0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += 16) {
        f2 o[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
            o[u] = s0 + u < S ? *reinterpret_cast<const f2*>(o_part + ((s0 + u) * stride + row) * kKvDim + 2 * lane)
                              : f2{0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            if (s0 + u < S) {
                const float ws = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s0 + u));
                acc += ws * o[u];
            }
        }
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.0f;
    const int64_t o = (int64_t)b * o_sb + (int64_t)hq * o_sh + 2 * lane;
    store_f(out, out_dtype, o, acc[0] * inv);
    store_f(out, out_dtype, o + 1, acc[1] * inv);
}

int auto_splits(int64_t B, int64_t Hkv, int64_t max_pages) {
    const int64_t want = (2 * 4 * (int64_t)num_cus() + B * Hkv - 1) / (B * Hkv);
    int64_t s = 1;
    while (s < want) s <<= 1;
    return (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(s, kKvMaxSplits), max_pages));
}

}  // namespace
}  // namespace exl3

using namespace exl3;

EXL3_API int64_t exl3_kv_page_bytes(void) { return kKvPageBytes; }

EXL3_API int exl3_kv_pack_pages(const void* k, const void* v, int kv_dtype, int64_t B, int64_t Hkv,
                                int64_t stride_b, int64_t stride_h, int64_t stride_t,
                                const int32_t* seq_lens, const int32_t* block_table,
                                int64_t bt_stride, int64_t max_pages, uint8_t* pool,
                                int64_t num_pages, void* stream) {
    EXL3_CHECK(k && v && seq_lens && block_table && pool, "kv pack: null pointer argument");
    EXL3_CHECK(kv_dtype >= 0 && kv_dtype <= 2, "kv pack: dtype must be 0 (fp16), 1 (bf16) or 2 (fp32)");
    EXL3_CHECK(B >= 1 && Hkv >= 1 && max_pages >= 1 && num_pages >= 1 && bt_stride >= max_pages,
               "kv pack: invalid geometry");
    EXL3_CHECK(B * max_pages * Hkv < ((int64_t)1 << 31) && num_pages < ((int64_t)1 << 31),
               "kv pack: problem too large");
    KvPackParams p = {};
    p.k = k;
    p.v = v;
    p.dtype = kv_dtype;
    p.sb = stride_b;
    p.sh = stride_h;
    p.st = stride_t;
    p.seq_lens = seq_lens;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.max_pages = (int)max_pages;
    p.pool = pool;
    p.page_stride = Hkv * (int64_t)kKvPageBytes;
    p.num_pages = (int)num_pages;
    p.B = (int)B;
    p.Hkv = (int)Hkv;
    const int64_t units = B * max_pages * Hkv;
    kv_pack_kernel<<<(unsigned)((units + 3) / 4), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(p);
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int exl3_kv_unpack_pages(const uint8_t* pool, int64_t num_pages, int64_t Hkv,
                                  const int32_t* seq_lens, const int32_t* block_table,
                                  int64_t bt_stride, int64_t B, int64_t max_pages, float* k_out,
                                  float* v_out, int64_t L, void* stream) {
    EXL3_CHECK(pool && seq_lens && block_table && k_out && v_out, "kv unpack: null pointer argument");
    EXL3_CHECK(B >= 1 && Hkv >= 1 && max_pages >= 1 && num_pages >= 1 && L >= 1 &&
                   bt_stride >= max_pages && B * max_pages * Hkv < ((int64_t)1 << 31),
               "kv unpack: invalid geometry");
    const int64_t units = B * max_pages * Hkv;
    kv_unpack_kernel<<<(unsigned)((units + 3) / 4), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        pool, Hkv * (int64_t)kKvPageBytes, (int)num_pages, (int)Hkv, seq_lens, block_table, bt_stride,
        (int)B, (int)max_pages, k_out, v_out, L);
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int64_t exl3_kv_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv,
                                               int64_t max_pages, int64_t n_splits) {
    if (B < 1 || Hq < 1 || Hkv < 1 || max_pages < 1 || n_splits < 0) return 0;
    const int64_t S = n_splits ? std::min(n_splits, max_pages) : auto_splits(B, Hkv, max_pages);
    return S * B * Hq * (kKvDim + 1) * (int64_t)sizeof(float);
}

EXL3_API int exl3_kv_decode(const void* q, int q_dtype, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t q_stride_b, int64_t q_stride_h, const uint8_t* pool,
                            int64_t num_pages, const int32_t* block_table, int64_t bt_stride,
                            int64_t max_pages, const int32_t* seq_lens, float sm_scale, void* out,
                            int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
                            int64_t n_splits, void* workspace, int64_t workspace_bytes,
                            void* stream) {
    EXL3_CHECK(q && pool && block_table && seq_lens && out, "kv decode: null pointer argument");
    EXL3_CHECK(q_dtype >= 0 && q_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
               "kv decode: dtype ids are 0 fp16, 1 bf16, 2 fp32");
    EXL3_CHECK(B >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0,
               "kv decode: query heads must be a positive multiple of the KV heads");
    EXL3_CHECK(Hq / Hkv <= kKvMaxGroup, "kv decode supports at most %d query heads per KV head",
               kKvMaxGroup);
    EXL3_CHECK(max_pages >= 1 && num_pages >= 1 && bt_stride >= max_pages && n_splits >= 0,
               "kv decode: invalid page geometry");
    EXL3_CHECK(n_splits <= kKvMaxSplits, "kv decode supports at most %d splits", kKvMaxSplits);
    EXL3_CHECK(std::isfinite(sm_scale), "kv decode: sm_scale must be finite");
    EXL3_CHECK(B * Hq * max_pages < ((int64_t)1 << 31), "kv decode: problem too large");
    const int S = n_splits ? (int)std::min(n_splits, max_pages) : auto_splits(B, Hkv, max_pages);
    const int64_t need = (int64_t)S * B * Hq * (kKvDim + 1) * (int64_t)sizeof(float);
    EXL3_CHECK(workspace && workspace_bytes >= need, "kv decode workspace too small: need %lld bytes",
               (long long)need);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    KvDecodeParams p = {};
    p.q = q;
    p.q_dtype = q_dtype;
    p.q_sb = q_stride_b;
    p.q_sh = q_stride_h;
    p.pool = pool;
    p.page_stride = Hkv * (int64_t)kKvPageBytes;
    p.num_pages = (int)num_pages;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.max_pages = (int)max_pages;
    p.seq_lens = seq_lens;
    p.B = (int)B;
    p.Hq = (int)Hq;
    p.Hkv = (int)Hkv;
    p.G = (int)(Hq / Hkv);
    p.S = S;
    p.pps = (int)((max_pages + S - 1) / S);
    p.scale_log2 = sm_scale * 1.4426950408889634f;
    p.masks = CodeMasks{0x000F000Fu, 0x00F000F0u, kMagic};
    p.o_part = reinterpret_cast<float*>(workspace);
    p.lse_part = p.o_part + (int64_t)S * B * Hq * kKvDim;
    profile_begin_call();
    profile_mark(0, st);
    const int64_t units = B * Hkv * S;
    kv_decode_kernel<4><<<(unsigned)((units + kKvWaves - 1) / kKvWaves), 64 * kKvWaves, 0, st>>>(p);
    EXL3_LAUNCHED();
    profile_mark(1, st);
    kv_merge_kernel<<<(unsigned)((B * Hq + 3) / 4), 256, 0, st>>>(p.o_part, p.lse_part, S, (int)B,
                                                                   (int)Hq, out, out_dtype,
                                                                   out_stride_b, out_stride_h);
    EXL3_LAUNCHED();
    profile_mark(2, st);
    return kOk;
}
