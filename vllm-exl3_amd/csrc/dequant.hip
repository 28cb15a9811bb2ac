// Bit-exact EXL3 trellis -> fp16 weight reconstruction on gfx950.
//
// Replaces the reference's host-only dequant_trellis/dequant_cpu
// (csrc/bindings.cpp:15-132), which copies device tensors to the host and
// decodes single-threaded.  One 256-thread workgroup owns one 128x128
// Hadamard block: it stages the block's 64 packed tiles in LDS, decodes them
// to fp32 in their swizzled positions, then runs the two fp32 butterfly
// passes as wavefront shuffles.  Every fp32 operation (each butterfly a+b /
// a-b, the norm and scale multiplies) is the same operation, on the same
// operands, as the reference's scalar loop, so the fp16 result is bit-exact.
#include "exl3_common.h"

namespace exl3 {
namespace {

constexpr int kBlock = 128;
constexpr int kLdsStride = kBlock + 1;  // column pass reads stride 129: conflict-free

// Tile index -> (row, col) within the 16x16 tile: the reference's fragment
// swizzle (csrc/bindings.cpp:37-77) as a bit permutation of the index.
__device__ __forceinline__ int tile_row(int b) {
    return (b & 1) | (((b >> 3) & 1) << 1) | (((b >> 4) & 1) << 2) | (((b >> 1) & 1) << 3);
}
__device__ __forceinline__ int tile_col(int b) {
    return ((b >> 5) & 1) | (((b >> 6) & 1) << 1) | (((b >> 7) & 1) << 2) | (((b >> 2) & 1) << 3);
}

// One 128-point unnormalised butterfly held as two values per lane
// (element l in v0, element l+64 in v1), strides 1..64 in the reference's
// order.  The upper element of each pair takes (lower - upper), exactly the
// reference's `a - b`.
__device__ __forceinline__ void butterfly128(float& v0, float& v1, int lane) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        float p0 = __shfl_xor(v0, s, 64);
        float p1 = __shfl_xor(v1, s, 64);
        if (lane & s) {
            v0 = p0 - v0;
            v1 = p1 - v1;
        } else {
            v0 = v0 + p0;
            v1 = v1 + p1;
        }
    }
    float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
}

template <int CB>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ trellis,
                                                     int tiles_n, int K,
                                                     const uint16_t* __restrict__ suh,
                                                     const uint16_t* __restrict__ svh,
                                                     uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ uint32_t lds_raw[];
    float* mat = reinterpret_cast<float*>(lds_raw);            // [128][129]
    uint32_t* words = lds_raw + kBlock * kLdsStride;           // [64][8K]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n32 = 8 * K;                                     // uint32 words per tile
    const int cb0 = blockIdx.x * 8;                            // first tile column
    const int kb0 = blockIdx.y * 8;                            // first tile row
    const int cols = tiles_n * 16;

    // Stage the 8x8 tiles: for each tile row the 8 tiles are contiguous.
    for (int w = tid; w < 64 * n32; w += 256) {
        int t = w / n32, i = w - t * n32;
        int kt = kb0 + (t >> 3), nt = cb0 + (t & 7);
        words[w] = trellis[((size_t)kt * tiles_n + nt) * n32 + i];
    }
    __syncthreads();

    // Decode: thread -> (tile, 64 consecutive indices).
    {
        const int t = tid >> 2;
        const uint32_t* tw = words + t * n32;
        const int rbase = (t >> 3) * 16, cbase = (t & 7) * 16;
        const uint32_t nbits = 256u * K;
        for (int j = 0; j < 64; ++j) {
            int idx = (tid & 3) * 64 + j;
            uint32_t bit = ((uint32_t)(idx + 1) * K + nbits - 16u) % nbits;
            uint32_t i0 = bit >> 5;
            uint32_t i1 = i0 + 1 == (uint32_t)n32 ? 0 : i0 + 1;
            uint32_t win = funnel(tw[i0], tw[i1], 48u - (bit & 31u)) & 0xFFFFu;
            float v = (float)decode_weight<CB>(win);
            mat[(rbase + tile_row(idx)) * kLdsStride + cbase + tile_col(idx)] = v;
        }
    }
    __syncthreads();

    // Pass 1: along each row (output dimension), then * norm.
    for (int r = wave * 32; r < wave * 32 + 32; ++r) {
        float v0 = mat[r * kLdsStride + lane];
        float v1 = mat[r * kLdsStride + lane + 64];
        butterfly128(v0, v1, lane);
        mat[r * kLdsStride + lane] = v0 * kHadNorm;
        mat[r * kLdsStride + lane + 64] = v1 * kHadNorm;
    }
    __syncthreads();

    // Pass 2: along each column (input dimension), then
    // ((v * norm) * suh[r]) * svh[c], one RNE to fp16 (kept in LDS as fp16
    // bit patterns reinterpreted through the float slots).
    const int row0 = blockIdx.y * kBlock, col0 = blockIdx.x * kBlock;
    const float su0 = (float)bits_to_half(suh[row0 + lane]);
    const float su1 = (float)bits_to_half(suh[row0 + lane + 64]);
    for (int c = wave * 32; c < wave * 32 + 32; ++c) {
        float v0 = mat[lane * kLdsStride + c];
        float v1 = mat[(lane + 64) * kLdsStride + c];
        butterfly128(v0, v1, lane);
        const float sv = (float)bits_to_half(svh[col0 + c]);
        float a0 = v0 * kHadNorm;
        float a1 = v1 * kHadNorm;
        a0 = a0 * su0;
        a1 = a1 * su1;
        a0 = a0 * sv;
        a1 = a1 * sv;
        mat[lane * kLdsStride + c] = __builtin_bit_cast(float, (uint32_t)half_to_bits(f32_to_f16_rne(a0)));
        mat[(lane + 64) * kLdsStride + c] = __builtin_bit_cast(float, (uint32_t)half_to_bits(f32_to_f16_rne(a1)));
    }
    __syncthreads();

    // Coalesced store: each thread writes 2 fp16 per step along a row.
    for (int e = tid; e < kBlock * kBlock / 2; e += 256) {
        int r = e >> 6, c = (e & 63) * 2;
        uint32_t lo = __builtin_bit_cast(uint32_t, mat[r * kLdsStride + c]) & 0xFFFFu;
        uint32_t hi = __builtin_bit_cast(uint32_t, mat[r * kLdsStride + c + 1]) & 0xFFFFu;
        *reinterpret_cast<uint32_t*>(out + (size_t)(row0 + r) * cols + col0 + c) = lo | (hi << 16);
    }
}

// Decode only (no rotation, no scales): fp16 codebook values at their
// swizzled positions.  Used to check the decode stage on its own.
template <int CB>
__global__ __launch_bounds__(256) void decode_tiles_kernel(const uint32_t* __restrict__ trellis,
                                                          int tiles_n, int K, int ntiles,
                                                          uint16_t* __restrict__ out) {
    const int t = blockIdx.x;  // one tile per block, 256 threads = 256 indices
    if (t >= ntiles) return;
    const int n32 = 8 * K;
    const uint32_t* tw = trellis + (size_t)t * n32;
    const int idx = threadIdx.x;
    const uint32_t nbits = 256u * K;
    uint32_t bit = ((uint32_t)(idx + 1) * K + nbits - 16u) % nbits;
    uint32_t i0 = bit >> 5;
    uint32_t i1 = i0 + 1 == (uint32_t)n32 ? 0 : i0 + 1;
    uint32_t win = funnel(tw[i0], tw[i1], 48u - (bit & 31u)) & 0xFFFFu;
    const int kt = t / tiles_n, nt = t - kt * tiles_n;
    const int cols = tiles_n * 16;
    out[(size_t)(kt * 16 + tile_row(idx)) * cols + nt * 16 + tile_col(idx)] =
        half_to_bits(decode_weight<CB>(win));
}

// ---------------------------------------------------------------------------
// n-gram embedding rows (ngram_dequant; pure-torch twin
// ngram_dequant_rows_torch, src/vllm_exl3/exl3.py:5170-5238): a packed row is
// one fp16 scale word plus a ring bitstream of 160 K-bit values (LSB-first
// in int16 words).  Element i's 16-bit mul1 state holds ring values i, i-1,
// i-2, ... (mod 160) in its K-bit groups 0, 1, 2, ...; the value is
// fp16(codebook(state) * scale + head_bias[head]).  One wave per row: the
// row's words are staged in LDS, lane l decodes elements l, l + 64, l + 128.
// ---------------------------------------------------------------------------
constexpr int kNgramDim = 160;
constexpr int kNgramMaxWords = 1 + kNgramDim * 8 / 16;  // K <= 8

__global__ __launch_bounds__(256) void ngram_kernel(const int16_t* __restrict__ packed, int64_t n_rows,
                                                   int64_t row_stride, int bits,
                                                   const int64_t* __restrict__ heads,
                                                   const uint16_t* __restrict__ head_bias,
                                                   int64_t num_heads, uint16_t* __restrict__ out) {
    __shared__ uint32_t lds[4][kNgramMaxWords + 1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + w;
    if (row >= n_rows) return;  // wave-uniform
    const int words = 1 + kNgramDim * bits / 16;
    const int16_t* src = packed + row * row_stride;
    for (int j = lane; j < words; j += 64) lds[w][j] = (uint16_t)src[j];
    if (lane == 0) lds[w][words] = 0;  // a 2-word read at the last word stays defined
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const float scale = (float)bits_to_half(lds[w][0]);
    const int64_t head = heads[row];
    const bool hok = head >= 0 && head < num_heads;
    const int groups = (16 + bits - 1) / bits;
    const uint32_t kmask = (1u << bits) - 1u;
    for (int i = lane; i < kNgramDim; i += 64) {
        uint32_t state = 0;
        for (int j = 0; j < groups; ++j) {
            int p = i - j;
            if (p < 0) p += kNgramDim;
            const int sb = p * bits;                 // first stream bit of ring value p
            const int wi = 1 + (sb >> 4), bi = sb & 15;
            const uint32_t two = lds[w][wi] | (lds[w][wi + 1] << 16);
            state |= ((two >> bi) & kmask) << (j * bits);
        }
        const float v = (float)decode_weight<kCbMul1>(state & 0xFFFFu);
        const float b = hok ? (float)bits_to_half(head_bias[head * kNgramDim + i]) : 0.0f;
        out[row * kNgramDim + i] = half_to_bits(f32_to_f16_rne(v * scale + b));
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

EXL3_API int exl3_dequant_trellis(const int16_t* trellis, int64_t tiles_k, int64_t tiles_n,
                                  int64_t K, int codebook, const uint16_t* suh,
                                  const uint16_t* svh, uint16_t* out, void* stream) {
    EXL3_CHECK(K == 2 || K == 3 || K == 4 || K == 8, "K must be one of 2, 3, 4, or 8");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(tiles_k > 0 && tiles_n > 0, "trellis dimensions must be positive");
    EXL3_CHECK((tiles_k * 16) % 128 == 0 && (tiles_n * 16) % 128 == 0,
               "trellis dimensions must reconstruct whole 128-element Hadamard blocks");
    EXL3_CHECK(tiles_k * 16 <= 65535 * 128 && tiles_n * 16 <= 0x7FFFFFFF / 128,
               "trellis dimensions exceed the launch grid");
    EXL3_CHECK(trellis && suh && svh && out, "null pointer argument");
    dim3 grid((unsigned)(tiles_n / 8), (unsigned)(tiles_k / 8));
    size_t lds = sizeof(float) * 128 * 129 + sizeof(uint32_t) * 64 * 8 * K;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint32_t* t32 = reinterpret_cast<const uint32_t*>(trellis);
    // The fp32 block alone is 66 KB of LDS: raise the dynamic-LDS cap once.
    static const hipError_t attr_status = [] {
        const int cap = 160 * 1024;
        hipError_t e = hipFuncSetAttribute((const void*)dequant_kernel<0>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, cap);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)dequant_kernel<1>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, cap);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)dequant_kernel<2>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, cap);
        if (e != hipSuccess) (void)hipGetLastError();
        return e;
    }();
    EXL3_HIP(attr_status);
    switch (codebook) {
        case 0: dequant_kernel<0><<<grid, 256, lds, s>>>(t32, (int)tiles_n, (int)K, suh, svh, out); break;
        case 1: dequant_kernel<1><<<grid, 256, lds, s>>>(t32, (int)tiles_n, (int)K, suh, svh, out); break;
        default: dequant_kernel<2><<<grid, 256, lds, s>>>(t32, (int)tiles_n, (int)K, suh, svh, out); break;
    }
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int exl3_decode_tiles(const int16_t* trellis, int64_t tiles_k, int64_t tiles_n, int64_t K,
                               int codebook, uint16_t* out, void* stream) {
    EXL3_CHECK(K >= 1 && K <= 8, "K must be in 1..8");
    EXL3_CHECK(codebook >= 0 && codebook <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
    EXL3_CHECK(tiles_k > 0 && tiles_n > 0 && tiles_k * tiles_n <= 0x7FFFFFFF,
               "trellis dimensions must be positive and fit the launch grid");
    EXL3_CHECK(trellis && out, "null pointer argument");
    int nt = (int)(tiles_k * tiles_n);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint32_t* t32 = reinterpret_cast<const uint32_t*>(trellis);
    switch (codebook) {
        case 0: decode_tiles_kernel<0><<<nt, 256, 0, s>>>(t32, (int)tiles_n, (int)K, nt, out); break;
        case 1: decode_tiles_kernel<1><<<nt, 256, 0, s>>>(t32, (int)tiles_n, (int)K, nt, out); break;
        default: decode_tiles_kernel<2><<<nt, 256, 0, s>>>(t32, (int)tiles_n, (int)K, nt, out); break;
    }
    EXL3_LAUNCHED();
    return kOk;
}

EXL3_API int exl3_ngram_dequant(const int16_t* packed, int64_t n_rows, int64_t row_stride, int bits,
                                const int64_t* heads, const uint16_t* head_bias, int64_t num_heads,
                                uint16_t* out, void* stream) {
    EXL3_CHECK(bits >= 1 && bits <= 8, "ngram_dequant supports 1 <= bits <= 8, got %d", bits);
    EXL3_CHECK(n_rows >= 0 && num_heads >= 1, "ngram_dequant: bad row or head count");
    EXL3_CHECK(row_stride >= 1 + kNgramDim * bits / 16, "ngram_dequant: rows need %d words",
               1 + kNgramDim * bits / 16);
    if (n_rows == 0) return kOk;
    EXL3_CHECK(packed && heads && head_bias && out, "null pointer argument");
    ngram_kernel<<<(unsigned)((n_rows + 3) / 4), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        packed, n_rows, row_stride, bits, heads, head_bias, num_heads, out);
    EXL3_LAUNCHED();
    return kOk;
}
