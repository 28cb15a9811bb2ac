/*
 * CPU oracle for the EXL3 trellis decode -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference's host dequantiser so that
 * the HIP kernels can be checked bit-for-bit.  Only tests/, the smoke entry
 * point and bench.py's cpu_baseline leg may load it; the product path never
 * does.  Build: `make -C oracle` (gcc -O2 -ffp-contract=off).
 *
 * Every function cites the reference file:line it follows
 * (paths relative to the vllm-exl3 repository root).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* IEEE binary16 -> binary32, exact.  csrc/exl3_dequant.cuh:25-38 */
float oc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: man * 2^-24, exact in binary32 */
            float v = ldexpf((float)man, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN kept
 * quiet.  csrc/exl3_dequant.cuh:40-86 (same result for every input; written
 * from the IEEE definition). */
uint16_t oc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e = (x >> 23) & 0xFFu;
    uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFFu) {
        if (m == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7C00u | 0x200u | (m >> 13));
    }
    int32_t ue = (int32_t)e - 127;          /* unbiased exponent */
    if (ue > 15) return (uint16_t)(sign | 0x7C00u);
    if (ue >= -14) {
        /* normal half candidate: 10 kept mantissa bits, 13 dropped */
        uint32_t keep = m >> 13;
        uint32_t drop = m & 0x1FFFu;
        uint32_t he = (uint32_t)(ue + 15);
        uint32_t out = (he << 10) | keep;
        if (drop > 0x1000u || (drop == 0x1000u && (keep & 1u))) out += 1; /* carry may bump exponent */
        if (out >= 0x7C00u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | out);
    }
    /* subnormal half: value = sig * 2^(ue-23); unit is 2^-24 */
    if (e == 0) return (uint16_t)sign; /* binary32 subnormals are far below 2^-25 */
    uint32_t sig = m | 0x800000u;
    int32_t shift = -ue - 1;                /* 14 .. ; sig >> shift counts 2^-24 units */
    if (shift >= 32) return (uint16_t)sign;
    uint32_t q = sig >> shift;
    uint32_t rem = sig & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q);
}

/* Procedural codebooks.  csrc/exl3_dequant.cuh:105-124,
 * src/vllm_exl3/dequant.py:99-112.
 *   cb 0 (3INST): x = w*89226354 + 64248484, masked, sum of halves
 *   cb 1 (MCG):   x = w*0xCBAC1FED,          masked, sum of halves
 *   cb 2 (mul1):  x = w*0x83DCD12D, byte sum s, half(s)*half(0x1eee)+half(0xc931)
 * Each returns the binary16 bit pattern after one RNE rounding. */
uint16_t oc_decode_codebook(uint16_t window, int cb) {
    uint32_t w = window;
    if (cb == 0 || cb == 1) {
        uint32_t x = (cb == 0) ? (w * 89226354u + 64248484u) : (w * 0xCBAC1FEDu);
        x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;   /* LOP3 0x6a == (a & b) ^ c */
        float s = oc_f16_to_f32((uint16_t)(x & 0xFFFFu)) + oc_f16_to_f32((uint16_t)(x >> 16));
        return oc_f32_to_f16(s);
    }
    uint32_t x = w * 0x83DCD12Du;
    uint32_t s = 0x6400u + (x & 0xFFu) + ((x >> 8) & 0xFFu) + ((x >> 16) & 0xFFu) + (x >> 24);
    float v = oc_f16_to_f32((uint16_t)s) * oc_f16_to_f32(0x1EEEu) + oc_f16_to_f32(0xC931u);
    return oc_f32_to_f16(v);
}

/* 16-bit window of the tile's circular bit stream starting at stream bit
 * `bit` (mod 256*K).  The tile is 8*K uint32 words, word i = u16[2i] |
 * u16[2i+1] << 16, bits numbered MSB-first inside each word.
 * csrc/exl3_dequant.cuh:141-159. */
uint16_t oc_read_window(const uint16_t* tile, int K, uint32_t bit) {
    uint32_t nbits = 256u * (uint32_t)K;
    uint32_t n32 = 8u * (uint32_t)K;
    bit %= nbits;
    uint32_t i0 = bit / 32u;
    uint32_t i1 = (i0 + 1u) % n32;
    uint64_t a = (uint64_t)tile[2 * i0] | ((uint64_t)tile[2 * i0 + 1] << 16);
    uint64_t b = (uint64_t)tile[2 * i1] | ((uint64_t)tile[2 * i1 + 1] << 16);
    uint64_t merged = (a << 32) | b;
    return (uint16_t)((merged >> (48u - (bit % 32u))) & 0xFFFFu);
}

/* Weight index i in [0,256) of a tile reads the window that ends at stream
 * bit (i+1)*K, i.e. starts at (i+257)*K-16 mod 256K.
 * csrc/exl3_dequant.cuh:161-166, csrc/bindings.cpp:44-46. */
uint16_t oc_decode_index(const uint16_t* tile, int K, int index, int cb) {
    uint32_t start = (uint32_t)(index + 257) * (uint32_t)K - 16u;
    return oc_decode_codebook(oc_read_window(tile, K, start), cb);
}

/* Position of weight index i inside the 16x16 tile (rows = input dim).
 * The reference's lane/fragment swizzle (csrc/bindings.cpp:37-77) is a pure
 * bit permutation of the 8-bit index:
 *   row = b0 | b3<<1 | b4<<2 | b1<<3,  col = b5 | b6<<1 | b7<<2 | b2<<3. */
void oc_tile_position(int index, int* row, int* col) {
    int b = index;
    *row = (b & 1) | (((b >> 3) & 1) << 1) | (((b >> 4) & 1) << 2) | (((b >> 1) & 1) << 3);
    *col = ((b >> 5) & 1) | (((b >> 6) & 1) << 1) | (((b >> 7) & 1) << 2) | (((b >> 2) & 1) << 3);
}

/* Literal restatement of the swizzle loop of csrc/bindings.cpp:51-75, used by
 * the tests to pin oc_tile_position (two independent spellings). */
void oc_tile_position_loop(int pos_row[256], int pos_col[256]) {
    for (int l = 0; l < 32; ++l) {
        if (l & 4) continue;
        int row0 = (l % 4) * 2, row2 = row0 + 8, col0 = (l / 8) * 2, col4 = col0 + 8;
        int rows[8] = {row0, row0 + 1, row2, row2 + 1, row0, row0 + 1, row2, row2 + 1};
        int cols[8] = {col0, col0, col0, col0, col4, col4, col4, col4};
        for (int j = 0; j < 8; ++j) {
            pos_row[l * 8 + j] = rows[j];
            pos_col[l * 8 + j] = cols[j];
            pos_row[(l + 4) * 8 + j] = rows[j];
            pos_col[(l + 4) * 8 + j] = cols[j] + 1;
        }
    }
}

/* In-place unnormalised Walsh-Hadamard butterfly, strides 1,2,..,n/2.
 * csrc/exl3_dequant.cuh:168-179. */
void oc_hadamard(float* v, int n) {
    for (int stride = 1; stride < n; stride <<= 1)
        for (int base = 0; base < n; base += stride << 1)
            for (int i = 0; i < stride; ++i) {
                float a = v[base + i], b = v[base + stride + i];
                v[base + i] = a + b;
                v[base + stride + i] = a - b;
            }
}

/* Decode tiles only (no Hadamard, no scales): out_f32[rows*cols] holds the
 * codebook values at their swizzled positions.  csrc/bindings.cpp:37-77. */
void oc_decode_tiles(const int16_t* trellis, int tiles_k, int tiles_n, int K, int cb,
                     float* out) {
    const int cols = tiles_n * 16;
    const size_t words = 16u * (size_t)K;
    for (int kt = 0; kt < tiles_k; ++kt)
        for (int nt = 0; nt < tiles_n; ++nt) {
            const uint16_t* tile = (const uint16_t*)(trellis + ((size_t)kt * tiles_n + nt) * words);
            for (int i = 0; i < 256; ++i) {
                int r, c;
                oc_tile_position(i, &r, &c);
                out[(size_t)(kt * 16 + r) * cols + nt * 16 + c] =
                    oc_f16_to_f32(oc_decode_index(tile, K, i, cb));
            }
        }
}

/* Full dequant: fp16 W[in,out] = diag(suh) H Wq H diag(svh) / 128 per
 * 128x128 block, with the reference's exact fp32 operation order:
 * pass 1 along each row (output dim) then x norm; pass 2 along each column
 * (input dim) then ((v*norm)*suh[r])*svh[c]; one RNE to fp16.
 * csrc/bindings.cpp:15-100. */
void oc_dequant(const int16_t* trellis, int tiles_k, int tiles_n, int K, int cb,
                const uint16_t* suh, const uint16_t* svh, uint16_t* out) {
    const int rows = tiles_k * 16, cols = tiles_n * 16;
    float* m = (float*)malloc(sizeof(float) * (size_t)rows * cols);
    oc_decode_tiles(trellis, tiles_k, tiles_n, K, cb, m);
    const float norm = 0.08838834764831845f;
    float line[128];
    for (int r0 = 0; r0 < rows; r0 += 128)
        for (int c0 = 0; c0 < cols; c0 += 128) {
            for (int r = 0; r < 128; ++r) {
                float* p = m + (size_t)(r0 + r) * cols + c0;
                for (int c = 0; c < 128; ++c) line[c] = p[c];
                oc_hadamard(line, 128);
                for (int c = 0; c < 128; ++c) p[c] = line[c] * norm;
            }
            for (int c = 0; c < 128; ++c) {
                for (int r = 0; r < 128; ++r) line[r] = m[(size_t)(r0 + r) * cols + c0 + c];
                oc_hadamard(line, 128);
                float sv = oc_f16_to_f32(svh[c0 + c]);
                for (int r = 0; r < 128; ++r) {
                    float v = line[r] * norm;
                    v = v * oc_f16_to_f32(suh[r0 + r]);
                    v = v * sv;
                    out[(size_t)(r0 + r) * cols + c0 + c] = oc_f32_to_f16(v);
                }
            }
        }
    free(m);
}
