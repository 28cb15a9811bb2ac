// Shared device helpers and host error plumbing for the MI355X (gfx950)
// EXL3 kernels.  Everything here is CDNA4-specific: 64-lane wavefronts,
// ds_bpermute/DPP cross-lane moves, v_bitop3 masks, MFMA f16 tiles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#define EXL3_API extern "C" __attribute__((visibility("default")))

namespace exl3 {

// --------------------------------------------------------------------------
// Host-side error reporting (thread-local message, negative status codes).
// --------------------------------------------------------------------------
enum Status : int { kOk = 0, kInvalid = -1, kHipError = -2, kWorkspace = -3 };

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* get_error();

#define EXL3_CHECK(cond, ...)              \
    do {                                   \
        if (!(cond)) {                     \
            ::exl3::set_error(__VA_ARGS__); \
            return ::exl3::kInvalid;       \
        }                                  \
    } while (0)

#define EXL3_HIP(call)                                                          \
    do {                                                                        \
        hipError_t _e = (call);                                                 \
        if (_e != hipSuccess) {                                                 \
            ::exl3::set_error("HIP error %s at %s:%d", hipGetErrorString(_e),   \
                              __FILE__, __LINE__);                              \
            return ::exl3::kHipError;                                           \
        }                                                                       \
    } while (0)

// Launch check: a launch failure is reported synchronously by the runtime.
#define EXL3_LAUNCHED() EXL3_HIP(hipGetLastError())

inline int num_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 256;
        return n > 0 ? n : 256;
    }();
    return cus;
}

// --------------------------------------------------------------------------
// Device helpers
// --------------------------------------------------------------------------
typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr float kHadNorm = 0.08838834764831845f;  // 1/sqrt(128) as fp32

__device__ __forceinline__ half_t bits_to_half(uint32_t b) {
    return __builtin_bit_cast(half_t, (uint16_t)b);
}
__device__ __forceinline__ uint16_t half_to_bits(half_t h) {
    return __builtin_bit_cast(uint16_t, h);
}

// fp32 -> fp16 with the fp32 value materialised first.  Without the register
// barrier the backend folds a preceding fp32 multiply into v_fma_mix*_f16,
// rounding the exact product once instead of rounding to fp32 and then to
// fp16 as a scalar CPU does (even under fp contract(off)).
__device__ __forceinline__ half_t f32_to_f16_rne(float x) {
    asm volatile("" : "+v"(x));
    return (half_t)x;
}

// Codebook ids (the reference's mcg/mul1 flags extended with 3INST):
// 0 = 3INST, 1 = MCG, 2 = mul1.
enum Codebook : int { kCb3Inst = 0, kCbMcg = 1, kCbMul1 = 2 };

// 32-bit codebook product for the two "sum of halves" codebooks, already
// masked: returns a packed pair (lo half, hi half) whose fp16 sum is the
// weight.  For 3INST the additive constant is folded in.
template <int CB>
__device__ __forceinline__ uint32_t cb_pair(uint32_t w) {
    uint32_t x = (CB == kCb3Inst) ? (w * 89226354u + 64248484u) : (w * 0xCBAC1FEDu);
    return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Exact decode of one 16-bit window to the fp16 weight (one RNE rounding).
template <int CB>
__device__ __forceinline__ half_t decode_weight(uint32_t w) {
    if constexpr (CB == kCbMul1) {
        uint32_t x = w * 0x83DCD12Du;
        uint32_t s = 0x6400u + (x & 0xFFu) + ((x >> 8) & 0xFFu) + ((x >> 16) & 0xFFu) + (x >> 24);
        // half(s)*half(0x1eee) is exact in fp32 and so is the sum with
        // half(0xc931) (|numerator| < 2^20 over 2^18), so one cvt rounds once.
        float v = (float)bits_to_half(s) * (float)bits_to_half(0x1EEEu) +
                  (float)bits_to_half(0xC931u);
        return (half_t)v;
    } else {
        uint32_t x = cb_pair<CB>(w);
        return bits_to_half(x & 0xFFFFu) + bits_to_half(x >> 16);
    }
}

// Funnel shift: bits [s, s+32) of the 64-bit value hi:lo.
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> s);
}

}  // namespace exl3
