// Seeded synthetic bits for the benchmark and the full-size tests.
//
// Word i of a fill is the SplitMix64 finaliser (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", OOPSLA 2014) of
// seed + (i + 1) * golden-ratio increment, high 32 bits: a counter-based
// generator, so the bits are the same on every device and every launch
// shape, and no library RNG kernel runs (profilers intercept those).
#include "exl3_common.h"

namespace exl3 {
namespace {

__global__ __launch_bounds__(256) void fill_hash_kernel(uint32_t* __restrict__ dst, int64_t n, uint64_t seed) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        uint64_t z = seed + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        dst[i] = (uint32_t)(z >> 32);
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

EXL3_API int exl3_fill_hash_u32(uint32_t* dst, int64_t n_words, uint64_t seed, void* stream) {
    EXL3_CHECK(n_words >= 0 && (n_words == 0 || dst), "fill: n_words must be >= 0 with a destination");
    if (n_words == 0) return kOk;
    const int64_t blocks = (n_words + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 4096 ? blocks : 4096);
    fill_hash_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(dst, n_words, seed);
    EXL3_LAUNCHED();
    return kOk;
}
