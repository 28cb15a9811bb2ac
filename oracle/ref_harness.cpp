// Harness over the reference's own host-side EXL3 primitives -- TEST
// INFRASTRUCTURE ONLY.  It compiles csrc/exl3_dequant.cuh where it lies under
// the reference checkout (nothing is copied) and exports its primitives with a
// C ABI so the tests can pin the oracle against the real reference code:
//   decode_codebook_bits  csrc/exl3_dequant.cuh:105-124 (all three codebooks)
//   read_window           csrc/exl3_dequant.cuh:141-159
//   hadamard              csrc/exl3_dequant.cuh:168-179
//   float_to_half_bits    csrc/exl3_dequant.cuh:40-86
//   half_bits_to_float    csrc/exl3_dequant.cuh:25-38
// The full dequant_cpu (csrc/bindings.cpp:15-100) is built separately by
// ref_dequant_harness.cpp (its translation unit needs the torch headers).
#include <cstddef>
#include <cstdint>
#include "exl3_dequant.cuh"

extern "C" {
uint16_t ref_decode_codebook_bits(uint16_t window, int cb) {
    return vllm_exl3::decode_codebook_bits(window, cb);
}
uint16_t ref_read_window(const uint16_t* packed, size_t words, size_t bit) {
    return vllm_exl3::read_window(packed, words, bit);
}
void ref_hadamard(float* values, int n) { vllm_exl3::hadamard(values, n); }
uint16_t ref_float_to_half_bits(float v) { return vllm_exl3::float_to_half_bits(v); }
float ref_half_bits_to_float(uint16_t b) { return vllm_exl3::half_bits_to_float(b); }
}
