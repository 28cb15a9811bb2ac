// Harness over the reference's own dequant_cpu (csrc/bindings.cpp:15-100) --
// TEST INFRASTRUCTURE ONLY.  The reference's translation unit is compiled
// where it lies under the reference checkout (nothing is copied), against the
// torch headers of this image.  Its Python module registration is compiled
// as an unused static function instead of the exported module init, so the
// addresses it takes of CUDA-only entry points (defined in the reference's
// .cu files, which cannot be built here) are never needed; the remaining
// CUDA entry points are called only from functions this harness never calls
// and stay unresolved (lazy binding).  Exported with a C ABI:
//   ref_dequant_cpu   trellis int16 [tiles_k, tiles_n, 16 K], suh / svh fp16
//                     bits, K, mcg -> fp16 [16 tiles_k, 16 tiles_n]
// Load it after torch (the library links libtorch) with RTLD_LAZY.
#include <torch/extension.h>
#undef PYBIND11_MODULE
#define PYBIND11_MODULE(name, variable) [[maybe_unused]] static void ref_module_unused(pybind11::module_& variable)
#include "bindings.cpp"

#include <cstring>

extern "C" int ref_dequant_cpu(const int16_t* trellis, int64_t tiles_k, int64_t tiles_n, const uint16_t* suh,
                               const uint16_t* svh, int64_t bits, int mcg, uint16_t* out) {
    auto t = torch::from_blob(const_cast<int16_t*>(trellis), {tiles_k, tiles_n, 16 * bits}, torch::kInt16);
    auto su = torch::from_blob(const_cast<uint16_t*>(suh), {tiles_k * 16}, torch::kHalf);
    auto sv = torch::from_blob(const_cast<uint16_t*>(svh), {tiles_n * 16}, torch::kHalf);
    auto r = dequant_cpu(t, su, sv, bits, mcg != 0);
    std::memcpy(out, r.data_ptr(), (size_t)r.numel() * 2);
    return 0;
}
