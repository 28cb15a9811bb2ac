// The large-m side of the dense EXL3 linear (implementation in fatgemm.hip):
// rotate the input rows, one fat GEMM, one output pass (128-Hadamard x svh,
// optional bias) - the weights are decoded once per 256 rows instead of being
// streamed once per 16 rows by the decode GEMV.
#pragma once

#include "exl3_common.h"

namespace exl3 {

// Rows from which exl3_linear takes the fat path (measured crossover on
// MI355X, bench.py --linear-crossover).
constexpr int64_t kLinearFatMinRows = 256;

size_t linear_fat_workspace_bytes(int64_t m, int64_t in_f, int64_t out_f);

// Arguments already validated by the caller; workspace of at least
// linear_fat_workspace_bytes().
int linear_fat(const void* x, int x_dtype, int64_t m, const int16_t* trellis, int64_t tiles_k,
               int64_t tiles_n, int64_t K, int codebook, const uint16_t* suh, const uint16_t* svh,
               const void* bias, int bias_dtype, void* out, int out_dtype, void* workspace,
               hipStream_t st);

}  // namespace exl3
