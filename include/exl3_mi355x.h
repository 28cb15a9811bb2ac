/*
 * exl3_mi355x.h -- C ABI of the MI355X-native (gfx950) EXL3 routed-expert
 * library libexl3_mi355x.so.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the default stream), launches
 * asynchronously on that stream, never synchronises and never allocates.
 * Scratch memory is passed in by the caller as a workspace whose size is
 * returned by the matching *_workspace_size() query; the workspace must be
 * zero-filled once when first allocated (kernels leave their counters at zero
 * again when they finish), and calls that share one workspace must be
 * ordered on one stream.
 *
 * Return value: 0 on success, a negative status on failure; the message is
 * available from exl3_last_error() (thread-local).  Validation failures
 * (-1) happen before any launch.
 *
 * fp16 / bf16 values are passed as uint16_t bit patterns.  Codebook ids:
 * 0 = 3INST, 1 = MCG, 2 = mul1 (the reference's `mcg`/`mul1` flag pair,
 * extended with 3INST).  Trellis tensors are int16 [in/16, out/16, 16*K],
 * the reference's packed layout (src/vllm_exl3/exl3.py:1541-1573).
 *
 * Each declaration names the reference interface it replaces; paths are
 * relative to the vllm-exl3 repository root.
 */
#ifndef EXL3_MI355X_H
#define EXL3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { EXL3_OK = 0, EXL3_EINVAL = -1, EXL3_EHIP = -2, EXL3_EWORKSPACE = -3 };
enum { EXL3_CB_3INST = 0, EXL3_CB_MCG = 1, EXL3_CB_MUL1 = 2 };

/* Last error message of the calling thread ("" when none). */
const char* exl3_last_error(void);

/* ABI revision; mirrors the reference module attribute P2B_MOE_ABI_VERSION
 * (csrc/bindings.cpp:243-257). */
int exl3_abi_version(void);

/* Decode a trellis into the fp16 weight matrix W[in, out] (row-major),
 * bit-exact with the reference host decoder: 128x128 block Hadamard on both
 * sides, x suh[in], x svh[out].  K in {2,3,4,8}; in and out multiples of 128.
 * Replaces vllm_exl3_c.dequant_trellis (csrc/bindings.cpp:117-132, whose math
 * is dequant_cpu, csrc/bindings.cpp:15-100). */
int exl3_dequant_trellis(const int16_t* trellis, int64_t tiles_k, int64_t tiles_n, int64_t K,
                         int codebook, const uint16_t* suh, const uint16_t* svh,
                         uint16_t* out_w, void* stream);

/* Decode stage only: codebook values (fp16) at their tile positions, no
 * Hadamard and no scales.  out_w is [tiles_k*16, tiles_n*16].  K in 1..8.
 * Replaces ExLlamaV3's `reconstruct` as called at src/vllm_exl3/exl3.py:3130-3156. */
int exl3_decode_tiles(const int16_t* trellis, int64_t tiles_k, int64_t tiles_n, int64_t K,
                      int codebook, uint16_t* out_w, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_H */
