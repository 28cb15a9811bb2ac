/*
 * exl3_mi355x.h -- C ABI of the MI355X-native (gfx950) EXL3 routed-expert
 * library libexl3_mi355x.so.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the default stream), launches
 * asynchronously on that stream, never synchronises and never allocates.
 * Scratch memory is passed in by the caller as a workspace whose size is
 * returned by the matching *_workspace_size() query; it needs no
 * initialisation, and calls that share one workspace must be ordered on one
 * stream.  No kernel waits on another workgroup: split-K partial sums are
 * finished by the next kernel in stream order.
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


/* ---------------------------------------------------------------------------
 * Dense EXL3 linear (fused input and output rotations).  x is [m, in]
 * (x_dtype 0 fp16, 1 bf16, 2 fp32; values are rounded to fp16 first, as the
 * reference casts at its boundary), out is [m, out] of out_dtype.  K in
 * {2,3,4}; 1 <= m <= 2^26.  Below 128 rows the decode GEMV streams the packed
 * trellis once per group of 16 rows; from 128 rows the input rows are
 * rotated once, one fat GEMM decodes the weights once per 256 rows on MFMA
 * (fp32 accumulation) and an output pass applies the rotation x svh.
 * exl3_linear adds an optional bias [out] (bias_dtype as x_dtype; NULL = no
 * bias) after the rotation, where the reference adds it after its forward
 * (Exl3LinearMethod.apply, src/vllm_exl3/exl3.py:6641-6654).
 * Replaces vllm_exl3_c.exl3_gemv (csrc/bindings.cpp:134-147,
 * csrc/exl3_gemv.cu:23-63), vllm_exl3_c.exl3_gemm (csrc/bindings.cpp:110-115,
 * csrc/exl3_gemm.cu:8-31) and the reconstruct + hgemm route of the dense
 * forward above 144 rows (_dense_forward, src/vllm_exl3/exl3.py:5797-5819). */
int64_t exl3_gemm_workspace_size(int64_t m, int64_t in_features, int64_t out_features);
int exl3_gemm(const void* x, int x_dtype, int64_t m, const int16_t* trellis, int64_t tiles_k,
              int64_t tiles_n, int64_t K, int codebook, const uint16_t* suh, const uint16_t* svh,
              void* out, int out_dtype, void* workspace, int64_t workspace_bytes, void* stream);
int exl3_linear(const void* x, int x_dtype, int64_t m, const int16_t* trellis, int64_t tiles_k,
                int64_t tiles_n, int64_t K, int codebook, const uint16_t* suh, const uint16_t* svh,
                const void* bias, int bias_dtype, void* out, int out_dtype, void* workspace,
                int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Batched decode GEMV: one linear per listed expert over the same input rows,
 * out[i] = exl3_gemm(x, W[expert_indices[i]]) as [n_sel, m, out_features]
 * of out_dtype.  Tables are int64 device arrays of device addresses with
 * n_ptr entries; expert_indices is a device int32 [n_sel]; an index outside
 * [0, n_ptr) yields zero rows.  K in {2,3,4}, any codebook, any m >= 1.
 * Replaces vllm_exl3_c.p2b_gemv_batched (csrc/bindings.cpp:149-156,
 * csrc/p2b_batched.cu:341-368; the reference fixes out_features at 2048 and
 * the codebook at MCG). */
int64_t exl3_gemv_batched_workspace_size(int64_t m, int64_t n_sel, int64_t in_features,
                                         int64_t out_features);
int exl3_gemv_batched(const void* x, int x_dtype, int64_t m, int64_t in_features,
                      int64_t out_features, const int64_t* trellis_tab, const int64_t* suh_tab,
                      const int64_t* svh_tab, int64_t n_ptr, const int32_t* expert_indices,
                      int64_t n_sel, int64_t K, int codebook, void* out, int out_dtype,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Routed-expert MoE forward for T decode rows in one launch sequence:
 * device-side routing sort -> fused gate/up GEMV + activation + down-input
 * rotation -> down GEMV -> per-token combine in slot order (no atomics in
 * the sum, bit-identical run to run).
 *   tables: int64 device arrays of device addresses, one entry per local
 *     expert (the reference's pointer tables, src/vllm_exl3/exl3.py:2475-2508);
 *     gate tables may be NULL when gateless != 0.
 *   k_gate/k_up/k_down: optional int8 per-expert K tables (NULL -> K_*).
 *   ids: [T, topk] int32 (ids_dtype 0) or int64 (1); ids outside [0, n_local)
 *     are non-local routes and contribute nothing.
 *   weights: [T, topk] fp16/bf16/fp32 routing weights.
 *   n_valid: optional device int32[1]; rows >= *n_valid are padding and
 *     produce exact zeros (never read on the host).
 *   act: 0 silu, 2 relu2 (gateless), 3 swiglu-oai; swiglu_limit 0 = no clamp.
 *   out: [T, hidden] of out_dtype.
 * Replaces vllm_exl3_c.p2b_fused_moe / p2b_fused_moe_mk / p2b_fused_moe_padded
 * (csrc/bindings.cpp:158-195; csrc/p2b_moe.cu:643-1071, 1295-2487) and the
 * decode rows of ExLlamaV3's exl3_moe / exl3_moe_mixedk
 * (src/vllm_exl3/exl3.py:3491-3579). */
int64_t exl3_moe_workspace_size(int64_t T, int64_t topk, int64_t n_local, int64_t hidden,
                                int64_t inter, int gateless);
int exl3_moe_forward(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
                     const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                     const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                     const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                     int64_t n_local, const int8_t* k_gate, const int8_t* k_up, const int8_t* k_down,
                     int64_t K_gate, int64_t K_up, int64_t K_down, int codebook, int gateless,
                     int act, float swiglu_limit, const void* ids, int ids_dtype,
                     const void* weights, int w_dtype, int64_t topk, const int32_t* n_valid,
                     void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* exl3_moe_forward without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The scratch is a
 * 64 MiB device array inside the library (each GPU the library runs on holds
 * it until the process ends); a call whose exl3_moe_workspace_size exceeds
 * 64 MiB fails with EXL3_EINVAL before any launch.  Allocates nothing; runs
 * on the device current on the calling thread.  All calls on one GPU share
 * the array: calls ordered on one stream are fine, calls that overlap (other
 * streams or threads) race.  Same arguments, validation and results as
 * exl3_moe_forward. */
int exl3_moe_forward_noalloc(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
                             const int64_t* gate_trellis, const int64_t* gate_suh,
                             const int64_t* gate_svh, const int64_t* up_trellis,
                             const int64_t* up_suh, const int64_t* up_svh,
                             const int64_t* down_trellis, const int64_t* down_suh,
                             const int64_t* down_svh, int64_t n_local, const int8_t* k_gate,
                             const int8_t* k_up, const int8_t* k_down, int64_t K_gate,
                             int64_t K_up, int64_t K_down, int codebook, int gateless, int act,
                             float swiglu_limit, const void* ids, int ids_dtype,
                             const void* weights, int w_dtype, int64_t topk,
                             const int32_t* n_valid, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Prefill ("fat") GEMM: out[M, N] = had128(A x Wq) * svh in fp32, where A is
 * fp16 [M, K_in] row-major and already input-rotated by the caller (x * suh
 * then the 128-block Hadamard), Wq the decoded trellis tiles.  K in {2,3,4},
 * any codebook; K_in and N multiples of 128.  Tiles of 256 rows x 256 columns
 * decode the packed bits once into LDS and feed v_mfma_f32_16x16x32_f16.
 * Replaces vllm_exl3_c.exl3_fat_gemm (csrc/bindings.cpp:259-261,
 * csrc/exl3_fat_gemm.cu:65-197, 277-287; K4 MCG only there). */
int exl3_fat_gemm(const uint16_t* a, int64_t M, const int16_t* trellis, int64_t tiles_k,
                  int64_t tiles_n, int64_t K, int codebook, const uint16_t* svh, float* out,
                  void* stream);

/* Scatter variant: out[token_idx[r], :] += route_weight[r] * row r of the
 * product (fp32 atomics; rows of one call are expected to carry distinct
 * tokens, as the reference assumes; rows whose token is outside
 * [0, out_rows) are dropped).  Needs a workspace of
 * exl3_fat_gemm_workspace_size(M, N, 1) bytes.
 * Replaces vllm_exl3_c.exl3_fat_gemm_scatter (csrc/bindings.cpp:262-265,
 * csrc/exl3_fat_gemm.cu:289-305). */
int64_t exl3_fat_gemm_workspace_size(int64_t M, int64_t out_features, int scatter);
int exl3_fat_gemm_scatter(const uint16_t* a, int64_t M, const int16_t* trellis, int64_t tiles_k,
                          int64_t tiles_n, int64_t K, int codebook, const uint16_t* svh,
                          const int64_t* token_idx, const uint16_t* route_weight, float* out,
                          int64_t out_rows, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Routed-expert MoE forward for prefill-sized batches, same arguments and
 * results as exl3_moe_forward (n_local <= 1023): device routing sort ->
 * gate/up input rotation per routed row -> grouped fat GEMM (gate, up) ->
 * activation + down input rotation -> grouped fat GEMM (down) -> per-token
 * combine in slot order (deterministic).
 * Replaces the prefill side of the reference's routed-expert dispatch:
 * apply_exl3_fused_moe / apply_exl3_batched_fat (src/vllm_exl3/exl3.py:
 * 2981-3599) with ExLlamaV3 exl3_moe / exl3_moe_mixedk and the per-expert
 * exl3_fat_gemm{,_scatter} host loop. */
int64_t exl3_moe_prefill_workspace_size(int64_t T, int64_t topk, int64_t n_local, int64_t hidden,
                                        int64_t inter, int gateless);
int exl3_moe_prefill(const void* x, int x_dtype, int64_t T, int64_t hidden, int64_t inter,
                     const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                     const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                     const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                     int64_t n_local, const int8_t* k_gate, const int8_t* k_up, const int8_t* k_down,
                     int64_t K_gate, int64_t K_up, int64_t K_down, int codebook, int gateless,
                     int act, float swiglu_limit, const void* ids, int ids_dtype,
                     const void* weights, int w_dtype, int64_t topk, const int32_t* n_valid,
                     void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* ---------------------------------------------------------------------------
 * Paged int4 KV cache (format defined by this build; the reference's own
 * 4-bit KV cache is NVFP4).  Per (token, KV head, 32-dim group) an fp16
 * scale and zero, codes 0..15; pages of 16 tokens; one page of one KV head
 * is exl3_kv_page_bytes() = 2560 bytes (K codes, V codes, K scale, K zero,
 * V scale, V zero).  The pool is uint8 [num_pages, num_kv_heads, 2560];
 * block_table is int32 [B, >= max_pages] (row stride bt_stride elements),
 * seq_lens int32 [B].  head_dim is 128.
 * ------------------------------------------------------------------------- */
int64_t exl3_kv_page_bytes(void);

/* Quantise K and V [B, num_kv_heads, L, 128] (element strides stride_b,
 * stride_h, stride_t; dtype 0 fp16, 1 bf16, 2 fp32) into the pages the block
 * table assigns to tokens [0, seq_lens[b]).  Token slots of a last page past
 * seq_lens[b] get code 0, scale 0, zero 0.
 * Replaces the cache write side of the reference's 4-bit KV overlay
 * (pack_q4_row / _q4_w1_kernel, src/vllm_exl3/minimax_q4kv_reference.py:
 * 297-326, src/vllm_exl3/minimax_q4kv_kernels.py:216-348). */
int exl3_kv_pack_pages(const void* k, const void* v, int kv_dtype, int64_t B, int64_t num_kv_heads,
                       int64_t stride_b, int64_t stride_h, int64_t stride_t,
                       const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                       int64_t max_pages, uint8_t* pool, int64_t num_pages, void* stream);

/* Dequantise the cached tokens back to fp32 K, V [B, num_kv_heads, L, 128]
 * (code * scale + zero); positions past seq_lens[b] are not written.
 * Replaces dequant_pool_pages (src/vllm_exl3/minimax_q4kv_reference.py:735-776). */
int exl3_kv_unpack_pages(const uint8_t* pool, int64_t num_pages, int64_t num_kv_heads,
                         const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                         int64_t B, int64_t max_pages, float* k_out, float* v_out, int64_t L,
                         void* stream);

/* Decode attention of one query token per sequence over its cached tokens
 * [0, seq_lens[b]): q [B, Hq, 128] (strides q_stride_b, q_stride_h), GQA with
 * Hq / num_kv_heads <= 16 query heads per KV head, softmax scale sm_scale.
 * Split-K over the pages (n_splits, 0 = chosen from the device size) with a
 * log-sum-exp merge into out [B, Hq, 128] (strides out_stride_b,
 * out_stride_h; dtype 0 fp16, 1 bf16, 2 fp32).  Workspace:
 * exl3_kv_decode_workspace_size(B, Hq, num_kv_heads, max_pages, n_splits).
 * Replaces q4_sparse_decode (the Triton _q4_decode_kernel and vLLM's split
 * merge, src/vllm_exl3/minimax_q4kv_kernels.py:385-506, 772-877) for the
 * dense int4 format above. */
int64_t exl3_kv_decode_workspace_size(int64_t B, int64_t Hq, int64_t num_kv_heads,
                                      int64_t max_pages, int64_t n_splits);
int exl3_kv_decode(const void* q, int q_dtype, int64_t B, int64_t Hq, int64_t num_kv_heads,
                   int64_t q_stride_b, int64_t q_stride_h, const uint8_t* pool, int64_t num_pages,
                   const int32_t* block_table, int64_t bt_stride, int64_t max_pages,
                   const int32_t* seq_lens, float sm_scale, void* out, int out_dtype,
                   int64_t out_stride_b, int64_t out_stride_h, int64_t n_splits, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * The reference's NVFP4 ("q4") paged KV cache, byte for byte: pool uint8
 * [pages][2*H][128][72] (slot 2h = K, 2h+1 = V of KV head h; a slot is a flat
 * 9216-byte region of 128 x 64 e2m1 data bytes then 1024 e4m3 scale bytes,
 * K scales linear, V scales token-quad swizzled).
 *   pack: k, v [B, H, L, 128] (dtype 0 fp16, 1 bf16, 2 fp32; element strides
 *     stride_b/h/t, unit dim stride); token p < seq_lens[b] of sequence b goes
 *     to slot p % 128 of page block_table[b * bt_stride + p / 128].  Replaces
 *     pack_q4_row / pack_slot_region_side (src/vllm_exl3/
 *     minimax_q4kv_reference.py:297-366); bit-exact.
 *   dequant: out fp32 [pages][2H][128][128].  Replaces dequant_pool_pages
 *     (minimax_q4kv_reference.py:735-776).
 *   sparse decode: q [total_q, Hq, 128] (strides q_stride_n/h), topk_idx
 *     int32 [Hkv][total_q][topk] (strides topk_stride_h/n, unit last stride)
 *     of logical block ids, block_table int32 [num_reqs][max_blocks],
 *     seq_lens int32 [num_reqs], total_q = num_reqs * decode_query_len;
 *     n_chunks splits of the top-k list, merged by log-sum-exp; out as q.
 *     Replaces q4_sparse_decode + _q4_decode_kernel
 *     (src/vllm_exl3/minimax_q4kv_kernels.py:385-506, 772-877). */
int64_t exl3_nvfp4_page_bytes(int64_t num_kv_heads);
int exl3_nvfp4_pack_pages(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                          int64_t stride_b, int64_t stride_h, int64_t stride_t, int64_t max_len,
                          const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                          int64_t max_blocks, void* pool, int64_t num_pages, void* stream);
int exl3_nvfp4_dequant_pages(const void* pool, int64_t num_pages, int64_t H, float* out,
                             void* stream);
/* Prefill staging: page list -> bf16 staging rows.  stage is bf16
 * [capacity][H][128][256] (contiguous): row r < n holds page pages[r]
 * (int32 when pages_dtype is 0, int64 when 1), K values in columns 0..127
 * and V values in 128..255, bit-identical to the bf16 cast of the fp32 pool
 * dequant (every e2m1 x e4m3 product is exact in bf16; a NaN scale code
 * gives 0x7FC0); row n is zeroed, as is a row whose page id lies outside
 * [0, num_pages).  Requires n + 1 <= capacity.  No host synchronisation.
 * Replaces q4_stage_pages + _q4_stage_kernel
 * (src/vllm_exl3/minimax_q4kv_kernels.py:509-566, 880-951). */
int exl3_nvfp4_stage_pages(const void* pool, int64_t num_pages, int64_t H, const void* pages,
                           int pages_dtype, int64_t n, void* stage, int64_t capacity, void* stream);
int64_t exl3_nvfp4_decode_workspace_size(int64_t total_q, int64_t Hq, int64_t n_chunks);
int exl3_nvfp4_sparse_decode(const void* q, int q_dtype, int64_t total_q, int64_t Hq, int64_t Hkv,
                             int64_t q_stride_n, int64_t q_stride_h, const void* pool,
                             int64_t num_pages, const int32_t* topk_idx, int64_t topk_stride_h,
                             int64_t topk_stride_n, int64_t max_topk, const int32_t* block_table,
                             int64_t bt_stride, int64_t max_blocks, const int32_t* seq_lens,
                             int64_t decode_query_len, float sm_scale, void* out, int out_dtype,
                             int64_t out_stride_n, int64_t out_stride_h, int64_t n_chunks,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* n-gram embedding rows: packed int16 [n_rows][row_stride] (word 0 an fp16
 * scale, then 160 K-bit ring values, K = bits in 1..8, row_stride >=
 * 1 + 10 * bits), heads int64 [n_rows], head_bias fp16 [num_heads][160] ->
 * out fp16 [n_rows][160] = fp16(mul1(state_i) * scale + head_bias[head]),
 * state_i's K-bit groups j = ring values (i - j) mod 160.  A head outside
 * [0, num_heads) contributes a zero bias.  Replaces exllamav3_ext's
 * ngram_dequant, whose pure-torch twin is ngram_dequant_rows_torch
 * (src/vllm_exl3/exl3.py:5170-5238). */
int exl3_ngram_dequant(const int16_t* packed, int64_t n_rows, int64_t row_stride, int bits,
                       const int64_t* heads, const uint16_t* head_bias, int64_t num_heads,
                       uint16_t* out, void* stream);

/* W1 write side of the NVFP4 pool: Gemma QK-norm + partial NeoX RoPE of the
 * fused bf16 rows qkv [num_tokens][row_width] = [q | k | v | index_q |
 * index_k] (128 dims per head; index heads only when num_index_heads > 0),
 * then q -> q_out bf16 [T][num_heads][128]; K (normed, roped) and V (as is)
 * -> q4 pack into slots 2h / 2h+1 of page slot_mapping[t] / 128, token
 * slot_mapping[t] % 128 (negative or out-of-pool entries skip); index_q ->
 * e4m3(bf16(v)) bytes into index_q_out [T][num_index_heads][128]; index_k ->
 * e4m3(clamp(v, +-448)) into row index_slot_mapping[t] of index_cache
 * [index_rows][128].  The processed K and index-K rows are written back into
 * qkv.  Norm weights ([128], w_dtype) and cos_sin_cache ([max_positions]
 * [rotary_dim] = cos | sin, cs_dtype): 0 fp16, 1 bf16, 2 fp32; rotary_dim a
 * multiple of 8 up to 128.  A token whose position is outside
 * [0, max_positions) is skipped.  Replaces q4_w1_insert + _q4_w1_kernel
 * (src/vllm_exl3/minimax_q4kv_kernels.py:216-348, 661-758). */
int exl3_nvfp4_w1_insert(void* qkv, int64_t num_tokens, int64_t row_width, const void* q_norm_w,
                         const void* k_norm_w, const void* index_q_norm_w,
                         const void* index_k_norm_w, int w_dtype, const void* cos_sin_cache,
                         int cs_dtype, int64_t max_positions, const int64_t* positions,
                         int64_t num_heads, int64_t num_kv_heads, int64_t num_index_heads,
                         int64_t rotary_dim, float eps, const int64_t* slot_mapping,
                         const int64_t* index_slot_mapping, void* pool, int64_t num_pages,
                         void* index_cache, int64_t index_rows, void* q_out, void* index_q_out,
                         void* stream);

/* ---------------------------------------------------------------------------
 * Instrumentation (no counterpart in the reference; used by the benchmark to
 * time individual kernels on their launch stream).  Between begin and end,
 * every instrumented call records HIP events at its phase boundaries:
 *   exl3_moe_forward: 0 route | 1 input rotation | 2 gate/up GEMV | 3 gate/up
 *                     finish + activation | 4 down GEMV | 5 combine
 *   exl3_gemm:        0 input rotation | 1 GEMV | 2 split finish (when split)
 *   exl3_moe_prefill: 0 route | 1 input rotation | 2 gate/up GEMMs | 3 activation
 *                     | 4 down GEMM | 5 combine
 *   exl3_fat_gemm{,_scatter}: 0 GEMM | 1 output rotation (+ scatter)
 *   exl3_kv_decode:   0 split-K attention | 1 merge
 *   exl3_nvfp4_sparse_decode: 0 block-sparse attention | 1 merge
 * Recording never synchronises.  exl3_profile_end waits for the events and
 * writes, per phase, the summed elapsed milliseconds over the recorded calls
 * (at most max_calls are recorded).  Not thread-safe. */
int exl3_profile_begin(int max_calls);
int exl3_profile_end(double* phase_ms, int max_phases, int* n_calls, int* n_phases);

/* ---------------------------------------------------------------------------
 * Seeded synthetic bits: dst[i] = high 32 bits of the SplitMix64 finaliser of
 * seed + (i + 1) * 0x9E3779B97F4A7C15, i < n_words.  Deterministic across
 * devices and launch shapes.  No counterpart in the reference: it generates
 * the benchmark's and the full-size tests' synthetic weights and caches on
 * the device without a library RNG kernel. */
int exl3_fill_hash_u32(uint32_t* dst, int64_t n_words, uint64_t seed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_H */
