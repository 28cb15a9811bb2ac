// Thin PyTorch-ROCm extension over the C ABI of libexl3_mi355x.so: the
// reference's compiled module surface (csrc/bindings.cpp:197-266 and the
// TORCH_CHECKs of csrc/p2b_moe.cu / csrc/exl3_fat_gemm.cu) with the same
// function names, argument names and error messages, plus this build's
// executor entries (moe_forward / moe_prefill, the dense linear with bias,
// decode_tiles, the n-gram rows).  Each function validates its tensors,
// takes the current HIP stream of the input's device and hands raw device
// pointers to the C ABI.  Host (CPU) tensors are staged through the current
// device for the entries whose reference contract accepts them.  There is
// no CPU compute path.
//
// The scratch workspaces live here: one buffer per (device, kind), grown on
// demand and never freed (a HIP graph captured while a buffer was current
// keeps its address), growth refused during graph capture.
#include <torch/extension.h>

#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPGraphsC10Utils.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "exl3_mi355x.h"

namespace py = pybind11;
using at::Tensor;

namespace {

constexpr int kCb3Inst = 0, kCbMcg = 1, kCbMul1 = 2;
constexpr int kActSilu = 0;

void status(int rc, const char* entry) {
    TORCH_CHECK(rc == 0, entry, ": ", exl3_last_error(), " (status ", rc, ")");
}

int dtype_id(at::ScalarType t, const char* what) {
    switch (t) {
        case at::kHalf: return 0;
        case at::kBFloat16: return 1;
        case at::kFloat: return 2;
        default: TORCH_CHECK(false, what, " must be float16, bfloat16 or float32");
    }
    return -1;
}

int codebook_id(bool mcg, bool mul1, const py::object& codebook) {
    if (!codebook.is_none()) {
        const int cb = codebook.cast<int>();
        TORCH_CHECK(cb >= 0 && cb <= 2, "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)");
        return cb;
    }
    TORCH_CHECK(!(mcg && mul1), "a tensor cannot carry both the mcg and the mul1 codebook marker");
    return mcg ? kCbMcg : (mul1 ? kCbMul1 : kCb3Inst);
}

// The device a call runs on: the tensor's, or the current HIP device for host
// tensors (the reference's CPU contract is served on the GPU).
at::Device gpu_device(const Tensor& t) {
    if (t.is_cuda()) return t.device();
    TORCH_CHECK(at::hasHIP() || torch::cuda::is_available(),
                "vllm_exl3_amd needs a HIP device; there is no CPU compute path");
    return at::Device(at::kCUDA, c10::hip::current_device());
}

void* stream_of(const at::Device& dev) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(dev.index()).stream());
}

const void* opt_ptr(const std::optional<Tensor>& t) { return t.has_value() ? t->data_ptr() : nullptr; }

// ---------------------------------------------------------------------------
// Workspaces
// ---------------------------------------------------------------------------
std::mutex g_ws_mu;
std::map<std::pair<std::string, std::string>, Tensor> g_ws;
std::vector<Tensor> g_retired;
int g_assume_capturing = -1;  // test hook: -1 ask the runtime, 0/1 forced

bool capturing(const at::Device& dev) {
    if (g_assume_capturing >= 0) return g_assume_capturing != 0;
    if (!dev.is_cuda()) return false;
    c10::hip::HIPGuard guard(dev.index());
    return c10::hip::currentStreamCaptureStatusMayInitCtx() != c10::hip::CaptureStatus::None;
}

// Per-(device, kind) scratch, grown on demand and never freed.  Like the
// reference's process-global temp caches (src/vllm_exl3/exl3.py:221-222,
// 2889) calls sharing a buffer must be ordered on one stream.  Growth keeps
// the old buffer alive (a captured graph may hold its address) and grows by
// at least half, so the retired buffers total less than twice the current
// one; growth is refused during graph capture.
Tensor workspace(const at::Device& dev, const std::string& kind, int64_t nbytes) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    const auto key = std::make_pair(dev.str(), kind);
    auto it = g_ws.find(key);
    if (it != g_ws.end() && it->second.numel() >= nbytes) return it->second;
    TORCH_CHECK(!capturing(dev), "EXL3 workspace '", kind, "' must grow to ", nbytes,
                " bytes during graph capture; run the call once eagerly at its largest size (or "
                "reserve_workspace) before capture");
    int64_t size = std::max<int64_t>(nbytes, 256);
    if (it != g_ws.end()) {
        size = std::max<int64_t>(size, it->second.numel() + it->second.numel() / 2);
        g_retired.push_back(it->second);
    }
    Tensor ws = at::empty({size}, at::TensorOptions().dtype(at::kByte).device(dev));
    g_ws[key] = ws;
    return ws;
}

Tensor workspace_py(const at::Device& dev, const std::string& kind, int64_t nbytes) {
    return workspace(dev, kind, nbytes);
}

void check(bool cond, const std::string& msg) { TORCH_CHECK(cond, msg); }

// ---------------------------------------------------------------------------
// Dequant and decode
// ---------------------------------------------------------------------------
Tensor dequant_trellis(const Tensor& trellis, const Tensor& suh, const Tensor& svh, int64_t K, bool mcg,
                       bool mul1, const py::object& codebook) {
    check(K == 2 || K == 3 || K == 4 || K == 8, "K must be one of 2, 3, 4, or 8");
    check(trellis.dim() == 3 && trellis.scalar_type() == at::kShort,
          "trellis must be int16 [rows/16, cols/16, 16*K]");
    check(trellis.size(2) == 16 * K, "trellis last dimension must be 16*K");
    check(trellis.size(0) > 0 && trellis.size(1) > 0, "trellis dimensions must be positive");
    check(suh.scalar_type() == at::kHalf && svh.scalar_type() == at::kHalf, "suh and svh must be float16");
    const int64_t rows = trellis.size(0) * 16, cols = trellis.size(1) * 16;
    check(suh.numel() >= rows && svh.numel() >= cols, "suh/svh are too short");
    check(rows % 128 == 0 && cols % 128 == 0,
          "trellis dimensions must reconstruct whole 128-element Hadamard blocks");
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = gpu_device(trellis);
    c10::hip::HIPGuard guard(dev.index());
    const Tensor t = trellis.to(dev).contiguous();
    const Tensor su = suh.to(dev).reshape(-1).slice(0, 0, rows).contiguous();
    const Tensor sv = svh.to(dev).reshape(-1).slice(0, 0, cols).contiguous();
    Tensor out = at::empty({rows, cols}, at::TensorOptions().dtype(at::kHalf).device(dev));
    status(exl3_dequant_trellis(static_cast<const int16_t*>(t.data_ptr()), t.size(0), t.size(1), K, cb,
                                static_cast<const uint16_t*>(su.data_ptr()),
                                static_cast<const uint16_t*>(sv.data_ptr()),
                                static_cast<uint16_t*>(out.data_ptr()), stream_of(dev)),
           "exl3_dequant_trellis");
    return trellis.is_cuda() ? out : out.to(trellis.device());
}

Tensor decode_tiles(const Tensor& trellis, int64_t K, bool mcg, bool mul1, const py::object& codebook) {
    check(1 <= K && K <= 8, "K must be in 1..8");
    check(trellis.dim() == 3 && trellis.scalar_type() == at::kShort && trellis.size(2) == 16 * K,
          "trellis must be int16 [rows/16, cols/16, 16*K]");
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = gpu_device(trellis);
    c10::hip::HIPGuard guard(dev.index());
    const Tensor t = trellis.to(dev).contiguous();
    Tensor out = at::empty({t.size(0) * 16, t.size(1) * 16}, at::TensorOptions().dtype(at::kHalf).device(dev));
    status(exl3_decode_tiles(static_cast<const int16_t*>(t.data_ptr()), t.size(0), t.size(1), K, cb,
                             static_cast<uint16_t*>(out.data_ptr()), stream_of(dev)),
           "exl3_decode_tiles");
    return trellis.is_cuda() ? out : out.to(trellis.device());
}

// ---------------------------------------------------------------------------
// Dense linear (GEMV / GEMM)
// ---------------------------------------------------------------------------
void check_linear(const Tensor& x, const Tensor& trellis, const Tensor& suh, const Tensor& svh, int64_t K) {
    check(K == 2 || K == 3 || K == 4, "native GEMV supports K in {2, 3, 4}");
    check(trellis.dim() == 3 && trellis.scalar_type() == at::kShort && trellis.size(2) == 16 * K,
          "trellis must be int16 [rows/16, cols/16, 16*K]");
    check(x.size(-1) == trellis.size(0) * 16, "x feature dimension does not match trellis");
    check((trellis.size(0) * 16) % 128 == 0 && (trellis.size(1) * 16) % 128 == 0,
          "trellis dimensions must reconstruct whole 128-element Hadamard blocks");
    check(suh.scalar_type() == at::kHalf && svh.scalar_type() == at::kHalf, "suh and svh must be float16");
    check(suh.numel() == trellis.size(0) * 16 && svh.numel() == trellis.size(1) * 16,
          "suh/svh do not match the trellis");
}

Tensor gemm_native(const Tensor& x2, const Tensor& trellis, const Tensor& suh, const Tensor& svh, int64_t K,
                   int cb, at::ScalarType out_dtype, const std::optional<Tensor>& bias) {
    const at::Device dev = x2.device();
    const int64_t m = x2.size(0), in_f = x2.size(1), out_f = trellis.size(1) * 16;
    const Tensor t = trellis.contiguous();
    const Tensor su = suh.reshape(-1).contiguous();
    const Tensor sv = svh.reshape(-1).contiguous();
    std::optional<Tensor> b;
    if (bias.has_value()) {
        check(bias->numel() == out_f && bias->device() == dev, "bias must hold out_features values on x's device");
        b = bias->reshape(-1).contiguous();
    }
    const int od = dtype_id(out_dtype, "out");
    const int xd = dtype_id(x2.scalar_type(), "x");
    const int bd = b.has_value() ? dtype_id(b->scalar_type(), "bias") : 0;
    Tensor out = at::empty({m, out_f}, at::TensorOptions().dtype(out_dtype).device(dev));
    const Tensor ws = workspace(dev, "gemm", exl3_gemm_workspace_size(m, in_f, out_f));
    status(exl3_linear(x2.data_ptr(), xd, m, static_cast<const int16_t*>(t.data_ptr()), t.size(0), t.size(1), K,
                       cb, static_cast<const uint16_t*>(su.data_ptr()), static_cast<const uint16_t*>(sv.data_ptr()),
                       opt_ptr(b), bd, out.data_ptr(), od, ws.data_ptr(), ws.numel(), stream_of(dev)),
           "exl3_linear");
    return out;
}

// Small-m GEMV with fused rotations.  csrc/bindings.cpp:134-147: fp16 [m, out]
// for device inputs; host inputs give the result in x's dtype on the host.
Tensor linear_gemv(const Tensor& x, const Tensor& trellis, const Tensor& suh, const Tensor& svh, int64_t K,
                 bool mcg, int64_t mmode, bool mul1, const py::object& codebook) {
    check(x.dim() >= 2, "x must have shape [..., in_features]");
    const int64_t m = x.numel() / x.size(-1);
    check(1 <= m && m <= 8, "native GEMV supports 1 <= m <= 8");
    check(mmode == 0 || mmode == 1, "mmode must be 0 or 1");
    check_linear(x, trellis, suh, svh, K);
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = gpu_device(x);
    c10::hip::HIPGuard guard(dev.index());
    const Tensor x2 = x.to(dev).contiguous().view({m, x.size(-1)});
    Tensor out = gemm_native(x2, trellis.to(dev), suh.to(dev), svh.to(dev), K, cb, at::kHalf, std::nullopt);
    return x.is_cuda() ? out : out.to(x.device(), x.scalar_type());
}

// Any-m EXL3 linear, csrc/bindings.cpp:110-115 (out_dtype and bias are
// keyword extensions; from 128 rows the weights are decoded once per 256 rows
// on MFMA, the reference's reconstruct + hgemm route, src/vllm_exl3/exl3.py:
// 5797-5819).
Tensor linear_gemm(const Tensor& x, const Tensor& trellis, const Tensor& suh, const Tensor& svh, int64_t K,
                 bool mcg, bool mul1, const py::object& codebook, at::ScalarType out_dtype,
                 const std::optional<Tensor>& bias) {
    check(x.dim() >= 1 && x.numel() > 0, "x must have shape [..., in_features]");
    check_linear(x, trellis, suh, svh, K);
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = gpu_device(x);
    c10::hip::HIPGuard guard(dev.index());
    const Tensor x2 = x.to(dev).contiguous().view({-1, x.size(-1)});
    std::optional<Tensor> b;
    if (bias.has_value()) b = bias->to(dev);
    Tensor out = gemm_native(x2, trellis.to(dev), suh.to(dev), svh.to(dev), K, cb, out_dtype, b);
    return x.is_cuda() ? out : out.to(x.device());
}

// One EXL3 linear per listed expert over the same rows (csrc/bindings.cpp:
// 149-156, csrc/p2b_batched.cu:341-368); out_features and the codebook are
// keyword extensions; an index outside the tables yields zero rows.
Tensor p2b_gemv_batched(const Tensor& x, const Tensor& trellis_ptrs, const Tensor& suh_ptrs,
                        const Tensor& svh_ptrs, const Tensor& expert_indices, int64_t K, bool mcg,
                        int64_t mmode, int64_t out_features, bool mul1, const py::object& codebook) {
    check(mmode == 0 || mmode == 1, "mmode must be 0 or 1");
    check(K == 2 || K == 3 || K == 4, "batched GEMV supports K=2,3,4");
    check(x.dim() >= 2 && x.numel() > 0, "x must have shape [..., in_features]");
    const at::Device dev = gpu_device(x);
    const std::pair<const Tensor*, const char*> tabs[3] = {
        {&trellis_ptrs, "trellis_ptrs"}, {&suh_ptrs, "suh_ptrs"}, {&svh_ptrs, "svh_ptrs"}};
    for (const auto& tn : tabs) {
        const Tensor& t = *tn.first;
        check(t.scalar_type() == at::kLong && t.dim() == 1 && t.is_cuda() && t.device() == dev,
              std::string(tn.second) + " must be an int64 device vector on x's device");
    }
    check(trellis_ptrs.numel() == suh_ptrs.numel() && suh_ptrs.numel() == svh_ptrs.numel() &&
              trellis_ptrs.numel() > 0,
          "pointer tables must have the same, non-zero length");
    check((expert_indices.scalar_type() == at::kInt || expert_indices.scalar_type() == at::kLong) &&
              expert_indices.is_cuda() && expert_indices.device() == dev && expert_indices.numel() > 0,
          "expert_indices must be a non-empty int32/int64 device tensor on x's device");
    const int64_t in_f = x.size(-1);
    check(in_f % 128 == 0 && out_features % 128 == 0, "batched GEMV feature dimensions must be multiples of 128");
    const int cb = codebook_id(mcg, mul1, codebook);
    c10::hip::HIPGuard guard(dev.index());
    const int64_t m = x.numel() / in_f, e = expert_indices.numel();
    const Tensor x2 = x.contiguous().view({m, in_f});
    const Tensor idx = expert_indices.reshape(-1).to(at::kInt).contiguous();
    const Tensor tp = trellis_ptrs.contiguous(), sp = suh_ptrs.contiguous(), vp = svh_ptrs.contiguous();
    Tensor out = at::empty({e, m, out_features}, at::TensorOptions().dtype(at::kHalf).device(dev));
    const Tensor ws = workspace(dev, "gemv_batched", exl3_gemv_batched_workspace_size(m, e, in_f, out_features));
    status(exl3_gemv_batched(x2.data_ptr(), dtype_id(x2.scalar_type(), "x"), m, in_f, out_features,
                             static_cast<const int64_t*>(tp.data_ptr()), static_cast<const int64_t*>(sp.data_ptr()),
                             static_cast<const int64_t*>(vp.data_ptr()), tp.numel(),
                             static_cast<const int32_t*>(idx.data_ptr()), e, K, cb, out.data_ptr(), 0,
                             ws.data_ptr(), ws.numel(), stream_of(dev)),
           "exl3_gemv_batched");
    return out;
}

// ---------------------------------------------------------------------------
// Routed-expert MoE executors
// ---------------------------------------------------------------------------
using MoeEntry = int (*)(const void*, int, int64_t, int64_t, int64_t, const int64_t*, const int64_t*,
                         const int64_t*, const int64_t*, const int64_t*, const int64_t*, const int64_t*,
                         const int64_t*, const int64_t*, int64_t, const int8_t*, const int8_t*, const int8_t*,
                         int64_t, int64_t, int64_t, int, int, int, float, const void*, int, const void*, int,
                         int64_t, const int32_t*, void*, int, void*, int64_t, void*);
using MoeWsQuery = int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t, int);

Tensor moe_call(MoeEntry entry, const char* entry_name, MoeWsQuery ws_query, const char* ws_kind,
                const Tensor& x, const Tensor& ids, const Tensor& weights, const py::dict& tables, int64_t n_local,
                int64_t intermediate_size, const py::object& K, const py::object& k_tables, int64_t codebook,
                bool gateless, int64_t act, double swiglu_limit, const std::optional<Tensor>& n_valid,
                std::optional<Tensor> out, at::ScalarType out_dtype) {
    check(x.dim() == 2 && x.is_cuda(), "fused MoE requires a CUDA [T, hidden] input");
    const int64_t T = x.size(0), hidden = x.size(1);
    check(ids.dim() == 2 && ids.size(0) == T, "fused MoE ids must be [T, topk]");
    check(ids.scalar_type() == at::kInt || ids.scalar_type() == at::kLong, "fused MoE ids must be int32 or int64");
    const int64_t topk = ids.size(1);
    check(weights.sizes() == ids.sizes(), "fused MoE requires one routing weight per expert index");
    const at::Device dev = x.device();
    const Tensor xs = x.contiguous(), ids_c = ids.contiguous(), w_c = weights.contiguous();
    static const char* names[9] = {"gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh",
                                   "up_svh", "down_trellis", "down_suh", "down_svh"};
    const int64_t* ptrs[9];
    for (int i = 0; i < 9; ++i) {
        ptrs[i] = nullptr;
        const bool has = tables.contains(names[i]) && !tables[names[i]].is_none();
        if (!has) {
            check(gateless && i < 3, std::string("fused MoE pointer table ") + names[i] + " missing");
            continue;
        }
        const Tensor t = tables[names[i]].cast<Tensor>();
        check(t.dim() == 1 && t.scalar_type() == at::kLong && t.is_contiguous() && t.device() == dev,
              "fused MoE pointer tables must be contiguous int64 vectors on the input device");
        check(t.numel() >= n_local, "fused MoE n_local must bound the pointer tables");
        ptrs[i] = static_cast<const int64_t*>(t.data_ptr());
    }
    const int8_t* kt[3] = {nullptr, nullptr, nullptr};
    if (!k_tables.is_none()) {
        const py::sequence kts = k_tables.cast<py::sequence>();
        for (size_t i = 0; i < kts.size() && i < 3; ++i) {
            if (kts[i].is_none()) continue;
            const Tensor t = kts[i].cast<Tensor>();
            check(t.scalar_type() == at::kChar && t.dim() == 1 && t.is_contiguous() && t.device() == dev &&
                      t.numel() >= n_local,
                  "fused MoE requires int8 device K tables with one entry per pointer-table slot");
            kt[i] = static_cast<const int8_t*>(t.data_ptr());
        }
    }
    if (n_valid.has_value()) {
        const Tensor& nv = *n_valid;
        check(nv.is_cuda() && nv.scalar_type() == at::kInt && nv.numel() == 1 && nv.is_contiguous() &&
                  nv.device() == dev,
              "padded fused MoE requires a contiguous int32 CUDA n_valid scalar tensor on x.device()");
    }
    if (!out.has_value()) out = at::empty({T, hidden}, at::TensorOptions().dtype(out_dtype).device(dev));
    check(out->dim() == 2 && out->size(0) == T && out->size(1) == hidden && out->is_contiguous() &&
              out->device() == dev,
          "fused MoE output shape must match input");
    const py::sequence Ks = K.cast<py::sequence>();
    check(Ks.size() == 3, "K must hold (K_gate, K_up, K_down)");
    const int64_t K0 = Ks[0].cast<int64_t>(), K1 = Ks[1].cast<int64_t>(), K2 = Ks[2].cast<int64_t>();
    const int64_t need = ws_query(T, topk, n_local, hidden, intermediate_size, gateless ? 1 : 0);
    check(need > 0, "fused MoE: unsupported geometry");
    c10::hip::HIPGuard guard(dev.index());
    const Tensor ws = workspace(dev, ws_kind, need);
    status(entry(xs.data_ptr(), dtype_id(xs.scalar_type(), "x"), T, hidden, intermediate_size, ptrs[0], ptrs[1],
                 ptrs[2], ptrs[3], ptrs[4], ptrs[5], ptrs[6], ptrs[7], ptrs[8], n_local, kt[0], kt[1], kt[2],
                 K0, K1, K2, (int)codebook, gateless ? 1 : 0,
                 (int)act, (float)swiglu_limit, ids_c.data_ptr(), ids_c.scalar_type() == at::kLong ? 1 : 0,
                 w_c.data_ptr(), dtype_id(w_c.scalar_type(), "routing weights"), topk,
                 n_valid.has_value() ? static_cast<const int32_t*>(n_valid->data_ptr()) : nullptr, out->data_ptr(),
                 dtype_id(out->scalar_type(), "out"), ws.data_ptr(), ws.numel(), stream_of(dev)),
           entry_name);
    return *out;
}

// All T decode rows of a routed-expert layer in one launch sequence (the
// streaming GEMV executor).  `tables` holds the nine int64 pointer tables,
// one entry per local expert; ids outside [0, n_local) are skipped.
Tensor moe_forward(const Tensor& x, const Tensor& ids, const Tensor& weights, const py::dict& tables,
                   int64_t n_local, int64_t intermediate_size, const py::object& K, const py::object& k_tables,
                   int64_t codebook, bool gateless, int64_t act, double swiglu_limit,
                   const std::optional<Tensor>& n_valid, const std::optional<Tensor>& out,
                   at::ScalarType out_dtype) {
    return moe_call(exl3_moe_forward, "exl3_moe_forward", exl3_moe_workspace_size, "moe", x, ids, weights, tables,
                    n_local, intermediate_size, K, k_tables, codebook, gateless, act, swiglu_limit, n_valid, out,
                    out_dtype);
}

// The same contract on the prefill executor (grouped MFMA fat GEMMs); the
// reference reaches this regime through apply_exl3_fused_moe /
// apply_exl3_batched_fat (src/vllm_exl3/exl3.py:2981-3599).
Tensor moe_prefill(const Tensor& x, const Tensor& ids, const Tensor& weights, const py::dict& tables,
                   int64_t n_local, int64_t intermediate_size, const py::object& K, const py::object& k_tables,
                   int64_t codebook, bool gateless, int64_t act, double swiglu_limit,
                   const std::optional<Tensor>& n_valid, const std::optional<Tensor>& out,
                   at::ScalarType out_dtype) {
    return moe_call(exl3_moe_prefill, "exl3_moe_prefill", exl3_moe_prefill_workspace_size, "moe_prefill", x, ids,
                    weights, tables, n_local, intermediate_size, K, k_tables, codebook, gateless, act, swiglu_limit,
                    n_valid, out, out_dtype);
}

// ---------------------------------------------------------------------------
// Prefill fat GEMM (csrc/bindings.cpp:259-265, csrc/exl3_fat_gemm.cu:277-305)
// ---------------------------------------------------------------------------
void check_fat(const Tensor& a, const Tensor& packed, const Tensor& out, const Tensor& svh, int64_t K) {
    check(a.is_cuda() && packed.is_cuda() && out.is_cuda() && svh.is_cuda(),
          "exl3_fat_gemm tensors must be CUDA tensors");
    check(a.is_contiguous() && packed.is_contiguous() && out.is_contiguous() && svh.is_contiguous(),
          "exl3_fat_gemm tensors must be contiguous");
    check(a.scalar_type() == at::kHalf, "a must be float16");
    check(packed.scalar_type() == at::kShort, "packed must be int16");
    check(out.scalar_type() == at::kFloat, "out must be float32");
    check(svh.scalar_type() == at::kHalf, "svh must be float16");
    check(a.dim() == 2 && packed.dim() == 3 && out.dim() == 2 && svh.dim() == 1,
          "exl3_fat_gemm expects rank-2/rank-3 tensors");
    check(K == 2 || K == 3 || K == 4, "exl3_fat_gemm supports K in {2, 3, 4}");
    check(a.size(1) == packed.size(0) * 16, "a K dimension does not match packed tensor");
    check(svh.numel() == packed.size(1) * 16, "svh N dimension does not match packed tensor");
    check(svh.numel() % 128 == 0 && a.size(1) % 128 == 0, "output dimension must be divisible by 128");
    check(packed.size(2) == 16 * K, "packed block width must be 16*K int16 words");
    check(a.device() == packed.device() && packed.device() == out.device() && out.device() == svh.device(),
          "exl3_fat_gemm tensors must share a device");
}

// out[M, N] = had128(a @ Wq) * svh in fp32 (a already input-rotated).
void fat_gemm(const Tensor& a, const Tensor& packed, Tensor& out, const Tensor& svh, int64_t K, bool mcg,
                   bool mul1, const py::object& codebook) {
    check_fat(a, packed, out, svh, K);
    check(out.size(0) == a.size(0) && out.size(1) == svh.numel(), "out shape must be [M, N]");
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = a.device();
    c10::hip::HIPGuard guard(dev.index());
    status(exl3_fat_gemm(static_cast<const uint16_t*>(a.data_ptr()), a.size(0),
                         static_cast<const int16_t*>(packed.data_ptr()), packed.size(0), packed.size(1), K, cb,
                         static_cast<const uint16_t*>(svh.data_ptr()), static_cast<float*>(out.data_ptr()),
                         stream_of(dev)),
           "exl3_fat_gemm");
}

// out[token_idx[r]] += route_weight[r] * (had128(a @ Wq) * svh)[r].
void fat_gemm_scatter(const Tensor& a, const Tensor& packed, Tensor& out, const Tensor& svh,
                           const Tensor& token_idx, const Tensor& route_weight, int64_t K, bool mcg, bool mul1,
                           const py::object& codebook) {
    check_fat(a, packed, out, svh, K);
    check(out.size(1) == svh.numel(), "out N dimension mismatch");
    check(token_idx.is_cuda() && route_weight.is_cuda(), "routing tensors must be CUDA tensors");
    check(token_idx.is_contiguous() && route_weight.is_contiguous(), "routing tensors must be contiguous");
    check(token_idx.scalar_type() == at::kLong, "token_idx must be int64");
    check(route_weight.scalar_type() == at::kHalf, "route_weight must be float16");
    check(token_idx.numel() == a.size(0) && route_weight.numel() == a.size(0), "routing tensors must have M elements");
    check(token_idx.device() == a.device() && route_weight.device() == a.device(),
          "routing tensors must share a device with a");
    const int cb = codebook_id(mcg, mul1, codebook);
    const at::Device dev = a.device();
    c10::hip::HIPGuard guard(dev.index());
    const Tensor ws = workspace(dev, "fat_scatter", exl3_fat_gemm_workspace_size(a.size(0), svh.numel(), 1));
    status(exl3_fat_gemm_scatter(static_cast<const uint16_t*>(a.data_ptr()), a.size(0),
                                 static_cast<const int16_t*>(packed.data_ptr()), packed.size(0), packed.size(1), K,
                                 cb, static_cast<const uint16_t*>(svh.data_ptr()),
                                 static_cast<const int64_t*>(token_idx.data_ptr()),
                                 static_cast<const uint16_t*>(route_weight.data_ptr()),
                                 static_cast<float*>(out.data_ptr()), out.size(0), ws.data_ptr(), ws.numel(),
                                 stream_of(dev)),
           "exl3_fat_gemm_scatter");
}

// ---------------------------------------------------------------------------
// The reference's fused decode entries (csrc/bindings.cpp:158-195)
// ---------------------------------------------------------------------------
void check_fused_common(const std::string& prefix, const Tensor& x, const Tensor& out, const std::vector<Tensor>& tabs,
                        int64_t intermediate_size, double swiglu_limit) {
    check(x.is_cuda() && x.scalar_type() == at::kHalf, prefix + " requires CUDA fp16 input");
    check(out.is_cuda() && out.scalar_type() == at::kHalf, prefix + " output must be CUDA fp16");
    check(out.sizes() == x.sizes(), prefix + " output shape must match input");
    check(x.dim() == 2 && x.size(1) > 0 && x.size(1) % 128 == 0,
          prefix + " hidden width must be a positive multiple of 128");
    check(intermediate_size > 0 && intermediate_size % 128 == 0,
          prefix + " local intermediate width must be a positive multiple of 128");
    check(std::isfinite(swiglu_limit) && swiglu_limit >= 0.0,
          prefix + " SwiGLU limit must be finite and nonnegative (0 disables clipping)");
    const int64_t n = tabs[0].numel();
    for (const Tensor& t : tabs)
        check(t.dim() == 1 && t.scalar_type() == at::kLong && t.numel() == n && n > 0,
              prefix + " pointer tables must be equally sized nonempty int64 vectors");
    check(x.is_contiguous() && out.device() == x.device() && out.is_contiguous(),
          prefix + " tensors must be contiguous and on the input CUDA device");
    for (const Tensor& t : tabs)
        check(t.device() == x.device() && t.is_contiguous(),
              prefix + " tensors must be contiguous and on the input CUDA device");
}

py::dict tables_dict(const std::vector<Tensor>& t) {
    py::dict d;
    static const char* names[9] = {"gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh",
                                   "up_svh", "down_trellis", "down_suh", "down_svh"};
    for (int i = 0; i < 9; ++i) d[names[i]] = t[i];
    return d;
}

void check_k_tables(const std::string& pre, const Tensor& kg, const Tensor& ku, const Tensor& kd, int64_t n) {
    for (const Tensor* t : {&kg, &ku, &kd})
        check(t->is_cuda() && t->dim() == 1 && t->is_contiguous() && t->scalar_type() == at::kChar && t->numel() == n,
              pre + " requires int8 CUDA K tables with one entry per pointer-table slot");
}

// One-row fused decode MoE, written into `out` in place (csrc/bindings.cpp:
// 158-167 / csrc/p2b_moe.cu:2431-2487: uniform K, ids index the tables).
Tensor p2b_fused_moe(const Tensor& x, Tensor& out, const Tensor& gt, const Tensor& gu, const Tensor& gv,
                     const Tensor& ut, const Tensor& uu, const Tensor& uv, const Tensor& dt, const Tensor& du,
                     const Tensor& dv, const Tensor& expert_indices, const Tensor& routing_weights, int64_t K_gate,
                     int64_t K_up, int64_t K_down, bool mcg, int64_t intermediate_size, double swiglu_limit,
                     const py::object& codebook) {
    const std::vector<Tensor> tabs = {gt, gu, gv, ut, uu, uv, dt, du, dv};
    const std::string pre = "fused MoE";
    check_fused_common(pre, x, out, tabs, intermediate_size, swiglu_limit);
    check(x.size(0) == 1, "fused MoE requires exactly one input row");
    check(K_gate == K_up && K_up == K_down && K_gate >= 2 && K_gate <= 4,
          "unsupported fused MoE K (uniform K in {2, 3, 4} required)");
    check(expert_indices.dim() == 1 && expert_indices.scalar_type() == at::kInt && expert_indices.numel() > 0,
          "fused MoE expert indices must be a nonempty int32 routing vector");
    check(routing_weights.scalar_type() == at::kHalf && routing_weights.numel() == expert_indices.numel(),
          "fused MoE requires one fp16 routing weight per expert index");
    check(expert_indices.device() == x.device() && routing_weights.device() == x.device() &&
              expert_indices.is_contiguous() && routing_weights.is_contiguous(),
          "fused MoE tensors must be contiguous and on the input CUDA device");
    const int cb = codebook_id(mcg, false, codebook);
    moe_forward(x, expert_indices.view({1, -1}), routing_weights.view({1, -1}), tables_dict(tabs), gt.numel(),
                intermediate_size, py::make_tuple(K_gate, K_up, K_down), py::none(), cb, false, kActSilu,
                swiglu_limit, std::nullopt, out, at::kFloat);
    return out;
}

// One-row mixed-K fused decode MoE with int8 per-expert K tables and the
// n_local sentinel (csrc/bindings.cpp:169-180 / csrc/p2b_moe.cu:1201-1265).
Tensor p2b_fused_moe_mk(const Tensor& x, Tensor& out, const Tensor& gt, const Tensor& gu, const Tensor& gv,
                        const Tensor& ut, const Tensor& uu, const Tensor& uv, const Tensor& dt, const Tensor& du,
                        const Tensor& dv, const Tensor& expert_indices, const Tensor& routing_weights,
                        const Tensor& k_gate_tbl, const Tensor& k_up_tbl, const Tensor& k_down_tbl, int64_t n_local,
                        bool mcg, int64_t intermediate_size, double swiglu_limit, const py::object& codebook) {
    const std::vector<Tensor> tabs = {gt, gu, gv, ut, uu, uv, dt, du, dv};
    const std::string pre = "mixed-K fused MoE";
    check_fused_common(pre, x, out, tabs, intermediate_size, swiglu_limit);
    check(x.size(0) == 1, pre + " requires exactly one input row");
    check(expert_indices.dim() == 1 && expert_indices.scalar_type() == at::kInt && expert_indices.numel() > 0,
          pre + " expert indices must be a nonempty int32 routing vector");
    check(routing_weights.scalar_type() == at::kHalf && routing_weights.numel() == expert_indices.numel(),
          pre + " requires one fp16 routing weight per expert index");
    check_k_tables(pre, k_gate_tbl, k_up_tbl, k_down_tbl, gt.numel());
    check(1 <= n_local && n_local <= gt.numel(),
          pre + " n_local must bound the pointer tables (1 <= n_local <= table length)");
    const int cb = codebook_id(mcg, false, codebook);
    moe_forward(x, expert_indices.view({1, -1}), routing_weights.view({1, -1}), tables_dict(tabs), n_local,
                intermediate_size, py::make_tuple(4, 4, 4), py::make_tuple(k_gate_tbl, k_up_tbl, k_down_tbl), cb,
                false, kActSilu, swiglu_limit, std::nullopt, out, at::kFloat);
    return out;
}

// Fixed-shape [MAX_T, MAX_K] decode MoE whose live row count is the device
// scalar n_valid (never read on the host); padded rows come out as exact
// zeros (csrc/bindings.cpp:182-195 / csrc/p2b_moe.cu:2346-2428).
Tensor p2b_fused_moe_padded(const Tensor& x, Tensor& out, const Tensor& gt, const Tensor& gu, const Tensor& gv,
                            const Tensor& ut, const Tensor& uu, const Tensor& uv, const Tensor& dt, const Tensor& du,
                            const Tensor& dv, const Tensor& expert_indices_padded,
                            const Tensor& routing_weights_padded, const Tensor& n_valid, const Tensor& k_gate_tbl,
                            const Tensor& k_up_tbl, const Tensor& k_down_tbl, int64_t n_local, int64_t max_k,
                            bool mcg, int64_t intermediate_size, double swiglu_limit, const py::object& codebook) {
    const std::vector<Tensor> tabs = {gt, gu, gv, ut, uu, uv, dt, du, dv};
    const std::string pre = "padded fused MoE";
    check_fused_common(pre, x, out, tabs, intermediate_size, swiglu_limit);
    check(expert_indices_padded.dim() == 2 && expert_indices_padded.scalar_type() == at::kInt &&
              expert_indices_padded.size(0) == x.size(0) && expert_indices_padded.size(1) >= 1,
          pre + " requires an int32 [MAX_T, MAX_K] routing grid whose rows match x");
    check(routing_weights_padded.scalar_type() == at::kHalf &&
              routing_weights_padded.sizes() == expert_indices_padded.sizes(),
          pre + " requires one fp16 routing weight per routing-grid slot");
    check_k_tables(pre, k_gate_tbl, k_up_tbl, k_down_tbl, gt.numel());
    check(1 <= n_local && n_local <= gt.numel(),
          pre + " n_local must bound the pointer tables (1 <= n_local <= table length)");
    check(max_k == expert_indices_padded.size(1), pre + " max_k must equal the routing grid's column count");
    const int cb = codebook_id(mcg, false, codebook);
    moe_forward(x, expert_indices_padded, routing_weights_padded, tables_dict(tabs), n_local, intermediate_size,
                py::make_tuple(4, 4, 4), py::make_tuple(k_gate_tbl, k_up_tbl, k_down_tbl), cb, false, kActSilu,
                swiglu_limit, n_valid, out, at::kFloat);
    return out;
}

// ---------------------------------------------------------------------------
// n-gram embedding rows (the contract of ngram_dequant_rows_torch,
// src/vllm_exl3/exl3.py:5212-5238)
// ---------------------------------------------------------------------------
constexpr int64_t kNgramRowDim = 160;

int64_t ngram_words_per_row(int64_t bits) { return 1 + kNgramRowDim * bits / 16; }

Tensor ngram_dequant_rows(const Tensor& packed, int64_t bits, const Tensor& heads, const Tensor& head_bias,
                          int64_t chunk) {
    (void)chunk;  // accepted for signature compatibility: one launch covers all rows
    check(packed.dim() == 2 && packed.scalar_type() == at::kShort && packed.is_cuda() && packed.stride(1) == 1,
          "ngram_dequant needs packed int16 (N, words) rows on the GPU");
    check(1 <= bits && bits <= 8, "ngram_dequant supports 1 <= bits <= 8");
    check(packed.size(1) >= ngram_words_per_row(bits),
          "ngram rows need " + std::to_string(ngram_words_per_row(bits)) + " words at " + std::to_string(bits) +
              " bits");
    const at::Device dev = packed.device();
    const int64_t n = packed.size(0);
    check(heads.dim() == 1 && heads.numel() == n && heads.device() == dev,
          "ngram_dequant heads must be one id per row on the rows' device");
    check(head_bias.dim() == 2 && head_bias.size(1) == kNgramRowDim && head_bias.device() == dev,
          "ngram_dequant head_bias must be (num_heads, 160) on the rows' device");
    c10::hip::HIPGuard guard(dev.index());
    const Tensor h = heads.to(at::kLong).contiguous();
    const Tensor hb = head_bias.to(at::kHalf).contiguous();
    Tensor out = at::empty({n, kNgramRowDim}, at::TensorOptions().dtype(at::kHalf).device(dev));
    if (n)
        status(exl3_ngram_dequant(static_cast<const int16_t*>(packed.data_ptr()), n, packed.stride(0), (int)bits,
                                  static_cast<const int64_t*>(h.data_ptr()),
                                  static_cast<const uint16_t*>(hb.data_ptr()), hb.size(0),
                                  static_cast<uint16_t*>(out.data_ptr()), stream_of(dev)),
               "exl3_ngram_dequant");
    return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    // torch's Python types (dtype defaults below) must exist before the defs
    py::module_::import("torch");
    m.doc() = "EXL3 routed-expert path on MI355X: the reference's native module surface over the C ABI";
    // Module attributes the plugin gates on (csrc/bindings.cpp:243-257).
    m.attr("P2B_MOE_ABI_VERSION") = 4;
    m.attr("P2B_MOE_MIXED_K") = true;
    m.attr("P2B_MOE_PADDED") = true;
    m.attr("NGRAM_ROW_DIM") = kNgramRowDim;

    m.def("dequant_trellis", &dequant_trellis, "Decode an EXL3 trellis tensor into an fp16 weight matrix",
          py::arg("trellis"), py::arg("suh"), py::arg("svh"), py::arg("K"), py::arg("mcg"), py::kw_only(),
          py::arg("mul1") = false, py::arg("codebook") = py::none());
    m.def("decode_tiles", &decode_tiles, "Codebook values at tile positions, no rotation", py::arg("trellis"),
          py::arg("K"), py::arg("mcg"), py::kw_only(), py::arg("mul1") = false, py::arg("codebook") = py::none());
    m.def("exl3_gemv", &linear_gemv, "Native small-m EXL3 GEMV", py::arg("x"), py::arg("trellis"), py::arg("suh"),
          py::arg("svh"), py::arg("K"), py::arg("mcg"), py::arg("mmode") = 1, py::kw_only(),
          py::arg("mul1") = false, py::arg("codebook") = py::none());
    m.def("exl3_gemm", &linear_gemm, "Native EXL3 linear (any m)", py::arg("x"), py::arg("trellis"), py::arg("suh"),
          py::arg("svh"), py::arg("K"), py::arg("mcg"), py::kw_only(), py::arg("mul1") = false,
          py::arg("codebook") = py::none(), py::arg("out_dtype") = at::kHalf, py::arg("bias") = py::none());
    m.def("p2b_gemv_batched", &p2b_gemv_batched, "Batched MoE EXL3 GEMV", py::arg("x"), py::arg("trellis_ptrs"),
          py::arg("suh_ptrs"), py::arg("svh_ptrs"), py::arg("expert_indices"), py::arg("K"), py::arg("mcg"),
          py::arg("mmode") = 1, py::kw_only(), py::arg("out_features") = 2048, py::arg("mul1") = false,
          py::arg("codebook") = py::none());
    m.def("moe_forward", &moe_forward, "Routed-expert decode layer step (streaming GEMV executor)", py::arg("x"),
          py::arg("ids"), py::arg("weights"), py::arg("tables"), py::arg("n_local"), py::arg("intermediate_size"),
          py::kw_only(), py::arg("K") = py::make_tuple(4, 4, 4), py::arg("k_tables") = py::none(),
          py::arg("codebook") = kCbMcg, py::arg("gateless") = false, py::arg("act") = kActSilu,
          py::arg("swiglu_limit") = 0.0, py::arg("n_valid") = py::none(), py::arg("out") = py::none(),
          py::arg("out_dtype") = at::kFloat);
    m.def("moe_prefill", &moe_prefill, "Routed-expert prefill layer step (grouped fat GEMM executor)",
          py::arg("x"), py::arg("ids"), py::arg("weights"), py::arg("tables"), py::arg("n_local"),
          py::arg("intermediate_size"), py::kw_only(), py::arg("K") = py::make_tuple(4, 4, 4),
          py::arg("k_tables") = py::none(), py::arg("codebook") = kCbMcg, py::arg("gateless") = false,
          py::arg("act") = kActSilu, py::arg("swiglu_limit") = 0.0, py::arg("n_valid") = py::none(),
          py::arg("out") = py::none(), py::arg("out_dtype") = at::kFloat);
    m.def("exl3_fat_gemm", &fat_gemm, "Native EXL3 fat GEMM for large prefill rows", py::arg("a"),
          py::arg("packed"), py::arg("out"), py::arg("svh"), py::arg("K"), py::arg("mcg"), py::arg("mul1"),
          py::kw_only(), py::arg("codebook") = py::none());
    m.def("exl3_fat_gemm_scatter", &fat_gemm_scatter, "Native EXL3 fat GEMM with token scatter", py::arg("a"),
          py::arg("packed"), py::arg("out"), py::arg("svh"), py::arg("token_idx"), py::arg("route_weight"),
          py::arg("K"), py::arg("mcg"), py::arg("mul1"), py::kw_only(), py::arg("codebook") = py::none());
    m.def("p2b_fused_moe", &p2b_fused_moe, "Fused MoE decode (one row, uniform K)", py::arg("x"), py::arg("out"),
          py::arg("gate_trellis_ptrs"), py::arg("gate_suh_ptrs"), py::arg("gate_svh_ptrs"),
          py::arg("up_trellis_ptrs"), py::arg("up_suh_ptrs"), py::arg("up_svh_ptrs"), py::arg("down_trellis_ptrs"),
          py::arg("down_suh_ptrs"), py::arg("down_svh_ptrs"), py::arg("expert_indices"),
          py::arg("routing_weights"), py::arg("K_gate"), py::arg("K_up"), py::arg("K_down"), py::arg("mcg"),
          py::arg("intermediate_size") = 2048, py::arg("swiglu_limit") = 0.0, py::kw_only(),
          py::arg("codebook") = py::none());
    m.def("p2b_fused_moe_mk", &p2b_fused_moe_mk, "Fused MoE decode with per-expert K tables", py::arg("x"),
          py::arg("out"), py::arg("gate_trellis_ptrs"), py::arg("gate_suh_ptrs"), py::arg("gate_svh_ptrs"),
          py::arg("up_trellis_ptrs"), py::arg("up_suh_ptrs"), py::arg("up_svh_ptrs"), py::arg("down_trellis_ptrs"),
          py::arg("down_suh_ptrs"), py::arg("down_svh_ptrs"), py::arg("expert_indices"),
          py::arg("routing_weights"), py::arg("k_gate_tbl"), py::arg("k_up_tbl"), py::arg("k_down_tbl"),
          py::arg("n_local"), py::arg("mcg"), py::arg("intermediate_size") = 2048, py::arg("swiglu_limit") = 0.0,
          py::kw_only(), py::arg("codebook") = py::none());
    m.def("p2b_fused_moe_padded", &p2b_fused_moe_padded, "Fused MoE decode on a fixed-shape padded grid",
          py::arg("x"), py::arg("out"), py::arg("gate_trellis_ptrs"), py::arg("gate_suh_ptrs"),
          py::arg("gate_svh_ptrs"), py::arg("up_trellis_ptrs"), py::arg("up_suh_ptrs"), py::arg("up_svh_ptrs"),
          py::arg("down_trellis_ptrs"), py::arg("down_suh_ptrs"), py::arg("down_svh_ptrs"),
          py::arg("expert_indices_padded"), py::arg("routing_weights_padded"), py::arg("n_valid"),
          py::arg("k_gate_tbl"), py::arg("k_up_tbl"), py::arg("k_down_tbl"), py::arg("n_local"), py::arg("max_k"),
          py::arg("mcg"), py::arg("intermediate_size") = 2048, py::arg("swiglu_limit") = 0.0, py::kw_only(),
          py::arg("codebook") = py::none());
    m.def("ngram_words_per_row", &ngram_words_per_row, "Packed int16 words per n-gram row", py::arg("bits"));
    m.def("ngram_dequant_rows", &ngram_dequant_rows, "n-gram embedding rows on the GPU", py::arg("packed"),
          py::arg("bits"), py::arg("heads"), py::arg("head_bias"), py::arg("chunk") = 8192);

    m.def("workspace", &workspace_py, "Per-(device, kind) scratch, grown on demand and never freed",
          py::arg("device"), py::arg("kind"), py::arg("nbytes"));
    m.def("reserve_workspace", &workspace_py, "Size a workspace ahead of graph capture", py::arg("device"),
          py::arg("kind"), py::arg("nbytes"));
    m.def("retired_workspaces", [] {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        return g_retired;
    }, "Superseded workspaces (kept alive: a captured graph may hold their addresses)");
    m.def("_reset_workspaces_for_tests", [] {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        g_ws.clear();
        g_retired.clear();
    });
    m.def("_assume_capturing_for_tests", [](int v) { g_assume_capturing = v; },
          "-1: ask the runtime whether the current stream captures; 0 / 1: assume it");
    m.def("abi_version", [] { return exl3_abi_version(); });
}
