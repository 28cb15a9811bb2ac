"""Drop-in for the reference's native module ``vllm_exl3_c``.

Same function names, keyword names, argument meaning and error behaviour as
the pybind exports of ``csrc/bindings.cpp:197-266``; every call validates its
tensors here (raising ``RuntimeError`` with the reference's message), then
hands raw device pointers to the C ABI of ``libexl3_mi355x.so`` on the current
HIP stream.  There is no CPU compute path: a missing library or a machine
without a GPU raises.
"""

from __future__ import annotations

import math

import torch

from . import _lib

# Module attributes the plugin gates on (csrc/bindings.cpp:243-257).
P2B_MOE_ABI_VERSION = 4
P2B_MOE_MIXED_K = True
P2B_MOE_PADDED = True

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def codebook_id(mcg: bool, mul1: bool = False, codebook: int | None = None) -> int:
    """Map the reference's (mcg, mul1) flags to a codebook id; `codebook`
    (0 = 3INST, 1 = MCG, 2 = mul1) overrides them."""
    if codebook is not None:
        _check(codebook in (0, 1, 2), "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)")
        return int(codebook)
    if mcg and mul1:
        raise RuntimeError("a tensor cannot carry both the mcg and the mul1 codebook marker")
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


def _gpu_device(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("vllm_exl3_amd needs a HIP device; there is no CPU compute path")
    return torch.device("cuda", torch.cuda.current_device())


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dequant_trellis(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                    mcg: bool, *, mul1: bool = False, codebook: int | None = None) -> torch.Tensor:
    """Decode a trellis into fp16 W[in, out]; result on trellis' device.

    csrc/bindings.cpp:117-132.  Runs on the GPU even for host tensors (they
    are staged through the current device)."""
    K = int(K)
    _check(K in (2, 3, 4, 8), "K must be one of 2, 3, 4, or 8")
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    _check(trellis.size(2) == 16 * K, "trellis last dimension must be 16*K")
    _check(trellis.size(0) > 0 and trellis.size(1) > 0, "trellis dimensions must be positive")
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16, "suh and svh must be float16")
    _check(suh.numel() >= trellis.size(0) * 16 and svh.numel() >= trellis.size(1) * 16,
           "suh/svh are too short")
    rows, cols = trellis.size(0) * 16, trellis.size(1) * 16
    _check(rows % 128 == 0 and cols % 128 == 0,
           "trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(trellis)
    t = trellis.to(dev).contiguous()
    su = suh.to(dev).reshape(-1)[:rows].contiguous()
    sv = svh.to(dev).reshape(-1)[:cols].contiguous()
    out = torch.empty((rows, cols), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("exl3_dequant_trellis", t.data_ptr(), t.size(0), t.size(1), K, cb,
                  su.data_ptr(), sv.data_ptr(), out.data_ptr(), stream_of(dev))
    return out if trellis.is_cuda else out.to(trellis.device)


def decode_tiles(trellis: torch.Tensor, K: int, mcg: bool, *, mul1: bool = False,
                 codebook: int | None = None) -> torch.Tensor:
    """Codebook values at tile positions, no rotation (ExLlamaV3 `reconstruct`
    as used at src/vllm_exl3/exl3.py:3130-3156)."""
    K = int(K)
    _check(1 <= K <= 8, "K must be in 1..8")
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16 and trellis.size(2) == 16 * K,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(trellis)
    t = trellis.to(dev).contiguous()
    out = torch.empty((t.size(0) * 16, t.size(1) * 16), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("exl3_decode_tiles", t.data_ptr(), t.size(0), t.size(1), K, cb,
                  out.data_ptr(), stream_of(dev))
    return out if trellis.is_cuda else out.to(trellis.device)


# ---------------------------------------------------------------------------
# Workspaces (no initialisation needed; split partials are finished by the
# next kernel in stream order)
# ---------------------------------------------------------------------------
_WORKSPACES: dict[tuple, torch.Tensor] = {}
# Superseded workspaces are never freed: a HIP graph captured while one of
# them was current keeps its address, and replays after a growth must not
# write into memory the caching allocator has handed to other tensors.
_RETIRED: list[torch.Tensor] = []

_DTYPE_ID = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _dtype_id(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DTYPE_ID:
        raise RuntimeError(f"{what} must be float16, bfloat16 or float32")
    return _DTYPE_ID[t.dtype]


def _capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


def workspace(device: torch.device, kind: str, nbytes: int) -> torch.Tensor:
    """Per-(device, kind) scratch, grown on demand and never freed.

    Like the reference's process-global temp caches (src/vllm_exl3/exl3.py:
    221-222, 2889) this is not thread-safe; calls sharing it must be ordered on
    one stream.  Growth keeps the old buffer alive (a captured graph may hold
    its address) and grows by at least half, so the retired buffers total
    less than twice the current one.  Growth is refused during graph capture:
    call once eagerly at the largest size first, or ``reserve_workspace``."""
    key = (str(device), kind)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if _capturing(device):
            raise RuntimeError(
                f"EXL3 workspace '{kind}' must grow to {int(nbytes)} bytes during graph capture; "
                "run the call once eagerly at its largest size (or reserve_workspace) before capture")
        size = max(int(nbytes), 256)
        if ws is not None:
            size = max(size, ws.numel() + ws.numel() // 2)
            _RETIRED.append(ws)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def reserve_workspace(device: torch.device, kind: str, nbytes: int) -> torch.Tensor:
    """Size a workspace ahead of graph capture (same rules as ``workspace``)."""
    return workspace(torch.device(device), kind, nbytes)


# ---------------------------------------------------------------------------
# GEMV / GEMM
# ---------------------------------------------------------------------------

def _gemm_native(x2: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                 K: int, cb: int, out_dtype: torch.dtype,
                 bias: torch.Tensor | None = None) -> torch.Tensor:
    dev = x2.device
    m, in_f = x2.shape
    out_f = trellis.size(1) * 16
    t = trellis.contiguous()
    su = suh.reshape(-1).contiguous()
    sv = svh.reshape(-1).contiguous()
    b = None
    if bias is not None:
        _check(bias.numel() == out_f and bias.device == dev, "bias must hold out_features values on x's device")
        b = bias.reshape(-1).contiguous()
    out = torch.empty((m, out_f), dtype=out_dtype, device=dev)
    lib = _lib.load()
    need = int(lib.exl3_gemm_workspace_size(m, in_f, out_f))
    ws = workspace(dev, "gemm", need)
    with torch.cuda.device(dev):
        _lib.call("exl3_linear", x2.data_ptr(), _dtype_id(x2, "x"), m, t.data_ptr(), t.size(0),
                  t.size(1), K, cb, su.data_ptr(), sv.data_ptr(),
                  b.data_ptr() if b is not None else None, _dtype_id(b, "bias") if b is not None else 0,
                  out.data_ptr(), _DTYPE_ID[out_dtype], ws.data_ptr(), ws.numel(), stream_of(dev))
    return out


def _check_linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                  K: int) -> None:
    _check(K in (2, 3, 4), "native GEMV supports K in {2, 3, 4}")
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16 and trellis.size(2) == 16 * K,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    _check(x.size(-1) == trellis.size(0) * 16, "x feature dimension does not match trellis")
    _check((trellis.size(0) * 16) % 128 == 0 and (trellis.size(1) * 16) % 128 == 0,
           "trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16, "suh and svh must be float16")
    _check(suh.numel() == trellis.size(0) * 16 and svh.numel() == trellis.size(1) * 16,
           "suh/svh do not match the trellis")


def exl3_gemv(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
              K: int, mcg: bool, mmode: int = 1, *, mul1: bool = False,
              codebook: int | None = None) -> torch.Tensor:
    """Small-m GEMV with fused rotations.  csrc/bindings.cpp:134-147.

    Returns fp16 [m, out] for device inputs; for host inputs the result comes
    back in x's dtype on the host (the reference's CPU contract)."""
    _check(x.dim() >= 2, "x must have shape [..., in_features]")
    m = x.numel() // x.size(-1)
    _check(1 <= m <= 8, "native GEMV supports 1 <= m <= 8")
    _check(mmode in (0, 1), "mmode must be 0 or 1")
    K = int(K)
    _check_linear(x, trellis, suh, svh, K)
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(x)
    x2 = x.to(dev).contiguous().view(m, x.size(-1))
    out = _gemm_native(x2, trellis.to(dev), suh.to(dev), svh.to(dev), K, cb, torch.float16)
    return out if x.is_cuda else out.to(x.device, x.dtype)


def exl3_gemm(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
              K: int, mcg: bool, *, mul1: bool = False, codebook: int | None = None,
              out_dtype: torch.dtype = torch.float16, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Any-m EXL3 linear: [m, out] of out_dtype (fp16 by default, as the
    reference).  csrc/bindings.cpp:110-115; from 128 rows the weights are
    decoded once per 256 rows on MFMA (the reference's reconstruct + hgemm
    route, src/vllm_exl3/exl3.py:5797-5819).  ``bias`` (keyword extension)
    is added after the output rotation."""
    K = int(K)
    _check(x.dim() >= 1 and x.numel() > 0, "x must have shape [..., in_features]")
    _check_linear(x, trellis, suh, svh, K)
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(x)
    x2 = x.to(dev).contiguous().view(-1, x.size(-1))
    out = _gemm_native(x2, trellis.to(dev), suh.to(dev), svh.to(dev), K, cb, out_dtype,
                       None if bias is None else bias.to(dev))
    return out if x.is_cuda else out.to(x.device)


def p2b_gemv_batched(x: torch.Tensor, trellis_ptrs: torch.Tensor, suh_ptrs: torch.Tensor,
                     svh_ptrs: torch.Tensor, expert_indices: torch.Tensor, K: int, mcg: bool,
                     mmode: int = 1, *, out_features: int = 2048, mul1: bool = False,
                     codebook: int | None = None) -> torch.Tensor:
    """One EXL3 linear per listed expert over the same rows: fp16
    [len(expert_indices), m, out_features], entry i equal to
    ``exl3_gemv(x, trellis[e_i], suh[e_i], svh[e_i], K, mcg)``.
    csrc/bindings.cpp:149-156, csrc/p2b_batched.cu:341-368.

    Same arguments as the reference (which fixes out_features at 2048 and the
    codebook at MCG); ``out_features`` and ``mul1``/``codebook`` are keyword
    extensions.  Pointer tables are int64 device tensors of device addresses
    owned by the caller; an index outside the tables yields zero rows.  One
    launch sequence on the current stream, no host synchronisation."""
    _check(mmode in (0, 1), "mmode must be 0 or 1")
    K = int(K)
    _check(K in (2, 3, 4), "batched GEMV supports K=2,3,4")
    _check(x.dim() >= 2 and x.numel() > 0, "x must have shape [..., in_features]")
    dev = _gpu_device(x)
    for t, nm in ((trellis_ptrs, "trellis_ptrs"), (suh_ptrs, "suh_ptrs"), (svh_ptrs, "svh_ptrs")):
        _check(t.dtype == torch.int64 and t.dim() == 1 and t.is_cuda and t.device == dev,
               f"{nm} must be an int64 device vector on x's device")
    _check(trellis_ptrs.numel() == suh_ptrs.numel() == svh_ptrs.numel() and trellis_ptrs.numel() > 0,
           "pointer tables must have the same, non-zero length")
    _check(expert_indices.dtype in (torch.int32, torch.int64) and expert_indices.is_cuda
           and expert_indices.device == dev and expert_indices.numel() > 0,
           "expert_indices must be a non-empty int32/int64 device tensor on x's device")
    in_f = x.size(-1)
    _check(in_f % 128 == 0 and int(out_features) % 128 == 0,
           "batched GEMV feature dimensions must be multiples of 128")
    cb = codebook_id(mcg, mul1, codebook)
    m = x.numel() // in_f
    e = expert_indices.numel()
    x2 = x.contiguous().view(m, in_f)
    idx = expert_indices.reshape(-1).to(torch.int32).contiguous()
    tp, sp, vp = (t.contiguous() for t in (trellis_ptrs, suh_ptrs, svh_ptrs))
    out = torch.empty((e, m, int(out_features)), dtype=torch.float16, device=dev)
    lib = _lib.load()
    need = int(lib.exl3_gemv_batched_workspace_size(m, e, in_f, int(out_features)))
    ws = workspace(dev, "gemv_batched", need)
    with torch.cuda.device(dev):
        _lib.call("exl3_gemv_batched", x2.data_ptr(), _dtype_id(x2, "x"), m, in_f, int(out_features),
                  tp.data_ptr(), sp.data_ptr(), vp.data_ptr(), tp.numel(), idx.data_ptr(), e, K, cb,
                  out.data_ptr(), _DTYPE_ID[torch.float16], ws.data_ptr(), ws.numel(), stream_of(dev))
    return out


# ---------------------------------------------------------------------------
# Routed-expert MoE
# ---------------------------------------------------------------------------
ACT_SILU, ACT_RELU2, ACT_SWIGLU_OAI = 0, 2, 3


def _moe_call(entry: str, ws_query: str, ws_kind: str, x: torch.Tensor, ids: torch.Tensor,
              weights: torch.Tensor, tables: dict[str, torch.Tensor], n_local: int,
              intermediate_size: int, K, k_tables, codebook: int, gateless: bool, act: int,
              swiglu_limit: float, n_valid: torch.Tensor | None, out: torch.Tensor | None,
              out_dtype: torch.dtype) -> torch.Tensor:
    _check(x.dim() == 2 and x.is_cuda, "fused MoE requires a CUDA [T, hidden] input")
    T, hidden = x.shape
    _check(ids.dim() == 2 and ids.size(0) == T, "fused MoE ids must be [T, topk]")
    _check(ids.dtype in (torch.int32, torch.int64), "fused MoE ids must be int32 or int64")
    topk = ids.size(1)
    _check(weights.shape == ids.shape, "fused MoE requires one routing weight per expert index")
    dev = x.device
    xs = x.contiguous()
    ids_c = ids.contiguous()
    w_c = weights.contiguous()
    names = ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
             "down_trellis", "down_suh", "down_svh")
    ptrs = []
    for nm in names:
        t = tables.get(nm)
        if t is None:
            _check(gateless and nm.startswith("gate"), f"fused MoE pointer table {nm} missing")
            ptrs.append(None)
            continue
        _check(t.dim() == 1 and t.dtype == torch.int64 and t.is_contiguous() and t.device == dev,
               "fused MoE pointer tables must be contiguous int64 vectors on the input device")
        _check(t.numel() >= n_local, "fused MoE n_local must bound the pointer tables")
        ptrs.append(t.data_ptr())
    kt = [None, None, None]
    if k_tables is not None:
        for i, t in enumerate(k_tables):
            if t is None:
                continue
            _check(t.dtype == torch.int8 and t.dim() == 1 and t.is_contiguous() and t.device == dev
                   and t.numel() >= n_local,
                   "fused MoE requires int8 device K tables with one entry per pointer-table slot")
            kt[i] = t.data_ptr()
    if n_valid is not None:
        _check(n_valid.is_cuda and n_valid.dtype == torch.int32 and n_valid.numel() == 1
               and n_valid.is_contiguous() and n_valid.device == dev,
               "padded fused MoE requires a contiguous int32 CUDA n_valid scalar tensor on x.device()")
    if out is None:
        out = torch.empty((T, hidden), dtype=out_dtype, device=dev)
    _check(out.shape == (T, hidden) and out.is_contiguous() and out.device == dev,
           "fused MoE output shape must match input")
    lib = _lib.load()
    need = int(getattr(lib, ws_query)(T, topk, n_local, hidden, intermediate_size, int(gateless)))
    _check(need > 0, "fused MoE: unsupported geometry")
    ws = workspace(dev, ws_kind, need)
    with torch.cuda.device(dev):
        _lib.call(entry, xs.data_ptr(), _dtype_id(xs, "x"), T, hidden,
                  int(intermediate_size), *ptrs, int(n_local), kt[0], kt[1], kt[2],
                  int(K[0]), int(K[1]), int(K[2]), int(codebook), int(gateless), int(act),
                  float(swiglu_limit), ids_c.data_ptr(), 1 if ids_c.dtype == torch.int64 else 0,
                  w_c.data_ptr(), _dtype_id(w_c, "routing weights"), topk,
                  n_valid.data_ptr() if n_valid is not None else None, out.data_ptr(),
                  _dtype_id(out, "out"), ws.data_ptr(), ws.numel(), stream_of(dev))
    return out


def moe_forward(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                tables: dict[str, torch.Tensor], n_local: int, intermediate_size: int, *,
                K: tuple[int, int, int] = (4, 4, 4), k_tables: tuple | None = None,
                codebook: int = CB_MCG, gateless: bool = False, act: int = ACT_SILU,
                swiglu_limit: float = 0.0, n_valid: torch.Tensor | None = None,
                out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """All T decode rows of a routed-expert layer in one launch sequence
    (streaming GEMV executor; weights are streamed once per 8 rows of a slot).

    ``tables`` holds the nine int64 pointer tables (keys gate_trellis, gate_suh,
    gate_svh, up_*, down_*), one entry per local expert.  ``ids`` [T, topk]
    local ids; ids outside [0, n_local) are skipped.  Returns [T, hidden]."""
    return _moe_call("exl3_moe_forward", "exl3_moe_workspace_size", "moe", x, ids, weights, tables,
                     n_local, intermediate_size, K, k_tables, codebook, gateless, act, swiglu_limit,
                     n_valid, out, out_dtype)


def moe_prefill(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                tables: dict[str, torch.Tensor], n_local: int, intermediate_size: int, *,
                K: tuple[int, int, int] = (4, 4, 4), k_tables: tuple | None = None,
                codebook: int = CB_MCG, gateless: bool = False, act: int = ACT_SILU,
                swiglu_limit: float = 0.0, n_valid: torch.Tensor | None = None,
                out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Same contract as :func:`moe_forward` on the prefill executor (grouped
    MFMA fat GEMMs: each routed expert's packed weights are decoded once per
    256 routed rows).  The reference reaches this regime through
    apply_exl3_fused_moe / apply_exl3_batched_fat (src/vllm_exl3/exl3.py:
    2981-3599); n_local <= 1023."""
    return _moe_call("exl3_moe_prefill", "exl3_moe_prefill_workspace_size", "moe_prefill", x, ids,
                     weights, tables, n_local, intermediate_size, K, k_tables, codebook, gateless,
                     act, swiglu_limit, n_valid, out, out_dtype)


# ---------------------------------------------------------------------------
# Prefill fat GEMM (csrc/bindings.cpp:259-265)
# ---------------------------------------------------------------------------

def _check_fat(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor,
               K: int) -> None:
    _check(a.is_cuda and packed.is_cuda and out.is_cuda and svh.is_cuda,
           "exl3_fat_gemm tensors must be CUDA tensors")
    _check(a.is_contiguous() and packed.is_contiguous() and out.is_contiguous()
           and svh.is_contiguous(), "exl3_fat_gemm tensors must be contiguous")
    _check(a.dtype == torch.float16, "a must be float16")
    _check(packed.dtype == torch.int16, "packed must be int16")
    _check(out.dtype == torch.float32, "out must be float32")
    _check(svh.dtype == torch.float16, "svh must be float16")
    _check(a.dim() == 2 and packed.dim() == 3 and out.dim() == 2 and svh.dim() == 1,
           "exl3_fat_gemm expects rank-2/rank-3 tensors")
    _check(K in (2, 3, 4), "exl3_fat_gemm supports K in {2, 3, 4}")
    _check(a.size(1) == packed.size(0) * 16, "a K dimension does not match packed tensor")
    _check(svh.numel() == packed.size(1) * 16, "svh N dimension does not match packed tensor")
    _check(svh.numel() % 128 == 0 and a.size(1) % 128 == 0,
           "output dimension must be divisible by 128")
    _check(packed.size(2) == 16 * K, "packed block width must be 16*K int16 words")
    _check(a.device == packed.device == out.device == svh.device,
           "exl3_fat_gemm tensors must share a device")


def exl3_fat_gemm(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor,
                  K: int, mcg: bool, mul1: bool, *, codebook: int | None = None) -> None:
    """out[M, N] = had128(a @ Wq) * svh in fp32 (a already input-rotated).
    csrc/bindings.cpp:259-261 / csrc/exl3_fat_gemm.cu:277-287; any K in
    {2,3,4} and codebook here."""
    K = int(K)
    _check_fat(a, packed, out, svh, K)
    _check(out.size(0) == a.size(0) and out.size(1) == svh.numel(), "out shape must be [M, N]")
    cb = codebook_id(mcg, mul1, codebook)
    dev = a.device
    with torch.cuda.device(dev):
        _lib.call("exl3_fat_gemm", a.data_ptr(), a.size(0), packed.data_ptr(), packed.size(0),
                  packed.size(1), K, cb, svh.data_ptr(), out.data_ptr(), stream_of(dev))


def exl3_fat_gemm_scatter(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor,
                          svh: torch.Tensor, token_idx: torch.Tensor, route_weight: torch.Tensor,
                          K: int, mcg: bool, mul1: bool, *, codebook: int | None = None) -> None:
    """out[token_idx[r]] += route_weight[r] * (had128(a @ Wq) * svh)[r].
    csrc/bindings.cpp:262-265 / csrc/exl3_fat_gemm.cu:289-305."""
    K = int(K)
    _check_fat(a, packed, out, svh, K)
    _check(out.size(1) == svh.numel(), "out N dimension mismatch")
    _check(token_idx.is_cuda and route_weight.is_cuda, "routing tensors must be CUDA tensors")
    _check(token_idx.is_contiguous() and route_weight.is_contiguous(),
           "routing tensors must be contiguous")
    _check(token_idx.dtype == torch.int64, "token_idx must be int64")
    _check(route_weight.dtype == torch.float16, "route_weight must be float16")
    _check(token_idx.numel() == a.size(0) and route_weight.numel() == a.size(0),
           "routing tensors must have M elements")
    _check(token_idx.device == a.device and route_weight.device == a.device,
           "routing tensors must share a device with a")
    cb = codebook_id(mcg, mul1, codebook)
    dev = a.device
    lib = _lib.load()
    need = int(lib.exl3_fat_gemm_workspace_size(a.size(0), svh.numel(), 1))
    ws = workspace(dev, "fat_scatter", need)
    with torch.cuda.device(dev):
        _lib.call("exl3_fat_gemm_scatter", a.data_ptr(), a.size(0), packed.data_ptr(),
                  packed.size(0), packed.size(1), K, cb, svh.data_ptr(), token_idx.data_ptr(),
                  route_weight.data_ptr(), out.data_ptr(), out.size(0), ws.data_ptr(), ws.numel(),
                  stream_of(dev))


def _check_fused_common(prefix: str, x, out, ptr_tables, intermediate_size, swiglu_limit) -> None:
    _check(x.is_cuda and x.dtype == torch.float16, f"{prefix} requires CUDA fp16 input")
    _check(out.is_cuda and out.dtype == torch.float16, f"{prefix} output must be CUDA fp16")
    _check(out.shape == x.shape, f"{prefix} output shape must match input")
    _check(x.dim() == 2 and x.size(1) > 0 and x.size(1) % 128 == 0,
           f"{prefix} hidden width must be a positive multiple of 128")
    _check(intermediate_size > 0 and intermediate_size % 128 == 0,
           f"{prefix} local intermediate width must be a positive multiple of 128")
    _check(math.isfinite(swiglu_limit) and swiglu_limit >= 0.0,
           f"{prefix} SwiGLU limit must be finite and nonnegative (0 disables clipping)")
    n = ptr_tables[0].numel()
    for t in ptr_tables:
        _check(t.dim() == 1 and t.dtype == torch.int64 and t.numel() == n and n > 0,
               f"{prefix} pointer tables must be equally sized nonempty int64 vectors")
    for t in (x, out, *ptr_tables):
        _check(t.device == x.device and t.is_contiguous(),
               f"{prefix} tensors must be contiguous and on the input CUDA device")


def _tables_dict(gt, gu, gv, ut, uu, uv, dt, du, dv) -> dict:
    return {"gate_trellis": gt, "gate_suh": gu, "gate_svh": gv, "up_trellis": ut, "up_suh": uu,
            "up_svh": uv, "down_trellis": dt, "down_suh": du, "down_svh": dv}


def p2b_fused_moe(x: torch.Tensor, out: torch.Tensor, gate_trellis_ptrs, gate_suh_ptrs,
                  gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs,
                  down_suh_ptrs, down_svh_ptrs, expert_indices: torch.Tensor,
                  routing_weights: torch.Tensor, K_gate: int, K_up: int, K_down: int, mcg: bool,
                  intermediate_size: int = 2048, swiglu_limit: float = 0.0, *,
                  codebook: int | None = None) -> torch.Tensor:
    """One-row fused decode MoE, written into ``out`` in place.

    csrc/bindings.cpp:158-167 / csrc/p2b_moe.cu:2431-2487 (uniform K; ids index
    the pointer tables directly; combine in slot order)."""
    tabs = (gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs,
            up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs)
    _check_fused_common("fused MoE", x, out, tabs, intermediate_size, swiglu_limit)
    _check(x.size(0) == 1, "fused MoE requires exactly one input row")
    _check(K_gate == K_up == K_down and K_gate in (2, 3, 4),
           "unsupported fused MoE K (uniform K in {2, 3, 4} required)")
    _check(expert_indices.dim() == 1 and expert_indices.dtype == torch.int32
           and expert_indices.numel() > 0,
           "fused MoE expert indices must be a nonempty int32 routing vector")
    _check(routing_weights.dtype == torch.float16
           and routing_weights.numel() == expert_indices.numel(),
           "fused MoE requires one fp16 routing weight per expert index")
    _check(expert_indices.device == x.device and routing_weights.device == x.device
           and expert_indices.is_contiguous() and routing_weights.is_contiguous(),
           "fused MoE tensors must be contiguous and on the input CUDA device")
    cb = codebook_id(mcg, False, codebook)
    moe_forward(x, expert_indices.view(1, -1), routing_weights.view(1, -1), _tables_dict(*tabs),
                gate_trellis_ptrs.numel(), intermediate_size, K=(K_gate, K_up, K_down),
                codebook=cb, swiglu_limit=swiglu_limit, out=out)
    return out


def p2b_fused_moe_mk(x: torch.Tensor, out: torch.Tensor, gate_trellis_ptrs, gate_suh_ptrs,
                     gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs,
                     down_suh_ptrs, down_svh_ptrs, expert_indices: torch.Tensor,
                     routing_weights: torch.Tensor, k_gate_tbl: torch.Tensor,
                     k_up_tbl: torch.Tensor, k_down_tbl: torch.Tensor, n_local: int, mcg: bool,
                     intermediate_size: int = 2048, swiglu_limit: float = 0.0, *,
                     codebook: int | None = None) -> torch.Tensor:
    """One-row mixed-K fused decode MoE with int8 per-expert K tables and the
    ``n_local`` sentinel.  csrc/bindings.cpp:169-180 / csrc/p2b_moe.cu:1201-1265."""
    tabs = (gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs,
            up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs)
    pre = "mixed-K fused MoE"
    _check_fused_common(pre, x, out, tabs, intermediate_size, swiglu_limit)
    _check(x.size(0) == 1, f"{pre} requires exactly one input row")
    _check(expert_indices.dim() == 1 and expert_indices.dtype == torch.int32
           and expert_indices.numel() > 0,
           f"{pre} expert indices must be a nonempty int32 routing vector")
    _check(routing_weights.dtype == torch.float16
           and routing_weights.numel() == expert_indices.numel(),
           f"{pre} requires one fp16 routing weight per expert index")
    for t in (k_gate_tbl, k_up_tbl, k_down_tbl):
        _check(t.is_cuda and t.dim() == 1 and t.is_contiguous() and t.dtype == torch.int8
               and t.numel() == gate_trellis_ptrs.numel(),
               f"{pre} requires int8 CUDA K tables with one entry per pointer-table slot")
    _check(1 <= n_local <= gate_trellis_ptrs.numel(),
           f"{pre} n_local must bound the pointer tables (1 <= n_local <= table length)")
    cb = codebook_id(mcg, False, codebook)
    moe_forward(x, expert_indices.view(1, -1), routing_weights.view(1, -1), _tables_dict(*tabs),
                int(n_local), intermediate_size, k_tables=(k_gate_tbl, k_up_tbl, k_down_tbl),
                codebook=cb, swiglu_limit=swiglu_limit, out=out)
    return out


def p2b_fused_moe_padded(x: torch.Tensor, out: torch.Tensor, gate_trellis_ptrs, gate_suh_ptrs,
                         gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs,
                         down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs,
                         expert_indices_padded: torch.Tensor, routing_weights_padded: torch.Tensor,
                         n_valid: torch.Tensor, k_gate_tbl: torch.Tensor, k_up_tbl: torch.Tensor,
                         k_down_tbl: torch.Tensor, n_local: int, max_k: int, mcg: bool,
                         intermediate_size: int = 2048, swiglu_limit: float = 0.0, *,
                         codebook: int | None = None) -> torch.Tensor:
    """Fixed-shape [MAX_T, MAX_K] decode MoE whose live row count is the device
    scalar ``n_valid`` (never read on the host); padded rows come out as exact
    zeros.  csrc/bindings.cpp:182-195 / csrc/p2b_moe.cu:2346-2428."""
    tabs = (gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs,
            up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs)
    pre = "padded fused MoE"
    _check_fused_common(pre, x, out, tabs, intermediate_size, swiglu_limit)
    _check(expert_indices_padded.dim() == 2 and expert_indices_padded.dtype == torch.int32
           and expert_indices_padded.size(0) == x.size(0) and expert_indices_padded.size(1) >= 1,
           f"{pre} requires an int32 [MAX_T, MAX_K] routing grid whose rows match x")
    _check(routing_weights_padded.dtype == torch.float16
           and routing_weights_padded.shape == expert_indices_padded.shape,
           f"{pre} requires one fp16 routing weight per routing-grid slot")
    for t in (k_gate_tbl, k_up_tbl, k_down_tbl):
        _check(t.is_cuda and t.dim() == 1 and t.is_contiguous() and t.dtype == torch.int8
               and t.numel() == gate_trellis_ptrs.numel(),
               f"{pre} requires int8 CUDA K tables with one entry per pointer-table slot")
    _check(1 <= n_local <= gate_trellis_ptrs.numel(),
           f"{pre} n_local must bound the pointer tables (1 <= n_local <= table length)")
    _check(max_k == expert_indices_padded.size(1),
           f"{pre} max_k must equal the routing grid's column count")
    cb = codebook_id(mcg, False, codebook)
    moe_forward(x, expert_indices_padded, routing_weights_padded, _tables_dict(*tabs),
                int(n_local), intermediate_size, k_tables=(k_gate_tbl, k_up_tbl, k_down_tbl),
                codebook=cb, swiglu_limit=swiglu_limit, n_valid=n_valid, out=out)
    return out


NGRAM_ROW_DIM = 160


def ngram_words_per_row(bits: int) -> int:
    """Packed int16 words per n-gram row: one fp16 scale word plus the K-bit
    ring bitstream (src/vllm_exl3/exl3.py:5174-5176)."""
    return 1 + NGRAM_ROW_DIM * int(bits) // 16


def ngram_dequant_rows(packed: torch.Tensor, bits: int, heads: torch.Tensor,
                       head_bias: torch.Tensor, chunk: int = 8192) -> torch.Tensor:
    """n-gram embedding rows on the GPU: packed int16 (N, words), heads (N,)
    int, head_bias (num_heads, 160) fp16 -> (N, 160) fp16 =
    codebook_mul1[state] * scale + head_bias[head] (the contract of
    ngram_dequant_rows_torch, src/vllm_exl3/exl3.py:5212-5238; ``chunk`` is
    accepted for signature compatibility, one launch covers all rows).
    Heads outside [0, num_heads) contribute a zero bias."""
    del chunk
    _check(packed.dim() == 2 and packed.dtype == torch.int16 and packed.is_cuda
           and packed.stride(1) == 1, "ngram_dequant needs packed int16 (N, words) rows on the GPU")
    _check(1 <= int(bits) <= 8, "ngram_dequant supports 1 <= bits <= 8")
    _check(packed.size(1) >= ngram_words_per_row(bits),
           f"ngram rows need {ngram_words_per_row(bits)} words at {bits} bits")
    dev = packed.device
    n = packed.size(0)
    _check(heads.dim() == 1 and heads.numel() == n and heads.device == dev,
           "ngram_dequant heads must be one id per row on the rows' device")
    _check(head_bias.dim() == 2 and head_bias.size(1) == NGRAM_ROW_DIM and head_bias.device == dev,
           "ngram_dequant head_bias must be (num_heads, 160) on the rows' device")
    h = heads.to(torch.int64).contiguous()
    hb = head_bias.to(torch.float16).contiguous()
    out = torch.empty((n, NGRAM_ROW_DIM), dtype=torch.float16, device=dev)
    if n:
        with torch.cuda.device(dev):
            _lib.call("exl3_ngram_dequant", packed.data_ptr(), n, packed.stride(0), int(bits),
                      h.data_ptr(), hb.data_ptr(), hb.size(0), out.data_ptr(), stream_of(dev))
    return out
