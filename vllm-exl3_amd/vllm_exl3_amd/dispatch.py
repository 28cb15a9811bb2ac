"""Routed-expert dispatch: the host side of the reference's
``apply_exl3_experts`` (src/vllm_exl3/exl3.py:3602-3703) over this build's
executors.

The decisions it owns, each restating the reference's rule:

* expert ids: global -> local with the ``n_local`` sentinel for invalid and
  non-local ids (``map_topk_to_local``, exl3.py:2332-2354), done on the device
  with no host synchronisation, so a decode step stays graph-capturable; the
  layer's ``expert_map`` is pinned on the activations' device once
  (``pin_exl3_expert_map``, exl3.py:2310-2330);
* activation and clamp limit from the layer (``resolve_moe_act``,
  exl3.py:1643-1670; ``resolve_moe_gate_params``, exl3.py:1691-1751);
* executor by rows per expert: the decode executor (streaming GEMV, weights
  read once per 8 rows of an expert; the reference's native p2b path is
  decode-only, exl3.py:2716-2773) while the average routed rows per local
  expert, T * topk / n_local, stay below ``prefill_rows_per_expert()``, the
  prefill executor (grouped MFMA GEMMs, weights decoded once per 256 rows of
  an expert; the reference's exl3_moe + fat-expert split, exl3.py:2981-3599)
  from there on.  The threshold is the measured crossover on MI355X
  (``bench.py --crossover``: 16-24 rows per expert on both the C1 and the C2
  layer geometry, e.g. C1 T=128 decode 330 us vs prefill 338 us, T=192
  453 vs 369; C2 T=256 756 vs 881, T=384 1093 vs 920).  The reference's per-expert fat split
  (``FAT_EXPERT_THRESHOLD``, exl3.py:140-143) needs a device-to-host read of
  the expert counts; the grouped prefill executor tiles every expert's rows
  in one launch, so no split (and no sync) is needed;
* failures: an executor error is recorded in ``layer._exl3_native_error``
  (exl3.py:3658-3673) and the call falls back to the other executor, then to
  the per-expert loop (``apply_exl3_python_loop``, exl3.py:2357-2413) whose
  projections are the layer's ``_exl3_inners`` (``Exl3Linear`` over the HIP
  GEMV/GEMM); ``layer._exl3_last_apply`` records the path that produced the
  result ("decode", "prefill" or "loop").

Nothing here computes on the CPU: the executors and ``Exl3Linear`` run HIP
kernels and raise when the library is missing.

Layer attributes read (the names the reference's layer carries):
``_exl3_ptrs`` (nine int64 pointer tables, exl3.py:2475-2508), ``_exl3_k`` or
``_exl3_k_tuple``, ``_exl3_k_tables`` (int8 per-expert K tables, mixed K),
``_exl3_intermediate_local``, ``_exl3_codebook_flags`` ((mcg, mul1) per
projection) or ``_exl3_codebook`` (0 = 3INST, 1 = MCG, 2 = mul1),
``_exl3_gateless``, ``_exl3_moe_act`` / ``moe_config.activation``,
``swiglu_limit`` / ``swiglu_alpha`` / ``swiglu_beta``, ``expert_map``,
``_exl3_inners``.
"""

from __future__ import annotations

import logging
import math
import os
from typing import Any

import torch

from . import vllm_exl3_c as C

logger = logging.getLogger(__name__)

MOE_ACT_SILU, MOE_ACT_RELU2_NOGATE, MOE_ACT_SWIGLU_OAI = 0, 2, 3
MINIMAX_SWIGLU_ALPHA_DEFAULT = 1.702
MINIMAX_SWIGLU_LIMIT_DEFAULT = 7.0
PTR_KEYS = ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
            "down_trellis", "down_suh", "down_svh")
_MCG_CODEBOOK_FLAGS = (True, False) * 3
# Average routed rows per local expert from which the prefill executor is
# faster than the decode executor (measured crossover on MI355X,
# bench.py --crossover).
_PREFILL_ROWS_PER_EXPERT_DEFAULT = 20.0


def prefill_rows_per_expert() -> float:
    """Rows per local expert at which dispatch switches to the prefill
    executor (``VLLM_EXL3_AMD_PREFILL_ROWS`` overrides the measured default)."""
    raw = os.environ.get("VLLM_EXL3_AMD_PREFILL_ROWS")
    if raw:
        try:
            return max(0.0, float(raw))
        except ValueError:
            logger.warning("Ignoring non-numeric VLLM_EXL3_AMD_PREFILL_ROWS=%r", raw)
    return _PREFILL_ROWS_PER_EXPERT_DEFAULT


# ---------------------------------------------------------------------------
# Expert ids
# ---------------------------------------------------------------------------

def pin_exl3_expert_map(layer: Any, device: torch.device) -> torch.Tensor | None:
    """The layer's ``expert_map`` as an int64 tensor on ``device``, copied
    once and cached on the layer (a copy under graph capture is forbidden).
    exl3.py:2310-2330."""
    emap = getattr(layer, "expert_map", None)
    if emap is None:
        return None
    cached = getattr(layer, "_exl3_pinned_expert_map", None)
    if (getattr(layer, "_exl3_raw_expert_map_id", None) == id(emap) and cached is not None
            and cached.device == device and cached.dtype == torch.long):
        return cached
    pinned = torch.as_tensor(emap).to(device=device, dtype=torch.long)
    layer._exl3_pinned_expert_map = pinned
    layer._exl3_raw_expert_map_id = id(emap)
    return pinned


def map_topk_to_local(ids: torch.Tensor, n_local: int,
                      expert_map: torch.Tensor | None) -> torch.Tensor:
    """ids (T, K) global ids -> local ids; invalid or non-local ids -> the
    ``n_local`` sentinel.  exl3.py:2332-2354 (same rule, device-side)."""
    flat = ids.reshape(-1)
    if expert_map is None:
        invalid = (flat < 0) | (flat >= n_local)
        return torch.where(invalid, flat.new_full(flat.shape, n_local), flat)
    if expert_map.device != flat.device or expert_map.dtype != torch.long:
        raise RuntimeError(
            "EXL3 expert_map is not pinned to the hidden-state device; "
            "call pin_exl3_expert_map before fused apply (CUDA graphs forbid the copy)")
    n_global = int(expert_map.numel())
    if n_global == 0:
        return flat.new_full(flat.shape, n_local)
    safe = flat.clamp(min=0, max=n_global - 1)
    mapped = expert_map[safe]
    invalid = (flat < 0) | (flat >= n_global) | (mapped < 0) | (mapped >= n_local)
    return torch.where(invalid, flat.new_full(flat.shape, n_local), mapped)


# ---------------------------------------------------------------------------
# Activation and clamp
# ---------------------------------------------------------------------------

def resolve_moe_act(layer: Any) -> int:
    """Kernel activation index from vLLM's MoE activation (exl3.py:1643-1670):
    silu -> 0, relu2_no_mul -> 2 (gateless), swigluoai[_uninterleave] -> 3;
    any other activation has no kernel and raises."""
    act = getattr(getattr(layer, "moe_config", None), "activation", None)
    value = getattr(act, "value", act)
    if value is None:
        return MOE_ACT_SILU
    if value == "silu":
        return MOE_ACT_SILU
    if value == "relu2_no_mul":
        return MOE_ACT_RELU2_NOGATE
    if value in ("swigluoai", "swigluoai_uninterleave"):
        return MOE_ACT_SWIGLU_OAI
    if str(value).endswith("_no_mul"):
        raise ValueError(f"EXL3 fused MoE has no kernel instance for non-gated activation {value!r}")
    raise ValueError(f"EXL3 fused MoE has no kernel instance for activation {value!r}; "
                     "known activations are silu, relu2_no_mul and swigluoai[_uninterleave]")


def _finite_float(raw) -> float | None:
    try:
        v = float(raw)
    except (TypeError, ValueError, OverflowError):
        return None
    return v if math.isfinite(v) else None


def resolve_moe_gate_params(layer: Any) -> tuple[float | None, float | None]:
    """(alpha, limit) of the layer's activation (exl3.py:1691-1751):
    SwiGLU-OAI requires alpha 1.702 and beta absent or 1.0 (the kernel
    hardcodes both) and defaults the limit to 7.0; silu and relu2 pass a
    positive finite ``swiglu_limit`` through (else no clamp)."""
    act = resolve_moe_act(layer)
    if act == MOE_ACT_SWIGLU_OAI:
        alpha = _finite_float(getattr(layer, "swiglu_alpha", None))
        alpha = MINIMAX_SWIGLU_ALPHA_DEFAULT if alpha is None else alpha
        if alpha != MINIMAX_SWIGLU_ALPHA_DEFAULT:
            raise ValueError(f"EXL3 swiglu_oai kernel hardcodes alpha={MINIMAX_SWIGLU_ALPHA_DEFAULT}; "
                             f"layer requests swiglu_alpha={alpha!r}")
        beta = _finite_float(getattr(layer, "swiglu_beta", None))
        if beta is not None and beta != 1.0:
            raise ValueError(f"EXL3 swiglu_oai kernel computes (up + 1) (beta=1.0); "
                             f"layer requests swiglu_beta={beta!r}")
        limit = _finite_float(getattr(layer, "swiglu_limit", None))
        return alpha, MINIMAX_SWIGLU_LIMIT_DEFAULT if limit is None else limit
    limit = _finite_float(getattr(layer, "swiglu_limit", None))
    return None, (limit if limit is not None and limit > 0 else None)


# ---------------------------------------------------------------------------
# Layer description for the executors
# ---------------------------------------------------------------------------

def layer_codebook(layer: Any) -> int:
    """One codebook id for all three projections, or raise (the executors
    take one codebook per layer; mixed codebooks go to the loop)."""
    cb = getattr(layer, "_exl3_codebook", None)
    if cb is not None:
        return int(cb)
    flags = tuple(getattr(layer, "_exl3_codebook_flags", _MCG_CODEBOOK_FLAGS))
    pairs = {(bool(flags[i]), bool(flags[i + 1])) for i in range(0, 6, 2)}
    if len(pairs) != 1:
        raise RuntimeError("EXL3 fused MoE: projections use different codebooks")
    mcg, mul1 = pairs.pop()
    return C.codebook_id(mcg, mul1)


def layer_k(layer: Any) -> tuple[tuple[int, int, int], tuple | None]:
    """(uniform K triple, per-expert K tables or None)."""
    tabs = getattr(layer, "_exl3_k_tables", None)
    kt = getattr(layer, "_exl3_k_tuple", None)
    if kt is None:
        k = int(getattr(layer, "_exl3_k", getattr(layer, "_exl3_bits", 4)) or 4)
        kt = (k, k, k)
    return tuple(int(v) for v in kt), (tuple(tabs) if tabs is not None else None)


def _executor_call(kind: str, x2d, local, weights, layer, act: int, limit: float | None):
    ptrs = getattr(layer, "_exl3_ptrs", None)
    if not isinstance(ptrs, dict) or any(k not in ptrs for k in PTR_KEYS if k.startswith(("up", "down"))):
        raise RuntimeError("EXL3 fused MoE: pointer tables were not built after weight load")
    n_local = int(getattr(layer, "_exl3_n_local", ptrs["up_trellis"].numel()))
    inter = int(getattr(layer, "_exl3_intermediate_local", 2048))
    K, k_tables = layer_k(layer)
    gateless = bool(getattr(layer, "_exl3_gateless", False)) or act == MOE_ACT_RELU2_NOGATE
    fn = C.moe_forward if kind == "decode" else C.moe_prefill
    return fn(x2d, local.view(x2d.shape[0], -1), weights, ptrs, n_local, inter, K=K,
              k_tables=k_tables, codebook=layer_codebook(layer), gateless=gateless, act=act,
              swiglu_limit=float(limit) if limit is not None and limit > 0 else 0.0,
              out_dtype=torch.float32)


# ---------------------------------------------------------------------------
# The per-expert loop (fallback)
# ---------------------------------------------------------------------------

class Exl3Linear:
    """One EXL3 projection on the GPU with the reference's LinearEXL3.forward
    call shape (``forward(x, params, out_dtype=...)``), over the HIP
    GEMV/GEMM (vllm_exl3_c.exl3_gemm)."""

    def __init__(self, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                 codebook: int):
        self.trellis, self.suh, self.svh = trellis, suh, svh
        self.K, self.codebook = int(K), int(codebook)

    def forward(self, x: torch.Tensor, _params: dict | None = None, *,
                out_dtype: torch.dtype = torch.float16,
                bias: torch.Tensor | None = None) -> torch.Tensor:
        return C.exl3_gemm(x, self.trellis, self.suh, self.svh, self.K, True,
                           codebook=self.codebook, out_dtype=out_dtype, bias=bias)


def apply_exl3_python_loop(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                           inners: list[dict[str, Any]], expert_map: torch.Tensor | None,
                           limit: float | None = None, *, act: int = MOE_ACT_SILU,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """Unique-expert loop with the reference's structure and rounding points
    (exl3.py:2357-2413): per local expert, gate/up projections of its rows in
    fp32 from fp16 inputs, clamp (gate from above, up symmetric), activation,
    down of the fp16 activation, weighted index_add into an fp32 output.
    Reads the unique expert ids on the host (a synchronising fallback)."""
    tokens, hidden = x2d.shape
    if out is None:
        out = torch.zeros(tokens, hidden, dtype=torch.float32, device=x2d.device)
    local_ids = map_topk_to_local(ids, len(inners), expert_map).reshape_as(ids)
    gateless = bool(inners) and inners[0].get("gate") is None
    clamp = limit is not None and limit > 0
    for raw in torch.unique(local_ids).tolist():
        e = int(raw)
        if e >= len(inners):
            continue
        token_idx, k_pos = (local_ids == e).nonzero(as_tuple=True)
        h = x2d.index_select(0, token_idx).contiguous().half()
        pack = inners[e]
        up = pack["up"].forward(h, {}, out_dtype=torch.float32)
        if gateless:
            if clamp:
                up = up.clamp(min=-limit, max=limit)
            a = torch.square(torch.relu(up))
        else:
            gate = pack["gate"].forward(h, {}, out_dtype=torch.float32)
            if clamp:
                gate = gate.clamp(max=limit)
                up = up.clamp(min=-limit, max=limit)
            if act == MOE_ACT_SWIGLU_OAI:
                a = (up + 1.0) * gate * torch.sigmoid(1.702 * gate)
            else:
                a = torch.nn.functional.silu(gate) * up
        down = pack["down"].forward(a.contiguous().half(), {}, out_dtype=torch.float32)
        scale = weights[token_idx, k_pos].unsqueeze(-1).to(torch.float32)
        out.index_add_(0, token_idx, down * scale)
    return out


# ---------------------------------------------------------------------------
# The routed-expert apply
# ---------------------------------------------------------------------------

def choose_executor(tokens: int, topk: int, n_local: int) -> str:
    """"prefill" once T * topk >= threshold * n_local, else "decode"."""
    return "prefill" if tokens * topk >= prefill_rows_per_expert() * n_local else "decode"


def apply_exl3_experts(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       layer: Any, *, limit: float | None = None,
                       executor: str | None = None) -> torch.Tensor:
    """Routed-expert apply of one layer: out[T, hidden] in x's dtype.

    ``executor`` forces "decode" or "prefill" (None: by row count).  The
    limit, when None, comes from the layer (``resolve_moe_gate_params``)."""
    layer._exl3_last_apply = None
    tokens, hidden = x.shape[-2], x.shape[-1]
    x2d = x.reshape(tokens, hidden)
    ids = topk_ids.reshape(tokens, -1).to(torch.long)
    weights = topk_weights.reshape(tokens, -1)
    act = getattr(layer, "_exl3_moe_act", None)
    if act is None:
        act = resolve_moe_act(layer)
    if limit is None:
        _, limit = resolve_moe_gate_params(layer)
    if limit is not None and (not math.isfinite(limit) or limit < 0):
        raise ValueError(f"EXL3 fused MoE limit must be finite and nonnegative, got {limit!r}")
    expert_map = pin_exl3_expert_map(layer, x2d.device)
    if executor not in (None, "decode", "prefill"):
        raise ValueError(f"executor must be 'decode' or 'prefill', got {executor!r}")
    if getattr(layer, "_exl3_ptrs", None) is not None:
        ptrs = layer._exl3_ptrs
        n_local = int(getattr(layer, "_exl3_n_local", ptrs["up_trellis"].numel()))
        first = executor or choose_executor(tokens, ids.shape[1], n_local)
        order = (first, "prefill" if first == "decode" else "decode")
        local = map_topk_to_local(ids, n_local, expert_map)
        for kind in order:
            try:
                out = _executor_call(kind, x2d, local, weights, layer, act, limit)
            except Exception as exc:  # recorded, then the next path is tried
                layer._exl3_native_error = repr(exc)
                logger.warning("EXL3 %s executor failed; falling back: %s", kind, exc)
                continue
            layer._exl3_last_apply = kind
            return out.to(dtype=x.dtype)
    inners = getattr(layer, "_exl3_inners", None)
    if not inners:
        raise RuntimeError("EXL3 experts were not built after weight load")
    out = apply_exl3_python_loop(x2d, ids, weights, inners, expert_map, limit, act=act)
    layer._exl3_last_apply = "loop"
    return out.to(dtype=x.dtype)
