"""EXL3 expert packs -> the executor's pointer tables.

Host-side loader for the checkpoint layout the reference plugin reads: one
tensor per (expert, projection, kind) named
``{prefix}.{e}.{w1|w3|w2}.{trellis|suh|svh|mcg|mul1}`` (w1 = gate, w3 = up,
w2 = down; ``tests/test_mixed_k_exl3.py:85-121`` of the reference writes
them in that form, ``src/vllm_exl3/exl3.py:113-117`` names the suffixes and
the codebook markers).  The loader checks every tensor the way the
reference's load path does, moves the packs to the device, and builds the
nine int64 pointer tables plus the per-expert K tables that
``vllm_exl3_c.moe_forward`` / ``moe_prefill`` take
(``build_exl3_fused_state``, ``src/vllm_exl3/exl3.py:2443-2600``).

Layout rules (``src/vllm_exl3/exl3.py:1541-1573``): a projection of ``in``
inputs and ``out`` outputs is an int16 trellis ``[in/16, out/16, 16*K]``
(K = bits per weight = ``trellis.shape[-1] // 16``), an fp16 ``suh[in]`` and
an fp16 ``svh[out]``.  Gate and up map hidden -> intermediate, down maps
intermediate -> hidden.  Codebook markers: an int32 ``mcg`` equal to
-877912083 (the MCG multiplier 0xCBAC1FED as a signed int32) selects MCG, an
int32 ``mul1`` equal to -2082680531 (0x83DCD12D) selects mul1; exactly one
marker per tensor set, with the known value
(``_check_moe_codebook_markers``, ``src/vllm_exl3/exl3.py:4282-4303``).
A pack with no marker is the 3INST codebook, which the reference's MoE path
rejects; ``allow_3inst=True`` accepts it (the benchmark's config C1 is
3INST).

Gateless layers (no w1 tensors) alias the up tables into the gate slots, as
the reference does (``src/vllm_exl3/exl3.py:2483-2485``).

The returned :class:`ExpertTables` owns the device tensors; keep it alive
while its tables are in use (the executor reads the pointees on every
call, also on graph replays).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Mapping

import torch

MCG_MARKER_SIGNED_INT32 = -877912083
MUL1_MARKER_SIGNED_INT32 = -2082680531
EXL3_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1")
PROJECTIONS = (("gate", "w1"), ("up", "w3"), ("down", "w2"))
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
# The executors stream K 2..4 and compute K 5/6 through per-expert K tables
# (the reference's mixed-K range, csrc/p2b_moe.cu:295-324).
K_SUPPORTED = (2, 3, 4, 5, 6)


class PackError(RuntimeError):
    """A checkpoint tensor does not match the EXL3 expert pack layout."""


@dataclass
class ExpertTables:
    tables: dict[str, torch.Tensor]
    k_tables: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None
    K: tuple[int, int, int]
    codebook: int
    gateless: bool
    hidden: int
    intermediate: int
    n_local: int
    ks: dict[str, list[int]] = field(default_factory=dict)
    _store: list = field(default_factory=list, repr=False)

    def forward_kwargs(self) -> dict:
        """Keyword arguments of moe_forward / moe_prefill for these packs."""
        return {"K": self.K, "k_tables": self.k_tables, "codebook": self.codebook,
                "gateless": self.gateless}

    def inners(self) -> list[dict]:
        """Per-expert projections as ``dispatch.Exl3Linear`` objects (the
        reference's ``layer._exl3_inners``, used by the per-expert loop)."""
        from .dispatch import Exl3Linear

        out, i = [], 0
        for e in range(self.n_local):
            d = {"gate": None}
            for p, _ in PROJECTIONS:
                if p == "gate" and self.gateless:
                    continue
                t, su, sv = self._store[i:i + 3]
                i += 3
                d[p] = Exl3Linear(t, su, sv, self.ks[p][e], self.codebook)
            out.append(d)
        return out

    def attach(self, layer):
        """Set the layer attributes ``dispatch.apply_exl3_experts`` reads
        (the names the reference's layer carries) and return the layer."""
        layer._exl3_ptrs = self.tables
        layer._exl3_k_tuple = self.K
        layer._exl3_k_tables = self.k_tables
        layer._exl3_codebook = self.codebook
        layer._exl3_gateless = self.gateless
        layer._exl3_intermediate_local = self.intermediate
        layer._exl3_hidden_size = self.hidden
        layer._exl3_n_local = self.n_local
        layer._exl3_inners = self.inners()
        layer._exl3_tables_owner = self
        return layer


def codebook_of(mcg: torch.Tensor | None, mul1: torch.Tensor | None, what: str,
                allow_3inst: bool = False) -> int:
    """Codebook id of one tensor set from its markers (0 = absent)."""
    def val(t):
        if t is None:
            return 0
        if t.numel() != 1 or t.dtype not in (torch.int32, torch.int64):
            raise PackError(f"EXL3 {what}: codebook marker must be one int32 value")
        return int(t.reshape(-1)[0].item())

    m, u = val(mcg), val(mul1)
    if m and u:
        raise PackError(f"EXL3 {what}: an expert tensor has both mcg and mul1 markers")
    if m:
        if m != MCG_MARKER_SIGNED_INT32:
            raise PackError(f"EXL3 {what}: mcg marker is not the MCG int32 "
                            f"{MCG_MARKER_SIGNED_INT32}; packed ABI mismatch")
        return CB_MCG
    if u:
        if u != MUL1_MARKER_SIGNED_INT32:
            raise PackError(f"EXL3 {what}: mul1 marker is not the mul1 int32 "
                            f"{MUL1_MARKER_SIGNED_INT32}; packed ABI mismatch")
        return CB_MUL1
    if not allow_3inst:
        raise PackError(f"EXL3 {what}: an expert tensor has no codebook marker "
                        "(mcg or mul1 never loaded)")
    return CB_3INST


def _check_proj(t: torch.Tensor, su: torch.Tensor, sv: torch.Tensor, n_in: int, n_out: int,
                what: str) -> int:
    if t.dtype != torch.int16 or t.dim() != 3:
        raise PackError(f"EXL3 {what}: trellis must be a 3-D int16 tensor, got "
                        f"{tuple(t.shape)} {t.dtype}")
    if t.shape[0] * 16 != n_in or t.shape[1] * 16 != n_out or t.shape[2] % 16:
        raise PackError(f"EXL3 {what}: trellis shape {tuple(t.shape)} does not match "
                        f"[{n_in // 16}, {n_out // 16}, 16*K]")
    K = int(t.shape[2]) // 16
    if K not in K_SUPPORTED:
        raise PackError(f"EXL3 {what}: K={K} bits per weight; the routed-expert executor "
                        f"supports K in {K_SUPPORTED}")
    if su.dim() != 1 or su.numel() != n_in or not su.is_floating_point():
        raise PackError(f"EXL3 {what}: suh must be a float vector of {n_in} input scales")
    if sv.dim() != 1 or sv.numel() != n_out or not sv.is_floating_point():
        raise PackError(f"EXL3 {what}: svh must be a float vector of {n_out} output scales")
    return K


def load_experts(get: Mapping[str, torch.Tensor] | Callable[[str], torch.Tensor | None],
                 prefix: str, n_experts: int, device, *, allow_3inst: bool = False
                 ) -> ExpertTables:
    """Build the executor's tables from ``n_experts`` packs named
    ``{prefix}.{e}.{w1|w3|w2}.{kind}``.

    ``get`` is a mapping (a state dict) or a function returning the tensor
    of a name or None.  Tensors are copied to ``device`` (fp16 scales,
    contiguous int16 trellis).  Raises :class:`PackError` on a missing
    tensor, a shape that does not fit, an unsupported K, a bad or missing
    codebook marker, or packs that mix codebooks (the kernels take one
    codebook per layer)."""
    if n_experts < 1:
        raise PackError("EXL3 experts: n_experts must be >= 1")
    if callable(get) and not isinstance(get, Mapping):
        fetch = get
    else:
        fetch = get.get  # type: ignore[union-attr]
    device = torch.device(device)

    def name(e, proj, kind):
        return f"{prefix}.{e}.{proj}.{kind}"

    has_gate = [fetch(name(e, "w1", "trellis")) is not None for e in range(n_experts)]
    if any(has_gate) and not all(has_gate):
        raise PackError("EXL3 experts: a layer must carry w1 for every expert or for none")
    gateless = not has_gate[0]

    up0 = fetch(name(0, "w3", "trellis"))
    dn0 = fetch(name(0, "w2", "trellis"))
    if up0 is None or dn0 is None:
        raise PackError(f"EXL3 experts: {name(0, 'w3', 'trellis')} / "
                        f"{name(0, 'w2', 'trellis')} missing")
    hidden, inter = int(up0.shape[0]) * 16, int(up0.shape[1]) * 16

    store: list[torch.Tensor] = []
    ptrs = {f"{p}_{a}": [] for p, _ in PROJECTIONS for a in ("trellis", "suh", "svh")}
    ks: dict[str, list[int]] = {p: [] for p, _ in PROJECTIONS}
    codebooks = set()
    for e in range(n_experts):
        for p, proj in PROJECTIONS:
            if p == "gate" and gateless:
                continue
            what = f"expert {e} {proj}"
            parts = {}
            for kind in EXL3_SUFFIXES:
                parts[kind] = fetch(name(e, proj, kind))
            for kind in ("trellis", "suh", "svh"):
                if parts[kind] is None:
                    raise PackError(f"EXL3 {what}: {name(e, proj, kind)} missing")
            n_in, n_out = (inter, hidden) if p == "down" else (hidden, inter)
            K = _check_proj(parts["trellis"], parts["suh"], parts["svh"], n_in, n_out, what)
            codebooks.add(codebook_of(parts["mcg"], parts["mul1"], what, allow_3inst))
            t = parts["trellis"].to(device=device).contiguous()
            su = parts["suh"].to(device=device, dtype=torch.float16).contiguous()
            sv = parts["svh"].to(device=device, dtype=torch.float16).contiguous()
            store += [t, su, sv]
            ptrs[f"{p}_trellis"].append(t.data_ptr())
            ptrs[f"{p}_suh"].append(su.data_ptr())
            ptrs[f"{p}_svh"].append(sv.data_ptr())
            ks[p].append(K)
    if len(codebooks) != 1:
        raise PackError("EXL3 experts: packs mix codebooks; a layer uses one codebook")
    if gateless:
        for a in ("trellis", "suh", "svh"):
            ptrs[f"gate_{a}"] = list(ptrs[f"up_{a}"])
        ks["gate"] = list(ks["up"])
    tables = {k: torch.tensor(v, dtype=torch.int64, device=device) for k, v in ptrs.items()}
    # uniform tables only when every K is one the uniform-K launch streams
    uniform = all(len(set(ks[p])) == 1 and ks[p][0] <= 4 for p, _ in PROJECTIONS)
    K = tuple(max(ks[p]) for p, _ in PROJECTIONS)
    k_tables = None if uniform else tuple(
        torch.tensor(ks[p], dtype=torch.int8, device=device) for p, _ in PROJECTIONS)
    return ExpertTables(tables=tables, k_tables=k_tables, K=K, codebook=codebooks.pop(),
                        gateless=gateless, hidden=hidden, intermediate=inter, n_local=n_experts,
                        ks=ks, _store=store)


def load_experts_safetensors(path: str, prefix: str, n_experts: int, device, *,
                             allow_3inst: bool = False) -> ExpertTables:
    """:func:`load_experts` over a safetensors file, reading only the named
    tensors (the file is memory-mapped, not loaded whole)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt", device="cpu") as f:
        keys = set(f.keys())
        return load_experts(lambda k: f.get_tensor(k) if k in keys else None, prefix, n_experts,
                            device, allow_3inst=allow_3inst)


def state_dict_of(experts: list, prefix: str, codebook: int) -> dict[str, torch.Tensor]:
    """The checkpoint tensors of synthetic packs (``synthetic.moe_layer``
    dicts of numpy arrays), named as the reference's checkpoints name them."""
    out = {}
    for e, pack in enumerate(experts):
        for p, proj in PROJECTIONS:
            if p not in pack:
                continue
            q = pack[p]
            base = f"{prefix}.{e}.{proj}"
            out[f"{base}.trellis"] = torch.from_numpy(q["trellis"]).clone()
            out[f"{base}.suh"] = torch.from_numpy(q["suh"]).clone()
            out[f"{base}.svh"] = torch.from_numpy(q["svh"]).clone()
            if codebook == CB_MCG:
                out[f"{base}.mcg"] = torch.tensor(MCG_MARKER_SIGNED_INT32, dtype=torch.int32)
            elif codebook == CB_MUL1:
                out[f"{base}.mul1"] = torch.tensor(MUL1_MARKER_SIGNED_INT32, dtype=torch.int32)
    return out
