"""Helpers shared by the GPU parity tests: dense references and error metrics.

The dense matrices come from the CPU oracle (oracle.dequant) at test sizes.
At the benchmark's full sizes they come from the HIP dequant, which the tests
pin bit-exact against the oracle; the products are then taken in fp32 by torch.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle as O
from vllm_exl3_amd import vllm_exl3_c as C


def rel_l2(got, want) -> float:
    got = torch.as_tensor(got).double().cpu()
    want = torch.as_tensor(want).double().cpu()
    return float((got - want).norm() / want.norm().clamp_min(1e-30))


def dense_cpu(experts: list, cb: int) -> list:
    out = []
    for pack in experts:
        d = {}
        for p in ("gate", "up", "down"):
            if p in pack:
                q = pack[p]
                d[p] = O.dequant(q["trellis"], q["suh"], q["svh"], q["K"], cb)
        out.append(d)
    return out


def dense_gpu(experts: list, cb: int, device, only=None) -> dict:
    out = {}
    for e, pack in enumerate(experts):
        if only is not None and e not in only:
            continue
        d = {}
        for p in ("gate", "up", "down"):
            if p in pack:
                q = pack[p]
                d[p] = C.dequant_trellis(torch.from_numpy(q["trellis"]).to(device),
                                         torch.from_numpy(q["suh"]).to(device),
                                         torch.from_numpy(q["svh"]).to(device), q["K"], True,
                                         codebook=cb)
        out[e] = d
    return out


def dense_of_layer(layer: dict, ks: list, cb: int):
    """dense(e) for a device layer built by synthetic.moe_layer_device: the
    expert's three projections dequantised on the GPU (the HIP dequant is
    pinned bit-exact to the oracle), one expert at a time to bound memory."""
    store = layer["_store"][3:]  # after the whole-layer buffers: (trellis, suh, svh) per projection

    def dense(e):
        d = {}
        for pi, p in enumerate(("gate", "up", "down")):
            t, su, sv = store[9 * e + 3 * pi: 9 * e + 3 * pi + 3]
            d[p] = C.dequant_trellis(t, su, sv, int(ks[e]), True, codebook=cb)
        return d
    return dense


def torch_moe_reference(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, dense,
                        n_local: int, limit: float = 0.0, act: str = "silu") -> torch.Tensor:
    """Same semantics as oracle.moe_reference, vectorised per expert in torch
    fp32.  ``dense`` maps an expert id to {'gate','up','down'} fp16 matrices:
    a dict, or a callable (experts are then materialised one at a time)."""
    T, H = x.shape
    xh = x.to(torch.float16).float()
    out = torch.zeros((T, H), dtype=torch.float32, device=x.device)
    ids = ids.long()
    valid = (ids >= 0) & (ids < n_local)
    for e in torch.unique(ids[valid]).tolist():
        t_idx, k_idx = (ids == e).nonzero(as_tuple=True)
        h = xh.index_select(0, t_idx)
        pk = dense(e) if callable(dense) else dense[e]
        u = (h @ pk["up"].float()).half().float()
        if "gate" not in pk:
            if limit > 0:
                u = u.clamp(-limit, limit)
            a = torch.relu(u) ** 2
        else:
            g = (h @ pk["gate"].float()).half().float()
            if limit > 0:
                g = g.clamp(max=limit)
                u = u.clamp(-limit, limit)
            if act == "swiglu_oai":
                a = (u + 1.0) * g * torch.sigmoid(1.702 * g)
            else:
                a = torch.nn.functional.silu(g) * u
        a = a.half().float()
        d = a @ pk["down"].float()
        out.index_add_(0, t_idx, d * weights[t_idx, k_idx].float().unsqueeze(-1))
    return out
