"""Seeded synthetic workloads for the benchmark configurations.

numpy's PCG64 generator makes every array bit-identical on every machine, so
the GPU box and the build container see the same inputs.  Shapes follow the
reference's packed layout: trellis int16 [in/16, out/16, 16*K], suh fp16 [in],
svh fp16 [out].
"""

from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def trellis(g: np.random.Generator, in_f: int, out_f: int, K: int) -> np.ndarray:
    """Uniformly random packed bits: any bitstream is a valid trellis."""
    return g.integers(0, 1 << 16, size=(in_f // 16, out_f // 16, 16 * K), dtype=np.uint16).view(np.int16)


def suh(g: np.random.Generator, n: int) -> np.ndarray:
    """Random +-1 input signs."""
    return np.where(g.random(n) < 0.5, -1.0, 1.0).astype(np.float16)


def svh(g: np.random.Generator, n: int, lo: float = 0.005, hi: float = 0.02) -> np.ndarray:
    """Random +-1 signs times U(lo, hi) output scales."""
    s = np.where(g.random(n) < 0.5, -1.0, 1.0)
    return (s * g.uniform(lo, hi, n)).astype(np.float16)


def linear(seed: int, in_f: int, out_f: int, K: int) -> dict:
    g = rng(seed)
    return {"trellis": trellis(g, in_f, out_f, K), "suh": suh(g, in_f), "svh": svh(g, out_f), "K": K}


def activations(seed: int, rows: int, cols: int) -> np.ndarray:
    """N(0,1) activations rounded to bf16, returned as float32 values."""
    x = rng(seed).standard_normal((rows, cols), dtype=np.float32)
    bits = x.view(np.uint32)
    # round-to-nearest-even to bf16
    bits = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return bits.view(np.float32)


# ---------------------------------------------------------------------------
# Routed-expert layers and routing
# ---------------------------------------------------------------------------

def moe_layer(seed: int, n_experts: int, hidden: int, inter: int, K, gateless: bool = False) -> list:
    """Per-expert packs: gate/up [hidden -> inter], down [inter -> hidden].

    ``K`` is an int (uniform) or a per-expert sequence of ints or of
    (K_gate, K_up, K_down) tuples."""
    g = rng(seed)
    experts = []
    for e in range(n_experts):
        ke = K if isinstance(K, int) else K[e]
        kg, ku, kd = (ke, ke, ke) if isinstance(ke, (int, np.integer)) else tuple(ke)
        pack = {}
        if not gateless:
            pack["gate"] = {"trellis": trellis(g, hidden, inter, int(kg)), "suh": suh(g, hidden),
                            "svh": svh(g, inter), "K": int(kg)}
        pack["up"] = {"trellis": trellis(g, hidden, inter, int(ku)), "suh": suh(g, hidden),
                      "svh": svh(g, inter), "K": int(ku)}
        pack["down"] = {"trellis": trellis(g, inter, hidden, int(kd)), "suh": suh(g, inter),
                        "svh": svh(g, hidden), "K": int(kd)}
        experts.append(pack)
    return experts


def mixed_k(seed: int, n_experts: int, probs=(0.4, 0.4, 0.2), ks=(2, 3, 4)) -> list:
    """Per-expert K drawn from the seed (e.g. 40% K2 / 40% K3 / 20% K4)."""
    return [int(k) for k in rng(seed).choice(ks, size=n_experts, p=probs)]


def softmax_topk(seed: int, tokens: int, n_experts: int, topk: int):
    """Router logits N(0,1) -> softmax -> top-k -> renormalised weights."""
    logits = rng(seed).standard_normal((tokens, n_experts)).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, ids, axis=1)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int64), w


def zipf_topk(seed: int, tokens: int, n_experts: int, topk: int, s: float = 1.1):
    """Skewed routing: each token draws top-k distinct experts with
    probability proportional to (rank+1)^-s over a seeded permutation of ids;
    weights are a softmax of N(0,1) logits at the chosen ids."""
    g = rng(seed)
    perm = g.permutation(n_experts)
    pr = (np.arange(n_experts) + 1.0) ** (-s)
    pr /= pr.sum()
    ids = np.empty((tokens, topk), dtype=np.int64)
    for t in range(tokens):
        ids[t] = perm[g.choice(n_experts, size=topk, replace=False, p=pr)]
    logits = g.standard_normal((tokens, topk)).astype(np.float32)
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w


class DeviceBits:
    """Seeded device-side bit streams from the library's counter-based fill
    (``exl3_fill_hash_u32``): no library RNG kernel runs, and the bits are the
    same on every device.  Each call draws a fresh stream (seed, counter)."""

    def __init__(self, seed: int, device):
        self.seed = int(seed) & 0xFFFFFFFF
        self.device = device
        self.n = 0

    def words(self, n: int):
        """n uint32 words as an int32 tensor."""
        import torch

        from . import _lib

        t = torch.empty(n, dtype=torch.int32, device=self.device)
        self.n += 1
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.call("exl3_fill_hash_u32", t.data_ptr(), n, (self.seed << 32) | self.n, stream)
        return t

    def uniform(self, n: int):
        """n float32 values uniform on (0, 1): (24 high bits + 0.5) / 2^24."""
        import torch

        w = self.words(n)
        return (torch.bitwise_right_shift(w, 8) & 0xFFFFFF).float().add_(0.5).mul_(2.0 ** -24)

    def signs(self, n: int):
        import torch

        return torch.where((self.words(n) & 1) == 1, -1.0, 1.0)

    def normal(self, shape):
        """Standard normal float32 values by the Box-Muller transform."""
        import math

        import torch

        n = int(np.prod(shape))
        u1, u2 = self.uniform(n), self.uniform(n)
        z = torch.sqrt(-2.0 * torch.log(u1)) * torch.cos((2.0 * math.pi) * u2)
        return z.view(*shape)


def moe_layer_device(seed: int, n_experts: int, hidden: int, inter: int, K, device) -> dict:
    """Like ``to_device(moe_layer(...))`` but generated on the device from
    ``DeviceBits`` (for multi-GB layers; the bits differ from the numpy
    generator's, the distributions are the same).  ``K`` is an int or a
    per-expert sequence of ints.  All trellis bits come from one fill and
    all scales from a few whole-layer tensor ops, so a layer costs a handful
    of kernel launches whatever its expert count."""
    import torch

    gen = DeviceBits(seed, device)
    names = ("gate", "up", "down")
    ks = [int(K if isinstance(K, (int, np.integer)) else K[e]) for e in range(n_experts)]
    shapes = []  # (expert, projection, in, out, K, trellis offset in int16, scale offsets)
    t_off = s_off = v_off = 0
    for e in range(n_experts):
        for p in names:
            i_f, o_f = (hidden, inter) if p != "down" else (inter, hidden)
            n = (i_f // 16) * (o_f // 16) * 16 * ks[e]
            shapes.append((e, p, i_f, o_f, ks[e], t_off, s_off, v_off))
            t_off += n + (-n) % 128  # keep every projection 256-byte aligned
            s_off += i_f
            v_off += o_f
    trellis_all = gen.words(t_off // 2).view(torch.int16)
    suh_all = gen.signs(s_off).half()
    svh_all = (gen.signs(v_off) * (0.005 + 0.015 * gen.uniform(v_off))).half()
    tabs = {f"{p}_{a}": [] for p in names for a in ("trellis", "suh", "svh")}
    store = [trellis_all, suh_all, svh_all]
    kt = {p: [] for p in names}
    for e, p, i_f, o_f, k, to, so, vo in shapes:
        n = (i_f // 16) * (o_f // 16) * 16 * k
        t = trellis_all[to:to + n].view(i_f // 16, o_f // 16, 16 * k)
        su = suh_all[so:so + i_f]
        sv = svh_all[vo:vo + o_f]
        store += [t, su, sv]
        tabs[f"{p}_trellis"].append(t.data_ptr())
        tabs[f"{p}_suh"].append(su.data_ptr())
        tabs[f"{p}_svh"].append(sv.data_ptr())
        kt[p].append(k)
    out = {k: torch.tensor(v, dtype=torch.int64, device=device) for k, v in tabs.items()}
    out["k_tables"] = tuple(torch.tensor(kt[p], dtype=torch.int8, device=device) for p in names)
    out["_store"] = store
    return out


def to_device(experts: list, device) -> dict:
    """Upload packs and build the nine int64 pointer tables plus int8 K tables.

    The returned dict owns the device tensors (keep it alive while the tables
    are in use)."""
    import torch

    store = []
    names = ("gate", "up", "down")
    gateless = "gate" not in experts[0]
    tabs = {f"{p}_{a}": [] for p in names for a in ("trellis", "suh", "svh")}
    ks = {p: [] for p in names}
    for pack in experts:
        for p in names:
            src = pack["up"] if (p == "gate" and gateless) else pack[p]
            t = torch.from_numpy(src["trellis"]).to(device)
            su = torch.from_numpy(src["suh"]).to(device)
            sv = torch.from_numpy(src["svh"]).to(device)
            store += [t, su, sv]
            tabs[f"{p}_trellis"].append(t.data_ptr())
            tabs[f"{p}_suh"].append(su.data_ptr())
            tabs[f"{p}_svh"].append(sv.data_ptr())
            ks[p].append(src["K"])
    out = {k: torch.tensor(v, dtype=torch.int64, device=device) for k, v in tabs.items()}
    out["k_tables"] = tuple(torch.tensor(ks[p], dtype=torch.int8, device=device) for p in names)
    out["_store"] = store
    return out


# ---------------------------------------------------------------------------
# KV cache decode workload (int4 paged cache)
# ---------------------------------------------------------------------------

def kv_inputs(seed: int, B: int, Hkv: int, L: int, D: int = 128, outlier_frac: float = 0.02,
              outlier_scale: float = 8.0):
    """K, V [B, Hkv, L, D] bf16-rounded N(0,1) values (float32 arrays) with a
    seeded ``outlier_frac`` of the channels of each head scaled by
    ``outlier_scale``."""
    g = rng(seed)
    n_out = max(1, int(round(outlier_frac * D)))
    out = []
    for _ in range(2):
        x = g.standard_normal((B, Hkv, L, D), dtype=np.float32)
        for h in range(Hkv):
            ch = g.choice(D, size=n_out, replace=False)
            x[:, h, :, ch] *= np.float32(outlier_scale)
        bits = x.view(np.uint32)
        bits = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        out.append(bits.view(np.float32))
    return out[0], out[1]


def block_table(seed: int, B: int, max_pages: int, num_pages: int | None = None) -> np.ndarray:
    """A random page assignment: every logical page of every sequence gets a
    distinct physical page (a seeded permutation of the pool)."""
    num_pages = num_pages or B * max_pages
    perm = rng(seed).permutation(num_pages)[:B * max_pages]
    return perm.reshape(B, max_pages).astype(np.int32)


def kv_inputs_device(seed: int, B: int, Hkv: int, L: int, device, D: int = 128,
                     outlier_frac: float = 0.02, outlier_scale: float = 8.0):
    """``kv_inputs`` generated on the device from ``DeviceBits`` (for the
    full-size workload; bf16 tensors [B, Hkv, L, D]); the outlier channels
    come from the numpy generator."""
    import torch

    gen = DeviceBits(seed, device)
    g = rng(seed)
    n_out = max(1, int(round(outlier_frac * D)))
    out = []
    for _ in range(2):
        x = gen.normal((B, Hkv, L, D))
        sc = np.ones((Hkv, D), np.float32)
        for h in range(Hkv):
            sc[h, g.choice(D, size=n_out, replace=False)] = outlier_scale
        x.mul_(torch.from_numpy(sc).to(device)[None, :, None, :])
        out.append(x.to(torch.bfloat16))
        del x
    return out[0], out[1]
