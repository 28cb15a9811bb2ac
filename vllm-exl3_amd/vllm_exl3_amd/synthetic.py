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
