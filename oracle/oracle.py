"""CPU oracle for the EXL3 routed-expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker: the product package never
imports it and fails loudly when its HIP library is missing.

Contents (each function cites the reference file:line it restates; paths are
relative to the vllm-exl3 repository root):

* bit-exact trellis decode and dequant via ``liboracle.so`` (C, built by
  ``make -C oracle``) -- ``csrc/exl3_dequant.cuh``, ``csrc/bindings.cpp:15-100``;
* dequant + fp32 matmul GEMV -- ``csrc/bindings.cpp:134-147``;
* the per-expert MoE loop -- ``src/vllm_exl3/exl3.py:2357-2413`` with the
  rounding points of ``tests/test_native_moe_contract.py:100-115``;
* routing helpers -- ``exl3.py:2332-2354``;
* the int4-asymmetric paged KV cache (a format this build defines; the
  reference's own KV format is NVFP4) and dense softmax attention.

Parity status of every function is listed in ``ORACLE_PINS`` below.
"""

from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent

# How each oracle function is pinned (a function without a check would read
# "parity unpinned").
ORACLE_PINS = {
    "f16<->f32": "reference golden vectors tests/test_dequant_parity.py:18-81, "
                 "numpy float16 casts over all 65536 patterns, oracle/_ref harness",
    "decode_codebook": "golden vectors tests/test_dequant_parity.py:84-104 (MCG, mul1); "
                       "all 65536 windows x 3 codebooks vs oracle/_ref (incl. 3INST)",
    "read_window": "every bit position of K=2,3,4,8 tiles vs oracle/_ref; brute-force bit list",
    "tile_position": "bijection + literal swizzle loop of csrc/bindings.cpp:51-75",
    "hadamard": "vs oracle/_ref (bit-exact); H.H = 128 I; float64 matrix form",
    "dequant": "bit-exact vs the reference's own dequant_cpu (csrc/bindings.cpp:15-100, compiled in "
               "place by oracle/ref_dequant_harness.cpp) for K 1..4, 8, MCG and mul1; float64 "
               "diag(suh) H Wq H diag(svh)/128 within one fp16 ulp; suh=svh=1 round trip; constant "
               "tile gives one non-zero per block",
    "moe_loop": "tests/test_oracle_moe.py: the reference's activation vectors "
                "(tests/test_activation_parity.py:46-81: 400.0, 99.9954605, five clamp "
                "boundaries, non-positive limits); SwiGLU-OAI and relu2 closed forms; a "
                "single-expert weight-1 reduction vs an independent torch float64 formula at "
                "both rounding-point settings; an exact-sum routing case after "
                "tests/test_routing_parity.py:84-111 with sentinels and an expert map; "
                "planted clamp/activation mistakes fail these checks",
    "map_topk_to_local": "tests/test_oracle_moe.py: exl3.py:2332-2354 cases (no map, map with "
                         "negative / out-of-range entries, ids past the map)",
    "kv_int4": "closed form + brute force on tiny pages (format defined in-repo)",
    "attention": "float64 textbook softmax attention; uniform-key closed form",
}


def _load_lib() -> ctypes.CDLL:
    path = _HERE / "liboracle.so"
    if not path.exists():
        raise RuntimeError(f"oracle library missing: run `make -C {_HERE}` ({path})")
    lib = ctypes.CDLL(str(path))
    u16, i32, f32 = ctypes.c_uint16, ctypes.c_int, ctypes.c_float
    p = ctypes.c_void_p
    lib.oc_f16_to_f32.restype = f32
    lib.oc_f16_to_f32.argtypes = [u16]
    lib.oc_f32_to_f16.restype = u16
    lib.oc_f32_to_f16.argtypes = [f32]
    lib.oc_decode_codebook.restype = u16
    lib.oc_decode_codebook.argtypes = [u16, i32]
    lib.oc_read_window.restype = u16
    lib.oc_read_window.argtypes = [p, i32, ctypes.c_uint32]
    lib.oc_decode_index.restype = u16
    lib.oc_decode_index.argtypes = [p, i32, i32, i32]
    lib.oc_tile_position.restype = None
    lib.oc_tile_position.argtypes = [i32, ctypes.POINTER(i32), ctypes.POINTER(i32)]
    lib.oc_tile_position_loop.restype = None
    lib.oc_tile_position_loop.argtypes = [p, p]
    lib.oc_hadamard.restype = None
    lib.oc_hadamard.argtypes = [p, i32]
    lib.oc_decode_tiles.restype = None
    lib.oc_decode_tiles.argtypes = [p, i32, i32, i32, i32, p]
    lib.oc_dequant.restype = None
    lib.oc_dequant.argtypes = [p, i32, i32, i32, i32, p, p, p]
    return lib


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = _load_lib()
    return _LIB


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


CODEBOOKS = {"3inst": 0, "mcg": 1, "mul1": 2}


# ---------------------------------------------------------------------------
# Trellis decode
# ---------------------------------------------------------------------------

def decode_codebook(window: int, cb: int) -> int:
    """fp16 bits of one window.  csrc/exl3_dequant.cuh:105-124."""
    return int(lib().oc_decode_codebook(window & 0xFFFF, cb))


def decode_codebook_table(cb: int) -> np.ndarray:
    """All 65536 windows -> fp16 bit patterns (uint16)."""
    L = lib()
    return np.array([L.oc_decode_codebook(w, cb) for w in range(65536)], dtype=np.uint16)


def read_window(tile_u16: np.ndarray, K: int, bit: int) -> int:
    """csrc/exl3_dequant.cuh:141-159 (circular MSB-first 16-bit window)."""
    t = np.ascontiguousarray(tile_u16, dtype=np.uint16)
    return int(lib().oc_read_window(_ptr(t), K, bit))


def tile_positions() -> tuple[np.ndarray, np.ndarray]:
    """(row, col) of each of the 256 tile indices.  csrc/bindings.cpp:37-77."""
    rows = np.zeros(256, dtype=np.int32)
    cols = np.zeros(256, dtype=np.int32)
    L = lib()
    r, c = ctypes.c_int(), ctypes.c_int()
    for i in range(256):
        L.oc_tile_position(i, ctypes.byref(r), ctypes.byref(c))
        rows[i], cols[i] = r.value, c.value
    return rows, cols


def tile_positions_loop() -> tuple[np.ndarray, np.ndarray]:
    rows = np.zeros(256, dtype=np.int32)
    cols = np.zeros(256, dtype=np.int32)
    lib().oc_tile_position_loop(_ptr(rows), _ptr(cols))
    return rows, cols


def hadamard_f32(v: np.ndarray) -> np.ndarray:
    """Unnormalised fp32 butterfly.  csrc/exl3_dequant.cuh:168-179."""
    out = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().oc_hadamard(_ptr(out), out.size)
    return out


def decode_tiles(trellis: np.ndarray, K: int, cb: int) -> np.ndarray:
    """Codebook values at swizzled positions, no rotation: fp32 [in, out]."""
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, w = t.shape
    assert w == 16 * K
    out = np.empty((tk * 16, tn * 16), dtype=np.float32)
    lib().oc_decode_tiles(_ptr(t), tk, tn, K, cb, _ptr(out))
    return out


def dequant(trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int, cb: int) -> np.ndarray:
    """Bit-exact fp16 W[in, out].  csrc/bindings.cpp:15-100 (+ cb 0 for 3INST)."""
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, w = t.shape
    if w != 16 * K:
        raise ValueError("trellis last dimension must be 16*K")
    if (tk * 16) % 128 or (tn * 16) % 128:
        raise ValueError("trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    su = np.ascontiguousarray(suh, dtype=np.float16).view(np.uint16)
    sv = np.ascontiguousarray(svh, dtype=np.float16).view(np.uint16)
    out = np.empty((tk * 16, tn * 16), dtype=np.uint16)
    lib().oc_dequant(_ptr(t), tk, tn, K, cb, _ptr(su), _ptr(sv), _ptr(out))
    return out.view(np.float16)


# ---------------------------------------------------------------------------
# Hadamard helpers (float64 closed forms used by the tests)
# ---------------------------------------------------------------------------

def hadamard_matrix(n: int = 128) -> np.ndarray:
    """Sylvester Walsh-Hadamard matrix (natural order), entries +-1."""
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def block_hadamard(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Normalised 128-block Hadamard along ``axis`` in float64."""
    x = np.moveaxis(np.asarray(x, dtype=np.float64), axis, -1)
    n = x.shape[-1]
    assert n % 128 == 0
    h = hadamard_matrix(128) / np.sqrt(128.0)
    y = (x.reshape(*x.shape[:-1], n // 128, 128) @ h).reshape(x.shape)
    return np.moveaxis(y, -1, axis)


# ---------------------------------------------------------------------------
# GEMV / MoE (reference eager semantics)
# ---------------------------------------------------------------------------

def gemv(x: np.ndarray, w16: np.ndarray) -> np.ndarray:
    """y = fp16(x) @ W in fp32.  csrc/bindings.cpp:144-146 (x cast to fp16 at
    the plugin boundary, exl3.py:2856)."""
    xf = np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    return xf @ np.asarray(w16, dtype=np.float32)


def map_topk_to_local(ids: np.ndarray, n_local: int,
                      expert_map: np.ndarray | None = None) -> np.ndarray:
    """Global expert ids -> local ids; invalid or non-local ids -> the
    ``n_local`` sentinel.  src/vllm_exl3/exl3.py:2332-2354: without a map an
    id is local when 0 <= id < n_local; with a map, ``expert_map[id]`` is the
    local id (negative = not on this rank), valid when 0 <= id < len(map) and
    0 <= map[id] < n_local."""
    ids = np.asarray(ids, dtype=np.int64)
    if expert_map is None:
        return np.where((ids < 0) | (ids >= n_local), n_local, ids)
    emap = np.asarray(expert_map, dtype=np.int64).reshape(-1)
    n_global = emap.size
    if n_global == 0:
        return np.full_like(ids, n_local)
    mapped = emap[np.clip(ids, 0, n_global - 1)]
    invalid = (ids < 0) | (ids >= n_global) | (mapped < 0) | (mapped >= n_local)
    return np.where(invalid, n_local, mapped)


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def moe_activation(g: np.ndarray | None, u: np.ndarray, act: str = "silu",
                   limit: float | None = None) -> np.ndarray:
    """The routed expert's activation in fp32, with the reference's clamp rules.

    src/vllm_exl3/exl3.py:2386-2410 (the eager loop) and csrc/p2b_moe.cu:
    755-768 (the kernel): a limit > 0 clamps the gate from above only and the
    up projection symmetrically; a limit of None, 0 or below is plain.
    * ``silu``: silu(g) * u;
    * ``swiglu_oai``: (u + 1) * g * sigmoid(1.702 g) (alpha 1.702, beta 1);
    * gateless (``g is None``): relu(u)^2 with the symmetric up clamp."""
    u = np.asarray(u, dtype=np.float32)
    clamp = limit is not None and limit > 0
    if g is None:
        if clamp:
            u = np.clip(u, np.float32(-limit), np.float32(limit))
        return np.square(np.maximum(u, np.float32(0))).astype(np.float32)
    g = np.asarray(g, dtype=np.float32)
    if clamp:
        g = np.minimum(g, np.float32(limit))
        u = np.clip(u, np.float32(-limit), np.float32(limit))
    if act == "swiglu_oai":
        sig = np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-1.702) * g))
        return ((u + np.float32(1.0)) * g * sig).astype(np.float32)
    if act != "silu":
        raise ValueError(f"unknown activation {act!r}")
    return (silu(g) * u).astype(np.float32)


def _f16(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def moe_reference(x: np.ndarray, ids: np.ndarray, weights: np.ndarray,
                  experts: list[dict], limit: float | None = None,
                  act: str = "silu", round_down: bool = False, gu_fp16: bool = True,
                  expert_map: np.ndarray | None = None) -> np.ndarray:
    """Per-route expert loop with fp32 accumulation: out[t] = sum over k of
    w[t,k] * down(act(gate(x_t), up(x_t))) for the local experts of row t.

    ``experts[e]`` holds dense matrices ``gate`` [H, I] (None for a gateless
    layer), ``up`` [H, I], ``down`` [I, H] (fp16 as ``dequant`` produces them;
    float32 matrices are used as given).  Rounding points, in order:

    1. x is rounded to fp16 (the plugin casts activations to fp16 before
       every EXL3 projection, exl3.py:2856 / 2396 ``.half()``);
    2. g = x @ gate and u = x @ up in fp32; with ``gu_fp16`` (default) each
       is rounded to fp16 -- the native kernel stores the GEMV tile results as
       fp16 (csrc/p2b_moe.cu:284) and the reference's native contract test
       rounds them (tests/test_native_moe_contract.py:104-105).  With
       ``gu_fp16=False`` they stay fp32, as in the eager loop
       (exl3.py:2392-2410, ``out_dtype=torch.float32``);
    3. the activation (``moe_activation``) in fp32, rounded to fp16 before
       the down projection (exl3.py:2410 ``.half()``);
    4. d = act @ down in fp32, rounded to fp16 when ``round_down`` (the
       contract test's ``.half()`` at tests/test_native_moe_contract.py:107);
    5. out[t] += fp32(w[t,k]) * d, in slot order k = 0, 1, ... (the
       deterministic combine order of csrc/p2b_moe.cu:1976-2008).

    Ids are mapped by ``map_topk_to_local`` (with ``expert_map`` when given);
    sentinel routes contribute nothing.
    """
    x = np.asarray(x)
    T, H = x.shape
    ids = map_topk_to_local(ids, len(experts), expert_map)
    out = np.zeros((T, H), dtype=np.float32)
    xh = _f16(x)
    for t in range(T):
        for k in range(ids.shape[1]):
            e = int(ids[t, k])
            if e >= len(experts):
                continue
            pack = experts[e]
            xv = xh[t:t + 1]
            u = xv @ np.asarray(pack["up"], dtype=np.float32)
            g = None
            if pack.get("gate") is not None:
                g = xv @ np.asarray(pack["gate"], dtype=np.float32)
            if gu_fp16:
                u = _f16(u)
                g = None if g is None else _f16(g)
            a = _f16(moe_activation(g, u, act, limit))
            d = a @ np.asarray(pack["down"], dtype=np.float32)
            if round_down:
                d = _f16(d)
            out[t] += np.float32(weights[t, k]) * d[0]
    return out


# ---------------------------------------------------------------------------
# int4-asymmetric paged KV cache (format defined in this build)
# ---------------------------------------------------------------------------

KV_GROUP = 32


def kv_quantize_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Quantise [..., D] rows per 32-element group.

    zero = fp16(min), scale = fp16((max - min) / 15) computed in fp32;
    q = clamp(rint((x - zero) / scale), 0, 15) in fp32 with the fp16-rounded
    zero and scale (scale 0 -> q 0).  Returns (q uint8 [..., D], scale fp16
    [..., D/32], zero fp16 [..., D/32]).
    """
    x = np.asarray(x, dtype=np.float32)
    D = x.shape[-1]
    g = x.reshape(*x.shape[:-1], D // KV_GROUP, KV_GROUP)
    mn = g.min(axis=-1)
    mx = g.max(axis=-1)
    zero = mn.astype(np.float16)
    scale = ((mx - mn) / np.float32(15.0)).astype(np.float32).astype(np.float16)
    zf = zero.astype(np.float32)[..., None]
    sf = scale.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(sf > 0, np.rint((g - zf) / np.where(sf > 0, sf, 1)), 0)
    q = np.clip(q, 0, 15).astype(np.uint8).reshape(x.shape)
    return q, scale, zero


def kv_dequantize_rows(q: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """x = q * scale + zero in fp32 (fp16 scale/zero widened exactly)."""
    D = q.shape[-1]
    qg = q.reshape(*q.shape[:-1], D // KV_GROUP, KV_GROUP).astype(np.float32)
    v = qg * scale.astype(np.float32)[..., None] + zero.astype(np.float32)[..., None]
    return v.reshape(q.shape).astype(np.float32)


def attention_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Dense softmax attention for one decode step, float64.

    q [B, Hq, D]; k, v [B, Hkv, L, D]; GQA with Hq/Hkv query heads per KV head.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    qg = q.reshape(B, Hkv, g, D)
    s = np.einsum("bhgd,bhld->bhgl", qg, k) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhgl,bhld->bhgd", p, v)
    return o.reshape(B, Hq, D)


# ---------------------------------------------------------------------------
# Paged int4 KV cache: page layout (format defined in this build)
# ---------------------------------------------------------------------------
# One page holds 16 tokens of one KV head in 2560 bytes (160 B per token):
#   [   0, 1024)  K codes: token-major nibbles in the order the QK matrix-core
#                 operand reads them (lane l = t + 16 j; 32-bit word g of the
#                 lane's 16 bytes holds dims 32 g + 8 j + p at bits 4 p).
#   [1024, 2048)  V codes: dim-major nibbles in the order the PV operand reads
#                 them (lane l = m + 16 j for dims 16 b + m and tokens
#                 4 j + i; word b // 2, bit 8 (b % 2) + (0, 16, 4, 20)[i]).
#   [2048, 2176)  K scale fp16 [4 token quads][4 groups][4 tokens] (token
#                 4 j + i at 16 j + 4 g + i: a decode lane's 16 scales, its
#                 four tokens in every group, are 32 contiguous bytes)
#   [2176, 2304)  K zero  fp16 [4 groups][16 tokens]
#   [2304, 2432)  V scale fp16 [4 token quads][4 groups][4 tokens]
#   [2432, 2560)  V zero  fp16 [4 groups][16 tokens]
# The pool is uint8 [num_pages, num_kv_heads, 2560]; a sequence's logical
# page i lives at physical page block_table[b, i].

KV_PAGE = 16
KV_HEAD_DIM = 128
KV_PAGE_BYTES = 2560
KV_OFF_KS, KV_OFF_KZ, KV_OFF_VS, KV_OFF_VZ = 2048, 2176, 2304, 2432
_V_BIT = (0, 16, 4, 20)


def kv_k_nibble_bit(t: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Bit offset (from the page start) of K code (token t, dim d)."""
    t, d = np.asarray(t), np.asarray(d)
    g, r = d // 32, d % 32
    j, p = r // 8, r % 8
    lane = t + 16 * j
    return (16 * lane + 4 * g) * 8 + 4 * p


def kv_v_nibble_bit(t: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Bit offset (from the page start) of V code (token t, dim d)."""
    t, d = np.asarray(t), np.asarray(d)
    b, m = d // 16, d % 16
    j, i = t // 4, t % 4
    lane = m + 16 * j
    return (1024 + 16 * lane + 4 * (b // 2)) * 8 + 8 * (b % 2) + np.asarray(_V_BIT)[i]


def _put_nibbles(page: np.ndarray, bits: np.ndarray, codes: np.ndarray) -> None:
    byte, sh = bits // 8, bits % 8
    np.bitwise_or.at(page, byte.ravel(), (codes.astype(np.uint8) << sh.astype(np.uint8)).ravel())


def _get_nibbles(page: np.ndarray, bits: np.ndarray) -> np.ndarray:
    byte, sh = bits // 8, bits % 8
    return (page[byte] >> sh.astype(np.uint8)) & 0xF


def kv_pack_pages(k: np.ndarray, v: np.ndarray, seq_lens: np.ndarray, block_table: np.ndarray,
                  num_pages: int) -> np.ndarray:
    """Quantise K, V [B, Hkv, L, 128] into a paged pool [num_pages, Hkv, 2560].

    Tokens at or past seq_lens[b] inside a sequence's last page are stored as
    code 0 with scale 0 and zero 0; pages no sequence uses stay zero."""
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, Hkv, L, D = k.shape
    assert D == KV_HEAD_DIM
    pool = np.zeros((num_pages, Hkv, KV_PAGE_BYTES), dtype=np.uint8)
    tt, dd = np.meshgrid(np.arange(KV_PAGE), np.arange(D), indexing="ij")
    kbits, vbits = kv_k_nibble_bit(tt, dd), kv_v_nibble_bit(tt, dd)
    for b in range(B):
        n = int(seq_lens[b])
        for lp in range((n + KV_PAGE - 1) // KV_PAGE):
            pg = int(block_table[b, lp])
            t0 = lp * KV_PAGE
            cnt = min(KV_PAGE, n - t0)
            for h in range(Hkv):
                page = pool[pg, h]
                for side, src, bits, off_s, off_z in ((0, k, kbits, KV_OFF_KS, KV_OFF_KZ),
                                                      (1, v, vbits, KV_OFF_VS, KV_OFF_VZ)):
                    rows = np.zeros((KV_PAGE, D), dtype=np.float32)
                    rows[:cnt] = src[b, h, t0:t0 + cnt]
                    q, s, z = kv_quantize_rows(rows)
                    q[cnt:] = 0
                    s[cnt:] = 0
                    z[cnt:] = 0
                    _put_nibbles(page, bits, q)
                    page[off_s:off_s + 128] = _scales_to_page(s).view(np.uint8).ravel()
                    page[off_z:off_z + 128] = np.ascontiguousarray(z.T).view(np.uint8).ravel()
    return pool


def _scales_to_page(s: np.ndarray) -> np.ndarray:
    """Scales [16 tokens, 4 groups] in page order [token quad][group][token % 4]."""
    return np.ascontiguousarray(s.reshape(4, 4, 4).transpose(0, 2, 1)).ravel()


def _scales_from_page(w: np.ndarray) -> np.ndarray:
    """Inverse of _scales_to_page: [16 tokens, 4 groups]."""
    return np.ascontiguousarray(w.reshape(4, 4, 4).transpose(0, 2, 1)).reshape(KV_PAGE, 4)


def kv_unpack_page(page: np.ndarray, side: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codes uint8 [16, 128], scale fp16 [16, 4], zero fp16 [16, 4]) of one page side."""
    tt, dd = np.meshgrid(np.arange(KV_PAGE), np.arange(KV_HEAD_DIM), indexing="ij")
    bits = kv_k_nibble_bit(tt, dd) if side == 0 else kv_v_nibble_bit(tt, dd)
    q = _get_nibbles(np.asarray(page, dtype=np.uint8), bits).astype(np.uint8)
    off_s, off_z = (KV_OFF_KS, KV_OFF_KZ) if side == 0 else (KV_OFF_VS, KV_OFF_VZ)
    s = _scales_from_page(np.ascontiguousarray(page[off_s:off_s + 128]).view(np.float16))
    z = np.ascontiguousarray(page[off_z:off_z + 128]).view(np.float16).reshape(4, KV_PAGE).T
    return q, s, z


def kv_unpack_pages(pool: np.ndarray, seq_lens: np.ndarray, block_table: np.ndarray,
                    L: int) -> tuple[np.ndarray, np.ndarray]:
    """Dequantised K, V [B, Hkv, L, 128] fp32 (zeros past seq_lens)."""
    B = len(seq_lens)
    Hkv = pool.shape[1]
    out = [np.zeros((B, Hkv, L, KV_HEAD_DIM), dtype=np.float32) for _ in range(2)]
    for b in range(B):
        n = int(seq_lens[b])
        for lp in range((n + KV_PAGE - 1) // KV_PAGE):
            pg = int(block_table[b, lp])
            t0 = lp * KV_PAGE
            cnt = min(KV_PAGE, n - t0)
            for h in range(Hkv):
                for side in (0, 1):
                    q, s, z = kv_unpack_page(pool[pg, h], side)
                    x = kv_dequantize_rows(q, s, z)
                    out[side][b, h, t0:t0 + cnt] = x[:cnt]
    return out[0], out[1]


def attention_decode_lens(q: np.ndarray, k: np.ndarray, v: np.ndarray, seq_lens: np.ndarray,
                          scale: float) -> np.ndarray:
    """``attention_decode`` with per-sequence lengths (keys [0, seq_lens[b]))."""
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(q.shape[0]):
        n = int(seq_lens[b])
        if n > 0:
            out[b:b + 1] = attention_decode(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], scale)
    return out


# ---------------------------------------------------------------------------
# n-gram embedding rows (mul1 codebook, 160-dim ring bitstream)
# ---------------------------------------------------------------------------
NGRAM_ROW_DIM = 160


def ngram_words_per_row(bits: int) -> int:
    """One fp16 scale word plus the K-bit ring bitstream (``exl3.py:5174-5176``)."""
    return 1 + NGRAM_ROW_DIM * int(bits) // 16


def ngram_bit_tables(bits: int) -> tuple[np.ndarray, np.ndarray]:
    """(word, bit) of state bit m of element i: ring position
    ((i - m // K) mod 160) * K + m % K, one word after the scale
    (``_ngram_bit_tables``, ``exl3.py:5196-5207``)."""
    i = np.arange(NGRAM_ROW_DIM)[:, None]
    m = np.arange(16)[None, :]
    sb = ((i - m // bits) % NGRAM_ROW_DIM) * bits + m % bits
    return 1 + (sb >> 4), sb & 15


def ngram_dequant_rows(packed: np.ndarray, bits: int, heads: np.ndarray,
                       head_bias: np.ndarray) -> np.ndarray:
    """fp16 [N, 160] = fp16(codebook_mul1[state] * scale + head_bias[head]),
    the product and the sum in fp32 (``ngram_dequant_rows_torch``,
    ``exl3.py:5212-5238``)."""
    packed = np.asarray(packed, dtype=np.int16)
    widx, bidx = ngram_bit_tables(bits)
    words = packed.astype(np.int64) & 0xFFFF
    state = (((words[:, widx] >> bidx) & 1) << np.arange(16)).sum(-1)
    cb = decode_codebook_table(2).view(np.float16)
    vals = cb[state].astype(np.float32)
    scale = packed[:, :1].copy().view(np.float16).astype(np.float32)
    bias = np.asarray(head_bias, dtype=np.float16)[np.asarray(heads, dtype=np.int64)].astype(np.float32)
    return ((vals * scale).astype(np.float32) + bias).astype(np.float16)
