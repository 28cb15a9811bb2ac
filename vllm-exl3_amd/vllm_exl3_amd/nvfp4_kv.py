"""The reference's NVFP4 ("q4") paged KV cache on the GPU: pack, pool
dequant, prefill staging and the block-sparse decode attention.

Host side of ``q4_sparse_decode`` (src/vllm_exl3/minimax_q4kv_kernels.py:
772-877) and of the reference packer / dequantiser
(src/vllm_exl3/minimax_q4kv_reference.py:297-366, 735-776) over the same
pool format, byte for byte: uint8 ``[pages, 2*num_kv_heads, 128, 72]``,
slot ``2h`` = K and ``2h+1`` = V of KV head h, each slot a flat 9216-byte
region (128 tokens x 64 data bytes, then 1024 e4m3 scale bytes).  Every call
runs the HIP kernels of ``libexl3_mi355x.so``; there is no CPU path.
Geometry errors raise ``ValueError`` before any launch; nothing synchronises
with the host, so a decode step can be captured in a HIP graph.
"""

from __future__ import annotations

import torch

from . import _lib
from .vllm_exl3_c import _DTYPE_ID, stream_of, workspace

PAGE_TOKENS = 128
HEAD_DIM = 128
ROW_BYTES = 72


def new_pool(num_pages: int, num_kv_heads: int, device) -> torch.Tensor:
    """A zeroed pool uint8 [num_pages, 2*num_kv_heads, 128, 72]."""
    return torch.zeros((num_pages, 2 * num_kv_heads, PAGE_TOKENS, ROW_BYTES), dtype=torch.uint8,
                       device=device)


def _check_pool(pool: torch.Tensor, num_kv_heads: int | None = None) -> None:
    if pool.dtype is not torch.uint8:
        raise ValueError("q4 decode requires the pool as raw uint8 bytes")
    if pool.dim() != 4 or pool.shape[2:] != (PAGE_TOKENS, ROW_BYTES) or pool.shape[1] % 2:
        raise ValueError("q4 pool geometry mismatch")
    if num_kv_heads is not None and pool.shape[1] != 2 * num_kv_heads:
        raise ValueError("q4 pool geometry mismatch")
    if pool.stride(3) != 1 or pool.stride(2) != ROW_BYTES or pool.stride(1) != PAGE_TOKENS * ROW_BYTES \
            or pool.stride(0) != pool.shape[1] * PAGE_TOKENS * ROW_BYTES:
        raise ValueError("q4 pool slot regions must be contiguous")
    if not pool.is_cuda:
        raise ValueError("the q4 pool lives in device memory")


def _i32(t: torch.Tensor, name: str, device) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.int64) or t.device != device:
        raise ValueError(f"{name} must be an int32/int64 tensor on the pool's device")
    return t.to(torch.int32)


def pack_pages(k: torch.Tensor, v: torch.Tensor, seq_lens: torch.Tensor,
               block_table: torch.Tensor, pool: torch.Tensor) -> None:
    """Quantise k, v [B, kv_heads, L, 128] (fp16/bf16/fp32, unit dim stride)
    into the pool: token p of sequence b goes to slot p % 128 of page
    block_table[b, p // 128]; only tokens [0, seq_lens[b]) are written."""
    _check_pool(pool)
    if k.shape != v.shape or k.dim() != 4 or k.size(3) != HEAD_DIM:
        raise ValueError("k and v must both be [B, kv_heads, L, 128]")
    if k.stride() != v.stride() or k.stride(3) != 1 or k.dtype != v.dtype or k.dtype not in _DTYPE_ID:
        raise ValueError("k and v must share a float dtype and strides, with unit dim stride")
    B, H, L, _ = k.shape
    if pool.shape[1] != 2 * H or k.device != pool.device or v.device != pool.device:
        raise ValueError("k/v geometry does not match the pool")
    sl = _i32(seq_lens, "seq_lens", pool.device).contiguous()
    bt = _i32(block_table, "block_table", pool.device)
    if sl.numel() != B or bt.dim() != 2 or bt.size(0) != B or bt.stride(1) != 1:
        raise ValueError("seq_lens [B] and block_table [B, max_blocks] (unit column stride) required")
    with torch.cuda.device(pool.device):
        _lib.call("exl3_nvfp4_pack_pages", k.data_ptr(), v.data_ptr(), _DTYPE_ID[k.dtype], B, H,
                  k.stride(0), k.stride(1), k.stride(2), L, sl.data_ptr(), bt.data_ptr(), bt.stride(0),
                  bt.size(1), pool.data_ptr(), pool.size(0), stream_of(pool.device))


def dequant_pool_pages(pool: torch.Tensor) -> torch.Tensor:
    """fp32 values [pages, 2*kv_heads, 128, 128] of every slot
    (``dequant_pool_pages``, minimax_q4kv_reference.py:735-776)."""
    _check_pool(pool)
    out = torch.empty((pool.size(0), pool.size(1), PAGE_TOKENS, HEAD_DIM), dtype=torch.float32,
                      device=pool.device)
    with torch.cuda.device(pool.device):
        _lib.call("exl3_nvfp4_dequant_pages", pool.data_ptr(), pool.size(0), pool.size(1) // 2,
                  out.data_ptr(), stream_of(pool.device))
    return out


def q4_stage_pages(buffer: torch.Tensor, pool: torch.Tensor, pages: torch.Tensor) -> int:
    """Dequantise ``pages`` of the q4 pool into staging rows ``buffer[:n]``
    and zero ``buffer[n]``; returns n = ``pages.numel()``.

    Same arguments, result and refusals as ``q4_stage_pages``
    (src/vllm_exl3/minimax_q4kv_kernels.py:880-951): ``buffer`` bf16
    [capacity, num_kv_heads, 128, 256] (K values in columns 0..127, V values
    in 128..255), ``pool`` uint8 [nb, 2*num_kv_heads, 128, 72] with
    contiguous 9216-byte slot regions, ``pages`` int32/int64 physical page
    ids.  The staged bytes equal the bf16 cast of ``dequant_pool_pages``
    (every e2m1 x e4m3 product is exact in bf16).  One launch, which also
    writes the zero row; page ids are read on the device only, so nothing
    synchronises with the host.  A page id outside [0, nb) stages a row of
    zeros."""
    for name, t in (("buffer", buffer), ("pages", pages)):
        if t.device != pool.device:
            raise ValueError(f"q4 KV refused: '{name}' is on {t.device}, expected {pool.device}")
    if not pool.is_cuda:
        raise ValueError(f"q4 KV refused: 'pool' must be on a cuda device, got {pool.device}")
    if pool.dtype is not torch.uint8:
        raise ValueError("q4 staging requires the pool as raw uint8 bytes, got "
                         f"{str(pool.dtype).replace('torch.', '')}; the overlay must re-view the "
                         "container before dispatch")
    if pool.dim() != 4 or pool.shape[2] != PAGE_TOKENS or pool.shape[3] != ROW_BYTES:
        raise ValueError("q4 pool must be [nb, 2*num_kv_heads, 128, 72]")
    if pool.stride(2) != ROW_BYTES or pool.stride(1) != PAGE_TOKENS * ROW_BYTES or pool.stride(3) != 1:
        raise ValueError("q4 pool slot regions must be contiguous")
    if buffer.dtype is not torch.bfloat16:
        raise ValueError(f"staging buffer must be bf16, got {str(buffer.dtype).replace('torch.', '')}")
    if pages.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"page ids must be int64/int32, got {str(pages.dtype).replace('torch.', '')}")
    num_kv_heads = pool.shape[1] // 2
    if buffer.dim() != 4 or buffer.shape[1] != num_kv_heads or buffer.shape[2] != PAGE_TOKENS \
            or buffer.shape[3] != 256:
        raise ValueError("staging buffer must be [capacity, num_kv_heads, 128, 256]")
    if not buffer.is_contiguous():
        raise ValueError("staging buffer must be contiguous")
    n = int(pages.numel())
    if n > buffer.shape[0] - 1:
        raise ValueError(f"staging buffer holds {buffer.shape[0] - 1} pages, need {n}")
    if pool.stride(0) != pool.shape[1] * PAGE_TOKENS * ROW_BYTES:
        pool = pool.contiguous()
    pg = pages.reshape(-1)
    if n and not pg.is_contiguous():
        pg = pg.contiguous()
    with torch.cuda.device(pool.device):
        _lib.call("exl3_nvfp4_stage_pages", pool.data_ptr(), pool.size(0), num_kv_heads,
                  pg.data_ptr() if n else 0, 1 if pg.dtype == torch.int64 else 0, n, buffer.data_ptr(),
                  buffer.size(0), stream_of(pool.device))
    return n


def _chunks(total_q: int, num_kv_heads: int, max_topk: int) -> int:
    """Shape-constant number of top-k chunks (graph safe): about 512
    workgroups in flight, a power of two, at most max_topk."""
    target = max(1, min(max_topk, 512 // max(1, total_q * num_kv_heads)))
    return 1 << (target.bit_length() - 1)


def q4_sparse_decode(q: torch.Tensor, pool: torch.Tensor, topk_idx: torch.Tensor,
                     block_table: torch.Tensor, seq_lens: torch.Tensor, num_kv_heads: int,
                     sm_scale: float, output: torch.Tensor, decode_query_len: int) -> None:
    """Block-sparse decode attention over the q4 pool, written into
    ``output`` [total_q, H, 128].  Same arguments and meaning as the
    reference: topk_idx [num_kv_heads, total_q, topk] logical block ids per
    query token (entries outside [0, n_blocks) skipped; the first
    min(topk, n_blocks) entries are examined), causal within the last block,
    query token i of request i // decode_query_len at position
    seq_len - decode_query_len + i % decode_query_len."""
    if q.dim() != 3 or q.size(2) != HEAD_DIM or q.stride(2) != 1:
        raise ValueError("q4 decode requires head_dim == 128")
    _check_pool(pool, num_kv_heads)
    total_q, Hq, _ = q.shape
    if Hq % num_kv_heads or Hq // num_kv_heads > 16:
        raise ValueError("q4 decode: Hq must be a multiple of num_kv_heads, at most 16 per KV head")
    if output.shape != q.shape or output.stride(2) != 1:
        raise ValueError("output must be [total_q, H, 128] with unit dim stride")
    if q.dtype not in _DTYPE_ID or output.dtype not in _DTYPE_ID:
        raise ValueError("q and output must be fp16, bf16 or fp32")
    dev = pool.device
    if q.device != dev or output.device != dev:
        raise ValueError("q and output must be on the pool's device")
    if seq_lens.dim() != 1 or total_q != seq_lens.numel() * decode_query_len:
        raise ValueError("total_q must equal len(seq_lens) * decode_query_len")
    if topk_idx.dim() != 3 or topk_idx.shape[:2] != (num_kv_heads, total_q):
        raise ValueError("topk_idx must be [num_kv_heads, total_q, topk]")
    tk = _i32(topk_idx, "topk_idx", dev)
    if tk.stride(2) != 1:
        tk = tk.contiguous()
    sl = _i32(seq_lens, "seq_lens", dev).contiguous()
    bt = _i32(block_table, "block_table", dev)
    if bt.dim() != 2 or bt.size(0) != sl.numel() or bt.stride(1) != 1:
        raise ValueError("block_table must be [num_reqs, max_blocks] with unit column stride")
    max_topk = tk.size(2)
    n_chunks = _chunks(total_q, num_kv_heads, max_topk)
    lib = _lib.load()
    need = int(lib.exl3_nvfp4_decode_workspace_size(total_q, Hq, n_chunks))
    ws = workspace(dev, "q4_decode", need)
    with torch.cuda.device(dev):
        _lib.call("exl3_nvfp4_sparse_decode", q.data_ptr(), _DTYPE_ID[q.dtype], total_q, Hq,
                  num_kv_heads, q.stride(0), q.stride(1), pool.data_ptr(), pool.size(0), tk.data_ptr(),
                  tk.stride(0), tk.stride(1), max_topk, bt.data_ptr(), bt.stride(0), bt.size(1),
                  sl.data_ptr(), int(decode_query_len), float(sm_scale), output.data_ptr(),
                  _DTYPE_ID[output.dtype], output.stride(0), output.stride(1), n_chunks,
                  ws.data_ptr(), ws.numel(), stream_of(dev))


def _w1_vec(t: torch.Tensor | None, name: str, dev, n: int | None = None) -> None:
    if t is None:
        raise ValueError(f"q4 W1 refused: {name} is required")
    if t.device != dev or not t.is_contiguous():
        raise ValueError(f"q4 W1 refused: {name} must be a contiguous tensor on qkv's device")
    if n is not None and t.numel() != n:
        raise ValueError(f"q4 W1 refused: {name} must hold {n} values")


def q4_w1_insert(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                 cos_sin_cache: torch.Tensor, positions: torch.Tensor, num_heads: int,
                 num_kv_heads: int, rotary_dim: int, eps: float,
                 index_q_norm_w: torch.Tensor | None, index_k_norm_w: torch.Tensor | None,
                 num_index_heads: int, slot_mapping: torch.Tensor | None,
                 index_slot_mapping: torch.Tensor | None, pool: torch.Tensor,
                 index_cache: torch.Tensor | None, block_size: int, q_out: torch.Tensor | None,
                 index_q_out: torch.Tensor | None, *, check_positions: bool | None = None) -> None:
    """The W1 write path: Gemma QK-norm + partial NeoX RoPE of the fused bf16
    rows ``qkv`` [T, (nq + 2 nkv [+ niq + 1]) * 128] = [q | k | v | index_q |
    index_k], then: q -> ``q_out`` (bf16 [T, nq*128]); K and V -> q4 pack into
    pool slots 2h / 2h+1 of page ``slot_mapping // 128`` (-1 skips); index_q
    -> e4m3(bf16(v)) bytes into ``index_q_out``; index_k -> e4m3(clamp(v,
    +-448)) into row ``index_slot_mapping`` of ``index_cache``.  The processed
    K and index-K rows are written back into ``qkv`` (bf16), as the
    reference kernel does.

    Same arguments and refusal rules as ``q4_w1_insert``
    (src/vllm_exl3/minimax_q4kv_kernels.py:661-758, validate_w1_call
    src/vllm_exl3/minimax_q4kv_reference.py:625-732): bf16 rows, 128-token
    blocks, rotary_dim % 8 == 0, fp8 e4m3 index buffers (float8_e4m3fn or
    their uint8 byte views); refusals raise ``ValueError("q4 W1 refused:
    ...")`` before any launch.  As in the reference, a ``slot_mapping`` (or
    ``index_slot_mapping``) of None means ``positions`` serves as the slot
    mapping.  ``check_positions`` (default: when the stream is not being
    captured) verifies on the host that every position has a cos/sin row;
    the kernel itself skips a token whose position has none."""
    dev = qkv.device
    errors = []
    if qkv.dtype is not torch.bfloat16:
        errors.append(f"q4 W1 requires bfloat16 qkv rows, got {qkv.dtype}")
    niq = int(num_index_heads)
    per = num_heads + 2 * num_kv_heads + (niq + 1 if niq > 0 else 0)
    if qkv.dim() != 2 or qkv.size(1) != per * HEAD_DIM:
        errors.append(f"q4 W1 qkv width {qkv.size(-1)} does not match the branch layout "
                      f"{per * HEAD_DIM}")
    if qkv.dim() == 2 and qkv.size(0) <= 0:
        errors.append("q4 W1 requires a positive token count")
    if not (0 < rotary_dim <= HEAD_DIM and rotary_dim % 8 == 0):
        errors.append(f"q4 W1 requires 0 < rotary_dim <= 128 and rotary_dim % 8 == 0, "
                      f"got {rotary_dim}")
    if block_size != PAGE_TOKENS:
        errors.append(f"q4 W1 requires block_size {PAGE_TOKENS}, got {block_size}")
    if q_out is None:
        errors.append("q4 W1 requires the bf16 q_out buffer")
    fp8 = getattr(torch, "float8_e4m3fn", None)
    for nm, t in (("index_cache", index_cache), ("index_q_out", index_q_out)):
        if niq > 0 and t is not None and t.dtype not in (fp8, torch.uint8):
            errors.append(f"q4 W1 requires the fp8 e4m3 {nm}, got {t.dtype}")
    if errors:
        raise ValueError("q4 W1 refused: " + "; ".join(errors))
    _check_pool(pool, num_kv_heads)
    if not qkv.is_cuda or not qkv.is_contiguous():
        raise ValueError("q4 W1 refused: qkv must be a contiguous device tensor")
    T = qkv.size(0)
    if q_out.dtype is not torch.bfloat16 or q_out.numel() != T * num_heads * HEAD_DIM:
        raise ValueError("q4 W1 refused: q_out must be bf16 [T, num_heads*128]")
    _w1_vec(q_out, "q_out", dev)
    _w1_vec(q_norm_w, "q_norm_w", dev, HEAD_DIM)
    _w1_vec(k_norm_w, "k_norm_w", dev, HEAD_DIM)
    if positions.dtype is not torch.int64:
        raise ValueError("q4 W1 refused: positions must be int64")
    _w1_vec(positions, "positions", dev, T)
    sm = positions if slot_mapping is None else slot_mapping
    ism = positions if index_slot_mapping is None else index_slot_mapping
    for nm, t in (("slot_mapping", sm), ("index_slot_mapping", ism)):
        if t.dtype is not torch.int64:
            raise ValueError(f"q4 W1 refused: {nm} must be int64")
        _w1_vec(t, nm, dev, T)
    if cos_sin_cache.dim() != 2 or cos_sin_cache.size(1) != rotary_dim:
        raise ValueError(f"q4 W1 refused: cos_sin_cache must be [rows, {rotary_dim}]")
    _w1_vec(cos_sin_cache, "cos_sin_cache", dev)
    dts = {q_norm_w.dtype, k_norm_w.dtype}
    iqw = ikw = idx_q = idx_c = None
    rows = 0
    if niq > 0:
        _w1_vec(index_q_norm_w, "index_q_norm_w", dev, HEAD_DIM)
        _w1_vec(index_k_norm_w, "index_k_norm_w", dev, HEAD_DIM)
        dts |= {index_q_norm_w.dtype, index_k_norm_w.dtype}
        _w1_vec(index_q_out, "index_q_out", dev, T * niq * HEAD_DIM)
        _w1_vec(index_cache, "index_cache", dev)
        if index_cache.numel() % HEAD_DIM:
            raise ValueError("q4 W1 refused: index_cache rows are 128 bytes")
        rows = index_cache.numel() // HEAD_DIM
        iqw, ikw = index_q_norm_w.data_ptr(), index_k_norm_w.data_ptr()
        idx_q, idx_c = index_q_out.data_ptr(), index_cache.data_ptr()
    if len(dts) != 1 or next(iter(dts)) not in _DTYPE_ID:
        raise ValueError("q4 W1 refused: norm weights must share one of fp16/bf16/fp32")
    if cos_sin_cache.dtype not in _DTYPE_ID:
        raise ValueError("q4 W1 refused: cos_sin_cache must be fp16/bf16/fp32")
    if check_positions is None:
        check_positions = not torch.cuda.is_current_stream_capturing()
    if check_positions:
        lo, hi = int(positions.min()), int(positions.max())
        if lo < 0 or hi >= cos_sin_cache.size(0):
            raise ValueError(f"positions [{lo}, {hi}] exceed the cos_sin_cache "
                             f"({cos_sin_cache.size(0)} rows)")
    with torch.cuda.device(dev):
        _lib.call("exl3_nvfp4_w1_insert", qkv.data_ptr(), T, qkv.size(1), q_norm_w.data_ptr(),
                  k_norm_w.data_ptr(), iqw, ikw, _DTYPE_ID[q_norm_w.dtype],
                  cos_sin_cache.data_ptr(), _DTYPE_ID[cos_sin_cache.dtype], cos_sin_cache.size(0),
                  positions.data_ptr(), num_heads, num_kv_heads, niq, rotary_dim, float(eps),
                  sm.data_ptr(), ism.data_ptr(), pool.data_ptr(), pool.size(0), idx_c, rows,
                  q_out.data_ptr(), idx_q, stream_of(dev))
