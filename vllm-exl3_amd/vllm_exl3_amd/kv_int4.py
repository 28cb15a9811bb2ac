"""Paged int4 KV cache: pack, unpack and split-K decode attention on the GPU.

The host side of the reference's 4-bit KV decode overlay
(``q4_sparse_decode``, src/vllm_exl3/minimax_q4kv_kernels.py:772-877) for the
int4-asymmetric format this build defines: per (token, KV head, 32-dim
group) an fp16 scale and zero, codes 0..15, 16-token pages of 2560 bytes per
KV head.  Like the reference wrapper it validates geometry before any launch
(raising ``ValueError``), never synchronises and picks a shape-constant split
count, so a decode step can be captured in a HIP graph.  Every call runs the
HIP kernels of ``libexl3_mi355x.so``; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .vllm_exl3_c import _DTYPE_ID, stream_of, workspace

PAGE_TOKENS = 16
HEAD_DIM = 128


def page_bytes() -> int:
    """Bytes of one page of one KV head (16 tokens x 160 B)."""
    return int(_lib.load().exl3_kv_page_bytes())


def new_pool(num_pages: int, num_kv_heads: int, device) -> torch.Tensor:
    """A zeroed uint8 pool [num_pages, num_kv_heads, page_bytes]."""
    return torch.zeros((num_pages, num_kv_heads, page_bytes()), dtype=torch.uint8, device=device)


def _check_tables(pool: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor) -> None:
    if pool.dtype is not torch.uint8 or pool.dim() != 3 or not pool.is_contiguous():
        raise ValueError("int4 KV pool must be a contiguous uint8 [pages, kv_heads, page_bytes] tensor")
    if pool.size(2) != page_bytes():
        raise ValueError(f"int4 KV pool pages must be {page_bytes()} bytes per KV head")
    if seq_lens.dtype is not torch.int32 or seq_lens.dim() != 1 or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 vector")
    if block_table.dtype is not torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 [B, max_pages] with unit column stride")
    if block_table.size(0) != seq_lens.numel():
        raise ValueError("block_table and seq_lens disagree on the batch size")
    for t, nm in ((seq_lens, "seq_lens"), (block_table, "block_table")):
        if t.device != pool.device:
            raise ValueError(f"{nm} must be on the pool's device")
    if not pool.is_cuda:
        raise ValueError("the int4 KV cache lives in device memory")


def pack_pages(k: torch.Tensor, v: torch.Tensor, seq_lens: torch.Tensor,
               block_table: torch.Tensor, pool: torch.Tensor) -> None:
    """Quantise k, v [B, kv_heads, L, 128] (fp16/bf16/fp32, unit dim stride)
    into the pool pages of tokens [0, seq_lens[b])."""
    _check_tables(pool, seq_lens, block_table)
    if k.shape != v.shape or k.dim() != 4 or k.size(3) != HEAD_DIM:
        raise ValueError("k and v must both be [B, kv_heads, L, 128]")
    if k.stride() != v.stride() or k.stride(3) != 1 or k.dtype != v.dtype:
        raise ValueError("k and v must share dtype and strides, with unit dim stride")
    if k.dtype not in _DTYPE_ID or k.device != pool.device:
        raise ValueError("k and v must be fp16/bf16/fp32 tensors on the pool's device")
    B, H = k.size(0), k.size(1)
    if H != pool.size(1) or B != seq_lens.numel():
        raise ValueError("k/v geometry does not match the pool and tables")
    with torch.cuda.device(pool.device):
        _lib.call("exl3_kv_pack_pages", k.data_ptr(), v.data_ptr(), _DTYPE_ID[k.dtype], B, H,
                  k.stride(0), k.stride(1), k.stride(2), seq_lens.data_ptr(), block_table.data_ptr(),
                  block_table.stride(0), block_table.size(1), pool.data_ptr(), pool.size(0),
                  stream_of(pool.device))


def unpack_pages(pool: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor,
                 L: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Dequantised fp32 K, V [B, kv_heads, L, 128]; positions past seq_lens are 0."""
    _check_tables(pool, seq_lens, block_table)
    B, H = seq_lens.numel(), pool.size(1)
    k = torch.zeros((B, H, L, HEAD_DIM), dtype=torch.float32, device=pool.device)
    v = torch.zeros_like(k)
    with torch.cuda.device(pool.device):
        _lib.call("exl3_kv_unpack_pages", pool.data_ptr(), pool.size(0), H, seq_lens.data_ptr(),
                  block_table.data_ptr(), block_table.stride(0), B, block_table.size(1),
                  k.data_ptr(), v.data_ptr(), L, stream_of(pool.device))
    return k, v


def int4_decode(q: torch.Tensor, pool: torch.Tensor, block_table: torch.Tensor,
                seq_lens: torch.Tensor, num_kv_heads: int, sm_scale: float,
                output: torch.Tensor, n_splits: int = 0) -> torch.Tensor:
    """One decode step of attention over the int4 cache.

    q, output [B, Hq, 128] (fp16/bf16/fp32, unit dim stride); GQA with
    Hq / num_kv_heads <= 16.  Same argument meaning as the reference's
    ``q4_sparse_decode`` minus the sparse top-k page list (this format is
    dense: every cached token [0, seq_lens[b]) is attended).  Writes
    ``output`` in place and returns it."""
    _check_tables(pool, seq_lens, block_table)
    if q.dim() != 3 or q.size(2) != HEAD_DIM or q.stride(2) != 1:
        raise ValueError("int4 decode requires q [B, H, 128] with unit dim stride")
    if output.shape != q.shape or output.stride(2) != 1:
        raise ValueError("output must be [B, H, 128] with unit dim stride")
    B, Hq, _ = q.shape
    if num_kv_heads != pool.size(1) or Hq % num_kv_heads or Hq // num_kv_heads > 16:
        raise ValueError("int4 decode: Hq must be a multiple of num_kv_heads, at most 16 per KV head")
    if B != seq_lens.numel():
        raise ValueError("q and seq_lens disagree on the batch size")
    if q.dtype not in _DTYPE_ID or output.dtype not in _DTYPE_ID:
        raise ValueError("q and output must be fp16, bf16 or fp32")
    if q.device != pool.device or output.device != pool.device:
        raise ValueError("q and output must be on the pool's device")
    lib = _lib.load()
    max_pages = block_table.size(1)
    need = int(lib.exl3_kv_decode_workspace_size(B, Hq, num_kv_heads, max_pages, int(n_splits)))
    ws = workspace(pool.device, "kv_decode", need)
    with torch.cuda.device(pool.device):
        _lib.call("exl3_kv_decode", q.data_ptr(), _DTYPE_ID[q.dtype], B, Hq, num_kv_heads,
                  q.stride(0), q.stride(1), pool.data_ptr(), pool.size(0), block_table.data_ptr(),
                  block_table.stride(0), max_pages, seq_lens.data_ptr(), float(sm_scale),
                  output.data_ptr(), _DTYPE_ID[output.dtype], output.stride(0), output.stride(1),
                  int(n_splits), ws.data_ptr(), ws.numel(), stream_of(pool.device))
    return output
