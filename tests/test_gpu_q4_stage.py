"""GPU parity of the q4 prefill staging (nvfp4_kv.q4_stage_pages, the
reference's q4_stage_pages + _q4_stage_kernel,
src/vllm_exl3/minimax_q4kv_kernels.py:509-566, 880-951): page list -> bf16
staging rows, bit-exact against the CPU oracle (the bf16 cast of the pinned
pool dequant), on packed pools and on raw random pool bytes (every e4m3
scale code, NaN codes included); page lists with repeats, int32 and int64
ids, the empty list, a full buffer, ids outside the pool; the wrapper's
refusals."""

import numpy as np
import pytest
import torch

import nvfp4 as N
from vllm_exl3_amd import nvfp4_kv as Q
from vllm_exl3_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _packed_pool(gpu, seed, H, n_pages):
    B, L = 2, n_pages * 64
    k, v = S.kv_inputs(seed, B, H, L)
    bt = S.block_table(seed + 1, B, (L + 127) // 128, n_pages)
    pool = Q.new_pool(n_pages, H, gpu)
    Q.pack_pages(torch.from_numpy(k).to(gpu).bfloat16(), torch.from_numpy(v).to(gpu).bfloat16(),
                 torch.tensor([L, L], dtype=torch.int32, device=gpu), torch.from_numpy(bt).to(gpu), pool)
    return pool


@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_stage_packed_pool_bit_exact(gpu, ids_dtype):
    H, nb = 4, 12
    pool = _packed_pool(gpu, 41, H, nb)
    pages = torch.tensor([5, 0, 11, 5, 3, 7, 7, 1], dtype=ids_dtype, device=gpu)
    buf = torch.full((12, H, 128, 256), 3.0, dtype=torch.bfloat16, device=gpu)
    n = Q.q4_stage_pages(buf, pool, pages)
    torch.cuda.synchronize()
    assert n == 8
    want = N.stage_pages(pool.cpu().numpy(), pages.cpu().numpy())
    got = _bits(buf)
    assert np.array_equal(got[:9], want)
    assert (got[9:] == 0x4040).all()  # rows past n + 1 untouched (3.0 in bf16)


def test_stage_raw_bytes_every_scale_code(gpu):
    """Arbitrary pool bytes: every e4m3 code incl. subnormals and the two NaN
    codes (staged as 0x7FC0)."""
    H, nb = 2, 5
    g = np.random.default_rng(42)
    raw = g.integers(0, 256, size=(nb, 2 * H, 128, 72), dtype=np.uint8)
    flat = raw.reshape(nb, 2 * H, -1)
    flat[0, 0, 8192:8192 + 256] = np.arange(256, dtype=np.uint8)  # every code in one slot
    pool = torch.from_numpy(raw).to(gpu)
    pages = torch.tensor([0, 4, 2, 0, 1, 3], dtype=torch.int64, device=gpu)
    buf = torch.empty((7, H, 128, 256), dtype=torch.bfloat16, device=gpu)
    assert Q.q4_stage_pages(buf, pool, pages) == 6
    want = N.stage_pages(raw, pages.cpu().numpy())
    got = _bits(buf)
    assert (want == 0x7FC0).any()
    assert np.array_equal(got, want)


def test_stage_empty_full_and_out_of_pool(gpu):
    H, nb = 1, 4
    pool = _packed_pool(gpu, 43, H, nb)
    buf = torch.full((4, H, 128, 256), 1.0, dtype=torch.bfloat16, device=gpu)
    # empty list: row 0 zeroed, nothing else touched
    assert Q.q4_stage_pages(buf, pool, torch.empty(0, dtype=torch.int64, device=gpu)) == 0
    torch.cuda.synchronize()
    assert not buf[0].any() and (buf[1:] == 1.0).all()
    # full buffer (capacity - 1 pages), one id past the pool and one negative
    pages = torch.tensor([3, nb, -2], dtype=torch.int32, device=gpu)
    assert Q.q4_stage_pages(buf, pool, pages) == 3
    want = N.stage_pages(pool.cpu().numpy(), pages.cpu().numpy())
    assert np.array_equal(_bits(buf), want)
    assert not buf[1].any() and not buf[2].any() and not buf[3].any()


def test_stage_large_slice(gpu):
    """A 30K-token prefix slice at the reference harness's 4 KV heads."""
    H, nb = 4, 240
    pool = _packed_pool(gpu, 44, H, nb)
    pages = torch.from_numpy(np.random.default_rng(45).permutation(nb)[:191]).to(gpu)
    buf = torch.empty((192, H, 128, 256), dtype=torch.bfloat16, device=gpu)
    assert Q.q4_stage_pages(buf, pool, pages) == 191
    vals = torch.from_numpy(N.dequant_pool(pool.cpu().numpy().reshape(nb, 2 * H, -1)))
    p = pages.cpu()
    want = torch.cat([vals[p, 0::2], vals[p, 1::2]], dim=-1).bfloat16()
    got = buf.cpu()
    assert torch.equal(got[:191].view(torch.int16), want.view(torch.int16))
    assert not got[191].any()


def test_stage_refusals(gpu):
    H = 2
    pool = Q.new_pool(3, H, gpu)
    buf = torch.empty((3, H, 128, 256), dtype=torch.bfloat16, device=gpu)
    pages = torch.tensor([0, 1], device=gpu)
    with pytest.raises(ValueError, match="raw uint8"):
        Q.q4_stage_pages(buf, pool.view(torch.int8), pages)
    with pytest.raises(ValueError, match=r"\[nb, 2\*num_kv_heads, 128, 72\]"):
        Q.q4_stage_pages(buf, pool.reshape(3, 2 * H, 9216), pages)
    with pytest.raises(ValueError, match="must be bf16"):
        Q.q4_stage_pages(buf.half(), pool, pages)
    with pytest.raises(ValueError, match="int64/int32"):
        Q.q4_stage_pages(buf, pool, pages.float())
    with pytest.raises(ValueError, match=r"\[capacity, num_kv_heads, 128, 256\]"):
        Q.q4_stage_pages(buf[:, :1], pool, pages)
    with pytest.raises(ValueError, match="holds 2 pages, need 3"):
        Q.q4_stage_pages(buf, pool, torch.tensor([0, 1, 2], device=gpu))
    with pytest.raises(ValueError, match="refused"):
        Q.q4_stage_pages(buf, pool, pages.cpu())
