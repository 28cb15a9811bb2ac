"""GPU parity of the paged int4 KV cache (pack, unpack, split-K decode attention).

Pack and unpack are checked bit-exact against the CPU oracle; decode against
the oracle's float64 softmax attention over the oracle-dequantised cache, with
relative L2 <= 2e-3.  At the BASELINE config-4 size the reference is torch
fp32 attention over the GPU-unpacked cache (unpack is pinned bit-exact at the
small sizes), plus the size-independent bound |x - deq(x)| <= scale/2 + fp16
rounding of scale and zero."""

import math

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import rel_l2
from vllm_exl3_amd import kv_int4 as KV
from vllm_exl3_amd import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _setup(gpu, seed, B, Hkv, L, seq, n_pages, dtype=torch.bfloat16):
    k, v = S.kv_inputs(seed, B, Hkv, L)
    max_pages = (L + 15) // 16
    bt = S.block_table(seed + 1, B, max_pages, n_pages)
    seq = np.asarray(seq, dtype=np.int32)
    pool = KV.new_pool(n_pages, Hkv, gpu)
    kt = torch.from_numpy(k).to(gpu).to(dtype)
    vt = torch.from_numpy(v).to(gpu).to(dtype)
    st = torch.from_numpy(seq).to(gpu)
    btt = torch.from_numpy(bt).to(gpu)
    KV.pack_pages(kt, vt, st, btt, pool)
    return k, v, seq, bt, pool, st, btt


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pack_bit_exact_vs_oracle(gpu, dtype):
    B, Hkv, L = 3, 2, 70
    seq = [70, 16, 1]
    k, v, seq, bt, pool, st, btt = _setup(gpu, 11, B, Hkv, L, seq, 16, dtype)
    want = O.kv_pack_pages(k, v, seq, bt, 16)
    got = pool.cpu().numpy()
    assert np.array_equal(got, want)
    kk, vv = KV.unpack_pages(pool, st, btt, L)
    wk, wv = O.kv_unpack_pages(want, seq, bt, L)
    assert np.array_equal(kk.cpu().numpy(), wk) and np.array_equal(vv.cpu().numpy(), wv)


def test_pack_edge_values(gpu):
    # constant groups (scale 0), a zero row, huge outliers, negative-only rows
    B, Hkv, L = 1, 1, 32
    k = np.zeros((B, Hkv, L, 128), np.float32)
    k[0, 0, 0] = 3.0
    k[0, 0, 1, :32] = np.linspace(-5, -1, 32)
    k[0, 0, 2] = np.where(np.arange(128) % 7 == 0, 900.0, -0.001)
    k[0, 0, 3:] = np.random.default_rng(0).standard_normal((29, 128))
    v = -k
    seq = np.array([32], np.int32)
    bt = np.array([[1, 0]], np.int32)
    pool = KV.new_pool(2, 1, gpu)
    KV.pack_pages(torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu),
                  torch.from_numpy(seq).to(gpu), torch.from_numpy(bt).to(gpu), pool)
    assert np.array_equal(pool.cpu().numpy(), O.kv_pack_pages(k, v, seq, bt, 2))


def _decode(gpu, q, pool, btt, st, Hkv, scale, out_dtype=torch.float32, n_splits=0):
    out = torch.empty(q.shape, dtype=out_dtype, device=gpu)
    return KV.int4_decode(q, pool, btt, st, Hkv, scale, out, n_splits=n_splits)


@pytest.mark.parametrize("G,n_splits", [(8, 0), (8, 1), (8, 3), (4, 0), (16, 2), (1, 0)])
def test_decode_vs_oracle(gpu, G, n_splits):
    B, Hkv, L = 3, 2, 300
    seq = [300, 17, 160]
    k, v, seq, bt, pool, st, btt = _setup(gpu, 20 + G, B, Hkv, L, seq, 64)
    kd, vd = O.kv_unpack_pages(O.kv_pack_pages(k, v, seq, bt, 64), seq, bt, L)
    q = S.activations(30 + G, B * Hkv * G, 128).reshape(B, Hkv * G, 128)
    scale = 1.0 / math.sqrt(128)
    want = O.attention_decode_lens(q, kd, vd, seq, scale)
    got = _decode(gpu, torch.from_numpy(q).to(gpu).bfloat16(), pool, btt, st, Hkv, scale,
                  n_splits=n_splits)
    assert rel_l2(got, want) <= TOL


def test_decode_dtypes_strides_and_empty_sequence(gpu):
    B, Hkv, G, L = 2, 2, 8, 64
    seq = [64, 0]
    k, v, seq, bt, pool, st, btt = _setup(gpu, 40, B, Hkv, L, seq, 8)
    kd, vd = O.kv_unpack_pages(O.kv_pack_pages(k, v, seq, bt, 8), seq, bt, L)
    qn = S.activations(41, B * Hkv * G, 128).reshape(B, Hkv * G, 128)
    want = O.attention_decode_lens(qn, kd, vd, seq, 0.1)
    # fp32 q viewed with a padded head stride, bf16 output
    qbig = torch.zeros((B, Hkv * G, 256), dtype=torch.float32, device=gpu)
    qbig[:, :, :128] = torch.from_numpy(qn).to(gpu)
    q = qbig[:, :, :128]
    got = _decode(gpu, q, pool, btt, st, Hkv, 0.1, out_dtype=torch.bfloat16)
    assert rel_l2(got[0].float(), want[0]) <= TOL + 4e-3  # bf16 output rounding
    assert torch.count_nonzero(got[1]) == 0


def test_decode_rejects_bad_geometry(gpu):
    pool = KV.new_pool(4, 2, gpu)
    st = torch.tensor([16], dtype=torch.int32, device=gpu)
    btt = torch.zeros((1, 1), dtype=torch.int32, device=gpu)
    q = torch.zeros((1, 6, 128), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        _decode(gpu, q, pool, btt, st, 4, 0.1)        # kv heads disagree with the pool
    with pytest.raises(ValueError):
        _decode(gpu, torch.zeros((1, 2, 64), device=gpu), pool, btt, st, 2, 0.1)
    with pytest.raises(ValueError):
        _decode(gpu, torch.zeros((1, 64, 128), device=gpu), pool, btt, st, 2, 0.1)  # G = 32


def test_decode_deterministic_and_graph_replay(gpu):
    B, Hkv, G, L = 4, 2, 8, 128
    seq = [128, 100, 33, 7]
    k, v, seq, bt, pool, st, btt = _setup(gpu, 50, B, Hkv, L, seq, 40)
    q = torch.from_numpy(S.activations(51, B * Hkv * G, 128).reshape(B, Hkv * G, 128)).to(gpu)
    q = q.bfloat16()
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu)
    KV.int4_decode(q, pool, btt, st, Hkv, 0.08, out)
    ref = out.clone()
    KV.int4_decode(q, pool, btt, st, Hkv, 0.08, out)
    assert torch.equal(out, ref)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        KV.int4_decode(q, pool, btt, st, Hkv, 0.08, out)
    for seed in (52, 53, 54):
        q.copy_(torch.from_numpy(S.activations(seed, B * Hkv * G, 128).reshape(B, Hkv * G, 128)))
        g.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        KV.int4_decode(q, pool, btt, st, Hkv, 0.08, eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_decode_config4_full_size(gpu):
    # B16, Hq64, Hkv8, d128, 32768 tokens, 16-token pages,
    # random block table, bf16 N(0,1) with 2% outlier channels x8.
    B, Hq, Hkv, L = 16, 64, 8, 32768
    max_pages = L // 16
    k, v = S.kv_inputs_device(4, B, Hkv, L, gpu)
    bt = torch.from_numpy(S.block_table(4, B, max_pages)).to(gpu)
    st = torch.full((B,), L, dtype=torch.int32, device=gpu)
    pool = KV.new_pool(B * max_pages, Hkv, gpu)
    KV.pack_pages(k, v, st, bt, pool)
    kd, vd = KV.unpack_pages(pool, st, bt, L)
    # size-independent pack bound on every element
    for x, xd in ((k, kd), (v, vd)):
        xf = x.float()
        g = xf.view(B, Hkv, L, 4, 32)
        mn, mx = g.amin(-1, keepdim=True), g.amax(-1, keepdim=True)
        sc = (mx - mn) / 15
        bound = sc / 2 + mn.abs() * 2.0 ** -10 + 15 * sc * 2.0 ** -10 + 1e-6
        assert bool(((g - xd.view(B, Hkv, L, 4, 32)).abs() <= bound).all())
    del k, v
    q = torch.from_numpy(S.activations(4, B * Hq, 128).reshape(B, Hq, 128)).to(gpu).bfloat16()
    scale = 1.0 / math.sqrt(128)
    got = _decode(gpu, q, pool, bt, st, Hkv, scale)
    G = Hq // Hkv
    worst = 0.0
    for b in range(B):
        qb = q[b].float().view(Hkv, G, 128)
        s = torch.matmul(qb, kd[b].transpose(1, 2).contiguous()) * scale     # [Hkv, G, L]
        p = torch.softmax(s, dim=-1)
        ob = torch.matmul(p, vd[b]).reshape(Hq, 128)
        worst = max(worst, rel_l2(got[b], ob))
    assert worst <= TOL, worst
