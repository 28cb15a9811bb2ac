"""GPU parity of the routed-expert prefill executor (grouped fat GEMMs).

Checked against the eager per-expert loop (oracle.moe_reference at small
sizes; its torch restatement over bit-exact dequantised weights at the
BASELINE config-2 size).  Tolerance: relative L2 <= 2e-3."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import dense_cpu, dense_gpu, rel_l2, torch_moe_reference
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _run(dl, x, ids, w, E, I, cb, K=(3, 3, 3), mixed=False, **kw):
    return C.moe_prefill(x, ids, w, dl, E, I, K=K, k_tables=dl["k_tables"] if mixed else None,
                         codebook=cb, **kw)


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", [2, 3, 4])
def test_prefill_small_vs_oracle(gpu, cb, K):
    E, H, I, topk, T = 5, 256, 384, 3, 37
    experts = S.moe_layer(300 + 3 * K + cb, E, H, I, K)
    x = S.activations(31 + K, T, H)
    ids, w = S.softmax_topk(41 + cb, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, cb))
    dl = S.to_device(experts, gpu)
    got = _run(dl, torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
               torch.from_numpy(w).to(gpu), E, I, cb, K=(K, K, K))
    assert rel_l2(got, want) <= TOL


def test_prefill_multi_tile_experts_and_edge_routes(gpu):
    # > 256 rows per expert (several row tiles), sentinels, int32 ids, padding
    E, H, I, topk, T = 4, 256, 256, 4, 300
    experts = S.moe_layer(12, E, H, I, 4)
    x = S.activations(13, T, H)
    ids, w = S.softmax_topk(14, T, E, topk)
    ids[5, 1] = -1
    ids[9, 0] = E + 3
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1))
    dl = S.to_device(experts, gpu)
    xt = torch.from_numpy(x).to(gpu)
    got = _run(dl, xt, torch.from_numpy(ids).to(gpu).int(), torch.from_numpy(w).to(gpu), E, I, 1,
               K=(4, 4, 4))
    assert rel_l2(got, want) <= TOL
    # device-side live-row count: rows >= n_valid are exact zeros, others unchanged
    n_valid = torch.tensor([200], dtype=torch.int32, device=gpu)
    got_p = _run(dl, xt, torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), E, I, 1,
                 K=(4, 4, 4), n_valid=n_valid)
    assert torch.count_nonzero(got_p[200:]) == 0
    want_p = O.moe_reference(x[:200], ids[:200], w[:200], dense_cpu(experts, 1))
    assert rel_l2(got_p[:200], want_p) <= TOL


def test_prefill_mixed_k_gateless_and_swiglu(gpu):
    E, H, I, topk, T = 6, 384, 256, 2, 50
    ks = [(2, 3, 4), 3, 4, (4, 2, 3), 2, 3]
    experts = S.moe_layer(21, E, H, I, ks)
    x = S.activations(22, T, H)
    ids, w = S.softmax_topk(23, T, E, topk)
    dl = S.to_device(experts, gpu)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1), limit=7.0, act="swiglu_oai")
    got = _run(dl, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
               torch.from_numpy(w).to(gpu), E, I, 1, mixed=True, act=C.ACT_SWIGLU_OAI,
               swiglu_limit=7.0)
    assert rel_l2(got, want) <= TOL
    gl = S.moe_layer(24, 3, H, I, 3, gateless=True)
    ids2, w2 = S.softmax_topk(25, T, 3, 2)
    want2 = O.moe_reference(x, ids2, w2, dense_cpu(gl, 0))
    got2 = _run(S.to_device(gl, gpu), torch.from_numpy(x).to(gpu), torch.from_numpy(ids2).to(gpu),
                torch.from_numpy(w2).to(gpu), 3, I, 0, gateless=True, act=C.ACT_RELU2)
    assert rel_l2(got2, want2) <= TOL


def test_prefill_matches_decode_executor_and_is_deterministic(gpu):
    E, H, I, topk, T = 16, 512, 512, 4, 64
    experts = S.moe_layer(33, E, H, I, 3)
    dl = S.to_device(experts, gpu)
    x = torch.from_numpy(S.activations(34, T, H)).to(gpu).bfloat16()
    ids_np, w_np = S.softmax_topk(35, T, E, topk)
    ids, w = torch.from_numpy(ids_np).to(gpu), torch.from_numpy(w_np).to(gpu)
    a = C.moe_prefill(x, ids, w, dl, E, I, K=(3, 3, 3), codebook=0)
    b = C.moe_prefill(x, ids, w, dl, E, I, K=(3, 3, 3), codebook=0)
    assert torch.equal(a, b), "repeated launches must be bit-identical"
    d = C.moe_forward(x, ids, w, dl, E, I, K=(3, 3, 3), codebook=0)
    assert rel_l2(a, d) <= TOL


def test_prefill_config2_full_size(gpu):
    # E128 top-8, H4096, I1024, K4 MCG, T=2048, Zipf(1.1) routing
    E, H, I, topk, T = 128, 4096, 1024, 8, 2048
    experts = S.moe_layer(2, E, H, I, 4)
    dl = S.to_device(experts, gpu)
    ids_np, w_np = S.zipf_topk(2, T, E, topk)
    x = torch.from_numpy(S.activations(2, T, H)).to(gpu).bfloat16()
    ids, w = torch.from_numpy(ids_np).to(gpu), torch.from_numpy(w_np).to(gpu)
    got = C.moe_prefill(x, ids, w, dl, E, I, K=(4, 4, 4), codebook=1)
    dense = dense_gpu(experts, 1, gpu)
    want = torch_moe_reference(x.float(), ids, w, dense, E)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("E,T,topk", [(128, 512, 8), (1000, 300, 8), (64, 3000, 6)])
def test_prefill_wide_router_bit_exact(gpu, monkeypatch, E, T, topk):
    """From 2048 routes the prefill routes with the multi-workgroup router
    (ranks per 1024-route workgroup, one scan, placement); EXL3_ROUTE_WIDE=0
    keeps the single-workgroup router.  Same stable order, so the outputs
    agree bit for bit; dropped ids and padded rows included.  E experts share four
    packs (pointer tables with repeated entries), so the reference needs
    four dequantisations."""
    H, I = 256, 256
    packs = S.moe_layer(700 + E, 4, H, I, 3)
    experts = [packs[e % 4] for e in range(E)]
    x = S.activations(701, T, H)
    ids, w = S.softmax_topk(702 + T, T, E, topk)
    ids[0, 0] = -1
    ids[1, 1] = E + 5
    n_live = T - 7
    dl = S.to_device(experts, gpu)
    args = (torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
            torch.from_numpy(w).to(gpu), dl, E, I)
    n_valid = torch.tensor([n_live], dtype=torch.int32, device=gpu)
    outs = []
    for wide in ("1", "0"):
        monkeypatch.setenv("EXL3_ROUTE_WIDE", wide)
        outs.append(C.moe_prefill(*args, K=(3, 3, 3), codebook=1, n_valid=n_valid))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.count_nonzero(outs[0][n_live:]) == 0
    dense = dense_cpu(packs, 1)
    want = O.moe_reference(x[:n_live], ids[:n_live], w[:n_live], [dense[e % 4] for e in range(E)])
    assert rel_l2(outs[0][:n_live], want) <= TOL
