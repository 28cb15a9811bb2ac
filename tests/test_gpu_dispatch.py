"""End-to-end GPU parity of the routed-expert dispatch
(vllm_exl3_amd.dispatch.apply_exl3_experts): a layer loaded from
checkpoint-named packs (mixed K including K5), global expert ids mapped
through a non-identity expert_map with non-local ids, on the decode
executor, the prefill executor and the per-expert loop, against the oracle's
eager loop with the same map.  Relative L2 <= 2e-3."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import dense_cpu, rel_l2
from vllm_exl3_amd import dispatch as D
from vllm_exl3_amd import packs as P
from vllm_exl3_amd import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 2e-3
PREFIX = "model.layers.7.mlp.experts"
N_LOCAL, H, I, TOPK = 6, 256, 384, 4
KS = [(2, 3, 4), 5, (4, 2, 3), 3, (3, 5, 2), 4]
# 12 global experts; local ids of this rank (negative: on another rank)
EMAP = np.array([3, -1, 0, 5, -1, 1, 4, -1, 2, -1, -1, 0], np.int64)


@pytest.fixture(scope="module")
def layer_and_dense(gpu):
    experts = S.moe_layer(81, N_LOCAL, H, I, KS)
    et = P.load_experts(P.state_dict_of(experts, PREFIX, P.CB_MCG), PREFIX, N_LOCAL, gpu)
    layer = et.attach(SimpleNamespace(expert_map=torch.from_numpy(EMAP)))
    return layer, dense_cpu(experts, 1)


def _inputs(seed, T):
    x = S.activations(seed, T, H)
    g = np.random.default_rng(seed)
    ids = g.integers(-1, len(EMAP) + 2, size=(T, TOPK))  # includes invalid and non-local ids
    w = g.random((T, TOPK)).astype(np.float32)
    return x, ids, w


@pytest.mark.parametrize("executor,T", [("decode", 5), ("prefill", 5), ("decode", 40),
                                        ("prefill", 300), (None, 3), (None, 400)])
def test_dispatch_with_expert_map(gpu, layer_and_dense, executor, T):
    layer, dense = layer_and_dense
    x, ids, w = _inputs(90 + T, T)
    want = O.moe_reference(x, ids, w, dense, expert_map=EMAP)
    xd = torch.from_numpy(x).to(gpu).bfloat16()
    got = D.apply_exl3_experts(xd, torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), layer,
                               executor=executor)
    assert got.dtype == torch.bfloat16
    assert layer._exl3_last_apply == (executor or D.choose_executor(T, TOPK, N_LOCAL))
    assert rel_l2(got.float(), want) <= TOL + 4e-3  # bf16 output rounding


def test_loop_fallback_on_gpu(gpu, layer_and_dense):
    """The per-expert loop over Exl3Linear projections (HIP GEMM, fp32 g/u as
    the reference's eager loop)."""
    layer, dense = layer_and_dense
    x, ids, w = _inputs(95, 7)
    inners = layer._exl3_inners
    # the loop streams K 2..4 only; map the K5 experts' ids away
    k5 = [e for e, k in enumerate(KS) if 5 in ((k,) if isinstance(k, int) else k)]
    emap = EMAP.copy()
    emap[np.isin(emap, k5)] = -1
    want = O.moe_reference(x, ids, w, dense, expert_map=emap, gu_fp16=False)
    got = D.apply_exl3_python_loop(torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                                   torch.from_numpy(w).to(gpu), inners,
                                   torch.from_numpy(emap).to(gpu))
    assert rel_l2(got, want) <= TOL


def test_dispatch_decode_graph_replay(gpu, layer_and_dense):
    layer, dense = layer_and_dense
    T = 4
    x, ids, w = _inputs(97, T)
    xd = torch.from_numpy(x).to(gpu)
    idd = torch.from_numpy(ids).to(gpu)
    wd = torch.from_numpy(w).to(gpu)

    def run():
        return D.apply_exl3_experts(xd, idd, wd, layer, executor="decode")

    run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = run()
    for rep in range(2):
        x, ids, w = _inputs(200 + rep, T)
        xd.copy_(torch.from_numpy(x))
        idd.copy_(torch.from_numpy(ids))
        wd.copy_(torch.from_numpy(w))
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_out.clone()
        eager = run()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        assert rel_l2(eager, O.moe_reference(x, ids, w, dense, expert_map=EMAP)) <= TOL
    del graph
