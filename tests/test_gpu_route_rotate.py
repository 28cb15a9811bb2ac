"""GPU parity of the decode step's three routing forms on the same inputs:
inline routing (steps of at most 64 routes: every gate/up GEMV workgroup
routes the step itself and rotates its rows from x; workgroup 0 writes the
router's tables), routing and the gate/up input rotation in one launch
(EXL3_MOE_INLINE_ROUTE=0; the GEMV stages its sorted rows through the
router's sorted row -> route map), and separate route and rotate launches
(also EXL3_MOE_ROUTE_ROTATE=0), against the oracle: uniform-K layers,
decode batch sizes, silu / clamped silu / SwiGLU-OAI / gateless relu2, int32
and int64 ids, sentinel ids, padded rows (n_valid), fp16/bf16/fp32 outputs.
Relative L2 <= 2e-3 against the oracle; the two launch sequences compute the
same rounding steps in the same order, so they agree bit for bit."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import dense_cpu, rel_l2
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _run(monkeypatch, mode, *a, **kw):
    """mode: "inline", True (route + rotate launch) or False (separate launches)."""
    monkeypatch.setenv("EXL3_MOE_INLINE_ROUTE", "1" if mode == "inline" else "0")
    monkeypatch.setenv("EXL3_MOE_ROUTE_ROTATE", "0" if mode is False else "1")
    out = C.moe_forward(*a, **kw)
    torch.cuda.synchronize()
    return out


CASES = [
    # T, E, H, I, topk, K, cb, act, limit, gateless
    (1, 8, 256, 384, 4, 3, 0, "silu", 0.0, False),
    (3, 6, 384, 256, 2, 2, 1, "silu", 1.0, False),
    (8, 8, 256, 256, 8, 4, 2, "swiglu_oai", 7.0, False),
    (16, 12, 512, 384, 4, 3, 1, "silu", 0.0, False),
    (40, 16, 256, 512, 6, 4, 0, "silu", 10.0, False),
    (5, 6, 256, 256, 3, 3, 1, "silu", 0.5, True),
]


@pytest.mark.parametrize("case", CASES)
def test_route_rotate_matches_oracle_and_separate_launches(gpu, monkeypatch, case):
    T, E, H, I, topk, K, cb, act, limit, gateless = case
    experts = S.moe_layer(300 + T, E, H, I, K, gateless=gateless)
    x = S.activations(301 + T, T, H)
    ids, w = S.softmax_topk(302 + T, T, E, topk)
    if T > 2:
        ids[1, 0] = -1          # invalid id
        ids[2, -1] = E + 3      # non-local id
        ids[0, 1] = ids[0, 0]   # one token routed twice to an expert
    act_name = "silu" if gateless else act
    want = O.moe_reference(x, ids, w, dense_cpu(experts, cb), limit=limit, act=act_name)
    dl = S.to_device(experts, gpu)
    act_id = C.ACT_RELU2 if gateless else (C.ACT_SWIGLU_OAI if act == "swiglu_oai" else C.ACT_SILU)
    args = (torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu).to(torch.int32),
            torch.from_numpy(w).to(gpu), dl, E, I)
    kw = dict(K=(K, K, K), codebook=cb, gateless=gateless, act=act_id, swiglu_limit=limit)
    inl = _run(monkeypatch, "inline", *args, **kw)
    fused = _run(monkeypatch, True, *args, **kw)
    six = _run(monkeypatch, False, *args, **kw)
    assert rel_l2(fused, want) <= TOL
    assert torch.equal(fused, six)
    assert torch.equal(inl, fused)
    again = _run(monkeypatch, "inline", *args, **kw)
    assert torch.equal(inl, again), "the decode step must be deterministic"


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_route_rotate_padded_and_routeless_rows(gpu, monkeypatch, out_dtype):
    """Rows at or beyond n_valid and rows whose every route is non-local come
    out as exact zeros; live rows match the oracle."""
    T, E, H, I, topk = 12, 8, 256, 256, 4
    experts = S.moe_layer(310, E, H, I, 4)
    x = S.activations(311, T, H)
    ids, w = S.softmax_topk(312, T, E, topk)
    ids[3, :] = E            # every route of token 3 is non-local
    n_live = 9
    dl = S.to_device(experts, gpu)
    n_valid = torch.tensor([n_live], dtype=torch.int32, device=gpu)
    out = torch.full((T, H), 5.0, dtype=out_dtype, device=gpu)
    args = (torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), dl, E, I)
    got = _run(monkeypatch, True, *args, K=(4, 4, 4), codebook=1, n_valid=n_valid, out=out)
    out2 = torch.full((T, H), 5.0, dtype=out_dtype, device=gpu)
    sep = _run(monkeypatch, False, *args, K=(4, 4, 4), codebook=1, n_valid=n_valid, out=out2)
    assert torch.equal(got, sep)
    out3 = torch.full((T, H), 5.0, dtype=out_dtype, device=gpu)
    inl = _run(monkeypatch, "inline", *args, K=(4, 4, 4), codebook=1, n_valid=n_valid, out=out3)
    assert torch.equal(inl, sep)
    assert torch.count_nonzero(got[n_live:]) == 0 and torch.count_nonzero(got[3]) == 0
    want = O.moe_reference(x[:n_live], ids[:n_live], w[:n_live], dense_cpu(experts, 1))
    tol = TOL if out_dtype == torch.float32 else TOL + 4e-3
    assert rel_l2(got[:n_live].float(), want) <= tol


@pytest.mark.parametrize("inline", [True, False])
def test_route_rotate_graph_replay(gpu, monkeypatch, inline):
    monkeypatch.setenv("EXL3_MOE_ROUTE_ROTATE", "1")
    monkeypatch.setenv("EXL3_MOE_INLINE_ROUTE", "1" if inline else "0")
    T, E, H, I, topk = 4, 8, 256, 384, 4
    experts = S.moe_layer(320, E, H, I, 3)
    dl = S.to_device(experts, gpu)
    dense = dense_cpu(experts, 0)
    x = torch.from_numpy(S.activations(321, T, H)).to(gpu)
    ids_np, w_np = S.softmax_topk(322, T, E, topk)
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(w_np).to(gpu)
    out = torch.empty((T, H), dtype=torch.float32, device=gpu)

    def run():
        C.moe_forward(x, ids, w, dl, E, I, K=(3, 3, 3), codebook=0, out=out)

    run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        xn = S.activations(330 + rep, T, H)
        idn, wn = S.softmax_topk(340 + rep, T, E, topk)
        x.copy_(torch.from_numpy(xn))
        ids.copy_(torch.from_numpy(idn))
        w.copy_(torch.from_numpy(wn))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        run()
        torch.cuda.synchronize()
        assert torch.equal(replayed, out)
        assert rel_l2(out, O.moe_reference(xn, idn, wn, dense)) <= TOL
    del graph
