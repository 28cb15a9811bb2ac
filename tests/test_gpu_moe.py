"""GPU parity of the routed-expert decode executor.

Checked against the per-expert eager loop (oracle.moe_reference at small
sizes; its torch restatement over bit-exact dequantised weights at the
benchmark's sizes).  Tolerance: relative L2 <= 2e-3."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import dense_cpu, dense_gpu, rel_l2, torch_moe_reference
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _layer(seed, E, H, I, K, cb, gateless=False):
    experts = S.moe_layer(seed, E, H, I, K, gateless=gateless)
    return experts


def _forward(dev_layer, x, ids, w, E, I, cb, K=(3, 3, 3), mixed=False, **kw):
    return C.moe_forward(x, ids, w, dev_layer, E, I, K=K,
                         k_tables=dev_layer["k_tables"] if mixed else None, codebook=cb, **kw)


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_moe_small_vs_oracle(gpu, gemv_policy, cb, T):
    E, H, I, topk = 6, 256, 384, 4
    experts = _layer(40 + T + cb, E, H, I, 3, cb)
    x = S.activations(5 + T, T, H)
    ids, w = S.softmax_topk(9 + T, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, cb))
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, cb)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("limit", [0.0, 1.0, 10.0])
def test_moe_clamp_repeated_ids_zero_weight(gpu, gemv_policy, limit):
    # Mirrors the reference's contract fixture (tests/test_native_moe_contract.py:
    # 54-151): two experts, repeated routes, last route zero weight, output
    # scales chosen so clipping engages.
    E, H, I, topk = 2, 4096, 1024, 6
    experts = _layer(77, E, H, I, 4, 1)
    for pk in experts:
        for proj, n_in, n_out, scale in (("gate", H, I, 8.0), ("up", H, I, 8.0), ("down", I, H, 1.0)):
            pk[proj]["suh"] = np.full(n_in, 1.0 / 64, dtype=np.float16)
            pk[proj]["svh"] = np.full(n_out, scale, dtype=np.float16)
    ids = (np.arange(topk) % E).reshape(1, topk).astype(np.int64)
    w = np.linspace(0.1, 0.9, topk).astype(np.float32).reshape(1, topk)
    w[0, -1] = 0
    w /= w.sum()
    x = S.activations(3, 1, H)
    dense = dense_cpu(experts, 1)
    want = O.moe_reference(x, ids, w, dense, limit=limit)
    if limit:
        xh = x.astype(np.float16).astype(np.float32)
        g = xh @ dense[0]["gate"].astype(np.float32)
        u = xh @ dense[0]["up"].astype(np.float32)
        assert ((g > limit) | (np.abs(u) > limit)).any(), "fixture must exercise clipping"
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, 1, K=(4, 4, 4), swiglu_limit=limit)
    assert rel_l2(got, want) <= TOL


def test_moe_mixed_k_and_sentinels(gpu, gemv_policy):
    E, H, I, topk, T = 8, 384, 256, 4, 5
    ks = [(2, 3, 4), 3, 4, (4, 2, 3), 2, 3, 4, 2]
    experts = _layer(91, E, H, I, ks, 1)
    x = S.activations(8, T, H)
    ids, w = S.softmax_topk(12, T, E, topk)
    ids[1, 2] = -1        # invalid id
    ids[3, 0] = E + 5     # non-local id
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1))
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, 1, mixed=True)
    assert rel_l2(got, want) <= TOL


def test_moe_mixed_k_whole_blocks(gpu, gemv_policy):
    # widths that are multiples of 512: every chunk takes the GEMV's
    # branch-free path, including the switch to an expert of another K
    E, H, I, topk, T = 8, 1024, 512, 4, 12
    ks = [2, 3, 4, (4, 2, 3), 2, 4, 3, (2, 4, 3)]
    experts = _layer(93, E, H, I, ks, 0)
    x = S.activations(10, T, H)
    ids, w = S.softmax_topk(14, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 0))
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, 0, mixed=True)
    assert rel_l2(got, want) <= TOL


def test_moe_gateless_relu2(gpu, gemv_policy):
    E, H, I, topk, T = 4, 256, 256, 2, 3
    experts = _layer(31, E, H, I, 3, 1, gateless=True)
    x = S.activations(4, T, H)
    ids, w = S.softmax_topk(5, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1))
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, 1, gateless=True, act=C.ACT_RELU2)
    assert rel_l2(got, want) <= TOL


def test_moe_swiglu_oai(gpu, gemv_policy):
    E, H, I, topk, T = 4, 256, 256, 2, 2
    experts = _layer(32, E, H, I, 4, 1)
    x = S.activations(6, T, H)
    ids, w = S.softmax_topk(7, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1), limit=7.0, act="swiglu_oai")
    dl = S.to_device(experts, gpu)
    got = _forward(dl, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                   torch.from_numpy(w).to(gpu), E, I, 1, K=(4, 4, 4), act=C.ACT_SWIGLU_OAI,
                   swiglu_limit=7.0)
    assert rel_l2(got, want) <= TOL


def test_moe_deterministic_and_graph_replay(gpu):
    E, H, I, topk, T = 8, 256, 256, 4, 6
    experts = _layer(55, E, H, I, 3, 0)
    dl = S.to_device(experts, gpu)
    dense = dense_gpu(experts, 0, gpu)
    x = torch.from_numpy(S.activations(1, T, H)).to(gpu)
    ids_np, w_np = S.softmax_topk(2, T, E, topk)
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(w_np).to(gpu)
    out = torch.empty((T, H), dtype=torch.float32, device=gpu)

    def run():
        _forward(dl, x, ids, w, E, I, 0, out=out)

    run()
    first = out.clone()
    run()
    assert torch.equal(first, out), "repeated launches must be bit-identical"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        x.copy_(torch.from_numpy(S.activations(100 + rep, T, H)))
        ids_np, w_np = S.softmax_topk(200 + rep, T, E, topk)
        ids.copy_(torch.from_numpy(ids_np))
        w.copy_(torch.from_numpy(w_np))
        graph.replay()
        torch.cuda.synchronize()
        want = torch_moe_reference(x, ids, w, dense, E)
        eager = out.clone()
        run()
        torch.cuda.synchronize()
        assert torch.equal(eager, out), "graph replay must match the eager launch bit-for-bit"
        assert rel_l2(out, want) <= TOL
    del graph


def test_p2b_fused_moe_dropin(gpu):
    E, H, I, topk = 4, 256, 256, 4
    experts = _layer(61, E, H, I, 2, 1)
    dl = S.to_device(experts, gpu)
    x = torch.from_numpy(S.activations(9, 1, H)).to(gpu).half()
    ids = torch.tensor([0, 2, 3, 2], dtype=torch.int32, device=gpu)
    w = torch.tensor([0.4, 0.3, 0.2, 0.1], dtype=torch.float16, device=gpu)
    out = torch.empty_like(x)
    tabs = [dl[k] for k in ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh",
                            "up_svh", "down_trellis", "down_suh", "down_svh")]
    r = C.p2b_fused_moe(x, out, *tabs, ids, w, 2, 2, 2, True, I, 0.0)
    assert r is out
    want = O.moe_reference(x.float().cpu().numpy(), ids.cpu().numpy()[None].astype(np.int64),
                           w.float().cpu().numpy()[None], dense_cpu(experts, 1))
    assert rel_l2(out.float(), want) <= 2e-3 + 1e-3  # fp16 output rounding
    # mixed-K entry with sentinel and the padded entry agree with the uniform one
    kt = dl["k_tables"]
    out_mk = torch.empty_like(x)
    ids_s = torch.tensor([0, 2, 3, E], dtype=torch.int32, device=gpu)
    C.p2b_fused_moe_mk(x, out_mk, *tabs, ids_s, w, *kt, E, True, I, 0.0)
    want_s = O.moe_reference(x.float().cpu().numpy(), np.array([[0, 2, 3, E]]),
                             w.float().cpu().numpy()[None], dense_cpu(experts, 1))
    assert rel_l2(out_mk.float(), want_s) <= 3e-3
    xp = torch.cat([x, torch.randn_like(x)], 0)
    ids_p = torch.stack([ids, ids]).contiguous()
    w_p = torch.stack([w, w]).contiguous()
    n_valid = torch.tensor([1], dtype=torch.int32, device=gpu)
    out_p = torch.full_like(xp, 7.0)
    C.p2b_fused_moe_padded(xp, out_p, *tabs, ids_p, w_p, n_valid, *kt, E, topk, True, I, 0.0)
    assert torch.equal(out_p[0], out[0])
    assert torch.count_nonzero(out_p[1]) == 0, "padded rows must be exact zeros"


@pytest.mark.parametrize("bad", ["rows", "width", "negative_limit", "nan_limit", "strided_pointers"])
def test_p2b_rejects_unsafe_calls_before_launch(gpu, bad):
    # Mirrors tests/test_native_moe_contract.py:228-248 of the reference.
    x = torch.zeros(1, 4096, dtype=torch.float16, device=gpu)
    out = torch.empty_like(x)
    ptrs = [torch.zeros(2, dtype=torch.int64, device=gpu) for _ in range(9)]
    ids = torch.zeros(1, dtype=torch.int32, device=gpu)
    weights = torch.ones(1, dtype=torch.float16, device=gpu)
    width, limit = 2048, 0.0
    if bad == "rows":
        x = x.repeat(2, 1)
    elif bad == "width":
        width = 1537
    elif bad == "negative_limit":
        limit = -1.0
    elif bad == "nan_limit":
        limit = float("nan")
    else:
        ptrs[0] = torch.zeros(4, dtype=torch.int64, device=gpu)[::2]
    with pytest.raises(RuntimeError, match="fused MoE"):
        C.p2b_fused_moe(x, out, *ptrs, ids, weights, 4, 4, 4, True, width, limit)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_moe_config1_full_size(gpu, gemv_policy, T):
    # E64 top-8, H2048, I1536, K3, 3INST, bf16 activations
    E, H, I, topk = 64, 2048, 1536, 8
    experts = S.moe_layer(1, E, H, I, 3)
    x = torch.from_numpy(S.activations(10 + T, T, H)).to(gpu).bfloat16()
    ids_np, w_np = S.softmax_topk(20 + T, T, E, topk)
    used = sorted(set(ids_np.ravel().tolist()))
    dense = dense_gpu(experts, 0, gpu, only=used)
    dl = S.to_device(experts, gpu)
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(w_np).to(gpu)
    got = _forward(dl, x, ids, w, E, I, 0)
    want = torch_moe_reference(x.float(), ids, w, dense, E)
    assert rel_l2(got, want) <= TOL


def test_moe_from_checkpoint_packs(gpu):
    # Packs named as the reference's checkpoints name them
    # (experts.{e}.{w1,w3,w2}.{trellis,suh,svh,mcg}), loaded into pointer and
    # K tables by vllm_exl3_amd.packs, then run through both executors.
    from vllm_exl3_amd import packs as P

    E, H, I, topk, T = 5, 256, 384, 3, 4
    ks = [(2, 3, 4), (4, 2, 3), (3, 3, 3), (2, 2, 2), (4, 4, 4)]
    experts = S.moe_layer(91, E, H, I, ks)
    prefix = "model.layers.3.mlp.experts"
    et = P.load_experts(P.state_dict_of(experts, prefix, P.CB_MCG), prefix, E, gpu)
    x = S.activations(92, T, H)
    ids, w = S.softmax_topk(93, T, E, topk)
    want = O.moe_reference(x, ids, w, dense_cpu(experts, 1))
    xd = torch.from_numpy(x).to(gpu).bfloat16()
    idd, wd = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    got = C.moe_forward(xd, idd, wd, et.tables, et.n_local, et.intermediate, **et.forward_kwargs())
    assert rel_l2(got, want) <= TOL
    got_p = C.moe_prefill(xd, idd, wd, et.tables, et.n_local, et.intermediate, **et.forward_kwargs())
    assert rel_l2(got_p, want) <= TOL


def test_graph_replay_after_workspace_growth(gpu):
    """A decode step captured at small T keeps replaying into live memory
    after an eager call at a larger T grew the shared workspace: the superseded
    workspace is kept, and replays stay bit-identical to eager launches."""
    E, H, I, topk, T = 8, 256, 256, 4, 2
    experts = _layer(58, E, H, I, 3, 0)
    dl = S.to_device(experts, gpu)
    dense = dense_gpu(experts, 0, gpu)
    x = torch.from_numpy(S.activations(11, T, H)).to(gpu)
    ids_np, w_np = S.softmax_topk(12, T, E, topk)
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(w_np).to(gpu)
    out = torch.empty((T, H), dtype=torch.float32, device=gpu)

    def run():
        _forward(dl, x, ids, w, E, I, 0, out=out)

    run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    # an eager call at a much larger T grows the workspace; then fill the
    # freed-and-reused memory pool with NaN
    Tb = 512
    xb = torch.from_numpy(S.activations(13, Tb, H)).to(gpu)
    ib, wb = S.softmax_topk(14, Tb, E, topk)
    _forward(dl, xb, torch.from_numpy(ib).to(gpu), torch.from_numpy(wb).to(gpu), E, I, 0)
    junk = [torch.full((1 << 20,), float("nan"), device=gpu) for _ in range(16)]
    for rep in range(2):
        x.copy_(torch.from_numpy(S.activations(300 + rep, T, H)))
        ids_np, w_np = S.softmax_topk(400 + rep, T, E, topk)
        ids.copy_(torch.from_numpy(ids_np))
        w.copy_(torch.from_numpy(w_np))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        run()
        torch.cuda.synchronize()
        assert torch.equal(replayed, out), "replay after workspace growth must match eager"
        assert rel_l2(out, torch_moe_reference(x, ids, w, dense, E)) <= TOL
    for j in junk:
        assert torch.isnan(j).all(), "a replay wrote into memory owned by other tensors"
    del graph
