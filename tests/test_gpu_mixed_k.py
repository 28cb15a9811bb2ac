"""GPU parity of mixed-K layers whose per-expert K tables hold values outside
{2, 3, 4}.

The reference's mixed-K tile switch computes K 5 and 6 with a generic tile
and writes zeros for any other table value (csrc/p2b_moe.cu:295-324), so a
projection of such an expert contributes a zero output.  Both executors
(decode, under both GEMV kernel choices, and prefill) are checked against the
oracle's eager loop with those projections' dense weights taken as zeros.
Tolerance: relative L2 <= 2e-3."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import rel_l2
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3
COMPUTED = (2, 3, 4, 5, 6)


def _dense(experts, cb):
    out = []
    for pack in experts:
        d = {}
        for p, q in pack.items():
            n_in, n_out = q["trellis"].shape[0] * 16, q["trellis"].shape[1] * 16
            if q["K"] in COMPUTED:
                d[p] = O.dequant(q["trellis"], q["suh"], q["svh"], q["K"], cb)
            else:
                d[p] = np.zeros((n_in, n_out), np.float16)
        out.append(d)
    return out


# K 7 and 1 stand for any unsupported table value (their projections are zero)
KS = [(5, 3, 4), 6, (2, 5, 3), (4, 4, 6), 3, (7, 2, 2), (2, 3, 1), (5, 6, 5)]


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_decode_mixed_k_beyond_4(gpu, gemv_policy, cb):
    E, H, I, topk, T = len(KS), 256, 384, 4, 6
    experts = S.moe_layer(71 + cb, E, H, I, KS)
    x = S.activations(72, T, H)
    ids, w = S.softmax_topk(73, T, E, topk)
    ids[0, :3] = [5, 6, 0]  # the zero-output experts are routed
    want = O.moe_reference(x, ids, w, _dense(experts, cb))
    dl = S.to_device(experts, gpu)
    got = C.moe_forward(torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
                        torch.from_numpy(w).to(gpu), dl, E, I, k_tables=dl["k_tables"], codebook=cb)
    assert rel_l2(got, want) <= TOL


def test_decode_mixed_k_split_tail(gpu, gemv_policy):
    """A decode step whose units outnumber the resident workgroups in both
    GEMV phases (the one-unit kernel then runs the later units in two halves
    of the input range), with K 5/6 units computed by the generic kernel and
    K 7 units zero: every workspace slot of every unit must be written once.
    128 experts share four packs (pointer tables with repeated entries), so
    the dense reference needs four dequantisations."""
    E, H, I, topk, T, cb = 128, 896, 512, 8, 48, 0
    packs = S.moe_layer(79, 4, H, I, [3, 5, (2, 6, 4), 7])
    experts = [packs[e % 4] for e in range(E)]
    dense = [{k: v.astype(np.float32) for k, v in d.items()} for d in _dense(packs, cb)]
    x = S.activations(80, T, H)
    ids, w = S.softmax_topk(81, T, E, topk)
    slots = len(set(ids.ravel().tolist()))
    resident = 3 * torch.cuda.get_device_properties(gpu).multi_processor_count
    assert slots * (H // 128) > resident and slots * 2 * (I // 128) > resident
    want = O.moe_reference(x, ids, w, [dense[e % 4] for e in range(E)])
    dl = S.to_device(experts, gpu)
    got = C.moe_forward(torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
                        torch.from_numpy(w).to(gpu), dl, E, I, k_tables=dl["k_tables"], codebook=cb)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_prefill_mixed_k_beyond_4(gpu, cb):
    E, H, I, topk, T = len(KS), 256, 384, 4, 40
    experts = S.moe_layer(74 + cb, E, H, I, KS)
    x = S.activations(75, T, H)
    ids, w = S.softmax_topk(76, T, E, topk)
    ids[0, :3] = [5, 6, 0]
    want = O.moe_reference(x, ids, w, _dense(experts, cb))
    dl = S.to_device(experts, gpu)
    got = C.moe_prefill(torch.from_numpy(x).to(gpu).bfloat16(), torch.from_numpy(ids).to(gpu),
                        torch.from_numpy(w).to(gpu), dl, E, I, k_tables=dl["k_tables"], codebook=cb)
    assert rel_l2(got, want) <= TOL


def test_mk_dropin_k5_k6_experts(gpu):
    """The reference-compatible p2b_fused_moe_mk entry with K5 and K6 experts
    routed, against the oracle."""
    E, H, I, topk = 4, 256, 256, 3
    experts = S.moe_layer(77, E, H, I, [5, (6, 5, 6), 3, 2])
    dl = S.to_device(experts, gpu)
    x = torch.from_numpy(S.activations(78, 1, H)).to(gpu).half()
    ids = torch.tensor([0, 1, 3], dtype=torch.int32, device=gpu)
    w = torch.tensor([0.5, 0.3, 0.2], dtype=torch.float16, device=gpu)
    tabs = [dl[k] for k in ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh",
                            "up_svh", "down_trellis", "down_suh", "down_svh")]
    out = torch.empty_like(x)
    C.p2b_fused_moe_mk(x, out, *tabs, ids, w, *dl["k_tables"], E, True, I, 0.0)
    want = O.moe_reference(x.float().cpu().numpy(), ids.cpu().numpy()[None].astype(np.int64),
                           w.float().cpu().numpy()[None], _dense(experts, 1))
    assert rel_l2(out.float(), want) <= TOL + 1e-3  # fp16 output rounding
