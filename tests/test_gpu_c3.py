"""Full-size GPU parity of BASELINE config 3: a mixed-K routed-MoE decode
layer, 256 experts with per-expert K drawn 40/40/20 over K2/K3/K4 (MCG) plus
one shared K4 expert routed as a ninth slot of weight 1, hidden 6144,
intermediate 2048, T = 64, uniform softmax top-8 routing - the workload the
benchmark times - under both decode GEMV kernels.

Reference: the eager per-expert loop (oracle.moe_reference's rounding points)
in torch fp32 over the routed experts' weights dequantised one expert at a
time by the HIP dequant (bit-exact to the oracle).  Relative L2 <= 2e-3."""

import numpy as np
import pytest
import torch

from moe_util import dense_of_layer, rel_l2, torch_moe_reference
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
E3, H3, I3, T3, TOPK = 256, 6144, 2048, 64, 8


@pytest.fixture(scope="module")
def c3(gpu):
    ks = S.mixed_k(3, E3) + [4]
    layer = S.moe_layer_device(3, E3 + 1, H3, I3, ks, gpu)
    ids_np, w_np = S.softmax_topk(3, T3, E3, TOPK)
    ids_np = np.concatenate([ids_np, np.full((T3, 1), E3, np.int64)], axis=1)
    w_np = np.concatenate([w_np, np.ones((T3, 1), np.float32)], axis=1)
    x = torch.from_numpy(S.activations(3, T3, H3)).to(gpu).bfloat16()
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(w_np).to(gpu)
    want = torch_moe_reference(x.float(), ids, w, dense_of_layer(layer, ks, 1), E3 + 1)
    torch.cuda.synchronize()
    yield layer, ks, x, ids, w, want
    del layer


def test_moe_config3_full_size(gpu, gemv_policy, c3):
    layer, ks, x, ids, w, want = c3
    assert sorted(set(ks)) == [2, 3, 4]
    got = C.moe_forward(x, ids, w, layer, E3 + 1, I3, K=(4, 4, 4), k_tables=layer["k_tables"],
                        codebook=1)
    torch.cuda.synchronize()
    err = rel_l2(got, want)
    print(f"C3 full size ({gemv_policy}): rel L2 {err:.3e}", flush=True)
    assert err <= 2e-3
