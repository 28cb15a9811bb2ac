"""Refusals of the W1 write drop-in (host checks, before any launch): the
messages of validate_w1_call (src/vllm_exl3/minimax_q4kv_reference.py:
625-732), raised as ValueError("q4 W1 refused: ...")."""

import pytest
import torch

from vllm_exl3_amd import nvfp4_kv as Q


def _args(**over):
    T, nq, nkv, niq = 3, 2, 1, 0
    a = dict(qkv=torch.zeros((T, (nq + 2 * nkv) * 128), dtype=torch.bfloat16),
             q_norm_w=torch.zeros(128), k_norm_w=torch.zeros(128),
             cos_sin_cache=torch.zeros((16, 64)), positions=torch.zeros(T, dtype=torch.int64),
             num_heads=nq, num_kv_heads=nkv, rotary_dim=64, eps=1e-6, index_q_norm_w=None,
             index_k_norm_w=None, num_index_heads=niq, slot_mapping=None, index_slot_mapping=None,
             pool=torch.zeros((1, 2, 128, 72), dtype=torch.uint8), index_cache=None, block_size=128,
             q_out=torch.zeros((T, nq * 128), dtype=torch.bfloat16), index_q_out=None)
    a.update(over)
    return a


@pytest.mark.parametrize("over, msg", [
    (dict(qkv=torch.zeros((3, 512), dtype=torch.float32)), "requires bfloat16 qkv rows"),
    (dict(qkv=torch.zeros((3, 640), dtype=torch.bfloat16)), "does not match the branch layout"),
    (dict(rotary_dim=60), "rotary_dim % 8 == 0"),
    (dict(rotary_dim=0), "rotary_dim % 8 == 0"),
    (dict(block_size=16), "block_size 128"),
    (dict(q_out=None), "requires the bf16 q_out buffer"),
    (dict(num_index_heads=1, qkv=torch.zeros((3, 768), dtype=torch.bfloat16),
          index_cache=torch.zeros((3, 128), dtype=torch.float16)), "fp8 e4m3 index_cache"),
])
def test_w1_refusals(over, msg):
    with pytest.raises(ValueError, match="q4 W1 refused") as ei:
        Q.q4_w1_insert(**_args(**over))
    assert msg in str(ei.value)


def test_w1_host_pool_must_be_device_memory():
    with pytest.raises(ValueError, match="device memory"):
        Q.q4_w1_insert(**_args())
