"""Expert pack loader: checkpoint names -> pointer tables (host side, CPU).

The marker constants are pinned by their closed form (the codebook
multipliers 0xCBAC1FED / 0x83DCD12D read as signed int32, the reference's
src/vllm_exl3/exl3.py:113-116); the table contents by the data pointers of
the tensors the loader keeps; the rejections by the reference's load checks
(src/vllm_exl3/exl3.py:4282-4303)."""

import numpy as np
import pytest
import torch

from vllm_exl3_amd import packs as P
from vllm_exl3_amd import synthetic as S

PREFIX = "layers.0.ffn.experts"


def _signed32(u):
    return u - (1 << 32) if u >= 1 << 31 else u


def test_marker_constants_are_the_signed_multipliers():
    assert P.MCG_MARKER_SIGNED_INT32 == _signed32(0xCBAC1FED)
    assert P.MUL1_MARKER_SIGNED_INT32 == _signed32(0x83DCD12D)


@pytest.mark.parametrize("cb", [P.CB_MCG, P.CB_MUL1])
def test_uniform_k_tables(cb):
    experts = S.moe_layer(3, 4, 256, 384, 3)
    sd = P.state_dict_of(experts, PREFIX, cb)
    et = P.load_experts(sd, PREFIX, 4, "cpu")
    assert et.codebook == cb and not et.gateless and et.k_tables is None
    assert et.K == (3, 3, 3) and et.hidden == 256 and et.intermediate == 384 and et.n_local == 4
    assert set(et.tables) == {f"{p}_{a}" for p in ("gate", "up", "down")
                              for a in ("trellis", "suh", "svh")}
    # every pointer is the address of a kept tensor holding the pack's bytes
    kept = {t.data_ptr(): t for t in et._store}
    for e in range(4):
        for p in ("gate", "up", "down"):
            t = kept[int(et.tables[f"{p}_trellis"][e])]
            assert np.array_equal(t.numpy(), experts[e][p]["trellis"])
            su = kept[int(et.tables[f"{p}_suh"][e])]
            assert su.dtype == torch.float16
            assert np.array_equal(su.numpy(), experts[e][p]["suh"])
            sv = kept[int(et.tables[f"{p}_svh"][e])]
            assert np.array_equal(sv.numpy(), experts[e][p]["svh"])


def test_mixed_k_tables_and_gateless_aliasing():
    ks = [(2, 3, 4), (4, 4, 2), (3, 2, 3)]
    experts = S.moe_layer(5, 3, 256, 256, ks, gateless=True)
    sd = P.state_dict_of(experts, PREFIX, P.CB_MCG)
    et = P.load_experts(sd, PREFIX, 3, "cpu")
    assert et.gateless
    # gateless: gate slots alias up (the reference's build_exl3_fused_state)
    for a in ("trellis", "suh", "svh"):
        assert torch.equal(et.tables[f"gate_{a}"], et.tables[f"up_{a}"])
    kg, ku, kd = et.k_tables
    assert ku.tolist() == [3, 4, 2] and kg.tolist() == ku.tolist() and kd.tolist() == [4, 2, 3]
    assert ku.dtype == torch.int8 and et.K == (4, 4, 4)
    assert et.forward_kwargs()["k_tables"] is et.k_tables


def test_3inst_needs_opt_in():
    experts = S.moe_layer(6, 2, 128, 128, 2)
    sd = P.state_dict_of(experts, PREFIX, P.CB_3INST)
    with pytest.raises(P.PackError, match="no codebook marker"):
        P.load_experts(sd, PREFIX, 2, "cpu")
    assert P.load_experts(sd, PREFIX, 2, "cpu", allow_3inst=True).codebook == P.CB_3INST


def _sd():
    experts = S.moe_layer(7, 2, 128, 256, 3)
    return P.state_dict_of(experts, PREFIX, P.CB_MCG)


@pytest.mark.parametrize("mutate, msg", [
    (lambda sd: sd.__setitem__(f"{PREFIX}.1.w2.mul1", torch.tensor(P.MUL1_MARKER_SIGNED_INT32, dtype=torch.int32)),
     "both mcg and mul1"),
    (lambda sd: sd.__setitem__(f"{PREFIX}.0.w3.mcg", torch.tensor(12345, dtype=torch.int32)),
     "packed ABI mismatch"),
    (lambda sd: sd.pop(f"{PREFIX}.1.w1.svh"), "missing"),
    (lambda sd: sd.pop(f"{PREFIX}.1.w1.trellis"), "w1 for every expert"),
    (lambda sd: sd.__setitem__(f"{PREFIX}.0.w2.trellis", torch.zeros((8, 16, 48), dtype=torch.int16)),
     "does not match"),
    (lambda sd: sd.__setitem__(f"{PREFIX}.0.w1.trellis", torch.zeros((8, 16, 112), dtype=torch.int16)),
     "supports K"),
    (lambda sd: sd.__setitem__(f"{PREFIX}.0.w1.trellis", torch.zeros((8, 16, 48), dtype=torch.int32)),
     "int16"),
    (lambda sd: sd.__setitem__(f"{PREFIX}.0.w3.suh", torch.ones(64, dtype=torch.float16)),
     "suh must be"),
])
def test_rejections(mutate, msg):
    sd = _sd()
    mutate(sd)
    with pytest.raises(P.PackError, match=msg):
        P.load_experts(sd, PREFIX, 2, "cpu")


def test_mixed_codebooks_rejected():
    experts = S.moe_layer(8, 2, 128, 128, 2)
    sd = P.state_dict_of(experts, PREFIX, P.CB_MCG)
    del sd[f"{PREFIX}.1.w2.mcg"]
    sd[f"{PREFIX}.1.w2.mul1"] = torch.tensor(P.MUL1_MARKER_SIGNED_INT32, dtype=torch.int32)
    with pytest.raises(P.PackError, match="mix codebooks"):
        P.load_experts(sd, PREFIX, 2, "cpu")


def test_safetensors_file(tmp_path):
    from safetensors.torch import save_file

    experts = S.moe_layer(9, 3, 128, 256, [2, 3, 4])
    sd = P.state_dict_of(experts, PREFIX, P.CB_MUL1)
    path = str(tmp_path / "experts.safetensors")
    save_file(sd, path)
    et = P.load_experts_safetensors(path, PREFIX, 3, "cpu")
    assert et.codebook == P.CB_MUL1 and et.k_tables[2].tolist() == [2, 3, 4]


def test_k5_k6_packs_always_get_k_tables():
    """K 5/6 run through the executors' per-expert K tables, so a layer with
    such a K gets tables even when its K is uniform."""
    sd = P.state_dict_of(S.moe_layer(10, 2, 128, 256, 5), PREFIX, P.CB_MCG)
    et = P.load_experts(sd, PREFIX, 2, "cpu")
    assert et.k_tables is not None and et.k_tables[0].tolist() == [5, 5]
    sd = P.state_dict_of(S.moe_layer(11, 2, 128, 256, [(6, 5, 4), 3]), PREFIX, P.CB_MCG)
    et = P.load_experts(sd, PREFIX, 2, "cpu")
    assert [t.tolist() for t in et.k_tables] == [[6, 3], [5, 3], [4, 3]]
    sd = P.state_dict_of(S.moe_layer(12, 2, 128, 256, 3), PREFIX, P.CB_MCG)
    assert P.load_experts(sd, PREFIX, 2, "cpu").k_tables is None


def test_attach_sets_dispatch_attributes():
    from types import SimpleNamespace

    sd = P.state_dict_of(S.moe_layer(13, 3, 128, 256, [2, 3, 4]), PREFIX, P.CB_MUL1)
    et = P.load_experts(sd, PREFIX, 3, "cpu")
    layer = et.attach(SimpleNamespace())
    assert layer._exl3_ptrs is et.tables and layer._exl3_n_local == 3
    assert layer._exl3_codebook == P.CB_MUL1 and layer._exl3_intermediate_local == 256
    assert len(layer._exl3_inners) == 3 and layer._exl3_inners[2]["down"].K == 4
    assert layer._exl3_inners[1]["up"].trellis.data_ptr() == int(et.tables["up_trellis"][1])
