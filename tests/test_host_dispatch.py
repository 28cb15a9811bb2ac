"""Host logic of the routed-expert dispatch (vllm_exl3_amd.dispatch) on the CPU,
with recording stand-ins for the two executors in the pattern of the
reference's tests/test_routing_parity.py:12-36 and fixed projections for the
per-expert loop as in tests/test_activation_parity.py:13-41."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from vllm_exl3_amd import dispatch as D


class _Recording:
    """Stand-in for vllm_exl3_c.moe_forward / moe_prefill: records the
    arguments and returns x * sum_k (id_k + 1) * w_k over the local routes
    (sentinels skipped), the reference test's exact-sum contract."""

    def __init__(self, kind: str, fail: bool = False):
        self.kind, self.fail, self.calls = kind, fail, []

    def __call__(self, x, ids, weights, tables, n_local, inter, **kw):
        self.calls.append({"ids": ids.clone(), "weights": weights.clone(), "n_local": n_local,
                           "inter": inter, **kw})
        if self.fail:
            raise RuntimeError(f"{self.kind} executor unavailable")
        valid = (ids >= 0) & (ids < n_local)
        contrib = torch.where(valid, (ids.float() + 1.0) * weights.float(), torch.zeros(()))
        return x.float() * contrib.sum(dim=1, keepdim=True)


def _layer(n_local=16, **attrs):
    ptrs = {k: torch.zeros(n_local, dtype=torch.int64) for k in D.PTR_KEYS}
    layer = SimpleNamespace(_exl3_ptrs=ptrs, _exl3_k=4, _exl3_intermediate_local=2048)
    for k, v in attrs.items():
        setattr(layer, k, v)
    return layer


@pytest.fixture
def rec(monkeypatch):
    dec, pre = _Recording("decode"), _Recording("prefill")
    monkeypatch.setattr(D.C, "moe_forward", dec)
    monkeypatch.setattr(D.C, "moe_prefill", pre)
    return dec, pre


@pytest.mark.parametrize("tokens", [1, 2, 4, 8])
@pytest.mark.parametrize("top_k", [1, 2, 3, 6, 8])
def test_routing_preserves_topk_and_all_contributions(rec, tokens, top_k):
    """tests/test_routing_parity.py:38-111: every row keeps its K routes and
    the output is their weighted sum."""
    dec, _ = rec
    hidden, n = 3, max(top_k + 2, 16)
    x = torch.arange(1, tokens * hidden + 1, dtype=torch.float32).reshape(tokens, hidden)
    ids = torch.arange(tokens * top_k, dtype=torch.long).reshape(tokens, top_k).remainder(n)
    w = torch.linspace(0.07, 0.97, steps=tokens * top_k).reshape(tokens, top_k)
    layer = _layer(n)
    out = D.apply_exl3_experts(x, ids, w, layer)
    assert layer._exl3_last_apply == "decode" and len(dec.calls) == 1
    call = dec.calls[0]
    assert torch.equal(call["ids"], ids) and torch.equal(call["weights"], w)
    assert call["n_local"] == n and call["inter"] == 2048 and call["K"] == (4, 4, 4)
    expected = x * ((ids.float() + 1.0) * w).sum(dim=1, keepdim=True)
    torch.testing.assert_close(out, expected, rtol=0, atol=0)


def test_expert_map_matches_oracle_mapping(rec):
    dec, _ = rec
    n_local = 6
    emap = torch.tensor([5, -1, 0, 3, 7, 1, 2, -4])
    ids = torch.tensor([[0, 1, 2, 9], [3, 4, 5, -2]])
    layer = _layer(n_local, expert_map=emap)
    D.apply_exl3_experts(torch.ones(2, 4), ids, torch.ones(2, 4), layer)
    want = O.map_topk_to_local(ids.numpy(), n_local, emap.numpy())
    np.testing.assert_array_equal(dec.calls[0]["ids"].numpy(), want)
    # the pinned map is cached on the layer and reused
    pinned = layer._exl3_pinned_expert_map
    D.apply_exl3_experts(torch.ones(2, 4), ids, torch.ones(2, 4), layer)
    assert layer._exl3_pinned_expert_map is pinned


def test_unpinned_map_is_refused():
    with pytest.raises(RuntimeError, match="not pinned"):
        D.map_topk_to_local(torch.zeros(2, 2, dtype=torch.long), 4, torch.zeros(4, dtype=torch.int32))


def test_executor_choice_by_rows_per_expert(rec, monkeypatch):
    dec, pre = rec
    thr = D.prefill_rows_per_expert()
    n_local, topk = 16, 2
    layer = _layer(n_local)
    t_switch = int(np.ceil(thr * n_local / topk))
    for T, kind in ((1, "decode"), (t_switch - 1, "decode"), (t_switch, "prefill"), (4 * t_switch, "prefill")):
        D.apply_exl3_experts(torch.ones(T, 8), torch.zeros(T, topk, dtype=torch.long),
                             torch.ones(T, topk), layer)
        assert layer._exl3_last_apply == kind, T
    monkeypatch.setenv("VLLM_EXL3_AMD_PREFILL_ROWS", "0.25")
    D.apply_exl3_experts(torch.ones(2, 8), torch.zeros(2, topk, dtype=torch.long), torch.ones(2, topk), layer)
    assert layer._exl3_last_apply == "prefill"
    D.apply_exl3_experts(torch.ones(2, 8), torch.zeros(2, topk, dtype=torch.long), torch.ones(2, topk), layer,
                         executor="decode")
    assert layer._exl3_last_apply == "decode"


class _FixedProjection:
    def __init__(self, value: float) -> None:
        self.value = value

    def forward(self, x, _params, *, out_dtype):
        return torch.full((x.shape[0], 1), self.value, dtype=out_dtype)


class _IdentityProjection:
    def forward(self, x, _params, *, out_dtype):
        return x.to(dtype=out_dtype)


def _loop_layer(gate, up, **attrs):
    inners = [{"gate": _FixedProjection(gate), "up": _FixedProjection(up), "down": _IdentityProjection()}]
    return SimpleNamespace(_exl3_inners=inners, **attrs)


def test_failures_are_recorded_and_fall_back(monkeypatch):
    dec, pre = _Recording("decode", fail=True), _Recording("prefill")
    monkeypatch.setattr(D.C, "moe_forward", dec)
    monkeypatch.setattr(D.C, "moe_prefill", pre)
    layer = _layer(4)
    D.apply_exl3_experts(torch.ones(1, 3), torch.zeros(1, 2, dtype=torch.long), torch.ones(1, 2), layer)
    assert layer._exl3_last_apply == "prefill" and "decode executor unavailable" in layer._exl3_native_error
    # both executors fail: the per-expert loop over the layer's projections
    pre.fail = True
    layer = _loop_layer(20.0, 20.0)
    layer._exl3_ptrs = _layer(1)._exl3_ptrs
    out = D.apply_exl3_experts(torch.zeros(1, 1), torch.tensor([[0]]), torch.tensor([[1.0]]), layer)
    assert layer._exl3_last_apply == "loop" and "prefill executor unavailable" in layer._exl3_native_error
    torch.testing.assert_close(out, torch.tensor([[400.0]]), rtol=0, atol=1e-4)


def test_loop_reproduces_reference_activation_vectors():
    """The loop's clamp and activation against the reference's known answers
    (tests/test_activation_parity.py:46-81)."""
    def run(g, u, limit, **attrs):
        return D.apply_exl3_experts(torch.zeros(1, 1), torch.tensor([[0]]), torch.tensor([[1.0]]),
                                    _loop_layer(g, u, **attrs), limit=limit)

    torch.testing.assert_close(run(20.0, 20.0, None), torch.tensor([[400.0]]), rtol=0, atol=1e-4)
    torch.testing.assert_close(run(20.0, 20.0, 10.0), torch.tensor([[99.9954605]]), rtol=0, atol=0.01)
    for g, u, lim in [(9.99, 20.0, 10.0), (10.0, -20.0, 10.0), (10.01, -20.0, 10.0),
                      (-10.01, 20.0, 10.0), (-9.99, -20.0, 10.0)]:
        want = torch.nn.functional.silu(torch.tensor(min(g, lim))) * min(max(u, -lim), lim)
        torch.testing.assert_close(run(g, u, lim), want.reshape(1, 1), rtol=0, atol=0.03)
    torch.testing.assert_close(run(20.0, 20.0, 0.0), run(20.0, 20.0, None), rtol=0, atol=1e-4)
    # the layer's swiglu_limit is used when the call passes none
    torch.testing.assert_close(run(20.0, 20.0, None, swiglu_limit=10.0),
                               torch.tensor([[99.9954605]]), rtol=0, atol=0.01)


def test_activation_and_gate_params(rec):
    dec, _ = rec

    def cfg(v):
        return SimpleNamespace(activation=SimpleNamespace(value=v))

    for value, act in (("silu", 0), ("relu2_no_mul", 2), ("swigluoai", 3), ("swigluoai_uninterleave", 3)):
        layer = _layer(moe_config=cfg(value))
        D.apply_exl3_experts(torch.ones(1, 4), torch.zeros(1, 1, dtype=torch.long), torch.ones(1, 1), layer)
        assert dec.calls[-1]["act"] == act
        assert dec.calls[-1]["gateless"] == (act == 2)
    # OAI: limit defaults to 7.0; alpha and beta are fixed by the kernel
    layer = _layer(moe_config=cfg("swigluoai"))
    D.apply_exl3_experts(torch.ones(1, 4), torch.zeros(1, 1, dtype=torch.long), torch.ones(1, 1), layer)
    assert dec.calls[-1]["swiglu_limit"] == 7.0
    with pytest.raises(ValueError, match="alpha"):
        D.resolve_moe_gate_params(_layer(moe_config=cfg("swigluoai"), swiglu_alpha=1.5))
    with pytest.raises(ValueError, match="beta"):
        D.resolve_moe_gate_params(_layer(moe_config=cfg("swigluoai"), swiglu_beta=0.5))
    with pytest.raises(ValueError, match="no kernel instance"):
        D.resolve_moe_act(_layer(moe_config=cfg("gelu")))
    assert D.resolve_moe_gate_params(_layer(swiglu_limit=-3.0)) == (None, None)
    assert D.resolve_moe_gate_params(_layer(swiglu_limit="nan")) == (None, None)
    assert D.resolve_moe_gate_params(_layer(swiglu_limit=10)) == (None, 10.0)


def test_codebook_and_k_description(rec):
    dec, _ = rec
    kt = tuple(torch.tensor([2, 5], dtype=torch.int8) for _ in range(3))
    layer = _layer(2, _exl3_codebook_flags=(False, True) * 3, _exl3_k_tuple=(3, 4, 2), _exl3_k_tables=kt)
    D.apply_exl3_experts(torch.ones(1, 4), torch.zeros(1, 1, dtype=torch.long), torch.ones(1, 1), layer)
    assert dec.calls[-1]["codebook"] == 2 and dec.calls[-1]["K"] == (3, 4, 2)
    assert dec.calls[-1]["k_tables"] is not None
    mixed = _layer(2, _exl3_codebook_flags=(True, False, False, True, True, False))
    with pytest.raises(RuntimeError, match="different codebooks"):
        D.layer_codebook(mixed)
