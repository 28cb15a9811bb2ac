"""Pins of the oracle's routed-expert loop (``oracle.moe_reference``) on the CPU.

The GPU MoE, prefill and smoke parity checks all compare against
``oracle.moe_reference`` or its torch twin ``moe_util.torch_moe_reference``,
so this file pins both:

* the reference's own known answers for the activation and clamp
  (tests/test_activation_parity.py:46-81), run through the oracle with scalar
  projections exactly as the reference runs them through its eager loop
  (fixed gate/up values, identity down, weight 1);
* SwiGLU-OAI and relu^2 against float64 closed forms;
* a single expert with weight 1 against an independently written torch
  float64 formula, at both rounding-point settings (fp16 g/u as the native
  kernel, fp32 g/u as the eager loop);
* an exact-sum routing case after tests/test_routing_parity.py:84-111
  (experts that scale x by e + 1, so the layer output is
  x * sum_k (id_k + 1) * w_k), with sentinel ids and an expert map;
* the id mapping of src/vllm_exl3/exl3.py:2332-2354;
* that mistakes planted in the oracle's activation (clamp direction, missing
  clamp, wrong OAI term) fail the checks above.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import torch_moe_reference


def _scalar_expert(gate: float | None, up: float, down: float = 1.0) -> dict:
    """An expert whose projections of x = [[1.0]] are exactly the given fp32
    values (the reference's _FixedProjection / _IdentityProjection)."""
    f = lambda v: np.array([[v]], dtype=np.float32)
    return {"gate": None if gate is None else f(gate), "up": f(up), "down": f(down)}


def run_activation(gate: float | None, up: float, limit: float | None, act: str = "silu") -> float:
    """tests/test_activation_parity.py:25-41: one token, one route, weight 1,
    through the eager-loop rounding points (g/u in fp32)."""
    out = O.moe_reference(np.ones((1, 1), np.float32), np.zeros((1, 1), np.int64),
                          np.ones((1, 1), np.float32), [_scalar_expert(gate, up)],
                          limit=limit, act=act, gu_fp16=False)
    return float(out[0, 0])


def _silu64(g: float) -> float:
    return g / (1.0 + math.exp(-g))


# --- the reference's activation vectors -----------------------------------

def check_reference_activation_vectors() -> None:
    """Every known answer of tests/test_activation_parity.py:46-81."""
    # :46-53 plain and clamped SwiGLU
    assert abs(run_activation(20.0, 20.0, None) - 400.0) <= 1e-4
    assert abs(run_activation(20.0, 20.0, 10.0) - 99.9954605) <= 0.01
    # :56-74 clamp boundaries and negative up
    for gate, up, limit in [(9.99, 20.0, 10.0), (10.0, -20.0, 10.0), (10.01, -20.0, 10.0),
                            (-10.01, 20.0, 10.0), (-9.99, -20.0, 10.0)]:
        expected = float(torch.nn.functional.silu(torch.tensor(min(gate, limit)))
                         * min(max(up, -limit), limit))
        got = run_activation(gate, up, limit)
        assert abs(got - expected) <= 0.03, (gate, up, limit, got, expected)
    # :77-81 a non-positive limit keeps plain SwiGLU
    plain = run_activation(20.0, 20.0, None)
    for limit in (0.0, -1.0):
        assert abs(run_activation(20.0, 20.0, limit) - plain) <= 1e-4


def test_reference_activation_vectors():
    check_reference_activation_vectors()


def test_swiglu_oai_closed_form():
    # (u + 1) * g * sigmoid(1.702 g), gate clamped from above, up symmetric
    cases = [(2.0, 3.0, None), (0.5, -0.25, None), (-3.0, 2.0, None), (30.0, 1.0, None),
             (20.0, -20.0, 7.0), (-20.0, 20.0, 7.0), (6.5, 6.5, 7.0)]
    for g, u, limit in cases:
        gc, uc = g, u
        if limit:
            gc = min(g, limit)
            uc = min(max(u, -limit), limit)
        want = (uc + 1.0) * gc / (1.0 + math.exp(-1.702 * gc))
        got = run_activation(g, u, limit, act="swiglu_oai")
        # one fp16 rounding of the activation before the (identity) down
        assert abs(got - want) <= max(abs(want), 1e-3) * 2 ** -10, (g, u, limit, got, want)
    # sigmoid saturates: large g gives (u + 1) * g
    assert run_activation(30.0, 1.0, None, act="swiglu_oai") == 60.0
    assert run_activation(0.0, 5.0, None, act="swiglu_oai") == 0.0


def test_relu2_gateless_closed_form():
    assert run_activation(None, 3.0, None) == 9.0
    assert run_activation(None, -2.0, None) == 0.0
    assert run_activation(None, 20.0, 10.0) == 100.0   # up clamped from above
    assert run_activation(None, -20.0, 10.0) == 0.0    # clamped from below, then relu
    assert run_activation(None, 1.5, 0.0) == 2.25      # limit 0 is no clamp


# --- single expert vs an independent float64 formula ------------------------

def _fp16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).to(torch.float64)


@pytest.mark.parametrize("gu_fp16", [True, False])
@pytest.mark.parametrize("act,limit", [("silu", None), ("silu", 1.0), ("swiglu_oai", 2.0),
                                       ("relu2", 0.5)])
def test_single_expert_reduction(gu_fp16, act, limit):
    rng = np.random.default_rng(5)
    H, I = 256, 128
    x = rng.standard_normal((1, H)).astype(np.float32)
    mk = lambda r, c, s: (rng.standard_normal((r, c)) * s).astype(np.float16)
    gate = None if act == "relu2" else mk(H, I, 0.1)
    up, down = mk(H, I, 0.1), mk(I, H, 0.1)
    got = O.moe_reference(x, np.array([[0]]), np.array([[1.0]], np.float32),
                          [{"gate": gate, "up": up, "down": down}], limit=limit,
                          act="silu" if act == "relu2" else act, gu_fp16=gu_fp16)
    # independent restatement: torch float64 with explicit fp16 rounding points
    xt = _fp16(torch.from_numpy(x))
    u = xt @ torch.from_numpy(up).double()
    g = None if gate is None else xt @ torch.from_numpy(gate).double()
    if gu_fp16:
        u = _fp16(u)
        g = None if g is None else _fp16(g)
    if limit:
        u = u.clamp(-limit, limit)
        g = None if g is None else g.clamp(max=limit)
    if act == "relu2":
        a = torch.relu(u) ** 2
    elif act == "swiglu_oai":
        a = (u + 1.0) * g * torch.sigmoid(1.702 * g)
    else:
        a = torch.nn.functional.silu(g) * u
    want = (_fp16(a) @ torch.from_numpy(down).double()).numpy()
    # the oracle computes in fp32; one act element may round to the other
    # fp16 neighbour, worth at most 1 ulp * |down row|
    err = np.abs(got - want).max()
    assert err <= 2e-3 * np.abs(want).max(), err
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-4, rel


# --- exact-sum routing ---------------------------------------------------------

def _scaling_experts(n: int, H: int = 3) -> list[dict]:
    """Expert e maps x -> (e + 1) * x exactly: a bias channel (x[:, H] = 1)
    drives the gate to 32, where silu(32) == 32 in fp32; up copies x; down
    scales by (e + 1) / 32 (exact in fp16 for e + 1 <= 32)."""
    experts = []
    for e in range(n):
        gate = np.zeros((H + 1, H), np.float16)
        gate[H, :] = 32.0
        up = np.zeros((H + 1, H), np.float16)
        up[np.arange(H), np.arange(H)] = 1.0
        down = np.zeros((H, H + 1), np.float16)
        down[np.arange(H), np.arange(H)] = (e + 1) / 32.0
        experts.append({"gate": gate, "up": up, "down": down})
    return experts


@pytest.mark.parametrize("tokens", [1, 2, 4, 8])
@pytest.mark.parametrize("top_k", [1, 3, 8])
def test_exact_sum_routing(tokens, top_k):
    """tests/test_routing_parity.py:84-111: every route contributes
    (id + 1) * w; the layer output is x * sum_k (id_k + 1) * w_k."""
    H = 3
    n = max(top_k + 2, 16)
    x = np.concatenate([np.arange(1, tokens * H + 1, dtype=np.float32).reshape(tokens, H),
                        np.ones((tokens, 1), np.float32)], axis=1)
    ids = (np.arange(tokens * top_k).reshape(tokens, top_k) % n).astype(np.int64)
    w = np.linspace(0.07, 0.97, tokens * top_k, dtype=np.float32).reshape(tokens, top_k)
    w16 = w.astype(np.float16).astype(np.float32)
    got = O.moe_reference(x, ids, w16, _scaling_experts(n, H))
    scale = ((ids + 1.0) * w16.astype(np.float64)).sum(axis=1)
    want = np.zeros((tokens, H + 1))
    want[:, :H] = x[:, :H] * scale[:, None]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=0)


def test_exact_sum_routing_sentinels_and_expert_map():
    H, n_local = 3, 6
    x = np.array([[1, 2, 3, 1], [4, 5, 6, 1]], np.float32)
    # global ids 0..9 -> local ids through the map; -1 / past the map / past
    # n_local are non-local
    emap = np.array([5, -1, 0, 3, 7, 1, 2, -4], np.int64)
    ids = np.array([[0, 1, 2, 9], [3, 4, 5, -2]], np.int64)
    w = np.array([[0.5, 0.25, 0.125, 2.0], [1.0, 4.0, 0.75, 8.0]], np.float32)
    got = O.moe_reference(x, ids, w, _scaling_experts(n_local, H), expert_map=emap)
    # row 0: global 0 -> local 5 (x6), 1 -> non-local, 2 -> local 0 (x1), 9 -> past the map
    # row 1: global 3 -> local 3 (x4), 4 -> 7 >= n_local, 5 -> local 1 (x2), -2 invalid
    s0 = 0.5 * 6 + 0.125 * 1
    s1 = 1.0 * 4 + 0.75 * 2
    want = np.zeros((2, H + 1), np.float32)
    want[0, :H] = x[0, :H] * s0
    want[1, :H] = x[1, :H] * s1
    np.testing.assert_array_equal(got, want)


def test_map_topk_to_local():
    ids = np.array([[-1, 0, 3, 4, 100]])
    np.testing.assert_array_equal(O.map_topk_to_local(ids, 4), [[4, 0, 3, 4, 4]])
    emap = np.array([2, -1, 0, 9])
    np.testing.assert_array_equal(O.map_topk_to_local(ids, 4, emap), [[4, 2, 4, 4, 4]])
    np.testing.assert_array_equal(O.map_topk_to_local(ids, 4, np.zeros(0, np.int64)),
                                  [[4, 4, 4, 4, 4]])


# --- the torch twin used at full sizes --------------------------------------

@pytest.mark.parametrize("act,limit,gateless", [("silu", 0.0, False), ("silu", 0.75, False),
                                                ("swiglu_oai", 1.5, False), ("silu", 0.5, True)])
def test_torch_twin_matches_oracle(act, limit, gateless):
    rng = np.random.default_rng(11)
    T, H, I, n, topk = 5, 128, 256, 6, 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    mk = lambda r, c: (rng.standard_normal((r, c)) * 0.08).astype(np.float16)
    experts = [{"gate": None if gateless else mk(H, I), "up": mk(H, I), "down": mk(I, H)}
               for _ in range(n)]
    ids = rng.integers(-1, n + 2, size=(T, topk))
    w = rng.random((T, topk)).astype(np.float32)
    want = O.moe_reference(x, ids, w, experts, limit=limit, act=act)
    dense = {e: {k: torch.from_numpy(v) for k, v in pk.items() if v is not None}
             for e, pk in enumerate(experts)}
    got = torch_moe_reference(torch.from_numpy(x), torch.from_numpy(ids), torch.from_numpy(w),
                              dense, n, limit=limit, act=act).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


# --- planted mistakes are caught -------------------------------------------

def _wrong_clamp_gate_below(g, u, act="silu", limit=None):
    if g is not None and limit is not None and limit > 0:
        g = np.maximum(np.asarray(g, np.float32), np.float32(-limit))  # wrong direction
        u = np.clip(np.asarray(u, np.float32), -limit, limit)
        return (O.silu(g) * u).astype(np.float32)
    return _ORIG_ACT(g, u, act, limit)


def _wrong_no_up_clamp(g, u, act="silu", limit=None):
    if g is not None and limit is not None and limit > 0:
        g = np.minimum(np.asarray(g, np.float32), np.float32(limit))
        return (O.silu(g) * np.asarray(u, np.float32)).astype(np.float32)
    return _ORIG_ACT(g, u, act, limit)


def _wrong_clamp_after_act(g, u, act="silu", limit=None):
    a = _ORIG_ACT(g, u, act, None)
    if limit is not None and limit > 0:
        a = np.clip(a, -limit, limit)
    return a


def _wrong_oai_minus_one(g, u, act="silu", limit=None):
    if act == "swiglu_oai":
        return _ORIG_ACT(g, np.asarray(u, np.float32) - np.float32(2.0), act, limit)
    return _ORIG_ACT(g, u, act, limit)


_ORIG_ACT = O.moe_activation


@pytest.mark.parametrize("mistake", [_wrong_clamp_gate_below, _wrong_no_up_clamp,
                                     _wrong_clamp_after_act])
def test_planted_clamp_mistakes_fail_the_vectors(monkeypatch, mistake):
    monkeypatch.setattr(O, "moe_activation", mistake)
    with pytest.raises(AssertionError):
        check_reference_activation_vectors()


def test_planted_oai_mistake_fails_the_closed_form(monkeypatch):
    monkeypatch.setattr(O, "moe_activation", _wrong_oai_minus_one)
    with pytest.raises(AssertionError):
        test_swiglu_oai_closed_form()


def test_planted_rounding_mistake_fails_the_reduction(monkeypatch):
    """Dropping the fp16 rounding of the activation is caught by the
    single-expert check (the formula there rounds it)."""
    orig = O._f16
    calls = {"n": 0}

    def skip_act_round(a):
        calls["n"] += 1
        # moe_reference rounds x, u, g, then the activation: skip the 4th
        return np.asarray(a, np.float32) if calls["n"] % 4 == 0 else orig(a)

    monkeypatch.setattr(O, "_f16", skip_act_round)
    with pytest.raises(AssertionError):
        test_single_expert_reduction(True, "silu", None)
