"""The compiled drop-in module exposes the reference's native-module surface
(csrc/bindings.cpp:197-266): every function with the same positional
parameter names in the same order (keyword-only extensions may follow), and
the capability attributes the plugin gates on (csrc/bindings.cpp:243-257).
Host only: reads the pybind signatures, calls nothing on a device."""

import re

import pytest

from vllm_exl3_amd import vllm_exl3_c as C

# the reference's py::arg lists, in order (csrc/bindings.cpp:198-265)
REFERENCE = {
    "dequant_trellis": ["trellis", "suh", "svh", "K", "mcg"],
    "exl3_gemv": ["x", "trellis", "suh", "svh", "K", "mcg", "mmode"],
    "exl3_gemm": ["x", "trellis", "suh", "svh", "K", "mcg"],
    "p2b_gemv_batched": ["x", "trellis_ptrs", "suh_ptrs", "svh_ptrs", "expert_indices", "K", "mcg", "mmode"],
    "p2b_fused_moe": ["x", "out", "gate_trellis_ptrs", "gate_suh_ptrs", "gate_svh_ptrs", "up_trellis_ptrs",
                      "up_suh_ptrs", "up_svh_ptrs", "down_trellis_ptrs", "down_suh_ptrs", "down_svh_ptrs",
                      "expert_indices", "routing_weights", "K_gate", "K_up", "K_down", "mcg",
                      "intermediate_size", "swiglu_limit"],
    "p2b_fused_moe_mk": ["x", "out", "gate_trellis_ptrs", "gate_suh_ptrs", "gate_svh_ptrs", "up_trellis_ptrs",
                         "up_suh_ptrs", "up_svh_ptrs", "down_trellis_ptrs", "down_suh_ptrs", "down_svh_ptrs",
                         "expert_indices", "routing_weights", "k_gate_tbl", "k_up_tbl", "k_down_tbl",
                         "n_local", "mcg", "intermediate_size", "swiglu_limit"],
    "p2b_fused_moe_padded": ["x", "out", "gate_trellis_ptrs", "gate_suh_ptrs", "gate_svh_ptrs",
                             "up_trellis_ptrs", "up_suh_ptrs", "up_svh_ptrs", "down_trellis_ptrs",
                             "down_suh_ptrs", "down_svh_ptrs", "expert_indices_padded",
                             "routing_weights_padded", "n_valid", "k_gate_tbl", "k_up_tbl", "k_down_tbl",
                             "n_local", "max_k", "mcg", "intermediate_size", "swiglu_limit"],
    "exl3_fat_gemm": ["a", "packed", "out", "svh", "K", "mcg", "mul1"],
    "exl3_fat_gemm_scatter": ["a", "packed", "out", "svh", "token_idx", "route_weight", "K", "mcg", "mul1"],
}


def _positional_names(fn) -> list[str]:
    """Parameter names before the keyword-only marker of a pybind signature."""
    first = fn.__doc__.strip().splitlines()[0]
    inner = first[first.index("(") + 1:first.rindex(") ->")]
    names = []
    for part in re.split(r",\s*(?![^\[]*\])", inner):
        part = part.strip()
        if part == "*":
            break
        names.append(part.split(":")[0].strip())
    return names


@pytest.mark.parametrize("name", sorted(REFERENCE))
def test_reference_function_surface(name):
    fn = getattr(C, name)
    assert callable(fn)
    assert _positional_names(fn) == REFERENCE[name]


def test_capability_attributes():
    assert C.P2B_MOE_ABI_VERSION == 4 and C.P2B_MOE_MIXED_K is True and C.P2B_MOE_PADDED is True


def test_module_is_the_compiled_extension():
    # no Python fallback: the exports are the extension's builtins
    assert type(C.p2b_fused_moe).__name__ == "builtin_function_or_method"
    assert C.p2b_fused_moe is C._C.p2b_fused_moe


def test_rejections_need_no_device():
    """Argument checks run before any device work: a CPU x is refused with the
    reference's message."""
    import torch

    x = torch.zeros(1, 256, dtype=torch.float16)
    tab = torch.zeros(4, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="fused MoE requires CUDA fp16 input"):
        C.p2b_fused_moe(x, x.clone(), *([tab] * 9), torch.zeros(2, dtype=torch.int32),
                        torch.zeros(2, dtype=torch.float16), 3, 3, 3, True)
