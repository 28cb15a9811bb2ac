"""Per-phase kernel timing through the library's event ring.

    with PhaseTimer(max_calls=100) as pt:
        for _ in range(100):
            vllm_exl3_c.moe_forward(...)
    pt.phase_ms  # summed milliseconds per phase; pt.calls recorded calls

Phases of exl3_moe_forward: 0 route, 1 gate/up GEMV, 2 down GEMV, 3 combine.
Events are recorded on the launch stream, so each phase time is that kernel's
duration plus the (small) gap before the next launch.
"""

from __future__ import annotations

import ctypes

from . import _lib

MOE_PHASES = ("route", "rotate", "gate_up", "act", "down", "combine")


class PhaseTimer:
    def __init__(self, max_calls: int, max_phases: int = 8):
        self.max_calls = int(max_calls)
        self.max_phases = int(max_phases)
        self.phase_ms: list[float] = []
        self.calls = 0

    def __enter__(self) -> "PhaseTimer":
        _lib.call("exl3_profile_begin", self.max_calls)
        return self

    def __exit__(self, *exc) -> None:
        arr = (ctypes.c_double * self.max_phases)()
        n_calls, n_phases = ctypes.c_int(), ctypes.c_int()
        _lib.call("exl3_profile_end", ctypes.addressof(arr), self.max_phases,
                  ctypes.addressof(n_calls), ctypes.addressof(n_phases))
        self.calls = n_calls.value
        self.phase_ms = [arr[i] for i in range(n_phases.value)]

    def mean_ms(self, phase: int) -> float:
        return self.phase_ms[phase] / max(self.calls, 1)
