"""MI355X-native (gfx950) EXL3 routed-expert compute path.

Modules:
  vllm_exl3_c  -- drop-in for the reference's native module (csrc/bindings.cpp)
  _lib         -- ctypes binding of the C ABI (include/exl3_mi355x.h)
  synthetic    -- seeded synthetic workloads for the five benchmark configs
"""

__all__ = ["vllm_exl3_c", "synthetic"]
