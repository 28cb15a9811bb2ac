"""Top-level alias so ``importlib.import_module("vllm_exl3_c")`` finds this build.

The reference plugin probes its native module by that name
(src/vllm_exl3/exl3.py:2146-2152) and requires a callable ``p2b_fused_moe``.
With ``vllm-exl3_amd/`` on ``sys.path`` this module is that drop-in: it
re-exports every name of :mod:`vllm_exl3_amd.vllm_exl3_c`.
"""

from vllm_exl3_amd.vllm_exl3_c import *  # noqa: F401,F403
from vllm_exl3_amd.vllm_exl3_c import (  # noqa: F401
    P2B_MOE_ABI_VERSION,
    P2B_MOE_MIXED_K,
    P2B_MOE_PADDED,
)
