"""Write NVFP4 KV pack fixtures from the reference's own packer.

Run in the build container only (the reference checkout does not travel):
    python tests/golden/make_nvfp4_vectors.py /root/reference
It imports src/vllm_exl3/minimax_q4kv_reference.py (pure torch) and stores,
for seeded rows that include e2m1 ties, RZ boundaries, saturation, zero and
tiny groups: the rows (as bf16 bit patterns), pack_q4_row's data and scale
bytes, and pack_slot_region_side's 9216-byte regions for K and V.  The
oracle in oracle/nvfp4.py is checked against these bytes.
"""

import importlib.util
import pathlib
import sys

import numpy as np
import torch


def load_reference(root: pathlib.Path):
    path = root / "src" / "vllm_exl3" / "minimax_q4kv_reference.py"
    spec = importlib.util.spec_from_file_location("q4kv_reference", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def rows_under_test() -> np.ndarray:
    g = np.random.default_rng(1234)
    rows = [g.standard_normal((96, 128)).astype(np.float32)]
    rows.append((g.standard_normal((16, 128)) * 40.0).astype(np.float32))     # scales > 1
    rows.append((g.standard_normal((16, 128)) * 1e-4).astype(np.float32))     # clamp 2^-9
    big = g.standard_normal((8, 128)).astype(np.float32)
    big[:, ::5] *= 3000.0                                                     # saturation
    rows.append(big)
    ties = np.zeros((8, 128), np.float32)
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    for r in range(8):
        for grp in range(8):
            v = np.zeros(16, np.float32)
            v[0] = 6.0                                   # amax 6 -> scale 1, recip 1
            v[1:8] = mids * (1 if (r + grp) % 2 == 0 else -1)
            v[8:15] = -mids
            ties[r, 16 * grp:16 * grp + 16] = v * (2.0 ** (r - 3))
    rows.append(ties)
    rz = np.zeros((8, 128), np.float32)
    for r in range(8):
        amax = np.float32(6.0 * (1.0 + (r + 1) / 16.0))  # scale 1 + k/16: inexact reciprocal
        for grp in range(8):
            v = np.linspace(-amax, amax, 16).astype(np.float32)
            v[3] = np.float32(0.75 * (1.0 + (r + 1) / 16.0))   # near the 0.75 boundary
            v[4] = np.float32(1.75 * (1.0 + (r + 1) / 16.0))
            rz[r, 16 * grp:16 * grp + 16] = v
    rows.append(rz)
    z = np.zeros((4, 128), np.float32)
    z[1] = -0.0
    z[2, :64] = 1e-30
    z[3, ::2] = -1e-3
    rows.append(z)
    x = np.concatenate(rows)
    # bf16 bit patterns (the packer rounds to bf16 first anyway)
    return torch.from_numpy(x).to(torch.bfloat16)


def main() -> int:
    root = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    ref = load_reference(root)
    xb = rows_under_test()
    data, scales = ref.pack_q4_row(xb)
    slot_rows = xb[:128]
    k_region = ref.pack_slot_region_side(slot_rows, 0)
    v_region = ref.pack_slot_region_side(slot_rows, 1)
    out = pathlib.Path(__file__).resolve().parent / "nvfp4_pack_vectors.npz"
    np.savez_compressed(
        out,
        rows_bf16=xb.view(torch.int16).numpy(),
        data=data.numpy(),
        scales=scales.numpy(),
        k_region=k_region.numpy(),
        v_region=v_region.numpy(),
    )
    print(f"wrote {out} ({xb.shape[0]} rows)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
