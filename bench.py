#!/usr/bin/env python3
"""Benchmark of the EXL3 routed-expert decode path on one MI355X.

Workload: one routed-MoE decode layer, 64 experts, top-8,
hidden 2048, per-expert intermediate 1536, fused gate/up + SiLU + down, K3
3INST trellis weights (seeded random bits, random suh/svh), bf16 activations
N(0,1), softmax top-8 routing.  A step is one layer forward for a batch of T
tokens; the headline is T = 16, with T = 1 and 4 reported alongside.

value = packed expert bytes touched per step (distinct routed experts x
3,560,448 B + activations) / time per step, inputs resident in HBM.
roofline = the dominant kernel (the gate/up GEMV) timed live with HIP events
on its launch stream, against the 8 TB/s HBM peak.
cpu_baseline = the CPU oracle's eager per-expert loop (single-threaded dequant
as the reference's host decoder, torch fp32 matmul on all host threads) on a
time-bounded sample of the same routed experts.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT / "vllm-exl3_amd", ROOT / "oracle"):
    sys.path.insert(0, str(p))

E, H, I, TOPK, K, CB = 64, 2048, 1536, 8, 3, 0
EXPERT_BYTES = 3 * H * I * K // 8 + 2 * 3 * (H + I)  # trellis + suh/svh of 3 projections
HBM_PEAK_GBS = 8000.0
# HBM bytes of one gate/up launch at T=16 (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000,
# factors from a 256 MiB copy), from profiles/moe_decode_c1_t16.md; re-measured
# with rocprofv3 --pmc whenever the kernel changes.
GATE_UP_TRAFFIC_T16 = 144_855_404 + 1_572_864


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def run_batch(C, S, torch, layer, T, steps, warmup, dev, PhaseTimer):
    from vllm_exl3_amd.profiling import MOE_PHASES

    x = torch.from_numpy(S.activations(10 + T, T, H)).to(dev).bfloat16()
    ids_np, w_np = S.softmax_topk(20 + T, T, E, TOPK)
    U = len(set(ids_np.ravel().tolist()))
    ids = torch.from_numpy(ids_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)

    def step():
        C.moe_forward(x, ids, w, layer, E, I, K=(K, K, K), codebook=CB, out=out)

    eager_ms, _ = time_steps(torch, step, steps, warmup)
    ms = graph_time(torch, step, steps, warmup)
    _, pt = time_steps(torch, step, steps, 1, PhaseTimer)
    step_bytes = U * EXPERT_BYTES + 2 * T * H + 4 * T * H
    gu_bytes = U * 2 * (H * I * K // 8 + 2 * (H + I)) + 2 * T * H  # gate+up trellis, scales, x
    gu_ms = pt.mean_ms(MOE_PHASES.index("gate_up"))
    return {
        "T": T, "distinct_experts": U, "us_per_step": ms * 1e3, "gbs": step_bytes / (ms * 1e-3) / 1e9,
        "eager_us_per_step": eager_ms * 1e3,
        "phase_us": {n: pt.mean_ms(i) * 1e3 for i, n in enumerate(MOE_PHASES)},
        "gate_up_bytes": gu_bytes, "gate_up_gbs": gu_bytes / (gu_ms * 1e-3) / 1e9,
        "ids": ids_np, "x": x,
    }


def cpu_baseline(S, O, torch, experts, ids_np, x, budget_s=12.0):
    """The reference's CPU eager path on the routed experts of the batch, in
    routing order, until the time budget is spent: per expert, the host
    dequant (single-threaded, as csrc/bindings.cpp:15-100) of gate/up/down and
    the fp32 matmuls of the per-expert loop (src/vllm_exl3/exl3.py:2357-2413)."""
    import numpy as np

    torch.set_num_threads(os.cpu_count() or 1)
    xf = x.float().cpu().to(torch.float16).float()
    order = []
    for e in ids_np.ravel().tolist():
        if e not in order:
            order.append(e)
    done, nbytes, t_dq, t_mm = 0, 0, 0.0, 0.0
    t0 = time.perf_counter()
    for e in order:
        pk = experts[e]
        t1 = time.perf_counter()
        w = {p: torch.from_numpy(O.dequant(pk[p]["trellis"], pk[p]["suh"], pk[p]["svh"], K, CB)
                                 .astype(np.float32)) for p in ("gate", "up", "down")}
        t2 = time.perf_counter()
        rows = torch.from_numpy(np.nonzero((ids_np == e).any(axis=1))[0])
        h = xf.index_select(0, rows)
        g = (h @ w["gate"]).half().float()
        u = (h @ w["up"]).half().float()
        a = (torch.nn.functional.silu(g) * u).half().float()
        _ = a @ w["down"]
        t3 = time.perf_counter()
        t_dq += t2 - t1
        t_mm += t3 - t2
        done += 1
        nbytes += EXPERT_BYTES
        if time.perf_counter() - t0 > budget_s:
            break
    total = t_dq + t_mm
    return {
        "value": nbytes / total / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{done} of {len(order)} routed experts of the T={ids_np.shape[0]} batch "
                   f"(dequant of gate/up/down single-threaded {t_dq:.2f} s + fp32 matmul "
                   f"{t_mm:.3f} s on {torch.get_num_threads()} threads; {cpu_model()}, "
                   f"os.cpu_count()={os.cpu_count()})"),
    }


# ---------------------------------------------------------------------------
# Other BASELINE configurations, reported beside the headline
# ---------------------------------------------------------------------------
FP16_PEAK_TFLOPS = 2500.0


def time_steps(torch, fn, steps, warmup, PhaseTimer=None):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    pt = None
    if PhaseTimer is not None:
        pt = PhaseTimer(max_calls=steps)
        pt.__enter__()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    if pt is not None:
        pt.__exit__(None, None, None)
    return start.elapsed_time(end) / steps, pt


def graph_time(torch, fn, steps, warmup):
    """Milliseconds per call of fn replayed from a HIP graph: every kernel of
    the step runs on every replay, only the host launch overhead is gone (a
    serving decode loop replays captured steps the same way)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    del g
    return ms


def prefill_c2(C, S, torch, dev, steps, warmup, PhaseTimer):
    """Config 2: routed-MoE prefill, E128 top-8, H4096, I1024, K4 MCG,
    T=2048 tokens with Zipf(1.1) expert popularity."""
    E2, H2, I2, T2, K2 = 128, 4096, 1024, 2048, 4
    layer2 = S.moe_layer_device(2, E2, H2, I2, K2, dev)
    ids_np, w_np = S.zipf_topk(2, T2, E2, TOPK)
    x = torch.from_numpy(S.activations(2, T2, H2)).to(dev).bfloat16()
    ids = torch.from_numpy(ids_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    out = torch.empty((T2, H2), dtype=torch.float32, device=dev)

    def step():
        C.moe_prefill(x, ids, w, layer2, E2, I2, K=(K2, K2, K2), codebook=1, out=out)

    ms, pt = time_steps(torch, step, steps, warmup, PhaseTimer)
    routes = T2 * TOPK
    flops = 2.0 * routes * (2 * H2 * I2 + I2 * H2)
    gu_flops = 2.0 * routes * 2 * H2 * I2
    names = ("route", "rotate_in", "gate_up_gemm", "act", "down_gemm", "combine")
    phase = {n: pt.mean_ms(i) * 1e3 for i, n in enumerate(names)}
    gemm_us = phase["gate_up_gemm"] + phase["down_gemm"]
    rows = np.bincount(ids_np.ravel(), minlength=E2)
    del layer2
    return {
        "workload": f"C2 routed-MoE prefill, E{E2} top-{TOPK}, H{H2} I{I2}, K{K2} MCG, T={T2}, Zipf(1.1)",
        "us_per_step": round(ms * 1e3, 2),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_fp16_peak": round(flops / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
        "gemm_tflops": round(flops / (gemm_us * 1e-6) / 1e12, 2),
        "gate_up_gemm_tflops": round(gu_flops / (phase["gate_up_gemm"] * 1e-6) / 1e12, 2),
        "flops_per_step": flops,
        "rows_per_expert": {"min": int(rows.min()), "max": int(rows.max())},
        "phase_us": {k: round(v, 2) for k, v in phase.items()},
    }


def decode_c3(C, S, torch, dev, steps, warmup, PhaseTimer):
    """Config 3: mixed-K routed-MoE decode, 256 routed experts (40/40/20
    K2/K3/K4, MCG) + 1 shared K4 expert (routed as a ninth slot of weight 1),
    top-8, H6144, I2048, T=64 uniform softmax routing."""
    from vllm_exl3_amd.profiling import MOE_PHASES

    E3, H3, I3, T3 = 256, 6144, 2048, 64
    ks = S.mixed_k(3, E3) + [4]
    layer3 = S.moe_layer_device(3, E3 + 1, H3, I3, ks, dev)
    ids_np, w_np = S.softmax_topk(3, T3, E3, TOPK)
    ids_np = np.concatenate([ids_np, np.full((T3, 1), E3, np.int64)], axis=1)
    w_np = np.concatenate([w_np, np.ones((T3, 1), np.float32)], axis=1)
    x = torch.from_numpy(S.activations(3, T3, H3)).to(dev).bfloat16()
    ids = torch.from_numpy(ids_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    out = torch.empty((T3, H3), dtype=torch.float32, device=dev)

    def step():
        C.moe_forward(x, ids, w, layer3, E3 + 1, I3, K=(4, 4, 4), k_tables=layer3["k_tables"],
                      codebook=1, out=out)

    eager_ms, _ = time_steps(torch, step, steps, warmup)
    ms = graph_time(torch, step, steps, warmup)
    _, pt = time_steps(torch, step, steps, 1, PhaseTimer)
    used = sorted(set(ids_np.ravel().tolist()))
    nbytes = sum(ks[e] * 3 * H3 * I3 // 8 + 6 * (H3 + I3) for e in used) + 2 * T3 * H3 + 4 * T3 * H3
    del layer3
    return {
        "workload": f"C3 mixed-K MoE decode, E{E3}+1 shared, top-{TOPK}, H{H3} I{I3}, "
                    f"K2/K3/K4 40/40/20 MCG, T={T3}",
        "us_per_step": round(ms * 1e3, 2),
        "eager_us_per_step": round(eager_ms * 1e3, 2),
        "timing": "HIP graph replay of the whole layer step; eager launches also reported",
        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": nbytes,
        "distinct_experts": len(used),
        "phase_us": {n: round(pt.mean_ms(i) * 1e3, 2)
                     for i, n in enumerate(MOE_PHASES)},
    }


def linear_c0(C, S, torch, dev, steps, warmup):
    """Config 0 on the GPU: one EXL3 linear 2048x2048, K4 MCG, batch 1 and 16."""
    lin = S.linear(0, 2048, 2048, 4)
    t = torch.from_numpy(lin["trellis"]).to(dev)
    su = torch.from_numpy(lin["suh"]).to(dev)
    sv = torch.from_numpy(lin["svh"]).to(dev)
    res = {}
    for m in (1, 16):
        x = torch.from_numpy(S.activations(100 + m, m, 2048)).to(dev).half()
        fn = lambda: C.exl3_gemm(x, t, su, sv, 4, True)  # noqa: E731
        eager_ms, _ = time_steps(torch, fn, steps, warmup)
        ms = graph_time(torch, fn, steps, warmup)
        nbytes = 2048 * 2048 * 4 // 8 + 2 * 4096 + 2 * m * 4096
        res[f"m={m}"] = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "eager_us": round(eager_ms * 1e3, 2)}
    return {"workload": "C0 EXL3 linear 2048x2048, K4 MCG, fp16 x",
            "timing": "HIP graph replay (rotate, GEMV, finish); eager launches also reported", **res}


def kv_decode_c4(S, torch, dev, steps, warmup, PhaseTimer):
    """Config 4: int4 paged KV-cache decode attention, B16, Hq64, Hkv8, d128,
    32768 cached tokens per sequence in 16-token pages, random block table."""
    from vllm_exl3_amd import kv_int4 as KV

    B4, Hq4, Hkv4, L4 = 16, 64, 8, 32768
    max_pages = L4 // 16
    k, v = S.kv_inputs_device(4, B4, Hkv4, L4, dev)
    bt = torch.from_numpy(S.block_table(4, B4, max_pages)).to(dev)
    st = torch.full((B4,), L4, dtype=torch.int32, device=dev)
    pool = KV.new_pool(B4 * max_pages, Hkv4, dev)
    KV.pack_pages(k, v, st, bt, pool)
    del k, v
    q = torch.from_numpy(S.activations(4, B4 * Hq4, 128).reshape(B4, Hq4, 128)).to(dev).bfloat16()
    out = torch.empty_like(q)
    scale = 1.0 / 128 ** 0.5
    ms, pt = time_steps(torch, lambda: KV.int4_decode(q, pool, bt, st, Hkv4, scale, out),
                        steps, warmup, PhaseTimer)
    cache_bytes = B4 * Hkv4 * L4 * 160
    nbytes = cache_bytes + 2 * q.numel() * 2 + bt.numel() * 4
    att_us = pt.mean_ms(0) * 1e3
    del pool
    return {
        "workload": f"C4 int4 paged KV decode attention, B{B4} Hq{Hq4} Hkv{Hkv4} d128, "
                    f"L={L4}, 16-token pages",
        "us_per_step": round(ms * 1e3, 2),
        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": nbytes,
        "attention_kernel_us": round(att_us, 2),
        "attention_kernel_gbs": round(cache_bytes / (att_us * 1e-6) / 1e9, 1),
        "merge_us": round(pt.mean_ms(1) * 1e3, 2),
    }


def crossover(args) -> int:
    """Median µs per call of moe_forward (decode executor) and moe_prefill
    (prefill executor) for T tokens, softmax top-8 routing, on two layer
    geometries; one JSON line per (geometry, T)."""
    import torch

    from vllm_exl3_amd import synthetic as S
    from vllm_exl3_amd import vllm_exl3_c as C

    dev = torch.device("cuda", 0)
    geoms = [("C1", 64, 2048, 1536, 3, 0), ("C2", 128, 4096, 1024, 4, 1)]
    for name, E_, H_, I_, K_, cb in geoms:
        layer = S.moe_layer_device(11, E_, H_, I_, K_, dev)
        for T in (8, 16, 32, 48, 64, 96, 128, 192, 256, 384, 512, 1024):
            x = torch.from_numpy(S.activations(T, T, H_)).to(dev).bfloat16()
            ids_np, w_np = S.softmax_topk(T, T, E_, TOPK)
            ids = torch.from_numpy(ids_np).to(dev)
            w = torch.from_numpy(w_np).to(dev)
            out = torch.empty((T, H_), dtype=torch.float32, device=dev)
            res = {"geometry": name, "T": T}
            for kind, fn in (("decode", C.moe_forward), ("prefill", C.moe_prefill)):
                call = lambda: fn(x, ids, w, layer, E_, I_, K=(K_, K_, K_), codebook=cb, out=out)  # noqa: E731
                res[kind + "_us"] = round(median_us(torch, call, 20, 3), 2)
            print(json.dumps(res), flush=True)
        del layer
        torch.cuda.empty_cache()
    return 0


def median_us(torch, fn, n, warmup):
    """Median of n single-call times (HIP events around each call)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in ev])) * 1e3


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batches", default="1,4,16",
                    help="decode batch sizes T to run; the headline is the largest")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", default="c0,c2,c3,c4",
                    help="other BASELINE configs reported beside the headline (c0,c2,c3,c4; '' = none)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    ap.add_argument("--fat-probe", default="", metavar="M,K,N",
                    help="only run the fat GEMM (K4 MCG) on one dense M x K x N problem with "
                         "host-generated inputs, 5 launches, and exit (for rocprofv3 --pmc runs)")
    ap.add_argument("--crossover", action="store_true",
                    help="only time the decode and the prefill executor over a range of T on the "
                         "C1 and C2 layer geometries (the dispatch threshold) and exit")
    args = ap.parse_args()
    if args.crossover:
        return crossover(args)
    if args.fat_probe:
        import numpy as np
        import torch

        sys.path.insert(0, str(ROOT / "vllm-exl3_amd"))
        from vllm_exl3_amd import synthetic as S
        from vllm_exl3_amd import vllm_exl3_c as C

        M, Kd, N = (int(v) for v in args.fat_probe.split(","))
        lin = S.linear(7, Kd, N, 4)
        dev = torch.device("cuda", 0)
        a = torch.from_numpy(S.activations(8, M, Kd)).to(dev).half()
        t = torch.from_numpy(lin["trellis"]).to(dev)
        sv = torch.from_numpy(lin["svh"]).to(dev)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        C.exl3_fat_gemm(a, t, out, sv, 4, True, False)
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(5):
            C.exl3_fat_gemm(a, t, out, sv, 4, True, False)
        ev[1].record()
        torch.cuda.synchronize()
        us = ev[0].elapsed_time(ev[1]) / 5 * 1e3
        print(json.dumps({"fat_probe": [M, Kd, N], "launches": 6, "us_per_launch": round(us, 2),
                          "tflops": round(2 * M * Kd * N / us / 1e6, 1)}), flush=True)
        return 0
    if args.copy_probe:
        import torch

        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 5}), flush=True)
        return 0
    if args.gpus != 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(the routed-expert layer would shard by expert; no collectives are built)", file=sys.stderr)
        return 2
    import torch

    from vllm_exl3_amd import synthetic as S
    from vllm_exl3_amd import vllm_exl3_c as C
    from vllm_exl3_amd.profiling import PhaseTimer

    dev = torch.device("cuda", 0)
    experts = S.moe_layer(1, E, H, I, K)
    layer = S.to_device(experts, dev)
    batches = sorted({int(b) for b in args.batches.split(",")})
    results = {T: run_batch(C, S, torch, layer, T, args.steps, args.warmup, dev, PhaseTimer)
               for T in batches}
    T_head = batches[-1]
    head = results[T_head]
    line = {
        "metric": "MoE-layer decode µs + packed-weight HBM GB/s; prefill TFLOP/s (EXL3 K2–K4)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "timing": "HIP graph replay of the whole layer step (route, rotate, gate/up, act, down, "
                  "combine); per-phase kernel times from a separate eager pass",
        "config": {
            "workload": f"C1 routed-MoE decode layer, E64 top-8, H2048 I1536, K3 3INST, bf16 x, T={T_head}",
            "experts": E, "topk": TOPK, "hidden": H, "intermediate": I, "K": K, "codebook": "3INST",
            "tokens": T_head, "distinct_experts": head["distinct_experts"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_wg_kernel<3INST, gate/up>",
            "achieved": round(head["gate_up_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["gate_up_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": GATE_UP_TRAFFIC_T16 if T_head == 16 else None,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, profiles/moe_decode_c1_t16.md",
            "bytes_per_launch": head["gate_up_bytes"],
            "us_per_launch": round(head["phase_us"]["gate_up"], 3),
        },
        "per_batch": {
            f"T={T}": {"us_per_step": round(r["us_per_step"], 2), "GB/s": round(r["gbs"], 1),
                       "eager_us_per_step": round(r["eager_us_per_step"], 2),
                       "distinct_experts": r["distinct_experts"],
                       "phase_us": {k: round(v, 2) for k, v in r["phase_us"].items()}}
            for T, r in results.items()
        },
    }
    others = {c.strip() for c in args.configs.split(",") if c.strip()}
    if "c0" in others:
        line["linear_c0"] = linear_c0(C, S, torch, dev, args.steps, args.warmup)
    if "c2" in others:
        line["prefill_c2"] = prefill_c2(C, S, torch, dev, max(5, args.steps // 5),
                                        min(args.warmup, 3), PhaseTimer)
    if "c3" in others:
        line["mixed_k_c3"] = decode_c3(C, S, torch, dev, args.steps, args.warmup, PhaseTimer)
    if "c4" in others:
        line["kv_decode_c4"] = kv_decode_c4(S, torch, dev, args.steps, args.warmup, PhaseTimer)
    if not args.no_cpu_baseline:
        import oracle as O

        line["cpu_baseline"] = cpu_baseline(S, O, torch, experts, head["ids"], head["x"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
