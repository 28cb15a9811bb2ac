#!/usr/bin/env python3
"""Benchmark of the EXL3 routed-expert decode path on one MI355X.

Workload: one routed-MoE decode layer, 64 experts, top-8,
hidden 2048, per-expert intermediate 1536, fused gate/up + SiLU + down, K3
3INST trellis weights (seeded random bits, random suh/svh), bf16 activations
N(0,1), softmax top-8 routing.  A step is one layer forward for a batch of T
tokens; the headline is T = 16, with T = 1 and 4 reported alongside.  Steps
rotate over ``--layers`` distinct layers (default 5, 1.14 GB of packed
experts), as consecutive layers of a model do, so the 256 MB Infinity Cache
cannot serve a step's weights from the previous step: every step reads its
experts from HBM.

value = packed expert bytes touched per step (distinct routed experts x
3,560,448 B + activations) / time per step, inputs resident in HBM.
roofline = the dominant kernel (the gate/up GEMV) timed live with HIP events
on its launch stream, against the 8 TB/s HBM peak.
cpu_baseline = the CPU oracle's eager per-expert loop (single-threaded dequant
as the reference's host decoder, torch fp32 matmul on all host threads) on a
time-bounded sample of the same routed experts; the other configurations'
CPU legs are reported under ``cpu_baselines``.
"""

from __future__ import annotations

import argparse
import ctypes
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
FP16_PEAK_TFLOPS = 2500.0  # MI355X published dense fp16/bf16 MFMA peak
FP16_FLOP_PER_CLK_CU = 4096  # gfx950: 4 SIMDs x 1024 dense fp16 FLOP per clock
# HBM bytes of one gate/up launch at T=16 (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000,
# factors from a 256 MiB copy), from profiles/moe_decode_c1_t16.md; re-measured
# with rocprofv3 --pmc whenever the kernel changes.
GATE_UP_TRAFFIC_T16 = 141_743_309 + 3_145_728


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def gpu_peaks() -> dict:
    """CU count and peak engine clock of device 0 (hipDeviceGetAttribute),
    and the fp16 dense MFMA peak they give beside the published figure."""
    out = {"published_tflops": FP16_PEAK_TFLOPS}
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        cus, khz = ctypes.c_int(), ctypes.c_int()
        # hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeClockRate (kHz)
        if hip.hipDeviceGetAttribute(ctypes.byref(cus), 63, 0) == 0 and \
                hip.hipDeviceGetAttribute(ctypes.byref(khz), 5, 0) == 0:
            out.update({"cus": cus.value, "peak_clock_mhz": khz.value / 1e3,
                        "fp16_flop_per_clk_cu": FP16_FLOP_PER_CLK_CU,
                        "computed_tflops": round(cus.value * FP16_FLOP_PER_CLK_CU * khz.value * 1e3 / 1e12, 1)})
    except OSError:
        pass
    return out


def step_stats(ms: list) -> dict:
    a = np.asarray(ms)
    return {"mean_ms": float(a.mean()), "median_ms": float(np.median(a)),
            "p95_ms": float(np.percentile(a, 95))}


def graph_time_rot(torch, fns, steps, warmup) -> dict:
    """Per-step times of fns[i % len(fns)] replayed from HIP graphs (one graph
    per function, captured once): every kernel of a step runs on every replay,
    only the host launch overhead is gone, as in a serving decode loop.  The K
    timed steps are bracketed by events (mean) and each has its own pair
    (median, p95)."""
    graphs = []
    for fn in fns:
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        graphs.append(g)
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        ev[i][0].record()
        graphs[i % len(graphs)].replay()
        ev[i][1].record()
    end.record()
    torch.cuda.synchronize()
    st = step_stats([a.elapsed_time(b) for a, b in ev])
    st["mean_ms"] = start.elapsed_time(end) / steps
    del graphs
    return st


def run_batch(C, S, torch, layers, T, steps, warmup, dev, PhaseTimer):
    from vllm_exl3_amd.profiling import MOE_PHASES

    x = torch.from_numpy(S.activations(10 + T, T, H)).to(dev).bfloat16()
    ids_np, w_np = S.softmax_topk(20 + T, T, E, TOPK)
    U = len(set(ids_np.ravel().tolist()))
    ids = torch.from_numpy(ids_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)

    def step_of(layer):
        return lambda: C.moe_forward(x, ids, w, layer, E, I, K=(K, K, K), codebook=CB, out=out)

    fns = [step_of(layer) for layer in layers]
    cnt = [0]

    def rotating():
        fns[cnt[0] % len(fns)]()
        cnt[0] += 1

    ms, _ = time_steps(torch, rotating, steps, warmup)
    st = event_stats(torch, rotating, steps, 1)
    gr = graph_time_rot(torch, fns, steps, warmup)
    _, pt = time_steps(torch, rotating, steps, 1, PhaseTimer)
    step_bytes = U * EXPERT_BYTES + 2 * T * H + 4 * T * H
    gu_bytes = U * 2 * (H * I * K // 8 + 2 * (H + I)) + 2 * T * H  # gate+up trellis, scales, x
    gu_ms = pt.mean_ms(MOE_PHASES.index("gate_up"))
    return {
        "T": T, "distinct_experts": U, "us_per_step": ms * 1e3, "gbs": step_bytes / (ms * 1e-3) / 1e9,
        "median_us": st["median_ms"] * 1e3, "p95_us": st["p95_ms"] * 1e3,
        "graph_us_per_step": gr["mean_ms"] * 1e3, "graph_median_us": gr["median_ms"] * 1e3,
        "phase_us": {n: pt.mean_ms(i) * 1e3 for i, n in enumerate(MOE_PHASES)},
        "gate_up_bytes": gu_bytes, "gate_up_gbs": gu_bytes / (gu_ms * 1e-3) / 1e9,
        "ids": ids_np, "x": x,
    }


def _dequant_f32(O, torch, q, K_, cb):
    return torch.from_numpy(O.dequant(q["trellis"], q["suh"], q["svh"], K_, cb).astype(np.float32))


def cpu_expert_loop(O, torch, experts, ks, cb, ids_np, x, budget_s, max_experts=None):
    """The reference's CPU eager path over the routed experts of a batch, in
    routing order, until the time budget is spent: per expert, the host
    dequant (single-threaded, as csrc/bindings.cpp:15-100) of gate/up/down and
    the fp32 matmuls of the per-expert loop (src/vllm_exl3/exl3.py:2357-2413).
    Returns (experts done, experts routed, dequant s, matmul s, packed bytes)."""
    torch.set_num_threads(os.cpu_count() or 1)
    xf = x.float().cpu().to(torch.float16).float()
    order = []
    for e in ids_np.ravel().tolist():
        if e not in order:
            order.append(e)
    done, nbytes, t_dq, t_mm = 0, 0, 0.0, 0.0
    t0 = time.perf_counter()
    for e in order:
        if max_experts is not None and done >= max_experts:
            break
        pk = experts[e]
        t1 = time.perf_counter()
        w = {p: _dequant_f32(O, torch, pk[p], ks[e], cb) for p in ("gate", "up", "down")}
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
        nbytes += sum(pk[p]["trellis"].nbytes + pk[p]["suh"].nbytes + pk[p]["svh"].nbytes
                      for p in ("gate", "up", "down"))
        if time.perf_counter() - t0 > budget_s:
            break
    return done, len(order), t_dq, t_mm, nbytes


def cpu_baseline(S, O, torch, experts, ids_np, x, budget_s=12.0):
    """C1 (the headline's CPU leg): the per-expert eager loop on a
    time-bounded sample of the T=16 batch's routed experts."""
    done, n, t_dq, t_mm, nbytes = cpu_expert_loop(O, torch, experts, [K] * E, CB, ids_np, x, budget_s)
    total = t_dq + t_mm
    return {
        "value": nbytes / total / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{done} of {n} routed experts of the T={ids_np.shape[0]} batch "
                   f"(dequant of gate/up/down single-threaded {t_dq:.2f} s + fp32 matmul "
                   f"{t_mm:.3f} s on {torch.get_num_threads()} threads; {cpu_model()}, "
                   f"os.cpu_count()={os.cpu_count()})"),
        "dequant_s": round(t_dq, 3), "matmul_s": round(t_mm, 4),
    }


def cpu_baselines(S, O, torch) -> dict:
    """CPU legs of C0, C2, C3 and C4 on the host cores (the reference's CPU
    eager path: single-threaded host dequant, torch fp32 matmul / attention on
    all threads), each on a bounded sample; dequant and matmul timed apart.
    Totals for a whole step are extrapolated from the sample and say so."""
    torch.set_num_threads(os.cpu_count() or 1)
    res = {"cores": torch.get_num_threads(), "cpu": cpu_model(), "os_cpu_count": os.cpu_count()}
    # C0: one 2048x2048 K4 MCG linear, m = 1 and 16
    lin = S.linear(0, 2048, 2048, 4)
    t0 = time.perf_counter()
    w = _dequant_f32(O, torch, lin, 4, 1)
    t_dq = time.perf_counter() - t0
    c0 = {"workload": "C0 2048x2048 K4 MCG", "dequant_s": round(t_dq, 4)}
    for m in (1, 16):
        xm = torch.from_numpy(S.activations(100 + m, m, 2048)).half().float()
        t1 = time.perf_counter()
        for _ in range(20):
            _ = xm @ w
        t_mm = (time.perf_counter() - t1) / 20
        nbytes = 2048 * 2048 * 4 // 8 + 2 * 4096 + 2 * m * 4096
        c0[f"m={m}"] = {"us": round((t_dq + t_mm) * 1e6, 1), "matmul_us": round(t_mm * 1e6, 1),
                        "gbs": round(nbytes / (t_dq + t_mm) / 1e9, 4)}
    res["c0"] = c0
    # C2: routed prefill, E128 K4 MCG, T=2048 Zipf: a sample of experts
    E2, H2, I2, T2 = 128, 4096, 1024, 2048
    ids2, _ = S.zipf_topk(2, T2, E2, TOPK)
    experts2 = S.moe_layer(2, 4, H2, I2, 4)  # the sample's packs (same shapes and K)
    order = []
    for e in ids2.ravel().tolist():
        if e not in order:
            order.append(e)
    x2 = torch.from_numpy(S.activations(2, T2, H2))
    t_dq = t_mm = 0.0
    flops = 0.0
    for i, e in enumerate(order[:4]):
        pk = experts2[i]
        t1 = time.perf_counter()
        ws = {p: _dequant_f32(O, torch, pk[p], 4, 1) for p in ("gate", "up", "down")}
        t2 = time.perf_counter()
        rows = torch.from_numpy(np.nonzero((ids2 == e).any(axis=1))[0])
        h = x2.index_select(0, rows).half().float()
        g = (h @ ws["gate"]).half().float()
        u = (h @ ws["up"]).half().float()
        _ = ((torch.nn.functional.silu(g) * u).half().float()) @ ws["down"]
        t_mm += time.perf_counter() - t2
        t_dq += t2 - t1
        flops += 2.0 * len(rows) * 3 * H2 * I2
    rows_all = np.bincount(ids2.ravel(), minlength=E2)
    per_dq = t_dq / 4
    tot_flops = 2.0 * T2 * TOPK * 3 * H2 * I2
    est_mm = t_mm / flops * tot_flops
    res["c2"] = {"workload": "C2 E128 K4 MCG, T=2048 Zipf", "sample": "4 most-routed experts",
                 "sample_rows": int(sum(rows_all[e] for e in order[:4])),
                 "dequant_s_per_expert": round(per_dq, 3), "matmul_s_sample": round(t_mm, 3),
                 "matmul_tflops": round(flops / t_mm / 1e12, 4),
                 "step_s_extrapolated": round(per_dq * E2 + est_mm, 2),
                 "tflops_extrapolated": round(tot_flops / (per_dq * E2 + est_mm) / 1e12, 5)}
    # C3: mixed-K decode, a K2, a K3 and a K4 expert dequantised
    H3, I3 = 6144, 2048
    ks3 = S.mixed_k(3, 256) + [4]
    per_k = {}
    for kk in (2, 3, 4):
        pk = S.moe_layer(30 + kk, 1, H3, I3, kk)[0]
        t1 = time.perf_counter()
        for p in ("gate", "up", "down"):
            _dequant_f32(O, torch, pk[p], kk, 1)
        per_k[kk] = time.perf_counter() - t1
    ids3, _ = S.softmax_topk(3, 64, 256, TOPK)
    used = sorted(set(ids3.ravel().tolist())) + [256]
    est_dq = sum(per_k[ks3[e]] for e in used)
    nbytes3 = sum(ks3[e] * 3 * H3 * I3 // 8 + 6 * (H3 + I3) for e in used)
    res["c3"] = {"workload": "C3 E256+1 mixed K2/3/4 MCG, T=64",
                 "dequant_s_per_expert": {f"K{kk}": round(v, 3) for kk, v in per_k.items()},
                 "step_s_extrapolated": round(est_dq, 2),
                 "gbs_extrapolated": round(nbytes3 / est_dq / 1e9, 4),
                 "note": "matmul of 64 rows is negligible beside the dequant"}
    # C4: int4 KV decode attention on the CPU, one KV head of one sequence
    # (its 8 query heads): oracle dequant of the int4 cache + fp32 attention
    L4, Hkv4, Hq4 = 32768, 8, 64
    kf, vf = S.kv_inputs(4, 1, 1, L4)
    kq, ksc, kz = O.kv_quantize_rows(kf)
    vq, vsc, vz = O.kv_quantize_rows(vf)
    q = torch.from_numpy(S.activations(4, Hq4 // Hkv4, 128))
    t1 = time.perf_counter()
    kd = torch.from_numpy(O.kv_dequantize_rows(kq, ksc, kz))[0]
    vd = torch.from_numpy(O.kv_dequantize_rows(vq, vsc, vz))[0]
    t2 = time.perf_counter()
    att = torch.softmax((q[None] @ kd.transpose(1, 2)) / 128 ** 0.5, dim=-1)
    _ = att @ vd
    t3 = time.perf_counter()
    n_units = 16 * Hkv4
    res["c4"] = {"workload": "C4 B16 Hq64 Hkv8 d128 L32768 int4 KV",
                 "sample": "1 KV head of 1 sequence (1 of 128 units)",
                 "dequant_s_per_unit": round(t2 - t1, 3), "attention_s_per_unit": round(t3 - t2, 4),
                 "step_s_extrapolated": round(n_units * (t3 - t1), 2),
                 "gbs_extrapolated": round(L4 * 160 / (t3 - t1) / 1e9, 4)}
    return res


# ---------------------------------------------------------------------------
# Other BASELINE configurations, reported beside the headline
# ---------------------------------------------------------------------------


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


def event_stats(torch, fn, steps, warmup) -> dict:
    """Eager per-call times: the K timed calls bracketed by events (mean)
    and each with its own pair (median, p95)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for a, b in ev:
        a.record()
        fn()
        b.record()
    end.record()
    torch.cuda.synchronize()
    st = step_stats([a.elapsed_time(b) for a, b in ev])
    st["mean_ms"] = start.elapsed_time(end) / steps
    return st


def prefill_c2(C, S, torch, dev, steps, warmup, PhaseTimer, zipf_s=1.1, peak_tflops=None):
    """Config 2: routed-MoE prefill, E128 top-8, H4096, I1024, K4 MCG,
    T=2048 tokens with Zipf(s) expert popularity (s = 1.1 as BASELINE names
    it; each token draws 8 distinct experts, so the head experts reach most
    tokens: 16..1848 rows; s = 0.4 gives 70..510 rows, closer to the stated
    ~0..~400 range).  The FLOP count is fixed by T x top-8 either way."""
    E2, H2, I2, T2, K2 = 128, 4096, 1024, 2048, 4
    layer2 = S.moe_layer_device(2, E2, H2, I2, K2, dev)
    ids_np, w_np = S.zipf_topk(2, T2, E2, TOPK, s=zipf_s)
    x = torch.from_numpy(S.activations(2, T2, H2)).to(dev).bfloat16()
    ids = torch.from_numpy(ids_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    out = torch.empty((T2, H2), dtype=torch.float32, device=dev)

    def step():
        C.moe_prefill(x, ids, w, layer2, E2, I2, K=(K2, K2, K2), codebook=1, out=out)

    st = event_stats(torch, step, steps, warmup)
    ms = st["mean_ms"]
    _, pt = time_steps(torch, step, steps, 1, PhaseTimer)
    routes = T2 * TOPK
    flops = 2.0 * routes * (2 * H2 * I2 + I2 * H2)
    gu_flops = 2.0 * routes * 2 * H2 * I2
    names = ("route", "rotate_in", "gate_up_gemm", "act", "down_gemm", "combine")
    phase = {n: pt.mean_ms(i) * 1e3 for i, n in enumerate(names)}
    gemm_us = phase["gate_up_gemm"] + phase["down_gemm"]
    rows = np.bincount(ids_np.ravel(), minlength=E2)
    del layer2
    res = {
        "workload": f"C2 routed-MoE prefill, E{E2} top-{TOPK}, H{H2} I{I2}, K{K2} MCG, T={T2}, Zipf({zipf_s})",
        "us_per_step": round(ms * 1e3, 2),
        "median_us": round(st["median_ms"] * 1e3, 2), "p95_us": round(st["p95_ms"] * 1e3, 2),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_fp16_peak": round(flops / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
        "gemm_tflops": round(flops / (gemm_us * 1e-6) / 1e12, 2),
        "gate_up_gemm_tflops": round(gu_flops / (phase["gate_up_gemm"] * 1e-6) / 1e12, 2),
        "flops_per_step": flops,
        "rows_per_expert": {"min": int(rows.min()), "median": float(np.median(rows)),
                            "max": int(rows.max())},
        "phase_us": {k: round(v, 2) for k, v in phase.items()},
    }
    if peak_tflops:
        res["frac_fp16_peak_computed"] = round(flops / (ms * 1e-3) / 1e12 / peak_tflops, 4)
    return res


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

    ms, _ = time_steps(torch, step, steps, warmup)
    st = event_stats(torch, step, steps, 1)
    gr = graph_time_rot(torch, [step], steps, warmup)
    _, pt = time_steps(torch, step, steps, 1, PhaseTimer)
    used = sorted(set(ids_np.ravel().tolist()))
    nbytes = sum(ks[e] * 3 * H3 * I3 // 8 + 6 * (H3 + I3) for e in used) + 2 * T3 * H3 + 4 * T3 * H3
    del layer3
    return {
        "workload": f"C3 mixed-K MoE decode, E{E3}+1 shared, top-{TOPK}, H{H3} I{I3}, "
                    f"K2/K3/K4 40/40/20 MCG, T={T3}",
        "us_per_step": round(ms * 1e3, 2),
        "median_us": round(st["median_ms"] * 1e3, 2), "p95_us": round(st["p95_ms"] * 1e3, 2),
        "graph_us_per_step": round(gr["mean_ms"] * 1e3, 2),
        "timing": "eager launches of the whole layer step; HIP graph replay also reported",
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
        ms, _ = time_steps(torch, fn, steps, warmup)
        st = event_stats(torch, fn, steps, 1)
        gr = graph_time_rot(torch, [fn], steps, warmup)
        nbytes = 2048 * 2048 * 4 // 8 + 2 * 4096 + 2 * m * 4096
        res[f"m={m}"] = {"us": round(ms * 1e3, 2), "median_us": round(st["median_ms"] * 1e3, 2),
                         "p95_us": round(st["p95_ms"] * 1e3, 2),
                         "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "graph_us": round(gr["mean_ms"] * 1e3, 2)}
    return {"workload": "C0 EXL3 linear 2048x2048, K4 MCG, fp16 x",
            "timing": "eager launches (rotate, GEMV, finish); HIP graph replay also reported", **res}


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
    call = lambda: KV.int4_decode(q, pool, bt, st, Hkv4, scale, out)  # noqa: E731
    ev = event_stats(torch, call, steps, warmup)
    ms = ev["mean_ms"]
    _, pt = time_steps(torch, call, steps, 1, PhaseTimer)
    cache_bytes = B4 * Hkv4 * L4 * 160
    nbytes = cache_bytes + 2 * q.numel() * 2 + bt.numel() * 4
    att_us = pt.mean_ms(0) * 1e3
    del pool
    return {
        "workload": f"C4 int4 paged KV decode attention, B{B4} Hq{Hq4} Hkv{Hkv4} d128, "
                    f"L={L4}, 16-token pages",
        "us_per_step": round(ms * 1e3, 2),
        "median_us": round(ev["median_ms"] * 1e3, 2), "p95_us": round(ev["p95_ms"] * 1e3, 2),
        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": nbytes,
        "attention_kernel_us": round(att_us, 2),
        "attention_kernel_gbs": round(cache_bytes / (att_us * 1e-6) / 1e9, 1),
        "merge_us": round(pt.mean_ms(1) * 1e3, 2),
    }


# The reference's published per-layer prefill times with the fast q4 staging
# and without staging (unquantised cache), GB10 (CHECKIN-Q4KV-1.md:1227-1235
# of the reference): the staging share is their difference.
Q4_REF_PREFILL_MS = {8192: (4.42, 3.99), 16384: (4.45, 4.31), 30720: (5.89, 4.83)}
Q4_STAGE_CAP = 192  # staging rows: 48 MiB at 4 KV heads (the reference's default cap)


def q4_stage_prefill(S, torch, dev, steps, warmup, PhaseTimer):
    """q4 prefill staging (q4_stage_pages) of an 8K / 16K / 30K-token prefix
    at the reference harness's 4 KV heads: every page of the prefix staged
    once, in slices of at most Q4_STAGE_CAP - 1 pages (one launch each),
    from a pool of 256 pages in a random page order."""
    from vllm_exl3_amd import nvfp4_kv as Q

    H, n_pool = 4, 256
    L = n_pool * 128
    k, v = S.kv_inputs_device(7, 1, H, L, dev)
    bt = torch.from_numpy(S.block_table(7, 1, n_pool)).to(dev)
    pool = Q.new_pool(n_pool, H, dev)
    Q.pack_pages(k, v, torch.tensor([L], dtype=torch.int32, device=dev), bt, pool)
    del k, v
    buf = torch.empty((Q4_STAGE_CAP, H, 128, 256), dtype=torch.bfloat16, device=dev)
    page_bytes = H * (2 * 9216 + 128 * 256 * 2)  # read both slots, write the K|V row
    out = {}
    for prefix, (ref_fast, ref_none) in Q4_REF_PREFILL_MS.items():
        nb = prefix // 128
        pages = bt[0, :nb].to(torch.int64)
        slices = [pages[i:i + Q4_STAGE_CAP - 1] for i in range(0, nb, Q4_STAGE_CAP - 1)]

        def call():
            for sl in slices:
                Q.q4_stage_pages(buf, pool, sl)

        ev = event_stats(torch, call, steps, warmup)
        torch.cuda.synchronize()
        with PhaseTimer(max_calls=steps * len(slices)) as pt:
            for _ in range(steps):
                call()
            torch.cuda.synchronize()
        kern_us = pt.mean_ms(0) * 1e3 * len(slices)  # phase 0 is one launch; means are per launch
        nbytes = nb * page_bytes + len(slices) * H * 128 * 256 * 2
        out[f"{prefix // 1024}K"] = {
            "pages": nb, "slices": len(slices),
            "call_us": round(ev["median_ms"] * 1e3, 2), "p95_us": round(ev["p95_ms"] * 1e3, 2),
            "kernel_us": round(kern_us, 2),
            "kernel_gbs": round(nbytes / (kern_us * 1e-6) / 1e9, 1),
            "frac_hbm_peak": round(nbytes / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes": nbytes,
            "ref_gb10_prefill_ms_fast_vs_unstaged": [ref_fast, ref_none],
            "ref_gb10_staging_share_ms": round(ref_fast - ref_none, 2),
        }
    del pool, buf
    return {"workload": "q4 prefill staging (q4_stage_pages), 4 KV heads, 128-token pages, "
                        "prefix pages in random pool order",
            "per_prefix": out}


def q4_sparse_decode_leg(S, torch, dev, steps, warmup, PhaseTimer):
    """NVFP4 block-sparse decode attention (q4_sparse_decode): 64 decode
    sequences, 24 query / 4 KV heads (one rank of a 48 / 8-head model at
    tensor parallel 2), 16 selected 128-token blocks per query token and KV
    head out of a 16,384-token context, pages in random pool order."""
    from vllm_exl3_amd import nvfp4_kv as Q

    B, Hq, Hkv, L, topk = 64, 24, 4, 16384, 16
    n_blocks = L // 128
    k, v = S.kv_inputs_device(9, B, Hkv, L, dev)
    bt = torch.from_numpy(S.block_table(9, B, n_blocks)).to(dev)
    sl = torch.full((B,), L, dtype=torch.int32, device=dev)
    pool = Q.new_pool(B * n_blocks, Hkv, dev)
    Q.pack_pages(k, v, sl, bt, pool)
    del k, v
    g = torch.Generator().manual_seed(10)
    tk = torch.stack([torch.stack([torch.randperm(n_blocks, generator=g)[:topk] for _ in range(B)])
                      for _ in range(Hkv)]).to(torch.int32).to(dev)  # [Hkv, B, topk]
    q = torch.from_numpy(S.activations(11, B * Hq, 128).reshape(B, Hq, 128)).to(dev).bfloat16()
    out = torch.empty_like(q)
    scale = 1.0 / 128 ** 0.5
    call = lambda: Q.q4_sparse_decode(q, pool, tk, bt, sl, Hkv, scale, out, 1)  # noqa: E731
    ev = event_stats(torch, call, steps, warmup)
    _, pt = time_steps(torch, call, steps, 1, PhaseTimer)
    kv_bytes = B * Hkv * topk * 2 * 9216  # K and V slot regions of every selected block
    nbytes = kv_bytes + 2 * q.numel() * 2
    att_us = pt.mean_ms(0) * 1e3
    del pool
    return {
        "workload": f"NVFP4 q4 sparse decode, B{B} Hq{Hq} Hkv{Hkv} d128, top-{topk} of {n_blocks} 128-token "
                    f"blocks per query and KV head",
        "us_per_step": round(ev["mean_ms"] * 1e3, 2),
        "median_us": round(ev["median_ms"] * 1e3, 2), "p95_us": round(ev["p95_ms"] * 1e3, 2),
        "bytes_per_step": nbytes,
        "gbs": round(nbytes / (ev["median_ms"] * 1e-3) / 1e9, 1),
        "decode_kernel_us": round(att_us, 2),
        "decode_kernel_gbs": round(kv_bytes / (att_us * 1e-6) / 1e9, 1),
        "frac_hbm_peak": round(kv_bytes / (att_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
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


def linear_crossover(args) -> int:
    """Median µs of exl3_gemm on its GEMV path and on its fat path (forced by
    EXL3_LINEAR_FAT_MIN_ROWS, which the library reads on every call) for m
    rows, on C0's 2048x2048 K4 MCG weights and a 4096x4096 K3 layer."""
    import torch

    from vllm_exl3_amd import synthetic as S
    from vllm_exl3_amd import vllm_exl3_c as C

    dev = torch.device("cuda", 0)
    for name, n, K_ in (("2048x2048 K4", 2048, 4), ("4096x4096 K3", 4096, 3)):
        lin = S.linear(0, n, n, K_)
        t, su, sv = (torch.from_numpy(lin[k]).to(dev) for k in ("trellis", "suh", "svh"))
        for m in (16, 32, 64, 96, 128, 192, 256, 512, 1024, 2048):
            x = torch.from_numpy(S.activations(m, m, n)).to(dev).half()
            res = {"linear": name, "m": m}
            for kind, rows in (("gemv", str(1 << 30)), ("fat", "1")):
                os.environ["EXL3_LINEAR_FAT_MIN_ROWS"] = rows
                res[kind + "_us"] = round(median_us(torch, lambda: C.exl3_gemm(x, t, su, sv, K_, True),
                                                    20, 3), 2)
            os.environ.pop("EXL3_LINEAR_FAT_MIN_ROWS", None)
            print(json.dumps(res), flush=True)
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
    ap.add_argument("--layers", type=int, default=5,
                    help="distinct C1 layers the decode steps rotate over (HBM-resident weights)")
    ap.add_argument("--configs", default="c0,c2,c3,c4,q4",
                    help="other BASELINE configs reported beside the headline (c0,c2,c3,c4 and q4, the "
                         "q4 prefill staging and sparse decode; '' = none)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    ap.add_argument("--fat-probe", default="", metavar="M,K,N",
                    help="only run the fat GEMM (K4 MCG) on one dense M x K x N problem with "
                         "host-generated inputs, 5 launches, and exit (for rocprofv3 --pmc runs)")
    ap.add_argument("--crossover", action="store_true",
                    help="only time the decode and the prefill executor over a range of T on the "
                         "C1 and C2 layer geometries (the dispatch threshold) and exit")
    ap.add_argument("--linear-crossover", action="store_true",
                    help="only time the dense linear's GEMV and fat paths over a range of m and exit")
    args = ap.parse_args()
    if args.crossover:
        return crossover(args)
    if args.linear_crossover:
        return linear_crossover(args)
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
    layers = [S.to_device(experts, dev)] + [S.moe_layer_device(100 + i, E, H, I, K, dev)
                                            for i in range(1, max(1, args.layers))]
    batches = sorted({int(b) for b in args.batches.split(",")})
    results = {T: run_batch(C, S, torch, layers, T, args.steps, args.warmup, dev, PhaseTimer)
               for T in batches}
    peaks = gpu_peaks()
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
        "timing": "eager launches of the whole layer step on one stream (K steps bracketed by HIP "
                  f"events), steps rotating over {len(layers)} distinct layers "
                  f"({len(layers) * E * EXPERT_BYTES / 1e9:.2f} GB of packed experts, beyond the "
                  "256 MB Infinity Cache); median/p95 from a second pass with an event pair per "
                  "step; HIP-graph replay reported beside it; per-phase kernel times from a third "
                  "eager pass",
        "median_ms_per_step": round(head["median_us"] / 1e3, 6),
        "p95_ms_per_step": round(head["p95_us"] / 1e3, 6),
        "config": {
            "workload": f"C1 routed-MoE decode layer, E64 top-8, H2048 I1536, K3 3INST, bf16 x, T={T_head}",
            "experts": E, "topk": TOPK, "hidden": H, "intermediate": I, "K": K, "codebook": "3INST",
            "tokens": T_head, "distinct_experts": head["distinct_experts"], "layers": len(layers),
        },
        "peaks": {"hbm_gbs": HBM_PEAK_GBS, "fp16": peaks},
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
                       "median_us": round(r["median_us"], 2), "p95_us": round(r["p95_us"], 2),
                       "graph_us_per_step": round(r["graph_us_per_step"], 2),
                       "graph_median_us": round(r["graph_median_us"], 2),
                       "distinct_experts": r["distinct_experts"],
                       "phase_us": {k: round(v, 2) for k, v in r["phase_us"].items()}}
            for T, r in results.items()
        },
    }
    others = {c.strip() for c in args.configs.split(",") if c.strip()}
    if "c0" in others:
        line["linear_c0"] = linear_c0(C, S, torch, dev, args.steps, args.warmup)
    if "c2" in others:
        pk = peaks.get("computed_tflops")
        line["prefill_c2"] = prefill_c2(C, S, torch, dev, max(5, args.steps // 5),
                                        min(args.warmup, 3), PhaseTimer, peak_tflops=pk)
        line["prefill_c2_flat"] = prefill_c2(C, S, torch, dev, max(5, args.steps // 5),
                                             min(args.warmup, 3), PhaseTimer, zipf_s=0.4, peak_tflops=pk)
    if "c3" in others:
        line["mixed_k_c3"] = decode_c3(C, S, torch, dev, args.steps, args.warmup, PhaseTimer)
    if "c4" in others:
        line["kv_decode_c4"] = kv_decode_c4(S, torch, dev, args.steps, args.warmup, PhaseTimer)
    if "q4" in others:
        line["q4_stage"] = q4_stage_prefill(S, torch, dev, args.steps, args.warmup, PhaseTimer)
        line["q4_sparse_decode"] = q4_sparse_decode_leg(S, torch, dev, args.steps, args.warmup, PhaseTimer)
    if not args.no_cpu_baseline:
        import oracle as O

        line["cpu_baseline"] = cpu_baseline(S, O, torch, experts, head["ids"], head["x"])
        if others:
            line["cpu_baselines"] = cpu_baselines(S, O, torch)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
