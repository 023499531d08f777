#!/usr/bin/env python3
"""Benchmark of the GPTQ-2D layer-quantization path on one MI355X.

One step quantizes one layer end to end on the GPU: the two feedback factors
L = ldl_of_inverse(A) and U = ldl_of_inverse(B)^T (blocked HIP Cholesky + triangular inverse, the
two factorisations concurrently on two streams) and the GPTQ-2D sweep of W with the INT4 quantizer fused into the HIP tile sweep.  The workload is the
headline layer of the benchmark definition, "H": W 8192 x 8192 fp32 ~ N(0, 0.02^2) with 0.5%
Student-t(3) x 0.1 outliers, Wishart-like Kronecker factors A, B (G 8192 x 32768 Gaussian, s_i =
i^-0.5, + 1e-2 I), INT4 symmetric per-row static scale (bf16-rounded abs-max of the row / 7.5,
zero point 0).  Inputs are synthetic (seeded numpy PCG64, instances.py) and resident in HBM before
the timed region, which covers --steps full steps after --warmup untimed ones.

Printed: one JSON line with the layer time (``value``, seconds per layer, lower is better), the
per-part breakdown, the roofline of the dominant kernel (the cross-tile feedback panels, fp32,
measured with HIP events around every launch inside the library during the timed steps) and the
CPU baseline: the restated reference PyTorch path (oracle: torch.linalg LDL + ``gptq_2d_torch``)
on the host cores, on a bounded sample (both LDLs in full, an evenly spaced sample of sweep stages
on the full-size tensors, extrapolated to all stages by each stage's exact work).
"""

from __future__ import annotations

import argparse
import functools
import json
import os
import pathlib
import platform
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT / "gptq-2d_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "layer quantize time (s) @8192² INT4; panel MFMA util %; Viterbi weights/s"
FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
# fp32 VALU without packed instructions (which this build does not use): half the published 157.3
# TFLOP/s vector figure, i.e. 78.6 TFLOP/s of FMA = 39.3e12 single fp32 operations per second.
VALU_FP32_OPS_PEAK = 39.3e12
# Outer block of the fused sweep, in antidiagonals (24 tile stages).  A longer outer block moves
# more of the cross-tile feedback into the few large outer flushes, which run closest to the MFMA
# peak, at the price of more in-block prep work per tile stage (whose MFMA pulls slow the in-tile
# sweeps beside them); sweep of the 8192^2 layer on one MI355X, best of four: 512 -> 19.7 ms,
# 640 -> 19.1, 704 -> 19.0, 768 -> 19.1, 832 -> 19.1, 1024 -> 19.6, 1536 -> 21.4, 2048 -> 23.9 ms.
# It changes the order of the fp32 additions only, not the algorithm.
OUTER_BLOCK = 768
# The 8192 x 28672 layers of C5a (1 x 32 super-entry rows, and the three-sided D-sided form) sweep fastest with
# longer blocks: C5a 768 -> 94.4 ms, 1024 -> 94.0, 1280 -> 95.2-95.9, 1536 -> 97.6, 2048 -> 104.3 (2 x 2-tile
# outer flushes; with 4 x 4 ones 1280 had been best at 97.6).
OUTER_BLOCK_WIDE = 1024
# HBM bytes per outer-flush launch at OUTER_BLOCK on the headline layer, mean over a step's 21
# launches: rocprofv3 FETCH_SIZE and WRITE_SIZE passes (one counter per run) over this benchmark,
# each scaled by what the same counter reads for a plain 256 MiB copy kernel in the same run
# (x1.9997 and x1.0000).  Counters cannot be read inside the timed run, so the figure is the
# measured one, with the command and per-kernel values in profiles/flush_traffic_H_int4.md; the
# algorithmic minimum (every operand once) is FLUSH_ALGORITHMIC_BYTES.
FLUSH_TRAFFIC_BYTES = 1.718e9
FLUSH_ALGORITHMIC_BYTES = 0.489e9
# The same two counter passes give the other kernels' HBM bytes, from which the line reports their achieved
# HBM rates against the live timings: a tile-stage launch at OUTER_BLOCK on the headline layer (FETCH_SIZE
# 13703.9 KiB x 1.9997 + WRITE_SIZE 2479.6 KiB, mean over a step's 511 launches) and one Viterbi call of the
# benchmark's search (FETCH_SIZE 132672.3 KiB x 2.0 + WRITE_SIZE 2081294.9 KiB: its step-minimum history);
# profiles/flush_traffic_H_int4.md, profiles/counters_H_int4.md and profiles/viterbi_hyb_counters.md.
TILE_STAGE_TRAFFIC_BYTES = 30.60e6
VITERBI_TRAFFIC_BYTES = 2.403e9
# fp32 VALU operations per trellis state evaluation of the plain search: 2 sub, 2 mul, 1 add (the squared
# distance), 1 add (the predecessor group's minimum), 1 min.
OPS_PER_STATE_EVAL = 7
# The benchmark's HYB table has 1024 distinct row pairs, so the search runs from per-step cost tables: each state
# evaluation gathers its 4-byte cost from LDS (8-byte reads for two states), adds the predecessor minimum and
# takes the running minimum.  Bound: the LDS gathers, against 64 banks x 4 B per clock per CU = 256 CUs x 256 B x
# 2.4 GHz; their random addresses make most LDS cycles bank-conflict stalls (profiles/viterbi_hyb_counters.md).
LDS_BYTES_PER_STATE_EVAL = 4
LDS_PEAK_TBS = 157.3


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="H", help="workload from instances.CONFIGS (default: the headline layer)")
    ap.add_argument("--cpu-stages", type=int, default=4096, help="sweep stages in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--configs", default="C2,C3,H64,C4,C5a,C5a3,C5b",
                    help="comma-separated other configurations to time after the headline layer ('' for none)")
    return ap.parse_args()


def _physical_cores():
    """(physical cores, logical CPUs) among the CPUs this process may run on (from /proc/cpuinfo)."""
    allowed = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else set(range(os.cpu_count() or 1))
    cores, proc, phys, core = set(), None, None, None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                proc, phys, core = int(val), None, None
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            if proc is not None and phys is not None and core is not None and proc in allowed:
                cores.add((phys, core))
                proc = None
    except OSError:
        pass
    return (len(cores) or len(allowed)), len(allowed)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _cpu_baseline(cfg, x, a, b, scale, zp, l_dev, u_dev, stages_in_sample):
    """The reference's PyTorch CPU path (restated in oracle/): LDL of both factors in full, and a sample of
    sweep stages on the full-size tensors extrapolated by exact per-stage work."""
    import torch

    from oracle import algorithms as OA
    from oracle import quantize as OQ
    from oracle import sweep as OS

    cores, logical = _physical_cores()
    threads = cores
    torch.set_num_threads(threads)
    ac, bc = a.cpu(), b.cpu()
    t0 = time.perf_counter()
    OA.ldl_of_inverse(ac)
    t_ldl_a = time.perf_counter() - t0
    t0 = time.perf_counter()
    OA.ldl_of_inverse(bc).t()
    t_ldl_b = time.perf_counter() - t0
    m, n = x.shape
    q = functools.partial(OQ.affine_quantizer, qmin=cfg.qmin, qmax=cfg.qmax)
    state = OS.TorchSweepState(x.cpu(), l_dev.cpu(), u_dev.cpu(), quantizer=q,
                               quantizer_inputs=(scale.cpu(), zp.cpu()))
    stages = m + n - 1
    sample = sorted({int(round(i * (stages - 1) / max(1, stages_in_sample - 1))) for i in range(stages_in_sample)})
    t_sample = 0.
    w_sample = 0
    for s in sample:
        t0 = time.perf_counter()
        state.run_stage(s)
        t_sample += time.perf_counter() - t0
        w_sample += OS.stage_work(m, n, s)
    w_total = sum(OS.stage_work(m, n, s) for s in range(stages))
    t_sweep = t_sample * w_total / w_sample
    value = t_ldl_a + t_ldl_b + t_sweep
    return {
        "value": value,
        "unit": "s/layer",
        "cores": threads,
        "kind": "port",
        "sample": (f"restated reference PyTorch path on {threads} threads ({cores} physical cores of the {logical} "
                   f"logical CPUs this process may use) of {_cpu_model()}: ldl_of_inverse(A) "
                   f"{t_ldl_a:.2f} s and ldl_of_inverse(B) {t_ldl_b:.2f} s in full; gptq_2d_torch {len(sample)} of "
                   f"{stages} stages on the full {m}x{n} tensors ({t_sample:.1f} s), extrapolated by exact "
                   f"per-stage work to {t_sweep:.1f} s"),
        "extrapolated": True,
    }


def _viterbi_bench(torch, dev, steps_timed=10, warmup=3):
    """Throughput of the trellis search on the longest antidiagonal of configuration C4: 512 super-entries
    of 16 x 16 (T = 256) with the HYB code, L = 16, K = 2, V = 2, tail-biting (two passes)."""
    import quantizer_trellis as QT

    rows, T, L, K, V = 512, 256, 16, 2, 2
    table = QT.hyb(L=L, device=dev)
    x = torch.randn(rows, T, generator=torch.Generator().manual_seed(0)).to(dev)
    out = torch.empty_like(x)
    scale = torch.ones(rows, device=dev)
    for _ in range(warmup):  # the clock settles over the first calls
        QT.trellis_quantize_hip(x, table, K, True, out=out, scale=scale)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps_timed):
        QT.trellis_quantize_hip(x, table, K, True, out=out, scale=scale)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / steps_timed / 1e3
    evals = rows * 2 * (T // V) * (1 << L)  # two passes, every state at every step
    hbm = {"traffic": VITERBI_TRAFFIC_BYTES, "traffic_unit": "B per call (rocprofv3, copy-calibrated)",
           "achieved_gbs": VITERBI_TRAFFIC_BYTES / sec / 1e9, "peak_gbs": HBM_PEAK_GBS}
    lds = evals * LDS_BYTES_PER_STATE_EVAL / sec / 1e12
    return {
        "workload": "C4 longest antidiagonal: 512 sequences of 256 (16x16 super-entries), HYB L=16 K=2 V=2, "
                    "tail-biting",
        "weights_per_s": rows * T / sec,
        "ms_per_call": sec * 1e3,
        "state_evals_per_s": evals / sec,
        "roofline": {"bound": "lds", "achieved": lds, "peak": LDS_PEAK_TBS,
                     "unit": "TB/s of 4-byte cost gathers (bank-conflicted random reads)", "frac": lds / LDS_PEAK_TBS},
        # the plain search's ceiling for comparison: 7 fp32 VALU operations per state evaluation
        "plain_search_valu_equivalent": {"achieved": evals * OPS_PER_STATE_EVAL / sec / 1e12,
                                         "peak": VALU_FP32_OPS_PEAK / 1e12, "unit": "Tops/s"},
        "hbm": hbm,
    }


def _tile_stage_line(sweep_ms, flush_ms, m, n):
    launches = (m + 31) // 32 + (n + 31) // 32 - 1
    us = 1e3 * (sweep_ms - flush_ms) / launches
    known = (m, n) == (8192, 8192) and OUTER_BLOCK == 768
    return {
        "launches": launches,
        "us_per_launch": round(us, 2),
        "traffic": TILE_STAGE_TRAFFIC_BYTES if known else None,
        "traffic_unit": "B per launch (rocprofv3, copy-calibrated)",
        "achieved_gbs": round(TILE_STAGE_TRAFFIC_BYTES / (us * 1e-6) / 1e9, 1) if known else None,
        "peak_gbs": HBM_PEAK_GBS,
        "bound": "latency (63 dependent in-tile steps per launch, one barrier each)",
    }


def _timed(torch, fn, steps, warmup=1):
    """Seconds per call of fn (synchronised around the timed calls), after warmup calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _config_lines(torch, dev, h_layer, names, steps=2):
    """Layer time (feedback factors + sweep, each timed on its own) of the other benchmark configurations on
    one GPU: C2 and C3 (fused sweep, affine INT quantizers), C4 (the headline layer's weights and factors in
    16 x 16 super-entries, HYB trellis search per stage), C5a (three-factor layer, 1 x 32 abs-max super-entries,
    fused), C5a3 (the same layer three-sided, D-sided sweep), C5b (eight 2048^2 layers in one captured graph
    replay), H64 (the headline layer in fp64)."""
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import instances
    import quantizer_int as QI

    lines = {}

    def line(workload, t_ldl, t_sweep, **extra):
        return {"workload": workload, "layer_s": round(t_ldl + t_sweep, 5), "factors_ms": round(1e3 * t_ldl, 3),
                "sweep_ms": round(1e3 * t_sweep, 3), **extra}

    for name in [nm for nm in ("C2", "C3") if nm in names]:
        cfg = instances.CONFIGS[name]
        x = instances.weights(cfg.m, cfg.n, cfg.seeds[0], cfg.outliers, cfg.bf16).float().to(dev)
        a = instances.wishart_factor(cfg.m, cfg.alpha, cfg.seeds[1], device=dev).float()
        b = instances.wishart_factor(cfg.n, cfg.alpha, cfg.seeds[2], device=dev).float()
        scale, zp = instances.quantizer_inputs(cfg, x)
        q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
        factors = lambda: LDL.feedback_factors_of_grams(a, b, check=False)
        lo, up = factors()
        t_ldl = _timed(torch, factors, steps)
        t_sw = _timed(torch, lambda: G.gptq_2d(x, lo, up, quantizer=q, quantizer_inputs=(scale, zp),
                                               outer_block_size=OUTER_BLOCK), steps)
        kind = "INT4 asymmetric per (row, 128 columns)" if cfg.quantizer == "int_g128" else (
            f"INT{(cfg.qmax - cfg.qmin + 1).bit_length() - 1} symmetric per row")
        lines[name] = line(f"{cfg.m}x{cfg.n} {kind}, fused sweep", t_ldl, t_sw)
        del x, a, b, scale, zp, lo, up

    x, a, b = h_layer
    m, n = x.shape
    if "H64" in names:
        _h64_line(torch, x, a, b, steps, lines, line)
    if "C4" in names:
        _c4_line(torch, dev, x, a, b, steps, lines, line)
    if "C5a" in names:
        _c5a_line(torch, dev, a, m, steps, lines, line)
    if "C5a3" in names:
        _c5a3_line(torch, dev, steps, lines, line)
    if "C5b" in names:
        _c5b_line(torch, dev, steps, lines, line)
    return lines


def _h64_line(torch, x, a, b, steps, lines, line):
    """The headline layer in fp64 end to end: the fp64 factors (strip Cholesky and inverse products on the fp64
    MFMA GEMM) and the fused fp64 sweep (push-form in-tile sweeps on VALU, flushes on fp64 MFMA)."""
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import instances
    import quantizer_int as QI

    cfg = instances.CONFIGS["H"]
    x64, a64, b64 = x.double(), a.double(), b.double()
    scale, zp = instances.quantizer_inputs(cfg, x64)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    factors = lambda: LDL.feedback_factors_of_grams(a64, b64, check=False)
    lo, up = factors()
    t_ldl = _timed(torch, factors, steps)
    t_sw = _timed(torch, lambda: G.gptq_2d(x64, lo, up, quantizer=q, quantizer_inputs=(scale, zp),
                                           outer_block_size=OUTER_BLOCK), steps)
    lines["H64"] = line(f"{x.size(0)}x{x.size(1)} INT4 symmetric per row in fp64 (factors and sweep)", t_ldl, t_sw)


def _c4_line(torch, dev, x, a, b, steps, lines, line):
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import quantizer_trellis as QT

    m, n = x.shape
    table = QT.hyb(L=16).to(dev)  # the tlut's k-means on the CPU (the pinned table), then moved
    scale = x.pow(2).mean().sqrt() / (0.9 * table.pow(2).mean().sqrt())
    q = functools.partial(QT.trellis_quantizer_super_entry_hip, table=table, K=2)
    factors = lambda: LDL.feedback_factors_of_grams(a, b, super_entry_shape=(16, 16), check=False)
    lo, up = factors()
    t_ldl = _timed(torch, factors, steps)
    t_sw = _timed(torch, lambda: G.gptq_2d_super_entry(x, lo, up, super_entry_shape=(16, 16), quantizer=q,
                                                       quantizer_inputs=(scale,)), 1)
    lines["C4"] = line(f"{m}x{n} HYB trellis L=16 K=2 V=2 tail-biting, 16x16 super-entries, per-stage HIP "
                       "search", t_ldl, t_sw)


def _c5a_line(torch, dev, a, m, steps, lines, line):
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import instances
    import quantizer_int as QI

    cfg = instances.THREE_FACTOR["C5a"]
    n = cfg.n1 * cfg.n2
    w = instances.weights(cfg.m, n, cfg.seeds[0], True, False).float().to(dev)
    a5 = a if cfg.seeds[1] == instances.CONFIGS["H"].seeds[1] and cfg.m == m else (
        instances.wishart_factor(cfg.m, cfg.alpha, cfg.seeds[1], device=dev).float())
    b1 = instances.wishart_factor(cfg.n1, cfg.alpha, cfg.seeds[2], device=dev).float()
    b2 = instances.wishart_factor(cfg.n2, cfg.alpha, cfg.seeds[3], device=dev).float()
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax, dtype=torch.bfloat16)

    def factors5():
        lo5 = LDL.ldl_of_inverse(a5, check=False)
        up5 = G.KroneckerU(LDL.ldl_of_inverse(b1, check=False).t().contiguous(),
                           LDL.ldl_of_inverse(b2, size=cfg.group, check=False).t().contiguous())
        return lo5, up5

    lo, up = factors5()
    t_ldl = _timed(torch, factors5, steps)
    t_sw = _timed(torch, lambda: G.gptq_2d_super_entry(w, lo, up, super_entry_shape=(1, cfg.group), quantizer=q,
                                                       outer_block_size=OUTER_BLOCK_WIDE), steps)
    lines["C5a"] = line(f"{cfg.m}x{n} = {cfg.m}x({cfg.n1}x{cfg.n2}), A (x) B1 (x) B2, INT4 abs-max per 1x{cfg.group} "
                        "super-entry (bf16 scales), fused sweep; U = U_B1 (x) U_B2 read from its two factors", t_ldl,
                        t_sw)


def _c5a3_line(torch, dev, steps, lines, line):
    """C5a's layer as the three-sided tensor X[i, b1, b2] (D-sided sweep), static abs-max INT4 scales per 32
    consecutive b2; factors are the three mode LDLs (A, B1, B2)."""
    import gptq_2d_ldl as LDL
    import gptq_d_sided as DS
    import instances
    import quantizer_int as QI

    cfg = instances.THREE_FACTOR["C5a"]
    x = instances.weights(cfg.m, cfg.n1 * cfg.n2, cfg.seeds[0], True, False).float().view(
        cfg.m, cfg.n1, cfg.n2).to(dev)
    grams = [instances.wishart_factor(k, cfg.alpha, s, device=dev).float()
             for k, s in zip((cfg.m, cfg.n1, cfg.n2), cfg.seeds[1:])]
    scale = instances.abs_max_group_scale(x, cfg.group, cfg.qmin, cfg.qmax)
    zero = torch.zeros_like(x)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    factors = lambda: [LDL.ldl_of_inverse(g, check=False) for g in grams]
    ls = factors()
    t_ldl = _timed(torch, factors, steps)
    t_sw = _timed(torch, lambda: DS.gptq_d_sided(x, ls, quantizer=q, quantizer_inputs=(scale, zero),
                                                 outer_block_size=OUTER_BLOCK_WIDE), steps)
    lines["C5a3"] = line(f"{cfg.m}x{cfg.n1}x{cfg.n2} three-sided (D-sided sweep on the two-sided engine, U = "
                         f"(L_B2 (x) L_B1)^T read from its two factors), static INT4 abs-max scale per {cfg.group} b2 "
                         "(bf16)",
                         t_ldl, t_sw)


def _c5b_line(torch, dev, steps, lines, line):
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import instances
    import quantizer_int as QI

    B, k = 8, 2048
    xb = torch.stack([instances.weights(k, k, 100 + i, True, False) for i in range(B)]).float().to(dev)
    ga = torch.stack([instances.wishart_factor(k, .5, 200 + i, device=dev) for i in range(B)]).float()
    gb = torch.stack([instances.wishart_factor(k, .5, 300 + i, device=dev) for i in range(B)]).float()
    sb = instances.abs_max_row_scale(xb, -8, 7).expand_as(xb).contiguous()
    zb = torch.zeros_like(xb)
    q = functools.partial(QI.affine_quantizer_hip, qmin=-8, qmax=7)
    factors_b = lambda: (LDL.ldl_of_inverse(ga, check=False), LDL.ldl_of_inverse(gb, check=False).transpose(-1, -2))
    lo, up = factors_b()
    up = up.contiguous()
    t_ldl = _timed(torch, factors_b, steps)
    replay = G.capture_gptq_2d(xb, lo, up, quantizer=q, quantizer_inputs=(sb, zb), outer_block_size=OUTER_BLOCK)
    t_sw = _timed(torch, lambda: replay(xb, lo, up, sb, zb), steps)
    lines["C5b"] = line(f"{B} x {k}x{k} INT4 per row, batched factors + one hipGraph replay of the fused sweep "
                        "(input copies included)", t_ldl, t_sw)


def main() -> int:
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the layer quantization runs on a single MI355X (--gpus {args.gpus} "
              "is not supported; independent layers shard across GPUs without any exchange)", file=sys.stderr)
        return 2

    import torch

    import _hip
    import gptq_2d as G
    import gptq_2d_ldl as LDL
    import instances
    import quantizer_int as QI

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = instances.CONFIGS[args.config]
    m, n = cfg.m, cfg.n

    # ---------------------------------------------------------------- inputs, resident in HBM
    w64 = instances.weights(m, n, cfg.seeds[0], cfg.outliers, cfg.bf16)
    x = w64.float().to(dev)
    del w64
    a = instances.wishart_factor(m, cfg.alpha, cfg.seeds[1], device=dev).float()
    b = instances.wishart_factor(n, cfg.alpha, cfg.seeds[2], device=dev).float()
    scale, zp = instances.quantizer_inputs(cfg, x)
    quant = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    torch.cuda.synchronize()

    def step(events=None):
        if events:
            events[0].record()
        lo, up = LDL.feedback_factors_of_grams(a, b, check=False)  # both factors, two streams
        if events:
            events[1].record()
        z = G.gptq_2d(x, lo, up, quantizer=quant, quantizer_inputs=(scale, zp), outer_block_size=OUTER_BLOCK)
        if events:
            events[2].record()
        return z, lo, up

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # ---------------------------------------------------------------- timed region
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    _hip.profile_start(1024, kinds=(_hip.PROF_FLUSH,))  # events only around the dominant kernel
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        z, lo, up = step(events[k])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    flush_ms, flush_flops, flush_n = _hip.profile_read(_hip.PROF_FLUSH)
    _hip.profile_stop()
    ms_per_step = 1e3 * elapsed / args.steps
    parts = {name: statistics.median(ev[i].elapsed_time(ev[i + 1]) for ev in events)
             for i, name in enumerate(("ldl_ms", "sweep_ms"))}

    # ---------------------------------------------------------------- sanity: INT4 codes, objective vs RTN
    codes = z / scale
    assert torch.equal(codes, codes.round()) and codes.min() >= cfg.qmin and codes.max() <= cfg.qmax, "bad codes"
    a64, b64 = a.double(), b.double()

    def objective(zz):
        r = (zz - x).double()
        return float(((a64 @ r) * (r @ b64)).sum())

    rtn = torch.clamp(torch.round(x / scale), cfg.qmin, cfg.qmax) * scale
    obj_ratio = objective(z) / objective(rtn)

    avg_us = 1e3 * flush_ms / max(1, flush_n)
    achieved = flush_flops / max(1, flush_n) / (avg_us * 1e-6) / 1e12 if flush_n else None
    roofline = {
        "bound": "mfma",
        "achieved": achieved,
        "peak": FP32_MFMA_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": achieved / FP32_MFMA_PEAK_TFLOPS if achieved else None,
        "traffic": FLUSH_TRAFFIC_BYTES if (m, n) == (8192, 8192) and OUTER_BLOCK == 768 else None,
        "traffic_unit": "B per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
        "traffic_algorithmic": FLUSH_ALGORITHMIC_BYTES if (m, n) == (8192, 8192) and OUTER_BLOCK == 768 else None,
        "kernel": "cross-tile feedback panels (flush), fp32",
        "launches": flush_n // max(1, args.steps),
        "avg_launch_us": avg_us,
        "flops_per_launch": flush_flops / max(1, flush_n),
    }
    stages = m + n - 1
    result = {
        "metric": METRIC,
        "value": ms_per_step / 1e3,
        "unit": "s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded PCG64 weights and Wishart-like Kronecker factors; no checkpoint)",
        "config": {
            "workload": f"{cfg.name}: {m}x{n} INT4 symmetric per-row static bf16 scale, Wishart-like A, B "
                        f"(s_i = i^-{cfg.alpha:g}, 1e-2 damping); LDL(A) || LDL(B) + fused GPTQ-2D sweep",
            "m": m, "n": n, "stages": stages, "quantizer": "affine INT4 [-8, 7], zero point 0",
            "outer_block_size": OUTER_BLOCK,
        },
        "breakdown": {
            **{k: round(v, 3) for k, v in parts.items()},
            "sweep_us_per_stage": round(1e3 * parts["sweep_ms"] / stages, 3),
            "flush_ms_per_step": round(flush_ms / args.steps, 3),
            "objective_vs_rtn": round(obj_ratio, 5),
        },
        # the tile stages: the sweep less its outer flushes, per launch (launch gaps included), and the HBM
        # rate of their measured bytes per launch
        "tile_stage": _tile_stage_line(parts["sweep_ms"], flush_ms / args.steps, m, n),
        "roofline": roofline,
        "viterbi_weights_per_s": None,
        "viterbi": None,
        "cpu_baseline": None,
    }
    names = [nm for nm in args.configs.split(",") if nm]
    if names:
        result["configs"] = _config_lines(torch, dev, (x, a, b), names)
    vit = _viterbi_bench(torch, dev)
    result["viterbi"] = vit
    result["viterbi_weights_per_s"] = vit["weights_per_s"]
    if not args.no_cpu:
        result["cpu_baseline"] = _cpu_baseline(cfg, x, a, b, scale, zp, lo, up, args.cpu_stages)
        result["gpu_vs_cpu_speedup"] = result["cpu_baseline"]["value"] / result["value"]
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
