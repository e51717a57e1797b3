#!/usr/bin/env python
"""Benchmark: the ten attention variants at B4 H16 S2048 D64 bf16 on one MI355X.

One step = one call of each of the ten variants (BASELINE.json parameters) on
inputs already resident in HBM: one q, k, v draw shared by the ten, as the
reference's benchmark does.  Prints ONE JSON line on stdout:
  value        whole-step algorithmic TFLOP/s (sum of the ten variants' FLOPs / step time)
  step_distinct_inputs  the same step with a q, k, v draw per variant (cold inputs)
  variants     per variant: us/call (median of 3 event loops, extra_bench.py:8-22),
               cold-cache us/call, TFLOP/s (algorithmic, visited-tile, dense),
               fraction of the bf16 MFMA peak and of the HBM roofline
  roofline     the dominant (slowest) variant's kernel, its average launch
               duration from HIP events around back-to-back loops of it
  northstar    the ten variants at the north-star shape B4 H16 S4096 D64: hot and
               cold us/call, % of bf16 MFMA peak (algorithmic and visited-tile
               FLOPs), % of the HBM roofline (8 TB/s and the measured copy rate),
               and which variants meet the >= 50 % visited-tile target
  cpu_baseline the reference's eager path (restated in oracle/) on the host CPU,
               on a bounded sample, with the GPU output checked on that sample;
               c1_fp32: BASELINE.json configs[0] (fp32 eager softcap) in full
Everything else goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "us/call + TFLOP/s (% bf16 MFMA peak) per variant, B4 H16 S2048 D64 bf16"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_name(op: str, B: int, H: int, S: int, D: int, params: dict) -> str:
    """rocprofv3's name of the kernel instantiation a variant launches."""
    from chia_proj_amd import plan
    from chia_proj_amd.accounting import core_plan_kwargs

    kw = core_plan_kwargs(op, H, params)
    p = plan(batch=B, heads=H, seqlen=S, head_dim=D, **kw)
    norm = {"softmax": 0, "sigmoid": 1, "relu": 2}[kw.get("norm", "softmax")]
    al = "true" if kw["alibi"] else "false"
    sc = "true" if kw.get("softcap", 0) else "false"
    if p["block_n"] == 32:  # the head_dim 128 one-block core
        return f"void chia::attn_fwd_q1_kernel<{D}, {norm}, {al}, {sc}>(chia::FwdParams)"
    return f"void chia::attn_fwd_kernel<{D}, {p['waves']}, {norm}, {al}, {sc}>(chia::FwdParams)"


def load_traffic(suite: str, op: str, kname: str):
    """HBM bytes per launch of `kname` on this suite's `op` workload, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (profiles/traffic.json), if recorded."""
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        rec = json.loads(path.read_text()).get(suite, {}).get(op)
    except (OSError, ValueError, AttributeError):
        return None
    if not rec or rec.get("kernel") != kname:
        return None
    return rec.get("bytes")


def cpu_baseline(cases, inputs, outputs, sample_heads: int = 16, reps: int = 5):
    """The reference's eager bf16 path (oracle.eager_bf16, extra_bench.py:37-50) on the
    host CPU for the first `sample_heads` head(s) of batch 0 of every variant, scaled
    to the full step; the same sample checks the GPU output against the fp32 oracle."""
    import torch

    import oracle  # the checker and the timed CPU path; used only in this leg
    from chia_proj_amd import gate
    from chia_proj_amd.accounting import work

    # one torch thread per core the process may run on; a host that caps its
    # share through OMP_NUM_THREADS (the GPU boxes: 16) is held to that cap
    affinity = len(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(affinity, cap) if cap > 0 else affinity
    torch.set_num_threads(threads)
    threads = torch.get_num_threads()
    total_s = 0.0
    total_flops = 0.0
    checks = {}
    for case in cases:
        q, k, v, params = inputs[case.name]
        B, H, S, D = case.shape
        qs, ks, vs = (t[:1, :sample_heads].cpu() for t in (q, k, v))
        p_sample = oracle.resolve_head_params(case.op, H, params, 0, sample_heads)
        oracle.eager_bf16(case.op, qs, ks, vs, **p_sample)  # warm-up
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            ref_eager = oracle.eager_bf16(case.op, qs, ks, vs, **p_sample)
            ts.append((time.perf_counter_ns() - t0) * 1e-9)
        t_sample = statistics.median(ts)
        scale = (B * H) / sample_heads
        total_s += t_sample * scale
        total_flops += work(case.op, B, H, S, D, params)["flops_alg"]
        ref32 = oracle.variant_ref(case.op, qs, ks, vs, **p_sample)
        got = outputs[case.name][:1, :sample_heads].float().cpu()
        unnorm = (case.op == "sigmoid_attn" and params.get("bias", 0.0) > -1.0) or (
            case.op == "relu_attn" and params.get("post_scale", 1.0) > 0.1)
        g = gate.north_star_gate(ref32, got, scale_aware=unnorm)
        checks[case.op] = {"ok": g.ok, "max_abs": round(g.stats.get("max_abs", float("nan")), 6),
                           "mean_abs": round(g.stats.get("mean_abs", float("nan")), 7),
                           "rel_vs_eager_bf16": round(gate.relerr(ref_eager.float(), got), 6)}
        log(f"  cpu {case.op:22s} sample {t_sample*1e3:8.1f} ms  gate {g.status} {g.stats}")
    return {
        "value": total_flops / total_s / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"each variant's reference bf16 eager path (oracle.eager_bf16, extra_bench.py:37-50) on "
                   f"{sample_heads} of the {cases[0].B * cases[0].H} (batch, head) slices, median of {reps} after 1 "
                   f"warm-up, scaled by B*H/{sample_heads} to the full step; torch CPU threads={threads} "
                   f"(sched_getaffinity: {affinity} cores, OMP_NUM_THREADS cap: {cap or 'none'})"),
        "step_s_scaled": total_s,
        "gate_on_sample": checks,
    }


def measure_cases(cases, calls, works, flusher, copy_gbps=None, tag=""):
    """Per variant: HIP-event median of 3 back-to-back loops (the reference's timer,
    extra_bench.py:8-22), the cold-cache median of single calls after a cache-evicting
    write (when `flusher` is given), TFLOP/s (algorithmic, visited-tile, dense), and
    the fractions of the bf16 MFMA peak and of the HBM roofline -- the 8 TB/s
    specification, and the box's measured copy rate when `copy_gbps` is given."""
    from chia_proj_amd.accounting import PEAK_HBM_GBPS, rates
    from chia_proj_amd.timing import cold_us, median_us

    rows, launch_us = {}, {}
    for c in cases:
        w = works[c.name]
        us = median_us(calls[c.name])
        r = rates(w, us)
        launch_us[c.name] = us
        row = {
            "us": round(us, 2),
            "tflops_alg": round(r["tflops_alg"], 2),
            "tflops_visited": round(r["tflops_visited"], 2),
            "tflops_dense": round(r["tflops_dense"], 2),
            "pct_mfma_peak_alg": round(100 * r["frac_mfma_alg"], 2),
            "pct_mfma_peak_visited": round(100 * r["frac_mfma_visited"], 2),
            "pct_hbm_roofline": round(100 * r["frac_hbm"], 2),
            "pct_roofline": round(100 * r["frac_roofline"], 2),
            "bound": w["bound"],
            "visible_pct": round(100 * w["visible_frac"], 2),
            "tile_wave": w["tile_wave"],
        }
        if copy_gbps:
            row["pct_hbm_copy"] = round(100 * r["gbps"] / copy_gbps, 2)
        if flusher is not None:
            cu = cold_us(calls[c.name], reps=15, flusher=flusher)
            rc = rates(w, cu)
            row["cold_us"] = round(cu, 2)
            row["cold_tflops_alg"] = round(rc["tflops_alg"], 2)
            row["cold_pct_mfma_peak_visited"] = round(100 * rc["frac_mfma_visited"], 2)
            row["cold_pct_hbm_roofline"] = round(100 * rc["frac_hbm"], 2)
            if copy_gbps:
                row["cold_pct_hbm_copy"] = round(100 * rc["gbps"] / copy_gbps, 2)
        rows[c.op] = row
        log(f"  {tag}{c.op:22s} {us:9.1f} us  alg {r['tflops_alg']:7.1f} TF/s ({100*r['frac_mfma_alg']:5.1f}% peak)  "
            f"visited {r['tflops_visited']:7.1f} ({100*r['frac_mfma_visited']:5.1f}%)  "
            f"HBM {100*r['frac_hbm']:5.1f}%  " + (f"cold {row['cold_us']:.1f} us" if "cold_us" in row else ""))
    return rows, launch_us


def prepare_cases(cases, dev):
    """Inputs, calls and work figures for a suite; one q, k, v draw per shape serves
    every variant (extra_bench.py:79-81), each variant keeping its own parameters.
    Also returns per-variant calls on each variant's own draw (cold inputs)."""
    from chia_proj_amd import OPS
    from chia_proj_amd.accounting import work
    from chia_proj_amd.workloads import draw_inputs

    inputs, calls, works, shared, distinct = {}, {}, {}, {}, {}
    for c in cases:
        q, k, v, params = draw_inputs(c, dev)
        distinct[c.name] = (lambda fn=OPS[c.op], q=q, k=k, v=v, p=params: fn(q, k, v, **p))
        q, k, v = shared.setdefault(tuple(q.shape), (q, k, v))
        inputs[c.name] = (q, k, v, params)
        calls[c.name] = (lambda fn=OPS[c.op], q=q, k=k, v=v, p=params: fn(q, k, v, **p))
        works[c.name] = work(c.op, c.B, c.H, c.S, c.D, params)
    return inputs, calls, works, distinct


NORTH_STAR_TARGET_PCT = 50.0  # >= 50 % of bf16 MFMA peak, visited-tile FLOPs


def northstar_report(dev, copy_gbps, cold: bool):
    """The north-star shape (B4 H16 S4096 D64, all ten variants, BASELINE parameters):
    hot and cold-cache us/call, % of the bf16 MFMA peak on algorithmic and visited-tile
    FLOPs, % of the HBM roofline (specification and measured copy), and which variants
    reach the north star's >= 50 % of MFMA peak on visited-tile FLOPs."""
    import torch

    from chia_proj_amd.timing import CacheFlusher
    from chia_proj_amd.workloads import north_star_suite

    cases = north_star_suite()
    log("[bench] north-star shape B4 H16 S4096 D64")
    inputs, calls, works, distinct = prepare_cases(cases, dev)
    del distinct
    flusher = CacheFlusher(device=dev) if cold else None
    rows, launch_us = measure_cases(cases, calls, works, flusher, copy_gbps, tag="ns ")
    del flusher, inputs, calls
    torch.cuda.empty_cache()
    met = [op for op, r in rows.items() if r["pct_mfma_peak_visited"] >= NORTH_STAR_TARGET_PCT]
    step_us = sum(launch_us.values())
    total = sum(w["flops_alg"] for w in works.values())
    return {
        "config": {"workload": "ten attention variants, B4 H16 S4096 D64 bf16, BASELINE.json parameters",
                   "batch": 4, "heads": 16, "seq_len": 4096, "head_dim": 64},
        "target": f">= {NORTH_STAR_TARGET_PCT:.0f}% of bf16 MFMA peak on visited-tile FLOPs (BASELINE.json north_star)",
        "variants": rows,
        "met_target": met,
        "sum_us": round(step_us, 2),
        "tflops_alg_over_sum": round(total / (step_us * 1e-6) / 1e12, 2),
    }


# The reference's published A100-SXM4-40GB latencies at its own shape (B2 H32 S2048 D128,
# reference constants): results/FINAL_flexattention.csv:2-11 (GraphSynth kernels and
# flex_attention).  Context for the reference-shape suite only, not a target.
A100_PUBLISHED_US = {
    "sigmoid_attn": (1073.2, None), "relu_attn": (472.8, None), "temp_perhead": (1863.6, 613.7),
    "bias_alibi": (841.4, 640.7), "bias_dilated": (1816.7, 570.6), "bias_local": (661.6, 402.1),
    "bias_block_diagonal": (289.4, 261.0), "bias_prefix_lm": (1389.7, 556.7), "softcap_gemma2": (901.0, 846.8),
    "bias_sliding_window": (433.0, 226.5),
}


# The reference's published A100 sequence sweep (results/FINAL_seqsweep.csv:2-31,
# GraphSynth kernels at B2 H32 D128): us/call where its status is "generalises",
# None where its kernel failed at that S ("AssertionError").  Context only.
A100_SEQSWEEP_US = {
    "sigmoid_attn": {1024: 312.5, 2048: 1074.1, 4096: 4343.5},
    "relu_attn": {1024: 151.0, 2048: 472.5, 4096: 1662.1},
    "temp_perhead": {1024: 530.2, 2048: 1867.4, 4096: 6892.3},
    "bias_alibi": {1024: 227.5, 2048: 843.1, 4096: 3222.8},
    "bias_dilated": {1024: 497.9, 2048: 1818.2, 4096: 7136.2},
    "bias_local": {1024: None, 2048: 663.0, 4096: None},
    "bias_block_diagonal": {1024: None, 2048: 289.8, 4096: None},
    "bias_prefix_lm": {1024: 663.8, 2048: 1389.6, 4096: 9608.3},
    "softcap_gemma2": {1024: 262.9, 2048: 900.9, 4096: 3329.6},
    "bias_sliding_window": {1024: None, 2048: 432.9, 4096: None},
}


def _load_best_modules():
    """op -> launch_kernel of the glob-compatible <op>_BEST.py modules, found and
    loaded as extra_bench.py:24-27,65-70 does."""
    import glob
    import importlib.util

    loaded = {}
    for path in glob.glob(str(REPO / "chia_proj_amd" / "kernels_mi355x" / "*_BEST.py")):
        bn = os.path.basename(path).replace("_BEST.py", "")
        op = "sigmoid_attn" if bn.startswith("sigmoid_") else bn.split("_gemini")[0]
        spec = importlib.util.spec_from_file_location("k" + str(abs(hash(path))), path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        loaded[op] = mod.launch_kernel
    return loaded


def reference_report(dev, args) -> int:
    """All ten variants at the reference's benchmark shape and constants (B2 H32 D128,
    extra_bench.py:5,32-62), called through the glob-compatible <op>_BEST.py modules
    loaded as extra_bench.py:24-27 loads them; HIP-event median and cold-cache us/call
    beside the reference's published A100 latencies (context, not a target).
    Suite "reference" is its benchmark at S = 2048 (FINAL_flexattention.csv);
    suite "seqsweep" its sequence sweep at S = 1024, 2048, 4096 (extra_bench.py:166-201,
    FINAL_seqsweep.csv), one q, k, v draw per S shared by the ten variants."""
    import torch

    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS, rates, work
    from chia_proj_amd.timing import CacheFlusher, cold_us, median_us
    from chia_proj_amd.workloads import REFERENCE_SWEEP_S, draw_inputs, reference_suite

    sweep = args.suite == "seqsweep"
    seq_lens = REFERENCE_SWEEP_S if sweep else (2048,)
    loaded = _load_best_modules()
    flusher = CacheFlusher(device=dev)
    rows, tot_us, tot_flops = {}, 0.0, 0.0
    for S in seq_lens:
        cases = reference_suite(S)
        q, k, v, _ = draw_inputs(cases[0], dev)
        if args.pmc_mode:  # for rocprofv3 --pmc: each variant twice after a cache flush, nothing timed
            for c in cases:
                for _ in range(2):
                    flusher()
                    loaded[c.op](q, k, v)
            torch.cuda.synchronize()
            continue
        for c in cases:
            fn = lambda f=loaded[c.op]: f(q, k, v)  # noqa: E731
            w = work(c.op, c.B, c.H, c.S, c.D, {})
            us = median_us(fn)
            cu = cold_us(fn, reps=15, flusher=flusher)
            r = rates(w, us)
            row = {"us": round(us, 2), "cold_us": round(cu, 2), "tflops_alg": round(r["tflops_alg"], 2),
                   "pct_mfma_peak_alg": round(100 * r["frac_mfma_alg"], 2)}
            if sweep:
                a100 = A100_SEQSWEEP_US[c.op][S]
                row["a100_graphsynth_us"] = a100
                row["a100_status"] = "generalises" if a100 is not None else "AssertionError"
                rows.setdefault(c.op, {})[str(S)] = row
            else:
                gs, flex = A100_PUBLISHED_US[c.op]
                row.update(a100_graphsynth_us=gs, a100_flex_attention_us=flex)
                rows[c.op] = row
                a100 = gs
            tot_us += us
            tot_flops += w["flops_alg"]
            log(f"  ref {c.op:22s} S{S:5d} {us:9.1f} us (cold {cu:8.1f})  alg {r['tflops_alg']:7.1f} TF/s "
                f"({100 * r['frac_mfma_alg']:5.1f}% peak)   A100 GraphSynth {a100} us")
        del q, k, v
        torch.cuda.empty_cache()
    if args.pmc_mode:
        print(json.dumps({"pmc_mode": True, "suite": args.suite, "seq_lens": list(seq_lens)}), flush=True)
        return 0
    shape = "B2 H32 S{1024,2048,4096} D128" if sweep else "B2 H32 S2048 D128"
    src = "results/FINAL_seqsweep.csv:2-31" if sweep else "results/FINAL_flexattention.csv:2-11"
    print(json.dumps({
        "metric": "reference benchmark shape: us/call + algorithmic TFLOP/s per variant", "unit": "us",
        "higher_is_better": False, "dtype": "bf16", "data": "synthetic (seeded N(0,1), one draw per S for the ten)",
        "n_gpus": 1,
        "config": {"workload": "ten variants through <op>_BEST.py::launch_kernel(q, k, v), reference constants, "
                               f"{shape} bf16", "suite": args.suite},
        "sum_us": round(tot_us, 2), "tflops_alg_over_sum": round(tot_flops / (tot_us * 1e-6) / 1e12, 2),
        "peak_bf16_tflops": PEAK_BF16_TFLOPS,
        "a100_context": f"{src} of the reference (A100-SXM4-40GB): context, not a target",
        "variants": rows,
    }), flush=True)
    return 0


def cpu_baseline_c1(reps: int = 5):
    """BASELINE.json configs[0] on the host: the reference's eager path in fp32 (Gemma-2
    softcap 50, causal, B1 H8 S512 D64; extra_bench.py:37-46,60 with every step in fp32),
    restated in oracle.variant_ref; median of `reps` after one warm-up."""
    import torch

    import oracle  # the timed CPU path of this leg only
    from chia_proj_amd.accounting import work
    from chia_proj_amd.workloads import baseline_configs, draw_inputs

    case = next(c for c in baseline_configs() if c.name.startswith("c1_"))
    q, k, v, params = draw_inputs(case, None, dtype=torch.float32)
    oracle.variant_ref(case.op, q, k, v, heads_per_chunk=case.H, **params)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter_ns()
        oracle.variant_ref(case.op, q, k, v, heads_per_chunk=case.H, **params)
        ts.append((time.perf_counter_ns() - t0) * 1e-9)
    t = statistics.median(ts)
    flops = work(case.op, case.B, case.H, case.S, case.D, params)["flops_alg"]
    log(f"  cpu c1 fp32 softcap 50 B1 H8 S512 D64: {t * 1e6:9.1f} us  {flops / t / 1e9:7.2f} GFLOP/s")
    return {"config": case.name, "dtype": "fp32", "us": round(t * 1e6, 2),
            "tflops_alg": round(flops / t / 1e12, 5), "cores": torch.get_num_threads(),
            "sample": f"the whole configuration (B1 H8 S512 D64), median of {reps} after 1 warm-up"}


def backward_report(cases, inputs, works, args) -> int:
    """Per variant: HIP-event median of torch.autograd.grad(o, (q, k, v), do) -- the
    chia_attn_bwd launches (row statistics, dQ, dK/dV) -- and its algorithmic rate,
    counting the 5 matmuls of the gradient (10 D per visible pair, 2.5x the forward)."""
    import torch

    from chia_proj_amd import OPS
    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS
    from chia_proj_amd.timing import median_us

    rows, total_us, total_flops = {}, 0.0, 0.0
    for c in cases:
        q, k, v, params = inputs[c.name]
        qg, kg, vg = (t.detach().requires_grad_(True) for t in (q, k, v))
        g = torch.Generator("cpu").manual_seed(4242)
        do = torch.randn(q.shape, generator=g).to(torch.bfloat16).to(q.device)
        o = OPS[c.op](qg, kg, vg, **params)
        if args.pmc_mode:  # two backward passes per variant for the counters, nothing timed
            for _ in range(2):
                torch.autograd.grad(o, (qg, kg, vg), do, retain_graph=True)
            torch.cuda.synchronize()
            continue
        us = median_us(lambda: torch.autograd.grad(o, (qg, kg, vg), do, retain_graph=True))
        flops = 2.5 * works[c.name]["flops_alg"]
        tf = flops / (us * 1e-6) / 1e12
        rows[c.op] = {"us": round(us, 2), "tflops_alg": round(tf, 2),
                      "pct_mfma_peak_alg": round(100 * tf / PEAK_BF16_TFLOPS, 2)}
        total_us += us
        total_flops += flops
        log(f"  backward {c.op:22s} {us:9.1f} us  alg {tf:7.1f} TF/s ({100 * tf / PEAK_BF16_TFLOPS:5.1f}% peak)")
    if args.pmc_mode:
        print(json.dumps({"pmc_mode": True, "backward": True, "variants": [c.op for c in cases]}), flush=True)
        return 0
    c0 = cases[0]
    print(json.dumps({
        "metric": "backward (dq, dk, dv) us/call + algorithmic TFLOP/s per variant",
        "value": round(total_flops / (total_us * 1e-6) / 1e12, 2), "unit": "TFLOP/s", "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic", "n_gpus": 1,
        "config": {"workload": f"backward of the ten variants, B{c0.B} H{c0.H} S{c0.S} D{c0.D} bf16",
                   "suite": args.suite},
        "variants": rows,
    }), flush=True)
    return 0


def flex_description(op: str, H: int, params: dict):
    """(score_mod, mask_mod, norm kwargs) for variant `op` with the suite's parameters,
    written as FlexAttention callables (extra_bench.py:85-95 style; sigmoid / ReLU via norm=)."""
    import torch

    p = dict(params)
    causal = lambda b, h, q, k: k <= q  # noqa: E731
    if op == "bias_sliding_window":
        w = p["window"]
        return None, lambda b, h, q, k: (k <= q) & (q - k < w), {}
    if op == "bias_local":
        w = p["window"]
        return None, lambda b, h, q, k: (q - k).abs() < w, {}
    if op == "bias_dilated":
        d, w = p["dilation"], p.get("window", 0)
        return None, lambda b, h, q, k: (k <= q) & ((q - k) % d == 0) & ((q - k < w) if w else (q >= 0)), {}
    if op == "bias_block_diagonal":
        blk, c = p["block"], p.get("causal", True)
        return None, lambda b, h, q, k: (q // blk == k // blk) & ((k <= q) if c else (q >= 0)), {}
    if op == "bias_prefix_lm":
        pre = p["prefix"]
        return None, lambda b, h, q, k: (k <= q) | (k < pre), {}
    if op == "bias_alibi":
        sl = torch.as_tensor(p["slopes"], dtype=torch.float32)
        return (lambda s, b, h, q, k: s + sl[h] * (k - q)), causal, {}
    if op == "softcap_gemma2":
        cap = p["softcap"]
        return (lambda s, b, h, q, k: torch.tanh(s / cap) * cap), causal, {}
    if op == "temp_perhead":
        t = torch.as_tensor(p["temperature"], dtype=torch.float32)
        if p.get("mode", "mul") == "div":
            return (lambda s, b, h, q, k: s / t[h]), causal, {}
        return (lambda s, b, h, q, k: s * t[h]), causal, {}
    if op == "relu_attn":
        return None, (None if not p.get("causal", True) else causal), dict(norm="relu", post_scale=p["post_scale"])
    if op == "sigmoid_attn":
        return None, (None if not p.get("causal", True) else causal), dict(norm="sigmoid", bias=p["bias"])
    raise KeyError(op)


def flex_report(cases, inputs, calls, args) -> int:
    """Per variant: the FlexAttention-style front end (chia_proj_amd.flex) against
    the direct variant call -- compile time of the callables (mask evaluation and
    fit, once) and HIP-event median per call of each path; the compiled call must
    return the direct call's output bit for bit."""
    import time

    import torch

    from chia_proj_amd.flex import create_block_mask, fit_score_mod, flex_attention
    from chia_proj_amd.timing import median_us

    rows = {}
    for c in cases:
        q, k, v, params = inputs[c.name]
        score_mod, mask_mod, norm_kw = flex_description(c.op, c.H, params)
        t0 = time.perf_counter()
        bm = create_block_mask(mask_mod, c.B, c.H, c.S, c.S, device=q.device) if mask_mod is not None else None
        fitted = fit_score_mod(score_mod, c.H, c.S, batch=c.B) if score_mod is not None else None
        compile_ms = (time.perf_counter() - t0) * 1e3
        flex_call = lambda: flex_attention(q, k, v, score_mod=fitted, block_mask=bm, **norm_kw)  # noqa: E731
        same = bool(torch.equal(flex_call(), calls[c.name]()))
        us_flex = median_us(flex_call)
        us_direct = median_us(calls[c.name])
        rows[c.op] = {"flex_us": round(us_flex, 2), "direct_us": round(us_direct, 2),
                      "compile_ms": round(compile_ms, 1), "identical_output": same,
                      "mask": bm.mask_kwargs() if bm is not None else None}
        log(f"  flex {c.op:22s} flex {us_flex:8.1f} us  direct {us_direct:8.1f} us  compile {compile_ms:7.1f} ms  "
            f"identical={same}")
    c0 = cases[0]
    print(json.dumps({
        "metric": "flex_attention front end us/call vs the direct variant call", "unit": "us",
        "higher_is_better": False, "dtype": "bf16", "data": "synthetic", "n_gpus": 1,
        "config": {"workload": f"ten variants as FlexAttention callables, B{c0.B} H{c0.H} S{c0.S} D{c0.D} bf16",
                   "suite": args.suite},
        "variants": rows,
    }), flush=True)
    return 0 if all(r["identical_output"] for r in rows.values()) else 1


def varlen_report(args) -> int:
    """Packed variable-length batch (attention_varlen): causal softmax, H16 D64,
    sequence lengths drawn in [256, 4096] up to 16384 tokens (the north-star
    shape's token count).  HIP-event median per call and algorithmic TFLOP/s
    (4 D per visible pair, summed over sequences), beside the same sequences
    padded to the longest (one fixed-length launch) and launched one by one."""
    import torch

    from chia_proj_amd import attention, attention_varlen, plan
    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS
    from chia_proj_amd.timing import median_us

    H, D, budget = 16, 64, 16384
    g = torch.Generator("cpu").manual_seed(2026)
    lens = []
    while sum(lens) < budget:
        lens.append(min(int(torch.randint(256, 4097, (1,), generator=g)), budget - sum(lens)))
    T, B, S = sum(lens), len(lens), max(lens)
    q, k, v = (torch.randn(T, H, D, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    pairs = sum(plan(batch=1, heads=1, seqlen=L, head_dim=D, causal=True)["pairs_visible"] for L in lens)
    flops = 4.0 * D * pairs * H
    packed = lambda: attention_varlen(q, k, v, cu, S, causal=True)  # noqa: E731
    pads = [torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).cuda().transpose(1, 2) for _ in range(3)]
    for b, (a0, a1) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        for t, src in zip(pads, (q, k, v)):
            t[b, :, :a1 - a0] = src[a0:a1].transpose(0, 1)
    padded = lambda: attention(*pads, causal=True)  # noqa: E731
    seqs = [(q[a:b].transpose(0, 1)[None], k[a:b].transpose(0, 1)[None], v[a:b].transpose(0, 1)[None])
            for a, b in zip(cu[:-1].tolist(), cu[1:].tolist())]
    each = lambda: [attention(*t, causal=True) for t in seqs]  # noqa: E731
    rows = {}
    for name, fn in (("packed", packed), ("padded_to_longest", padded), ("one_launch_per_sequence", each)):
        us = median_us(fn)
        tf = flops / (us * 1e-6) / 1e12
        rows[name] = {"us": round(us, 2), "tflops_alg": round(tf, 2),
                      "pct_mfma_peak_alg": round(100 * tf / PEAK_BF16_TFLOPS, 2)}
        log(f"  varlen {name:26s} {us:9.1f} us  alg {tf:7.1f} TF/s")
    print(json.dumps({
        "metric": "packed variable-length causal softmax, algorithmic TFLOP/s", "value": rows["packed"]["tflops_alg"],
        "unit": "TFLOP/s", "higher_is_better": True, "dtype": "bf16", "data": "synthetic", "n_gpus": 1,
        "config": {"workload": f"{B} sequences of 256..4096 tokens ({T} tokens), H{H} D{D}, causal softmax",
                   "lengths": lens},
        "paths": rows,
    }), flush=True)
    return 0


def fp8_report(cases, inputs, works, args) -> int:
    """Per variant: the FP8 forward (attention_fp8, e4m3 q / k / v quantised per
    tensor from the suite's inputs) against the bf16 forward on the same inputs,
    then the FP8 forward on e5m2 inputs: HIP-event median per call and
    algorithmic TFLOP/s (4 D per visible pair)."""
    import torch

    from chia_proj_amd import OPS, attention_fp8, core_kwargs, quantize_fp8
    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS
    from chia_proj_amd.timing import median_us

    PEAK_FP8_TFLOPS = 2 * PEAK_BF16_TFLOPS
    rows, tot_fp8, tot_bf16, tot_flops = {}, 0.0, 0.0, 0.0
    for c in cases:
        q, k, v, params = inputs[c.name]
        kw = core_kwargs(c.op, c.H, **params)
        (q8, qd), (k8, kd), (v8, vd) = (quantize_fp8(t) for t in (q, k, v))
        us8 = median_us(lambda: attention_fp8(q8, k8, v8, q_descale=qd, k_descale=kd, v_descale=vd, **kw))
        us16 = median_us(lambda: OPS[c.op](q, k, v, **params))
        (q5, qd5), (k5, kd5), (v5, vd5) = (quantize_fp8(t, dtype=torch.float8_e5m2) for t in (q, k, v))
        us5 = median_us(lambda: attention_fp8(q5, k5, v5, q_descale=qd5, k_descale=kd5, v_descale=vd5, **kw))
        flops = works[c.name]["flops_alg"]
        tf8, tf16 = flops / (us8 * 1e-6) / 1e12, flops / (us16 * 1e-6) / 1e12
        rows[c.op] = {"fp8_us": round(us8, 2), "bf16_us": round(us16, 2), "fp8_tflops_alg": round(tf8, 2),
                      "pct_fp8_peak": round(100 * tf8 / PEAK_FP8_TFLOPS, 2), "speedup": round(us16 / us8, 3),
                      "e5m2_us": round(us5, 2)}
        tot_fp8 += us8
        tot_bf16 += us16
        tot_flops += flops
        log(f"  fp8 {c.op:22s} {us8:8.1f} us ({tf8:7.1f} TF/s, {100 * tf8 / PEAK_FP8_TFLOPS:5.1f}% of fp8 peak)"
            f"   bf16 {us16:8.1f} us   x{us16 / us8:5.2f}   e5m2 {us5:8.1f} us")
    c0 = cases[0]
    print(json.dumps({
        "metric": "fp8 forward (e4m3 q, k, v) algorithmic TFLOP/s over the ten variants",
        "value": round(tot_flops / (tot_fp8 * 1e-6) / 1e12, 2), "unit": "TFLOP/s", "higher_is_better": True,
        "dtype": "fp8_e4m3", "data": "synthetic", "n_gpus": 1,
        "config": {"workload": f"ten variants, B{c0.B} H{c0.H} S{c0.S} D{c0.D}, e4m3 per-tensor scales",
                   "suite": args.suite},
        "bf16_same_step_us": round(tot_bf16, 2), "fp8_step_us": round(tot_fp8, 2), "variants": rows,
    }), flush=True)
    return 0


def configs_report(args) -> int:
    """Every BASELINE.json configuration on its own shape (workloads.baseline_configs): HIP-event
    median per call, algorithmic TFLOP/s and % of the bf16 MFMA peak, and the HBM roofline."""
    import torch

    from chia_proj_amd import OPS
    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS, PEAK_HBM_GBPS, work
    from chia_proj_amd.timing import median_us
    from chia_proj_amd.workloads import baseline_configs, draw_inputs

    rows = {}
    for c in baseline_configs():
        q, k, v, params = draw_inputs(c, "cuda")
        fn = lambda: OPS[c.op](q, k, v, **params)  # noqa: E731
        us = median_us(fn)
        w = work(c.op, c.B, c.H, c.S, c.D, params)
        tf = w["flops_alg"] / (us * 1e-6) / 1e12
        gbps = w["bytes"] / (us * 1e-6) / 1e9
        rows[c.name] = {"op": c.op, "shape": [c.B, c.H, c.S, c.D], "us": round(us, 2), "tflops_alg": round(tf, 2),
                        "pct_mfma_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2),
                        "pct_hbm_roofline": round(100 * gbps / PEAK_HBM_GBPS, 2)}
        log(f"  {c.name:36s} {us:9.1f} us  {tf:7.1f} TF/s ({100 * tf / PEAK_BF16_TFLOPS:5.1f}% MFMA, "
            f"{100 * gbps / PEAK_HBM_GBPS:5.1f}% HBM)")
        del q, k, v
        torch.cuda.empty_cache()
    print(json.dumps({"metric": "BASELINE.json configurations: us/call + TFLOP/s per configuration", "unit": "us",
                      "higher_is_better": False, "dtype": "bf16", "data": "synthetic", "n_gpus": 1,
                      "configs": rows}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--suite", default="headline", choices=["headline", "northstar", "reference", "seqsweep"],
                    help="headline: the metric's shape (default); northstar: B4 H16 S4096 D64; reference: the "
                         "reference's own shape and constants through its loader (own JSON line); seqsweep: "
                         "the same at S = 1024, 2048, 4096, as the reference's sequence sweep")
    ap.add_argument("--no-northstar", action="store_true",
                    help="skip the north-star object (B4 H16 S4096 D64) of the default headline run")
    ap.add_argument("--variants", default="", help="comma-separated subset of variants (profiling runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--no-calibration", action="store_true")
    ap.add_argument("--report", default="", help="also write the JSON line to this file")
    ap.add_argument("--backward", action="store_true",
                    help="time the backward (chia_attn_bwd: dq, dk, dv) of each variant instead of the forward step; "
                         "prints its own JSON line (not the headline metric)")
    ap.add_argument("--flex", action="store_true",
                    help="time the FlexAttention-style front end (score_mod / mask_mod callables compiled to the "
                         "core) against the direct variant calls; prints its own JSON line")
    ap.add_argument("--varlen", action="store_true",
                    help="time a packed variable-length batch (attention_varlen) against padding and per-sequence "
                         "launches; prints its own JSON line")
    ap.add_argument("--fp8", action="store_true",
                    help="time the FP8 (e4m3) forward of each variant against the bf16 forward; prints its own "
                         "JSON line")
    ap.add_argument("--configs", action="store_true",
                    help="time every BASELINE.json configuration on its own shape; prints its own JSON line")
    ap.add_argument("--pmc-mode", action="store_true",
                    help="for rocprofv3 --pmc: launch each variant twice after a cache flush, then a calibration "
                         "kernel that reads and writes 512 MiB, and exit (with --backward: two backward passes per variant)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the attention kernels shard over "
                                   "(batch, head) with no exchange, so --gpus N > 1 is not provided"}))
        return 2

    import torch

    from chia_proj_amd.accounting import PEAK_BF16_TFLOPS, PEAK_HBM_GBPS
    from chia_proj_amd.timing import CacheFlusher, copy_calibration
    from chia_proj_amd.workloads import headline_suite, north_star_suite

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.varlen:
        return varlen_report(args)
    if args.configs:
        return configs_report(args)
    if args.suite in ("reference", "seqsweep"):
        return reference_report(dev, args)
    cases = headline_suite() if args.suite == "headline" else north_star_suite()
    if args.variants:
        keep = set(args.variants.split(","))
        cases = [c for c in cases if c.op in keep]
        if not cases:
            raise SystemExit(f"no variant matches {args.variants}")

    log(f"[bench] device {torch.cuda.get_device_name(0)}  suite={args.suite}  variants={len(cases)}")
    inputs, calls, works, distinct = prepare_cases(cases, dev)
    if args.backward:
        return backward_report(cases, inputs, works, args)
    if args.flex:
        return flex_report(cases, inputs, calls, args)
    if args.fp8:
        return fp8_report(cases, inputs, works, args)
    outputs = {c.name: calls[c.name]() for c in cases}
    torch.cuda.synchronize()

    if args.pmc_mode:
        flusher = CacheFlusher(nbytes=1 << 30, device=dev)
        for c in cases:
            for _ in range(2):
                flusher()
                calls[c.name]()
        x = torch.empty(128 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        y = torch.empty_like(x)
        flusher()
        torch.add(x, 1.0, out=y)  # counter calibration: 512 MiB read, 512 MiB written
        torch.cuda.synchronize()
        print(json.dumps({"pmc_mode": True, "variants": [c.op for c in cases], "calibration_bytes": 2 * x.numel() * 4}))
        return 0

    # The box's achievable HBM rate (a copy larger than the Infinity Cache), so the
    # HBM fractions can be stated against it as well as against the 8 TB/s spec.
    calib = None if args.no_calibration else copy_calibration(device=dev)
    if calib:
        log(f"[bench] copy calibration: {calib['GBps']:.0f} GB/s = {100*calib['frac_of_peak']:.1f}% of 8 TB/s")
        if calib["frac_of_peak"] >= 1.0:
            log("[bench] WARNING: copy exceeded 100% of peak: timer not trustworthy")
    copy_gbps = calib["GBps"] if calib else None

    # ---- per-variant: median of 3 event loops (reference timer), cold cache ----
    # Each loop runs one variant back to back between two events, so the
    # per-launch average is the kernel's own duration (rocprofv3 agrees).
    flusher = None if args.no_cold else CacheFlusher(device=dev)
    variants, launch_us = measure_cases(cases, calls, works, flusher, copy_gbps)
    del flusher

    # ---- timed steps: W warm-up, then K steps bracketed by synchronize ----------
    # (after the per-variant loops, which leave the GPU at its working clock)
    # Events only at the two ends: an event recorded between launches is a
    # barrier packet that idles the GPU for a few microseconds.
    for _ in range(args.warmup):
        for c in cases:
            calls[c.name]()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        for c in cases:
            calls[c.name]()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = start.elapsed_time(end) / args.steps
    log(f"[bench] {args.steps} steps: {step_ms:.3f} ms/step (event), wall {wall*1e3/args.steps:.3f} ms/step")

    # The same step with each variant on its own q, k, v: ten inputs of 48 MB
    # (headline) exceed the 256 MB Infinity Cache, so every launch starts cold.
    for _ in range(args.warmup):
        for c in cases:
            distinct[c.name]()
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        for c in cases:
            distinct[c.name]()
    end.record()
    torch.cuda.synchronize()
    step_distinct_ms = start.elapsed_time(end) / args.steps
    del distinct
    log(f"[bench] distinct inputs per variant: {step_distinct_ms:.3f} ms/step")

    # ---- dominant kernel roofline (HIP events around its back-to-back loops) ----
    dom = max(cases, key=lambda c: launch_us[c.name])
    w = works[dom.name]
    avg = launch_us[dom.name]
    kname = kernel_name(dom.op, dom.B, dom.H, dom.S, dom.D, inputs[dom.name][3])
    if w["bound"] == "mfma":
        achieved, peak, unit, per_launch = w["flops_alg"] / (avg * 1e-6) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", w["flops_alg"]
    else:
        achieved, peak, unit, per_launch = w["bytes"] / (avg * 1e-6) / 1e9, PEAK_HBM_GBPS, "GB/s", w["bytes"]
    roofline = {
        "bound": w["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
        "frac": round(achieved / peak, 4), "traffic": load_traffic(args.suite, dom.op, kname),
        "kernel": kname, "variant": dom.op, "avg_launch_us": round(avg, 2),
        "algorithmic_per_launch": per_launch,
    }

    northstar = None
    if args.suite == "headline" and not args.no_northstar and not args.variants:
        northstar = northstar_report(dev, copy_gbps, cold=not args.no_cold)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (reference eager path on the host)")
        cpu = cpu_baseline(cases, inputs, outputs)
        cpu["c1_fp32"] = cpu_baseline_c1()

    total_flops = sum(works[c.name]["flops_alg"] for c in cases)
    c0 = cases[0]
    line = {
        "metric": METRIC,
        "value": round(total_flops / (step_ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v drawn once per shape and shared by the variants, as in the "
                "reference benchmark; BASELINE.json variant parameters)",
        "config": {
            "workload": (f"ten attention variants, one call each per step, B{c0.B} H{c0.H} S{c0.S} D{c0.D} bf16"
                         + (f" (subset: {args.variants})" if args.variants else "")),
            "batch": c0.B, "heads": c0.H, "seq_len": c0.S, "head_dim": c0.D, "suite": args.suite,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "step_distinct_inputs": {"ms_per_step": round(step_distinct_ms, 4),
                                 "value": round(total_flops / (step_distinct_ms * 1e-3) / 1e12, 2),
                                 "note": "each variant on its own q, k, v draw: every launch reads cold inputs"},
        "variants": variants,
        "northstar": northstar,
        "copy_calibration": calib,
        "peak": {"bf16_mfma_tflops": PEAK_BF16_TFLOPS, "hbm_gbps": PEAK_HBM_GBPS},
    }
    text = json.dumps(line)
    print(text, flush=True)
    if args.report:
        Path(args.report).parent.mkdir(parents=True, exist_ok=True)
        Path(args.report).write_text(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
