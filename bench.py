#!/usr/bin/env python3
"""Benchmark: DiT evals/s (8 s audio, CFG batch 2) on one MI355X, plus the 24-step CFG sampler.

Workload (the measured configuration): one 21-block MMDiT velocity evaluation at 8 s — audio rows
La=256, text rows Lt=141 (S=397 joint tokens), B=2 (cond + uncond arm), H=1024, 16 heads x 64,
FFN 4096, 7 joint + 14 fused blocks, BF16 weights ~N(0, 0.02) from seed 4242, synthetic N(0,1)
inputs. A "step" is one evaluation, replayed as a hipGraph with every input already in HBM.

Also reported: the 24-step CFG Euler sampler at the same size (ms, graph replay), per-kernel
statistics of one evaluation (HIP event pairs on the library's stream), the roofline of the
dominant kernel, and the CPU oracle timed on this host as a baseline.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]
"""
import argparse
import importlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2500.0      # MI355X dense FP16/BF16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sampler-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--eager", action="store_true",
                    help="launch kernel by kernel instead of replaying hipGraphs (for profilers that do not follow graphs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (one process, one MI355X); --gpus %d is not supported"
              % args.gpus, file=sys.stderr)
        return 2

    tsn = importlib.import_module("thinksound-native_amd")
    spec = tsn.default_spec(1)
    S = spec.La + spec.Lt
    log("bench: workload one eval, B=%d La=%d Lt=%d S=%d" % (spec.B, spec.La, spec.Lt, S))
    t0 = time.time()
    w16 = tsn.synth_weights(spec, 4242, 0.0)
    log("bench: synthetic weights %.1f s (%d params)" % (time.time() - t0, w16.size))

    rt = tsn.Runtime(0)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(w16)
    inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
    z, tt, text, pooled = (rt.array(inp[k]) for k in ("z", "t", "text", "pooled"))
    v = rt.empty((spec.B, spec.La, spec.latent))

    # ---------------- timed region: K graph replays of one evaluation ----------------
    if args.eager:
        step = lambda: m.forward_ex(z, tt, text, pooled, v)
    else:
        m.capture_forward(z, tt, text, pooled, v)
        step = m.replay
    for _ in range(args.warmup):
        step()
    rt.sync()
    wall0 = time.perf_counter()
    rt.begin()
    for _ in range(args.steps):
        step()
    gpu_ms = rt.commit()
    wall_ms = (time.perf_counter() - wall0) * 1e3
    ms_per_eval = gpu_ms / args.steps
    evals_per_s = 1e3 / ms_per_eval
    log("bench: %d evals in %.3f ms (events), %.3f ms wall -> %.4f ms/eval, %.1f evals/s"
        % (args.steps, gpu_ms, wall_ms, ms_per_eval, evals_per_s))

    # ---------------- per-kernel statistics (one eager eval, warm) ----------------
    stats = None
    for _ in range(3):
        stats = m.profile_forward(z, tt, text, pooled, v)
    stats.sort(key=lambda k: -k["ms"])
    tot_ms = sum(k["ms"] for k in stats)
    for k in stats:
        log("  %-28s %4d launches %8.3f ms  %7.1f TFLOP/s  %7.1f GB/s"
            % (k["name"], k["launches"], k["ms"], k["flops"] / (k["ms"] * 1e9) if k["ms"] else 0,
               k["bytes"] / (k["ms"] * 1e6) if k["ms"] else 0))
    dom = stats[0]
    bound = "mfma" if dom["flops"] > 0 and dom["flops"] / max(dom["bytes"], 1) > 300 else (
        "mfma" if dom["name"].startswith(("gemm", "flash")) else "hbm")
    avg_launch_ms = dom["ms"] / dom["launches"]
    if bound == "mfma":
        achieved = (dom["flops"] / dom["launches"]) / (avg_launch_ms * 1e-3) / 1e12
        peak, unit = PEAK_F16_TFLOPS, "TFLOP/s"
    else:
        achieved = (dom["bytes"] / dom["launches"]) / (avg_launch_ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    eval_flops = sum(k["flops"] for k in stats)

    # ---------------- the 24-step CFG sampler (graph replay) ----------------
    P = spec.B // 2
    x0 = inp["z"][0::2].copy()
    x = rt.array(x0)
    if args.eager:
        run_sampler = lambda: m.sample(x, text, pooled, 24, 5.0)
    else:
        m.capture_sample(x, text, pooled, 24, 5.0)
        run_sampler = m.replay
    run_sampler()
    rt.sync()
    samp = []
    for _ in range(args.sampler_reps):
        x.upload(x0)
        rt.begin()
        run_sampler()
        samp.append(rt.commit())
    sampler_ms = statistics.median(samp)
    log("bench: 24-step sampler %.3f ms (median of %d; min %.3f)" % (sampler_ms, len(samp), min(samp)))

    # ---------------- CPU baseline: the oracle, one full evaluation ----------------
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle
        if not os.path.exists(pyoracle.LIB_PATH):
            pyoracle.build()
        w32 = tsn.bf16_to_f32(w16)
        c0 = time.perf_counter()
        pyoracle.dit_forward(spec, w32, inp["z"], inp["t"], inp["text"], inp["pooled"])
        cpu_s = time.perf_counter() - c0
        cpu = {"value": round(1.0 / cpu_s, 4), "unit": "evals/s", "cores": pyoracle.num_threads(), "kind": "port",
               "sample": "one full 21-block evaluation of the timed workload (B=2, La=256, Lt=141), f32, %.2f s"
                         % cpu_s}
        log("bench: CPU oracle %.2f s per eval on %d threads" % (cpu_s, pyoracle.num_threads()))

    out = {
        "metric": "DiT evals/s (8 s, CFG batch 2); 24-step sampler ms; % BF16 MFMA peak",
        "value": round(evals_per_s, 2),
        "unit": "evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_eval, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) inputs, BF16 N(0,0.02) random-init weights)",
        "config": {"workload": "one 21-block DiT velocity evaluation, 8 s audio, CFG batch 2",
                   "B": spec.B, "La": spec.La, "Lt": spec.Lt, "S": S, "H": spec.H, "heads": spec.NH,
                   "ffn": spec.F, "joint_blocks": spec.n_joint, "fused_blocks": spec.n_fused},
        "sampler_ms": round(sampler_ms, 3),
        "sampler_config": "24 Euler steps, CFG 5.0, 1 prompt x 2 arms, same model and sizes",
        "eval_gflop": round(eval_flops / 1e9, 2),
        "mfma_frac_eval": round(eval_flops / (ms_per_eval * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
        "roofline": {"kernel": dom["name"], "bound": bound, "achieved": round(achieved, 2), "peak": peak,
                     "unit": unit, "frac": round(achieved / peak, 4), "traffic": None,
                     "launches_per_eval": dom["launches"], "avg_launch_us": round(avg_launch_ms * 1e3, 3)},
        "kernels": [{"name": k["name"], "launches": k["launches"], "ms": round(k["ms"], 4),
                     "share": round(k["ms"] / tot_ms, 4)} for k in stats],
        "cpu_baseline": cpu,
        "accumulate": "f32 (f16 MFMA operands from BF16 weights; f32 residual stream)",
        "launch": "eager" if args.eager else "hipGraph replay",
    }
    print(json.dumps(out), flush=True)
    m.close()
    rt.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
