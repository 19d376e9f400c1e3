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
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2500.0      # MI355X dense FP16/BF16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
PEAK_F32_TFLOPS = 157.3       # MI355X dense FP32 MFMA
PEAK_CLK_GHZ = 2.4            # MI355X peak engine clock (2.5 PF = 256 CUs x 4096 flop/clock x 2.4 GHz)
CAL_COPY_FLOATS = 16 << 20    # calibration copy: 64 MiB read + 64 MiB written
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_dit_eval_b2_la256.txt")
CPU_SAMPLE_S = 10.0           # CPU baseline: whole evaluations until this much time has passed


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _demangled_tail(mangled):
    """last component (with integer template arguments) of an Itanium nested name: _ZN..k..ILi1ELi4EE.. -> k<1, 4>"""
    i, name, args = 3, mangled, []
    while i < len(mangled) and mangled[i].isdigit():
        j = i
        while mangled[j].isdigit():
            j += 1
        n = int(mangled[i:j])
        name, args, i = mangled[j:j + n], [], j + n
        if mangled.startswith("IL", i):   # integer template arguments L<type><value>E ... E
            i += 1
            while mangled.startswith("L", i):
                e = mangled.index("E", i)
                args.append(mangled[i + 2:e].replace("n", "-"))
                i = e + 1
            i += 1
    return name + ("<%s>" % ", ".join(args) if args else "")


def short_kernel_name(full):
    """'void ns::(anonymous namespace)::k<1, 4>(Args)' -> 'k<1, 4>' (the library's own kernel names)."""
    if full.startswith("_ZN"):
        return _demangled_tail(full)
    depth, end = 0, len(full)
    for i, ch in enumerate(full):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and i > 0 and full[i - 1] != ":":
            end = i
            break
    name = full[:end].strip()
    if name.startswith("void "):
        name = name[5:]
    depth, cut = 0, 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == ":" and depth == 0:
            cut = i + 1
    return name[cut:]


def read_counter_csv(path, counter):
    """Per-dispatch values of one counter from a rocprofv3 counter-collection CSV -> {kernel: [values]}."""
    import csv
    out = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            out.setdefault(short_kernel_name(row["Kernel_Name"]), []).append(float(row["Counter_Value"]))
    return out


def pmc_summary(fetch_csv, write_csv, cmd):
    """Text summary of FETCH_SIZE / WRITE_SIZE (KiB per dispatch) per kernel, scaled by the ratio of
    the calibration copy's known bytes to what the same counter reads for it."""
    fetch = read_counter_csv(fetch_csv, "FETCH_SIZE")
    write = read_counter_csv(write_csv, "WRITE_SIZE")
    cal_kib = CAL_COPY_FLOATS * 4 / 1024.0
    cf = cal_kib / statistics.mean(fetch["copy_kernel"])
    cw = cal_kib / statistics.mean(write["copy_kernel"])
    lines = ["# HBM traffic per dispatch, one 21-block DiT evaluation (B=2, La=256, Lt=141, S=397)",
             "# commands (rocprofv3 counter passes, one counter each):",
             "#   " + cmd.replace("{C}", "FETCH_SIZE"),
             "#   " + cmd.replace("{C}", "WRITE_SIZE"),
             "# calibration: copy_kernel of %d MiB read + %d MiB written reads FETCH %.1f KiB, WRITE %.1f KiB"
             % (cal_kib / 1024, cal_kib / 1024, statistics.mean(fetch["copy_kernel"]),
                statistics.mean(write["copy_kernel"])),
             "# scale factors: fetch %.4f, write %.4f (traffic = FETCH*1024*fetch_scale + WRITE*1024*write_scale)"
             % (cf, cw),
             "%-28s %10s %14s %14s %16s" % ("kernel", "dispatches", "FETCH KiB/d", "WRITE KiB/d", "traffic B/d")]
    for k in sorted(set(fetch) & set(write), key=lambda n: -statistics.mean(fetch[n])):
        fk, wk = statistics.mean(fetch[k]), statistics.mean(write[k])
        lines.append("%-28s %10d %14.1f %14.1f %16.0f" % (k, len(fetch[k]), fk, wk, fk * 1024 * cf + wk * 1024 * cw))
    return "\n".join(lines) + "\n"


def read_traffic(kernel):
    """traffic (HBM bytes per dispatch) of a kernel from the committed counter summary, or None"""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.rsplit(None, 4)
                if not line.startswith("#") and len(parts) == 5 and parts[0] == kernel:
                    return float(parts[4])
    except OSError:
        pass
    return None


def stats_summary(stats_csv, cmd, title="eager launches of the DiT evaluation (B=2, La=256, Lt=141, S=397)"):
    """Text summary of a rocprofv3 --kernel-trace --stats kernel_stats.csv"""
    import csv
    rows = []
    with open(stats_csv, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((short_kernel_name(r["Name"]), int(r["Calls"]), float(r["TotalDurationNs"]) / 1e6,
                         float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3,
                         float(r["Percentage"])))
    lines = ["# rocprofv3 kernel statistics, " + title,
             "# command: " + cmd,
             "%-28s %8s %12s %10s %10s %10s %7s" % ("kernel", "calls", "total ms", "avg us", "min us", "max us", "%")]
    for r in sorted(rows, key=lambda r: -r[2]):
        lines.append("%-28s %8d %12.3f %10.3f %10.3f %10.3f %7.2f" % r)
    return "\n".join(lines) + "\n"


def profile_pass(which):
    """workload for rocprofv3 --kernel-trace: eager launches only. vae: five 8 s decodes (T=172);
    enc: five CLIP and five T5 encodes of 77 tokens at the reference sizes; ref: five evaluations
    of the reference checkpoint's graph at 8 s, B = 2 (one CFG pair)"""
    tsn = importlib.import_module("thinksound-native_amd")
    rt = tsn.Runtime(0)
    if which == "ref":
        spec = tsn.ref_spec_for_duration(8, 2)
        m = tsn.RefDitModel(rt, spec)
        m.upload_weights(tsn.ref_synth_weights(spec, 4242, 0.0))
        inp = tsn.ref_synth_inputs(spec, 4242, cfg_pairs=True)
        d = {k: rt.array(v) for k, v in inp.items()}
        v = rt.empty((spec.B, spec.T, spec.latent))
        for i in range(5):
            m.forward_ex(d["x"], d["t"], d["clip_pp"], d["text_pp"], d["gcmlp"], d["sync_gather"], v)
            rt.sync()
            log("profile pass: reference graph eval %d done" % i)
        m.close()
    elif which == "vae":
        spec = tsn.vae_spec_for_duration(8)
        m = tsn.VaeModel(rt, spec)
        m.upload_weights(tsn.vae_synth_weights(spec, 4242))
        z = rt.array(tsn.synth_normal_f32(4242, 2000, 0.0, 1.0, (spec.T, spec.latent)))
        a = rt.empty((tsn.vae_audio_len(spec), spec.out_ch))
        for i in range(5):
            m.decode(z, a)
            rt.sync()
            log("profile pass: vae decode %d done" % i)
        m.close()
    else:
        for name, spec, synth, cls in (("clip", tsn.clip_spec_default(), tsn.clip_synth_weights, tsn.ClipModel),
                                       ("t5", tsn.t5_spec_default(), tsn.t5_synth_weights, tsn.T5Model)):
            m = cls(rt, spec)
            m.upload_weights(synth(spec, 4242))
            ids = np.arange(spec.ctx, dtype=np.int32) % (spec.vocab - 1) + 1
            width = spec.H if name == "clip" else spec.d
            a, g = rt.empty((spec.ctx, width)), rt.empty((width,))
            for i in range(5):
                if name == "clip":
                    m.encode(ids, a, g)
                else:
                    m.encode(ids, a)
                rt.sync()
                log("profile pass: %s encode %d done" % (name, i))
            m.close()
    rt.close()
    return 0


PMC_WORKLOADS = {"8s": 1, "b16": 4, "30s": 3}   # counter-pass workload -> tsn_dit_default_spec index


def pmc_pass(which="8s"):
    """workload for counter runs: three eager evaluations of the 8 s (B = 2), batch-16 or 30 s
    workload, each followed by a calibration copy of 64 MiB"""
    import numpy as np
    tsn = importlib.import_module("thinksound-native_amd")
    spec = tsn.default_spec(PMC_WORKLOADS[which])
    rt = tsn.Runtime(0)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(tsn.synth_weights(spec, 4242, 0.0))
    inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
    z, tt, text, pooled = (rt.array(inp[k]) for k in ("z", "t", "text", "pooled"))
    v = rt.empty((spec.B, spec.La, spec.latent))
    a = rt.array(np.ones(CAL_COPY_FLOATS, np.float32))
    b = rt.empty((CAL_COPY_FLOATS,))
    for i in range(3):
        m.forward_ex(z, tt, text, pooled, v)
        rt.copy(a, b, CAL_COPY_FLOATS)
        rt.sync()
        log("pmc pass %s: eval %d done" % (which, i))
    m.close()
    rt.close()
    return 0


N_SIMD = 1024   # 256 CUs x 4 SIMDs
N_XCC = 8


def read_counter_rows(path):
    """{kernel: {counter: [values per dispatch]}, plus '__dur_ns': [durations]} from a counter CSV"""
    import csv
    out = {}
    seen = set()
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            k = short_kernel_name(row["Kernel_Name"])
            d = out.setdefault(k, {})
            d.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
            key = (row["Dispatch_Id"], k)
            if key not in seen:
                seen.add(key)
                d.setdefault("__dur_ns", []).append(float(row["End_Timestamp"]) - float(row["Start_Timestamp"]))
    return out


def pmc_util_summary(sq_csv, dram_csv, title, cmd):
    """Per-kernel MFMA utilisation (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x 1024 SIMDs, the
    MfmaUtil metric), executed f16 MFMA flops (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512), instruction mix, and
    memory-side traffic (TCC_EA0_RDREQ_DRAM / WRREQ_DRAM requests, scaled to bytes by the 64 MiB
    calibration copy) per dispatch."""
    sq, dr = read_counter_rows(sq_csv), read_counter_rows(dram_csv)
    mean = statistics.mean
    cal_bytes = CAL_COPY_FLOATS * 4.0
    rd_b = cal_bytes / mean(dr["copy_kernel"]["TCC_EA0_RDREQ_DRAM_sum"])
    wr_b = cal_bytes / mean(dr["copy_kernel"]["TCC_EA0_WRREQ_DRAM_sum"])
    lines = ["# rocprofv3 counters per dispatch, " + title,
             "# commands (two counter passes):",
             "#   " + cmd.replace("{P}", "SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA "
                                          "SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_LDS SQ_WAVES GRBM_GUI_ACTIVE"),
             "#   " + cmd.replace("{P}", "TCC_EA0_RDREQ_DRAM_sum TCC_EA0_WRREQ_DRAM_sum"),
             "# mfma_util = SQ_VALU_MFMA_BUSY_CYCLES / (%d SIMDs x GRBM_GUI_ACTIVE / %d XCCs) (rocprofv3's MfmaUtil; its"
             " GRBM_GUI_ACTIVE window holds about 6 us more than the dispatch, see clk)" % (N_SIMD, N_XCC),
             "# mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (%d SIMDs x dispatch duration x %.1f GHz peak clock): the"
             " fraction of the dispatch's peak MFMA cycles spent busy" % (N_SIMD, PEAK_CLK_GHZ),
             "# clk = GRBM_GUI_ACTIVE / %d / dispatch duration (GHz-equivalent)" % N_XCC,
             "# exec TF/s = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 flops / dispatch duration (executed MFMA work, hi|lo"
             " operands counted twice)",
             "# valu/wave, mfma/wave, lds/wave = SQ_INSTS_VALU, SQ_INSTS_MFMA, SQ_INSTS_LDS over SQ_WAVES",
             "# DRAM MB = TCC_EA0_RDREQ_DRAM x %.1f B + TCC_EA0_WRREQ_DRAM x %.1f B (bytes per request from the 64 MiB"
             " calibration copy; memory-side requests past L2, MALL hits included)" % (rd_b, wr_b),
             "%-26s %5s %8s %6s %9s %9s %9s %9s %8s %9s %9s %7s" % (
                 "kernel", "disp", "avg us", "clk", "mfma_util", "mfma_busy", "exec TF/s", "valu/wave", "mfma/wv",
                 "lds/wave", "DRAM MB", "GB/s")]
    rows = []
    for k, d in sq.items():
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in d:
            continue
        dur = mean(d["__dur_ns"])
        gui = mean(d["GRBM_GUI_ACTIVE"]) / N_XCC
        util = mean(d["SQ_VALU_MFMA_BUSY_CYCLES"]) / (N_SIMD * gui) if gui > 0 else 0.0
        busy = mean(d["SQ_VALU_MFMA_BUSY_CYCLES"]) / (N_SIMD * dur * PEAK_CLK_GHZ)
        flops = mean(d["SQ_INSTS_VALU_MFMA_MOPS_F16"]) * 512
        waves = max(mean(d["SQ_WAVES"]), 1.0)
        dm = dr.get(k, {})
        dram = (mean(dm["TCC_EA0_RDREQ_DRAM_sum"]) * rd_b + mean(dm["TCC_EA0_WRREQ_DRAM_sum"]) * wr_b) if dm else 0.0
        rows.append((k, len(d["__dur_ns"]), dur / 1e3, gui / dur, util, busy, flops / dur / 1e3,
                     mean(d["SQ_INSTS_VALU"]) / waves, mean(d["SQ_INSTS_MFMA"]) / waves,
                     mean(d["SQ_INSTS_LDS"]) / waves, dram / 1e6, dram / dur))
    for r in sorted(rows, key=lambda r: -r[1] * r[2]):
        lines.append("%-26s %5d %8.2f %6.2f %9.3f %9.3f %9.1f %9.0f %8.0f %9.0f %9.2f %7.0f" % r)
    return "\n".join(lines) + "\n"


STALL_COUNTERS = ("SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_WAIT_INST_LDS SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS "
                  "SQ_ACTIVE_INST_ANY SQ_LDS_IDX_ACTIVE")


def pmc_stall_summary(csv_path, title, cmd):
    """Per-kernel shares of resident wave-cycles (SQ_WAVE_CYCLES) from one counter pass: waiting on
    anything (SQ_WAIT_ANY: s_waitcnt on memory or LDS, barriers, dependencies), waiting for an
    instruction to issue (SQ_WAIT_INST_ANY, of which LDS: SQ_WAIT_INST_LDS), and issuing VALU, LDS or
    any instruction (SQ_ACTIVE_INST_*), per dispatch."""
    d_all = read_counter_rows(csv_path)
    mean = statistics.mean
    cols = [("wait_any", "SQ_WAIT_ANY"), ("wait_inst", "SQ_WAIT_INST_ANY"), ("wait_lds", "SQ_WAIT_INST_LDS"),
            ("act_valu", "SQ_ACTIVE_INST_VALU"), ("act_lds", "SQ_ACTIVE_INST_LDS"), ("act_any", "SQ_ACTIVE_INST_ANY")]
    lines = ["# rocprofv3 wave-state counters per dispatch, " + title,
             "# command: " + cmd.replace("{P}", STALL_COUNTERS),
             "# each column = counter / SQ_WAVE_CYCLES (the waves' resident cycles, summed over waves):",
             "#   " + ", ".join("%s = %s" % c for c in cols),
             "%-28s %5s %8s " % ("kernel", "disp", "avg us") + " ".join("%9s" % c[0] for c in cols)]
    rows = []
    for k, d in d_all.items():
        if "SQ_WAVE_CYCLES" not in d or mean(d["SQ_WAVE_CYCLES"]) <= 0:
            continue
        wc = mean(d["SQ_WAVE_CYCLES"])
        rows.append((k, len(d["__dur_ns"]), mean(d["__dur_ns"]) / 1e3) +
                    tuple(mean(d[c]) / wc if c in d else float("nan") for _, c in cols))
    for r in sorted(rows, key=lambda r: -r[1] * r[2]):
        lines.append("%-28s %5d %8.2f " % r[:3] + " ".join("%9.3f" % v for v in r[3:]))
    return "\n".join(lines) + "\n"


# GEMM shapes of the DiT workloads (name, M, N, K) for the vendor yardstick
YARDSTICK_SHAPES = [("8 s fused FFN1", 794, 4096, 1024), ("8 s fused FFN2", 794, 1024, 4096),
                    ("8 s fused QKV", 794, 3072, 1024), ("8 s fused out-projection", 794, 1024, 1024),
                    ("8 s joint FFN1 audio (K = 3 x 1024)", 512, 4096, 3072),
                    ("30 s fused FFN1", 2202, 4096, 1024), ("30 s fused QKV", 2202, 3072, 1024),
                    ("batch-16 fused FFN1", 6352, 4096, 1024), ("batch-16 fused FFN2", 6352, 1024, 4096),
                    ("batch-16 fused QKV", 6352, 3072, 1024), ("batch-16 joint FFN1 audio", 4096, 4096, 3072),
                    ("square 4096", 4096, 4096, 4096), ("square 8192", 8192, 8192, 8192)]


def vendor_yardstick():
    """Measurement only, never a product path: the vendor f16 GEMM (torch.nn.functional.linear, which
    runs hipBLASLt on this image) against this library's tsn_gemm on f16 X and f16 W with f16 Y, at
    the DiT's GEMM shapes; HIP events around 50 calls after 5 warm-up calls, same process, same GPU."""
    import torch
    tsn = importlib.import_module("thinksound-native_amd")
    assert torch.cuda.is_available()
    dev = torch.device("cuda:0")
    rt = tsn.Runtime(0)
    rng = np.random.default_rng(5)
    lines = ["# vendor yardstick: f16 GEMM Y[M,N] = X[M,K] W[N,K]^T, f16 operands and output, f32 accumulation",
             "# vendor = torch %s torch.nn.functional.linear (hipBLASLt); tsn = tsn_gemm (xdtype f16, wdtype f16, "
             "ydtype f16); mean of 50 calls, HIP events" % torch.__version__,
             "# command: python3 bench.py --vendor-yardstick",
             "%-36s %5s %5s %5s %10s %9s %10s %9s %8s" % ("shape", "M", "N", "K", "vendor us", "TFLOP/s",
                                                           "tsn us", "TFLOP/s", "tsn/vnd")]
    for name, M, N, K in YARDSTICK_SHAPES:
        x = torch.randn(M, K, device=dev, dtype=torch.float16)
        w = torch.randn(N, K, device=dev, dtype=torch.float16)
        for _ in range(5):
            y = torch.nn.functional.linear(x, w)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(50):
            y = torch.nn.functional.linear(x, w)
        e1.record()
        torch.cuda.synchronize()
        vus = e0.elapsed_time(e1) / 50 * 1e3
        del x, w, y
        X = rt.array(rng.standard_normal((M, K)).astype(np.float16))
        W = rt.array((0.05 * rng.standard_normal((N, K))).astype(np.float16))
        Y = rt.empty((M, N), np.float16)
        for _ in range(5):
            rt.gemm(1, W, X, 1, Y, 1, None, M, N, K)
        rt.sync()
        rt.begin()
        for _ in range(50):
            rt.gemm(1, W, X, 1, Y, 1, None, M, N, K)
        tus = rt.commit() / 50 * 1e3
        for a in (X, W, Y):
            a.free()
        fl = 2.0 * M * N * K
        lines.append("%-36s %5d %5d %5d %10.2f %9.1f %10.2f %9.1f %8.2f" % (
            name, M, N, K, vus, fl / vus / 1e6, tus, fl / tus / 1e6, tus / vus))
        log(lines[-1])
    rt.close()
    print("\n".join(lines), flush=True)
    return 0


UTIL_FILE = os.path.join(ROOT, "profiles", "mfma_util_dit_eval_b2_la256.txt")


def read_util_row(kernel, path=UTIL_FILE):
    """(mfma_busy, DRAM bytes per dispatch) of a kernel from a committed counter summary, or None"""
    try:
        with open(path) as f:
            for line in f:
                parts = line.rsplit(None, 11)
                if not line.startswith("#") and len(parts) == 12 and parts[0] == kernel:
                    return float(parts[5]), float(parts[10]) * 1e6
    except (OSError, ValueError):
        pass
    return None


def write_ref_gguf(tsn, spec, w16, path):
    """the reference-size checkpoint as a BF16 GGUF (tensor names, dims and dit.* metadata of the
    reference's file) holding the bits of w16; returns the file size"""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_writer as gw
    sd = spec.as_dict()
    meta = [("dit.hidden_dim", gw.KV_U32, spec.H), ("dit.num_heads", gw.KV_U32, spec.NH),
            ("dit.depth", gw.KV_U32, spec.n_joint + spec.n_fused), ("dit.fused_depth", gw.KV_U32, spec.n_fused),
            ("dit.latent_dim", gw.KV_U32, spec.latent)]
    return gw.write_bf16(path, [(n, gw.ref_ne(n, k, sd), w16[o:o + k]) for n, k, o in tsn.ref_manifest(spec)], meta)


def gguf_load_pass(path):
    """child process: a fresh runtime loads the reference-size GGUF; prints the load time and the
    process's peak resident host memory as one JSON line"""
    def vm_kb(key):   # this process image's own figures (getrusage's maxrss carries the parent's over exec)
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split()[1])
        return float("nan")
    tsn = importlib.import_module("thinksound-native_amd")
    rt = tsn.Runtime(0)
    rss0 = vm_kb("VmRSS")
    t0 = time.perf_counter()
    spec = tsn.ref_spec_from_gguf(path, 2, 172, 64, 154)
    m = tsn.RefDitModel(rt, spec)
    m.load_gguf(path)
    rt.sync()
    dt = time.perf_counter() - t0
    print(json.dumps({"load_s": dt, "rss_before_mb": rss0 / 1024.0, "rss_peak_mb": vm_kb("VmHWM") / 1024.0}),
          flush=True)
    m.close()
    rt.close()
    return 0


def bench_ref(tsn, rt, args):
    """The reference checkpoint's own three-stream graph at 8 s (B=2, T=172, C=64, TS=154): the
    checkpoint is written as a reference-size BF16 GGUF and loaded through tsn_refdit_load_gguf
    (raw payloads to HBM, converted on the device; load time, rate and the loading process's peak
    host memory measured, the latter in a child process), then graph replays of one evaluation,
    the 24-step sampler, and per-kernel statistics."""
    import tempfile
    spec = tsn.ref_spec_for_duration(8, 2)
    t0 = time.time()
    w16 = tsn.ref_synth_weights(spec, 4242, 0.0)
    log("bench ref: synthetic weights %.1f s (%d params)" % (time.time() - t0, w16.size))
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    load = None
    try:
        t0 = time.time()
        size = write_ref_gguf(tsn, spec, w16, path)
        nparams = int(w16.size)
        del w16
        log("bench ref: wrote %.2f GB GGUF in %.1f s" % (size / 1e9, time.time() - t0))
        child = subprocess.run([sys.executable, os.path.abspath(__file__), "--gguf-load-pass", path],
                               capture_output=True, text=True, timeout=300)
        cj = json.loads(child.stdout.strip().splitlines()[-1]) if child.returncode == 0 else None
        if cj is None:
            log("bench ref: load child failed: %s" % child.stderr[-500:])
        t0 = time.perf_counter()
        m = tsn.RefDitModel(rt, tsn.ref_spec_from_gguf(path, spec.B, spec.T, spec.C, spec.TS))
        m.load_gguf(path)
        rt.sync()
        load_s = time.perf_counter() - t0
    finally:
        os.remove(path)
    load = {"file_bytes": size, "params": nparams, "tensor_type": "BF16", "load_s": round(load_s, 4),
            "gb_per_s": round(size / load_s / 1e9, 2),
            "fresh_process_load_s": round(cj["load_s"], 4) if cj else None,
            "fresh_process_rss_peak_mb": round(cj["rss_peak_mb"], 1) if cj else None,
            "fresh_process_rss_before_load_mb": round(cj["rss_before_mb"], 1) if cj else None,
            "path": "tsn_refdit_load_gguf: tensor payloads read from the file into two pinned 32 MiB buffers in "
                    "turn and copied to HBM as stored (BF16), then converted and laid out on the device; "
                    "no host f32 copy"}
    log("bench ref: GGUF load %.3f s (%.2f GB/s); fresh process %s" % (load_s, size / load_s / 1e9, cj))
    inp = tsn.ref_synth_inputs(spec, 4242, cfg_pairs=True)
    d = {k: rt.array(v) for k, v in inp.items()}
    args_in = (d["clip_pp"], d["text_pp"], d["gcmlp"], d["sync_gather"])
    v = rt.empty((spec.B, spec.T, spec.latent))
    m.capture_forward(d["x"], d["t"], *args_in, v)
    for _ in range(args.warmup):
        m.replay()
    rt.sync()
    n = max(1, args.steps // 2)
    rt.begin()
    for _ in range(n):
        m.replay()
    ms = rt.commit() / n
    stats = None
    for _ in range(3):
        stats = m.profile_forward(d["x"], d["t"], *args_in, v)
    stats.sort(key=lambda k: -k["ms"])
    tot = sum(k["ms"] for k in stats)
    flops = sum(k["flops"] for k in stats)
    for k in stats[:8]:
        log("  ref %-28s %4d launches %8.3f ms  %7.1f TFLOP/s" % (k["name"], k["launches"], k["ms"],
                                                                   k["flops"] / (k["ms"] * 1e9) if k["ms"] else 0))
    x0 = inp["x"][0::2].copy()
    x = rt.array(x0)
    m.capture_sample(x, *args_in, 24, 5.0)
    m.replay()
    rt.sync()
    samp = []
    for _ in range(args.sampler_reps):
        x.upload(x0)
        rt.begin()
        m.replay()
        samp.append(rt.commit())
    sampler_ms = statistics.median(samp)
    log("bench ref: %.4f ms/eval (%.1f evals/s), 24-step sampler %.3f ms" % (ms, 1e3 / ms, sampler_ms))
    m.close()
    return {"workload": "reference checkpoint graph, one evaluation at 8 s, CFG batch 2",
            "B": spec.B, "T": spec.T, "C": spec.C, "TS": spec.TS, "H": spec.H, "ffn": spec.F,
            "joint_blocks": spec.n_joint, "fused_blocks": spec.n_fused,
            "evals_per_s": round(1e3 / ms, 2), "ms_per_eval": round(ms, 5), "sampler_ms": round(sampler_ms, 3),
            "eval_gflop": round(flops / 1e9, 2),
            "mfma_frac_eval": round(flops / (ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
            "kernels": [{"name": k["name"], "launches": k["launches"], "ms": round(k["ms"], 4),
                         "share": round(k["ms"] / tot, 4)} for k in stats[:10]],
            "gguf_load": load,
            "launch": "hipGraph replay"}


def bench_vae(tsn, rt, args):
    """The reference's VAE decoder at 8 s (T = 172 latent rows -> 352,256 stereo samples): graph
    replays of one decode, per-kernel statistics, and the oracle timed on a 4-row latent."""
    spec = tsn.vae_spec_for_duration(8)
    w = tsn.vae_synth_weights(spec, 4242)
    m = tsn.VaeModel(rt, spec)
    m.upload_weights(w)
    latent = tsn.synth_normal_f32(4242, 2000, 0.0, 1.0, (spec.T, spec.latent))
    z = rt.array(latent)
    n_audio = tsn.vae_audio_len(spec)
    audio = rt.empty((n_audio, spec.out_ch))
    m.capture_decode(z, audio)
    for _ in range(3):
        m.replay()
    rt.sync()
    n = 10
    rt.begin()
    for _ in range(n):
        m.replay()
    ms = rt.commit() / n
    stats = None
    for _ in range(2):
        stats = m.profile_decode(z, audio)
    stats.sort(key=lambda k: -k["ms"])
    tot = sum(k["ms"] for k in stats)
    flops = sum(k["flops"] for k in stats)
    for k in stats[:6]:
        log("  vae %-28s %4d launches %8.3f ms  %7.1f TFLOP/s (f32 GEMM)  %7.1f GB/s"
            % (k["name"], k["launches"], k["ms"], k["flops"] / (k["ms"] * 1e9) if k["ms"] else 0,
               k["bytes"] / (k["ms"] * 1e6) if k["ms"] else 0))
    dom = stats[0]
    dom_tf = dom["flops"] / (dom["ms"] * 1e9) if dom["ms"] else 0.0
    log("bench vae: %.3f ms per 8 s decode (%.0fx real time), %.1f GFLOP (f32 GEMM)" % (ms, 8e3 / ms, flops / 1e9))
    cpu = None
    if not args.no_cpu:
        import pyoracle
        cspec = spec.copy(T=4)
        cw = w   # the manifest does not depend on T
        cl = latent[:4].copy()
        k, c0 = 0, time.perf_counter()
        while True:
            pyoracle.vae_decode(cspec.as_dict(), cw, cl)
            k += 1
            cs = time.perf_counter() - c0
            if cs >= CPU_SAMPLE_S / 2:
                break
        cpu = {"value": round(k * 4 * 2048 / cs, 1), "unit": "audio samples/s", "cores": pyoracle.num_threads(),
               "kind": "port", "sample": "%d decodes of a 4-row latent (8192 samples), f32 host C++ oracle, %.2f s"
                                         % (k, cs)}
        log("bench vae: CPU oracle %d decodes of 4 rows in %.2f s" % (k, cs))
    m.close()
    return {"workload": "VAE decode of an 8 s latent (T=172 -> 352256 samples x 2 channels)",
            "T": spec.T, "widths": list(spec.width), "strides": list(spec.stride),
            "ms_per_decode": round(ms, 4), "audio_samples_per_s": round(n_audio / (ms * 1e-3), 1),
            "realtime_factor": round(8e3 / ms, 1), "gflop_f32": round(flops / 1e9, 2),
            "f32_tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "mfma_frac_f16_executed": round(3 * flops / (ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
            "dominant": {"kernel": dom["name"], "f32_tflops": round(dom_tf, 2),
                         "mfma_frac_f16_executed": round(3 * dom_tf / PEAK_F16_TFLOPS, 4)},
            "kernels": [{"name": k["name"], "launches": k["launches"], "ms": round(k["ms"], 4),
                         "share": round(k["ms"] / tot, 4)} for k in stats[:8]],
            "arithmetic": "f32-accurate: three f16 MFMA products per term (hi/lo split of both operands)",
            "cpu_baseline": cpu, "launch": "hipGraph replay"}


def bench_workloads(tsn, rt, args):
    """The other configured workloads, reported beside the metric: the 30 s clip (La=960, S=1101) and
    the 16-sample batch (8 prompts x CFG, prompt p's latent and text features from seed p + 1), each
    as one evaluation and the 24-step sampler; graph replays, synthetic BF16 weights."""
    out = {}
    for wl, name in ((3, "clip_30s"), (4, "batch16")):
        spec = tsn.default_spec(wl)
        m = tsn.DitModel(rt, spec)
        m.upload_weights(tsn.synth_weights(spec, 4242, 0.0))
        if wl == 4:
            inp = tsn.synth_prompt_inputs(spec, list(range(1, spec.B // 2 + 1)))
        else:
            inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
        z, tt, text, pooled = (rt.array(inp[k]) for k in ("z", "t", "text", "pooled"))
        v = rt.empty((spec.B, spec.La, spec.latent))
        m.capture_forward(z, tt, text, pooled, v)
        for _ in range(5):
            m.replay()
        rt.sync()
        n = 20
        rt.begin()
        for _ in range(n):
            m.replay()
        ms = rt.commit() / n
        stats = m.profile_forward(z, tt, text, pooled, v)
        flops = sum(k["flops"] for k in stats)
        for k in sorted(stats, key=lambda k: -k["ms"])[:6]:
            log("  %s %-28s %4d launches %8.3f ms  %7.1f TFLOP/s  %7.1f GB/s"
                % (name, k["name"], k["launches"], k["ms"], k["flops"] / (k["ms"] * 1e9) if k["ms"] else 0,
                   k["bytes"] / (k["ms"] * 1e6) if k["ms"] else 0))
        r = {"B": spec.B, "La": spec.La, "Lt": spec.Lt, "ms_per_eval": round(ms, 4),
             "evals_per_s": round(1e3 / ms, 2), "eval_gflop": round(flops / 1e9, 1),
             "mfma_frac_eval": round(flops / (ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)}
        if wl in (3, 4):
            x0 = inp["z"][0::2].copy()
            x = rt.array(x0)
            m.capture_sample(x, text, pooled, 24, 5.0)
            m.replay()
            rt.sync()
            x.upload(x0)
            rt.begin()
            m.replay()
            r["sampler_ms"] = round(rt.commit(), 3)
        log("bench %s: %.4f ms/eval, %.1f GFLOP, %.1f%% of the f16 MFMA peak%s"
            % (name, ms, flops / 1e9, 100 * r["mfma_frac_eval"],
               (", 24-step sampler %.2f ms" % r["sampler_ms"]) if "sampler_ms" in r else ""))
        out[name] = r
        m.close()
    return out


def bench_joint_block(tsn, rt, args):
    """One joint block at 8 s (B=2, La=256, Lt=141) on the stream rows X [B, S, H]: its adaLN
    modulation GEMV, LN, QKV, attention, out-projection, FFNs and gated residuals, eager launches
    timed by events (the entry point copies X in and out)."""
    spec = tsn.default_spec(0)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(tsn.synth_weights(spec, 4242, 0.0))
    S = spec.La + spec.Lt
    X = rt.array(tsn.synth_normal_f32(4242, tsn.IDX_X, 0.0, 1.0, (spec.B, S, spec.H)))
    g = rt.array(tsn.synth_normal_f32(4242, tsn.IDX_G, 0.0, 1.0, (spec.B, spec.H)))
    for _ in range(5):
        m.joint_block(0, X, g)
    rt.sync()
    n = 50
    rt.begin()
    for _ in range(n):
        m.joint_block(0, X, g)
    ms = rt.commit() / n
    B, La, Lt, H, F = spec.B, spec.La, spec.Lt, spec.H, spec.F
    flops = 2.0 * B * (La * 3 * H * H + Lt * 3 * H * H + La * H * H + Lt * H * H + La * F * 3 * H + La * H * 3 * F
                       + Lt * F * H * 2) + 4.0 * B * spec.NH * S * S * 64
    m.close()
    log("bench joint block: %.4f ms, %.2f GFLOP, %.1f%% of the f16 MFMA peak"
        % (ms, flops / 1e9, flops / (ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS * 100))
    return {"B": B, "La": La, "Lt": Lt, "ms": round(ms, 4), "gflop": round(flops / 1e9, 2),
            "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4), "launch": "eager"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(tsn, pyoracle):
    """The CPU oracle on every configured workload, on this host's cores: the single joint block and
    the 24-step 8 s sampler in full; the 30 s clip and the 16-sample batch as one evaluation each, the
    24-step sampler projected as 24 x that (the oracle's cost per step does not depend on the step)."""
    out = {"cores": pyoracle.num_threads(), "cpu": cpu_model(), "kind": "port"}
    spec = tsn.default_spec(0)
    w32 = tsn.bf16_to_f32(tsn.synth_weights(spec, 4242, 0.0))
    S = spec.La + spec.Lt
    X = tsn.synth_normal_f32(4242, tsn.IDX_X, 0.0, 1.0, (spec.B, S, spec.H))
    g = tsn.synth_normal_f32(4242, tsn.IDX_G, 0.0, 1.0, (spec.B, spec.H))
    c0 = time.perf_counter()
    pyoracle.joint_block(spec, w32, 0, X, g)
    out["joint_block_8s_b2"] = {"ms": round((time.perf_counter() - c0) * 1e3, 1), "measured": "full"}
    del w32
    spec = tsn.default_spec(2)
    w32 = tsn.bf16_to_f32(tsn.synth_weights(spec, 4242, 0.0))
    inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
    c0 = time.perf_counter()
    pyoracle.dit_sample(spec, w32, inp["z"][0::2].copy(), inp["text"], inp["pooled"], 24, 5.0)
    out["sampler_8s_24steps"] = {"ms": round((time.perf_counter() - c0) * 1e3, 1), "measured": "full"}
    del w32
    for wl, name in ((3, "clip_30s"), (4, "batch16")):
        spec = tsn.default_spec(wl)
        w32 = tsn.bf16_to_f32(tsn.synth_weights(spec, 4242, 0.0))
        inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
        c0 = time.perf_counter()
        pyoracle.dit_forward(spec, w32, inp["z"], inp["t"], inp["text"], inp["pooled"])
        ms = (time.perf_counter() - c0) * 1e3
        out[name] = {"eval_ms": round(ms, 1), "measured": "one evaluation",
                     "sampler_24steps_ms_projected": round(24 * ms, 1)}
        del w32
    log("bench: CPU oracle baselines %s" % json.dumps(out))
    return out


def f32_to_bf16(x):
    """round-to-nearest-even f32 -> bf16 bits (uint16)"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bench_bf16_gemm(tsn, rt, args):
    """The bf16-operand mode beside f16: tsn_gemm on the same pipelined kernel and tiles, f16 X and W
    against bf16 X and W (f32 Y), at the 8 s evaluation's FFN1 and QKV shapes and the batch-16 FFN1
    shape; eager launches timed by events, 20 each"""
    out = {}
    for name, (M, N, K) in (("ffn1_8s_794x4096x1024", (794, 4096, 1024)), ("qkv_8s_794x3072x1024", (794, 3072, 1024)),
                            ("ffn1_b16_6352x4096x1024", (6352, 4096, 1024))):
        xf = tsn.synth_normal_f32(4242, 3100, 0.0, 1.0, (M, K))
        wf = tsn.synth_normal_f32(4242, 3101, 0.0, 0.02, (N, K))
        y = rt.empty((M, N))
        row = {}
        for tag, dt, conv in (("f16", tsn.F16, lambda a: a.astype(np.float16)), ("bf16", tsn.BF16, f32_to_bf16)):
            X, W = rt.array(conv(xf)), rt.array(conv(wf))
            for _ in range(3):
                rt.gemm(dt, W, X, dt, y, tsn.F32, None, M, N, K)
            rt.sync()
            n = 20
            rt.begin()
            for _ in range(n):
                rt.gemm(dt, W, X, dt, y, tsn.F32, None, M, N, K)
            ms = rt.commit() / n
            tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
            row[tag] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac_peak": round(tf / PEAK_F16_TFLOPS, 4)}
            X.free()
            W.free()
        y.free()
        row["bf16_over_f16"] = round(row["bf16"]["tflops"] / row["f16"]["tflops"], 3)
        out[name] = row
    log("bench bf16 gemm: %s" % json.dumps(out))
    return out


def bench_hbm(tsn, rt, args):
    """The HBM-bound norm kernel on a large shape: adaLN (LayerNorm + broadcast shift/scale) over
    65536 rows x 1024, f32 in, f16 out; algorithmic bytes = rows*H*(4 + 2) + modulation, 20 launches"""
    rows, H = 65536, 1024
    x = rt.array(tsn.synth_normal_f32(4242, 3000, 0.0, 1.0, (rows, H)))
    mod = rt.array(tsn.synth_normal_f32(4242, 3001, 0.0, 0.1, (6 * H,)))
    y = rt.empty((rows, H), np.float16)
    for _ in range(3):
        rt.adaln_ln(x, mod, y, 1, rows, H, 0, 6, 0, 1e-5)
    rt.sync()
    n = 20
    rt.begin()
    for _ in range(n):
        rt.adaln_ln(x, mod, y, 1, rows, H, 0, 6, 0, 1e-5)
    ms = rt.commit() / n
    gbs = (rows * H * 6.0 + 2 * H * 4.0) / (ms * 1e-3) / 1e9
    log("bench hbm: adaLN 65536 x 1024 %.1f us, %.0f GB/s (%.1f%% of 8 TB/s)" % (ms * 1e3, gbs, gbs / 80.0))
    return {"adaln_ln_65536x1024_f16": {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                                         "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}}


def bench_encoders(tsn, rt, args):
    """The reference's text encoders, once per prompt: CLIP (24 layers, H 1024) and T5 v1.1 XL (24 layers,
    d 2048, d_ff 5120) over 77 tokens, f32 synthetic weights; eager launches, median of 5."""
    out = {}
    for name, spec, synth, cls in (("clip", tsn.clip_spec_default(), tsn.clip_synth_weights, tsn.ClipModel),
                                   ("t5", tsn.t5_spec_default(), tsn.t5_synth_weights, tsn.T5Model)):
        w = synth(spec, 4242)
        m = cls(rt, spec)
        m.upload_weights(w)
        del w
        ids = np.arange(spec.ctx, dtype=np.int32) % (spec.vocab - 1) + 1
        width = spec.H if name == "clip" else spec.d
        a = rt.empty((spec.ctx, width))
        g = rt.empty((width,))
        run = (lambda: m.encode(ids, a, g)) if name == "clip" else (lambda: m.encode(ids, a))
        for _ in range(2):
            run()
        rt.sync()
        ts = []
        for _ in range(5):
            rt.begin()
            run()
            ts.append(rt.commit())
        stats = m.profile_encode(ids, a, g) if name == "clip" else m.profile_encode(ids, a)
        flops = sum(k["flops"] for k in stats)
        wbytes = 4.0 * (int(lib_total(tsn, name, spec)))
        ms = statistics.median(ts)
        gemm = [k for k in stats if k["name"] == "gemm_f32_kernel"][0]
        for k in sorted(stats, key=lambda k: -k["ms"]):
            log("  %s %-24s %4d launches %8.3f ms" % (name, k["name"], k["launches"], k["ms"]))
        log("bench %s: %.3f ms per prompt, %.1f GFLOP, gemm_f32 %.3f ms (%d launches, %.1f TFLOP/s)"
            % (name, ms, flops / 1e9, gemm["ms"], gemm["launches"], gemm["flops"] / (gemm["ms"] * 1e9)))
        out[name] = {"ms_per_prompt": round(ms, 4), "gflop": round(flops / 1e9, 2), "weights_gb_f32": round(wbytes / 1e9, 3),
                     "weight_read_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1),
                     "gemm_f32": {"launches": gemm["launches"], "ms": round(gemm["ms"], 4),
                                  "tflops": round(gemm["flops"] / (gemm["ms"] * 1e9), 2),
                                  "frac_fp32_mfma_peak": round(gemm["flops"] / (gemm["ms"] * 1e9) / PEAK_F32_TFLOPS, 4)}}
        m.close()
    out["workload"] = "CLIP and T5 text encoders over 77 tokens, one prompt each, f32"
    out["launch"] = "eager"
    return out


def lib_total(tsn, name, spec):
    man = tsn.clip_manifest(spec) if name == "clip" else tsn.t5_manifest(spec)
    return man[-1][1] + man[-1][2]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sampler-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-all", action="store_true",
                    help="also time the CPU oracle on the other workloads: the joint block and the 24-step 8 s "
                         "sampler in full, the 30 s and batch-16 evaluations once (about 3 minutes)")
    ap.add_argument("--no-ref", action="store_true", help="skip the reference checkpoint graph section")
    ap.add_argument("--no-vae", action="store_true", help="skip the VAE decoder section")
    ap.add_argument("--no-enc", action="store_true", help="skip the text-encoder section")
    ap.add_argument("--no-wl", action="store_true", help="skip the 30 s and batch-16 workload section")
    ap.add_argument("--eager", action="store_true",
                    help="launch kernel by kernel instead of replaying hipGraphs (for profilers that do not follow graphs)")
    ap.add_argument("--pmc-pass", nargs="?", const="8s", choices=sorted(PMC_WORKLOADS),
                    help="only run three eager evaluations (8 s B=2, batch 16 or 30 s) and 64 MiB calibration "
                         "copies (workload for rocprofv3 --pmc)")
    ap.add_argument("--pmc-util-summary", nargs=4, metavar=("SQ_CSV", "DRAM_CSV", "TITLE", "CMD"),
                    help="print the MFMA-utilisation and DRAM summary of two counter CSVs (no GPU use)")
    ap.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "CMD"),
                    help="print the traffic summary of two counter-collection CSVs (no GPU use)")
    ap.add_argument("--pmc-stall-summary", nargs=3, metavar=("CSV", "TITLE", "CMD"),
                    help="print the wait-counter summary (SQ_WAIT_ANY, SQ_WAIT_INST_ANY over SQ_WAVE_CYCLES) of a "
                         "counter CSV (no GPU use)")
    ap.add_argument("--vendor-yardstick", action="store_true",
                    help="only time the vendor f16 GEMM (torch -> hipBLASLt) beside tsn_gemm at the DiT's GEMM shapes "
                         "(measurement only)")
    ap.add_argument("--stats-summary", nargs=2, metavar=("STATS_CSV", "CMD"),
                    help="print the summary of a rocprofv3 kernel_stats.csv (no GPU use)")
    ap.add_argument("--stats-title", default=None, help="workload line of --stats-summary")
    ap.add_argument("--gguf-load-pass", metavar="GGUF",
                    help="only load a reference-graph GGUF checkpoint in a fresh runtime and print the load time "
                         "and peak host memory (run by the benchmark as a child process)")
    ap.add_argument("--profile-pass", choices=["vae", "enc", "ref"],
                    help="only run eager VAE decodes, text-encoder passes or reference-graph evaluations "
                         "(workload for rocprofv3 --kernel-trace)")
    args = ap.parse_args()
    if args.pmc_summary:
        sys.stdout.write(pmc_summary(*args.pmc_summary))
        return 0
    if args.pmc_util_summary:
        sys.stdout.write(pmc_util_summary(*args.pmc_util_summary))
        return 0
    if args.pmc_stall_summary:
        sys.stdout.write(pmc_stall_summary(*args.pmc_stall_summary))
        return 0
    if args.stats_summary:
        if args.stats_title:
            sys.stdout.write(stats_summary(*args.stats_summary, title=args.stats_title))
        else:
            sys.stdout.write(stats_summary(*args.stats_summary))
        return 0
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (one process, one MI355X); --gpus %d is not supported"
              % args.gpus, file=sys.stderr)
        return 2

    if args.vendor_yardstick:
        return vendor_yardstick()
    if args.gguf_load_pass:
        return gguf_load_pass(args.gguf_load_pass)
    if args.pmc_pass:
        return pmc_pass(args.pmc_pass)
    if args.profile_pass:
        return profile_pass(args.profile_pass)

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
    # the denominators this GPU actually reaches (f16 MFMA chains, 1 GiB device copy)
    meas_tflops, meas_gbs = rt.probe_peaks()
    log("bench: measured peaks %.0f TFLOP/s dense f16 MFMA, %.0f GB/s device copy" % (meas_tflops, meas_gbs))
    meas_peak = meas_tflops if bound == "mfma" else meas_gbs
    traffic = read_traffic(dom["name"])
    util = read_util_row(dom["name"])
    if traffic is not None:
        log("bench: %s HBM traffic %.0f B/dispatch (counters), algorithmic %.0f B/dispatch"
            % (dom["name"], traffic, dom["bytes"] / dom["launches"]))

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

    # ---------------- the reference checkpoint's graph (reported beside the metric) ----------------
    ref = None
    if not args.no_ref and not args.eager:
        ref = bench_ref(tsn, rt, args)

    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle
        if not os.path.exists(pyoracle.LIB_PATH):
            pyoracle.build()
    vae = None
    if not args.no_vae and not args.eager:
        vae = bench_vae(tsn, rt, args)
    enc = None
    if not args.no_enc and not args.eager:
        enc = bench_encoders(tsn, rt, args)
    wls = None
    if not args.no_wl and not args.eager:
        wls = bench_workloads(tsn, rt, args)
        wls["joint_block"] = bench_joint_block(tsn, rt, args)
        wls["hbm_kernels"] = bench_hbm(tsn, rt, args)
        wls["bf16_gemm"] = bench_bf16_gemm(tsn, rt, args)

    # ---------------- CPU baseline: the oracle, one full evaluation ----------------
    cpu = None
    cpu_all = None
    if not args.no_cpu:
        import pyoracle
        w32 = tsn.bf16_to_f32(w16)
        n_ev = 0
        c0 = time.perf_counter()
        while True:
            pyoracle.dit_forward(spec, w32, inp["z"], inp["t"], inp["text"], inp["pooled"])
            n_ev += 1
            cpu_s = time.perf_counter() - c0
            if cpu_s >= CPU_SAMPLE_S:
                break
        cpu = {"value": round(n_ev / cpu_s, 4), "unit": "evals/s", "cores": pyoracle.num_threads(), "kind": "port",
               "cpu": cpu_model(),
               "sample": "%d full 21-block evaluations of the timed workload (B=2, La=256, Lt=141), f32 host C++ "
                         "oracle, %.2f s" % (n_ev, cpu_s)}
        log("bench: CPU oracle %d evals in %.2f s on %d threads" % (n_ev, cpu_s, pyoracle.num_threads()))
        if args.cpu_all:
            cpu_all = cpu_baselines(tsn, pyoracle)

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
        "measured_peaks": {"mfma_f16_tflops": round(meas_tflops, 1), "copy_gbs": round(meas_gbs, 1)},
        "roofline": {"kernel": dom["name"], "bound": bound, "achieved": round(achieved, 2), "peak": peak,
                     "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
                     "mfma_busy_counter": util[0] if util else None,
                     "traffic_dram_requests": round(util[1]) if util else None,
                     "peak_measured": round(meas_peak, 1), "frac_of_measured": round(achieved / meas_peak, 4),
                     "launches_per_eval": dom["launches"], "avg_launch_us": round(avg_launch_ms * 1e3, 3)},
        "kernels": [{"name": k["name"], "launches": k["launches"], "ms": round(k["ms"], 4),
                     "share": round(k["ms"] / tot_ms, 4)} for k in stats],
        "cpu_baseline": cpu,
        "cpu_baselines_other_workloads": cpu_all,
        "reference_graph": ref,
        "vae_decoder": vae,
        "text_encoders": enc,
        "other_workloads": wls,
        "accumulate": "f32 (f16 MFMA operands from BF16 weights; f32 residual stream)",
        "launch": "eager" if args.eager else "hipGraph replay",
    }
    print(json.dumps(out), flush=True)
    m.close()
    rt.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
