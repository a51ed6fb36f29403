#!/usr/bin/env python3
"""Benchmark of the MI355X Q4_K/Q6_K fused-dequant matmul (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2] [--no-cpu] [--no-extras]

A step is one pass of the hot path over one batch of synthetic input: one qk_matmul /
qk_gemv_group call through the C ABI (M=1: the single-token GEMV kernel alone; M=2..4: an
activation prepass kernel + the GEMV kernel; M>=16: a prepass + the GEMM kernel).
The K timed steps are captured once into a HIP graph and replayed, so the host launch rate does
not limit the kernels; every step uses a different weight copy from a ring of >= 8 copies
(>= 512 MiB) so the 256 MiB Infinity Cache cannot serve repeats.  Inputs are resident in HBM
before the timed region; timing uses HIP events on the launch stream.

value = algorithmic bytes per step (GGUF weight bytes + fp32 x + fp32 y) / time per step for the
default workload c2.  roofline.achieved divides the same bytes by the dominant kernel's mean
duration: for an M=1 call (one kernel) that is the graph-timed step itself, which rocprofv3's kernel
trace reproduces within ~2 %; HIP events around single eager launches (also reported) add the
dispatch latency on top.  Default workload c2 (Q6_K GEMV M=1 K=17408 N=5120).  The other configs are
reported under "extras": c1 (Q4_K GEMV), c3a/c3b (M=4), c4 (M=512 prefill GEMM, TFLOPS) and c5
(the 497-matmul decode step of a synthetic 64-layer stack, ~15.5 GB of weights).  The CPU
baseline times the reference's own AVX-512 matvec (oracle/_ref, compiled from the reference
headers) on the host cores, or the repository's CPU restatement when that cannot run; it is a
reported baseline, not the target.
"""
import argparse
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen3.8_27b_reference_amd")
HBM_PEAK_GBS = 8000.0
SEED_BASE = 0x5EED0000000000C0
T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K = 8, 12, 13, 14
TYPE_NAME = {T_Q8_0: "Q8_0", T_Q4_K: "Q4_K", T_Q5_K: "Q5_K", T_Q6_K: "Q6_K"}
LAYOUT_GGUF, LAYOUT_T16 = 0, 1
MALL_BYTES = 256 << 20

# BASELINE configs (BASELINE.json "configs"), GEMV family
CONFIGS = {
    "c1": dict(desc="Q4_K GEMV M=1 K=5120 N=17408 (ffn_gate)", kind="gemv", type=T_Q4_K, K=5120, N=17408, M=1, cid=1),
    "c2": dict(desc="Q6_K GEMV M=1 K=17408 N=5120 (ffn_down)", kind="gemv", type=T_Q6_K, K=17408, N=5120, M=1, cid=2),
    "c3a": dict(desc="Q4_K gate+up GLU M=4 K=5120 N=17408x2", kind="glu", type=T_Q4_K, K=5120, N=17408, M=4, cid=3),
    "c3b": dict(desc="Q4_K GEMV M=4 K=5120 N=5120", kind="gemv", type=T_Q4_K, K=5120, N=5120, M=4, cid=3),
    "c4": dict(desc="Q4_K prefill GEMM M=512 K=5120 N=17408", kind="gemm", type=T_Q4_K, K=5120, N=17408, M=512,
               cid=4),
    # the other types of a Q4_K_M file at the shapes they take there (extras, not BASELINE configs):
    # Q5_K ffn_down, Q8_0 attn_output / ssm_out
    "q5k": dict(desc="Q5_K GEMV M=1 K=17408 N=5120 (ffn_down)", kind="gemv", type=T_Q5_K, K=17408, N=5120, M=1,
                cid=6),
    "q8_0": dict(desc="Q8_0 GEMV M=1 K=6144 N=5120 (attn_output)", kind="gemv", type=T_Q8_0, K=6144, N=5120, M=1,
                 cid=7),
    "q5k_m4": dict(desc="Q5_K GEMV M=4 K=17408 N=5120", kind="gemv", type=T_Q5_K, K=17408, N=5120, M=4, cid=8),
    # the largest single matmul of a decode step: the Q6_K output projection (1.04 GB)
    "lm_head": dict(desc="Q6_K GEMV M=1 K=5120 N=248320 (output projection)", kind="gemv", type=T_Q6_K, K=5120,
                    N=248320, M=1, cid=11),
    "q5k_m512": dict(desc="Q5_K prefill GEMM M=512 K=17408 N=5120", kind="gemm", type=T_Q5_K, K=17408, N=5120,
                     M=512, cid=9),
    "q8_0_m512": dict(desc="Q8_0 prefill GEMM M=512 K=6144 N=5120", kind="gemm", type=T_Q8_0, K=6144, N=5120,
                      M=512, cid=10),
}
FP16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA headline
SWEEP_LAYERS = 64
# The reference's own published GEMV bandwidth for the same shapes (RTX 6000D).
REF_PUBLISHED_GBS = {"c1": 1192.0, "c2": 1214.0}
KERNEL_NAME = {T_Q4_K: "k_gemv_q4k", T_Q6_K: "k_gemv_q6k"}  # M = 2..4 (after the k_prep_q4/q6 prepass)
KERNEL_SINGLE = "k_gemv1"  # M = 1: one kernel, x converted inside
KERNEL_GEMM = "k_gemm"


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def algorithmic_bytes(cfg, rb):
    nmat = 2 if cfg["kind"] == "glu" else 1
    return nmat * cfg["N"] * rb + cfg["M"] * cfg["K"] * 4 + cfg["M"] * cfg["N"] * 4


def sweep_matrices():
    """The decode-step matmuls of a synthetic 64-layer stack with the reference's layer map and shapes
    (qwen_cpu/qwen.cpp:608-631: linear-attention layers unless (l+1) % 4 == 0) and a Q4_K_M-like type
    mix: Q4_K everywhere except ffn_down on even layers and attn_v on layers 7, 15, ..., 63 (Q6_K),
    plus the Q6_K output projection 248320 x 5120.  Returns [(name, type, k, n)]."""
    mats = []
    for l in range(SWEEP_LAYERS):
        if (l + 1) % 4:
            mats += [(f"{l}.qkv", T_Q4_K, 5120, 10240), (f"{l}.gate_z", T_Q4_K, 5120, 6144),
                     (f"{l}.alpha", T_Q4_K, 5120, 48), (f"{l}.beta", T_Q4_K, 5120, 48),
                     (f"{l}.ssm_out", T_Q4_K, 6144, 5120)]
        else:
            mats += [(f"{l}.q", T_Q4_K, 5120, 12288), (f"{l}.k", T_Q4_K, 5120, 1024),
                     (f"{l}.v", T_Q6_K if (l + 1) % 8 == 0 else T_Q4_K, 5120, 1024), (f"{l}.o", T_Q4_K, 6144, 5120)]
        mats += [(f"{l}.gate", T_Q4_K, 5120, 17408), (f"{l}.up", T_Q4_K, 5120, 17408),
                 (f"{l}.down", T_Q6_K if l % 2 == 0 else T_Q4_K, 17408, 5120)]
    mats.append(("output", T_Q6_K, 5120, 248320))
    return mats


def sweep_groups(mats):
    """The launches of one decode step, grouped as the reference's forward pass groups them for
    T < 16 (qwen_cuda/qwen.cpp:262-312): matrices that read the same activation share one launch
    ({qkv, gate_z, alpha, beta} on linear-attention layers, {q, k, v} on full-attention layers),
    ffn gate and up form one GLU launch with one output, and ssm_out / o, down and the output
    projection run alone.  Returns [(glu, [matrix indices])]."""
    groups, i = [], 0
    while i < len(mats):
        name = mats[i][0].split(".")[-1]
        if name == "qkv":
            groups.append((False, [i, i + 1, i + 2, i + 3])); i += 4
        elif name == "q":
            groups.append((False, [i, i + 1, i + 2])); i += 3
        elif name == "gate":
            groups.append((True, [i, i + 1])); i += 2
        else:
            groups.append((False, [i])); i += 1
    return groups


class SweepWorkload:
    """one decode step = every matmul of the synthetic stack at M=1, launched in
    layer order with the reference's grouping (one x per launch, one y per matrix, one y per GLU
    pair; one copy of the weights: the stack is far larger than the MALL)."""

    def __init__(self, hip, hiprt, qk, stream):
        self.hip, self.qk, self.stream = hip, qk, stream
        self.mats = sweep_matrices()
        self.groups = sweep_groups(self.mats)
        self.copies = 1
        seed = SEED_BASE | 5
        rng = np.random.default_rng(seed)
        self.bufs, self.W = [], []
        self.weight_bytes = 0
        block0 = 0
        big = max(n * qk.row_bytes(t, k) for _, t, k, n in self.mats)
        tmp = hiprt.Buf(hip, big)
        for _, typ, k, n in self.mats:
            rb = qk.row_bytes(typ, k)
            nblk = n * (k // 256)
            qk.synth_fill(typ, seed, block0, nblk, tmp.ptr)
            block0 += nblk
            dst = hiprt.Buf(hip, n * rb)
            self.W.append(qk.repack(qk.weight_view(tmp.ptr, typ, k, n, LAYOUT_GGUF), dst.ptr, LAYOUT_T16))
            hip.sync()
            self.bufs.append(dst)
            self.weight_bytes += n * rb
        tmp.close()
        # one activation per launch and one output per matrix (per pair for a GLU launch)
        self.launches, self.act_bytes = [], 0
        for glu, idx in self.groups:
            k = self.mats[idx[0]][2]
            x = hiprt.Buf.of(hip, rng.standard_normal(k).astype(np.float32))
            outs = idx[:1] if glu else idx
            ys = [hiprt.Buf(hip, self.mats[j][3] * 4) for j in outs]
            self.bufs += [x] + ys
            self.launches.append((glu, [self.W[j] for j in idx], x, ys))
            self.act_bytes += 4 * k + sum(4 * self.mats[j][3] for j in outs)
        self.bytes_per_step = self.weight_bytes + self.act_bytes

    def launch(self, i):
        for glu, ws, x, ys in self.launches:
            if len(ws) == 1:
                self.qk.matmul(ws[0], x.ptr, 1, ys[0].ptr, self.stream)
            else:
                self.qk.gemv_group(ws, [y.ptr for y in ys], glu, x.ptr, 1, self.stream)

    def close(self):
        for b in self.bufs:
            b.close()


class GemvWorkload:
    """Weight ring + activations for one GEMV config, resident in HBM."""

    def __init__(self, hip, hiprt, qk, cfg, stream):
        self.hip, self.qk, self.cfg, self.stream = hip, qk, cfg, stream
        typ, K, N, M = cfg["type"], cfg["K"], cfg["N"], cfg["M"]
        self.rb = qk.row_bytes(typ, K)
        self.wbytes = N * self.rb
        self.nmat = 2 if cfg["kind"] == "glu" else 1
        # enough copies that repeats cannot hit the 256 MiB MALL (two suffice past it)
        self.copies = max(8 if self.wbytes * self.nmat < MALL_BYTES else 2,
                          math.ceil(2 * MALL_BYTES / (self.wbytes * self.nmat)))
        seed = SEED_BASE | cfg["cid"]
        nblk = N * (K // 256)
        tmp = hiprt.Buf(hip, self.wbytes)
        self.bufs, self.W = [], []
        for c in range(self.copies):
            ws = []
            for j in range(self.nmat):
                qk.synth_fill(typ, seed, (c * self.nmat + j) * nblk, nblk, tmp.ptr)
                dst = hiprt.Buf(hip, self.wbytes)
                view = qk.weight_view(tmp.ptr, typ, K, N, LAYOUT_GGUF)
                ws.append(qk.repack(view, dst.ptr, LAYOUT_T16))
                hip.sync()
                self.bufs.append(dst)
            self.W.append(ws)
        tmp.close()
        rng = np.random.default_rng(seed)
        self.x_host = rng.standard_normal((M, K)).astype(np.float32)
        self.x = hiprt.Buf.of(hip, self.x_host)
        self.y = hiprt.Buf(hip, M * N * 4)
        self.bytes_per_step = algorithmic_bytes(cfg, self.rb)

    def launch(self, i):
        ws = self.W[i % self.copies]
        if self.nmat == 2:
            self.qk.gemv_group(ws, [self.y.ptr], True, self.x.ptr, self.cfg["M"], self.stream)
        else:
            self.qk.matmul(ws[0], self.x.ptr, self.cfg["M"], self.y.ptr, self.stream)

    def close(self):
        for b in self.bufs:
            b.close()
        self.x.close()
        self.y.close()


def time_workload(hip, wl, steps, warmup, stream):
    """Warmup eagerly, capture exactly `steps` launches into one graph, replay it three times
    untimed, then time exactly one replay (`steps` steps) with events on the launch stream,
    bracketed by device synchronisations.  Returns ms per step."""
    for i in range(warmup):
        wl.launch(i)
    hip.stream_sync(stream)
    hip.begin_capture(stream)
    for i in range(steps):
        wl.launch(i)
    graph, gexec = hip.end_capture(stream)
    for _ in range(3):  # untimed replays: the first replays after a new workload run slow (clocks, TLB)
        hip.graph_launch(gexec, stream)
    hip.sync()
    e0, e1 = hip.event_create(), hip.event_create()
    hip.event_record(e0, stream)
    hip.graph_launch(gexec, stream)
    hip.event_record(e1, stream)
    hip.event_sync(e1)
    hip.sync()
    ms = hip.elapsed_ms(e0, e1) / steps
    hip.event_destroy(e0)
    hip.event_destroy(e1)
    hip.graph_destroy(graph, gexec)
    return ms


def kernel_event_ms(hip, wl, n, stream):
    """Mean and median latency of one eager launch, each bracketed by its own pair of HIP events on
    the launch stream (kernel duration plus the dispatch latency)."""
    evs = [(hip.event_create(), hip.event_create()) for _ in range(n)]
    for i in range(4):
        wl.launch(i)
    hip.stream_sync(stream)
    for i, (e0, e1) in enumerate(evs):
        hip.event_record(e0, stream)
        wl.launch(i)
        hip.event_record(e1, stream)
    hip.stream_sync(stream)
    ts = [hip.elapsed_ms(e0, e1) for e0, e1 in evs]
    for e0, e1 in evs:
        hip.event_destroy(e0)
        hip.event_destroy(e1)
    return float(np.mean(ts)), float(np.median(ts))


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, calibrated
    on a copy kernel), read from the committed summary profiles/<kernel>_<workload>_traffic.md."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.md")  # e.g. k_gemv_q6k_c2
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(cfg_name, cfg, gpu_y, gpu_x, budget_s):
    """Times the CPU matvec for the same config on the host cores (bounded sample) and checks the
    GPU result against it on the same inputs."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib

    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    typ, K, N, M = cfg["type"], cfg["K"], cfg["N"], cfg["M"]
    o = oracle_lib.Oracle()
    kind = "port"
    runner = o
    if oracle_lib.ref_available():
        runner = oracle_lib.RefLib()
        kind = "reference"
    runner.init(threads)
    seed = SEED_BASE | cfg["cid"]
    nblk = N * (K // 256)
    ncop = 8
    ws = [o.fill(typ, seed, c * nblk, nblk) for c in range(ncop)]  # same bytes as the GPU ring
    rb = o.row_bytes(typ, K)
    # parity of the GPU result (copy 0) against the CPU path on the same inputs
    y0 = runner.matmul(typ, ws[0], K, N, gpu_x)
    parity = float(np.linalg.norm(gpu_y.astype(np.float64) - y0) / np.linalg.norm(y0))
    runner.matmul(typ, ws[1], K, N, gpu_x)  # warm
    times = []
    t_start = time.perf_counter()
    i = 0
    while time.perf_counter() - t_start < budget_s and i < 100000:
        t0 = time.perf_counter()
        runner.matmul(typ, ws[i % ncop], K, N, gpu_x)
        times.append(time.perf_counter() - t0)
        i += 1
    t_med = float(np.median(times))
    nbytes = algorithmic_bytes(cfg, rb)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(nbytes / t_med / 1e9, 2),
        "unit": "GB/s",
        "cores": runner.threads,
        "kind": kind,
        "sample": f"{len(times)} matvecs of {cfg_name} ({cfg['desc']}) cycling {ncop} weight copies, "
                  f"median {t_med * 1e6:.0f} us; {model}; avx512={oracle_lib.cpu_has_avx512()}",
        "parity_gpu_vs_cpu_normwise": parity,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-sweep", action="store_true", help="skip config 5 (allocates ~15.5 GB)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 16 device-to-device copies of 256 MiB (reference dispatches for the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE calibration) and exit")
    ap.add_argument("--sweep-steps", type=int, default=10)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)

    hiprt = _load("qk_hiprt", os.path.join(PKG, "hiprt.py"))
    qkmod = _load("qk_binding", os.path.join(PKG, "qk.py"))
    hip = hiprt.Hip()
    if hip.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy:
        nbytes = 256 << 20
        src, dst = hiprt.Buf(hip, nbytes), hiprt.Buf(hip, nbytes)
        hip.memset(src.ptr, 1, nbytes)
        for _ in range(16):
            hip.dtod(dst.ptr, src.ptr, nbytes)
        hip.sync()
        print(json.dumps({"calibration": "device-to-device copy", "bytes_per_copy": nbytes, "copies": 16}))
        return
    qk = qkmod.Lib()
    stream = hip.stream_create()
    qk.init_stream(stream)

    def run(name):
        cfg = CONFIGS[name]
        wl = GemvWorkload(hip, hiprt, qk, cfg, stream)
        ms = time_workload(hip, wl, args.steps, args.warmup, stream)
        gbs = wl.bytes_per_step / (ms * 1e-3) / 1e9
        out = dict(ms_per_step=ms, gbs=gbs, bytes_per_step=wl.bytes_per_step, copies=wl.copies)
        if name == args.workload:
            out["kernel_ms_mean"], out["kernel_ms_median"] = kernel_event_ms(hip, wl, 200, stream)
        # GPU output of copy 0 for the CPU-side check
        wl.launch(0)
        hip.stream_sync(stream)
        out["y0"] = wl.y.get(np.float32, (cfg["M"], cfg["N"]))
        out["x"] = wl.x_host
        wl.close()
        return out

    main_cfg = CONFIGS[args.workload]
    r = run(args.workload)
    gemm = main_cfg["kind"] == "gemm"
    # every GEMV config runs the int8 kernel (up to four tokens per launch, gate/up pairs included)
    single = not gemm
    kname = KERNEL_GEMM if gemm else KERNEL_SINGLE if single else KERNEL_NAME[main_cfg["type"]]
    if gemm:  # the M=512 prefill line is MFMA-bound: TFLOP/s against the dense fp16 peak
        flops = 2.0 * main_cfg["M"] * main_cfg["N"] * main_cfg["K"]
        value = flops / (r["ms_per_step"] * 1e-3) / 1e12
        achieved = value  # two kernels per call: the prepass (~5 % of the step) is included
        unit, peak, bound = "TFLOP/s", FP16_DENSE_PEAK_TFLOPS, "mfma"
        timed = "one qk_matmul call = k_gemm_prep_x (x -> fp16 image) + k_gemm"
        dtype = "f16 MFMA operands (weights dequantized with fp16 scales, x rounded to fp16), f32 accumulate"
    else:
        value = r["gbs"]
        achieved = value
        unit, peak, bound = "GB/s", HBM_PEAK_GBS, "hbm"
        if single:
            timed = "one qk_matmul call = k_gemv1 alone (x converted into the int8 image inside)"
            dtype = "i8 MFMA (quant ints; x as two int8 parts per super-block), i32 dot products, f32 scaling"
        else:
            timed = f"one qk_matmul call = k_prep_q{4 if main_cfg['type'] == T_Q4_K else 6} + {kname}"
            dtype = "f16 MFMA operands (exact quant ints, x as fp16 hi+lo pair), f32 accumulate"
    result = {
        "metric": "Q4_K/Q6_K GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOPS at M=512",
        "value": round(value, 1),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(value / REF_PUBLISHED_GBS[args.workload], 3)
                        if args.workload in REF_PUBLISHED_GBS else None),
        "dtype": dtype,
        "data": "synthetic (splitmix64 GGUF blocks, N(0,1) fp32 activations)",
        "config": {"workload": f"{args.workload}: {main_cfg['desc']}", "type": TYPE_NAME[main_cfg["type"]],
                   "M": main_cfg["M"], "K": main_cfg["K"], "N": main_cfg["N"],
                   "weight_copies": r["copies"], "layout": "T16", "timing": "hipGraph of K launches, hipEvents"},
        "pct_of_peak": round(100 * value / peak, 1),
        "roofline": {
            "bound": bound,
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": traffic_from_profiles(kname.split("<")[0], args.workload),
            "kernel": kname,
            "kernel_us": round(r["ms_per_step"] * 1e3, 2),
            "single_launch_us_mean": round(r["kernel_ms_mean"] * 1e3, 2),
            "timed_unit": f"{timed}; achieved = algorithmic {'flops' if gemm else 'bytes'} per call / mean "
                          "duration per call over the K graph-replayed launches, HIP events on the launch stream "
                          "(rocprofv3 kernel trace agrees, profiles/); single_launch_us_mean = one eager launch "
                          "between two events, dispatch latency included",
            "bytes_per_launch": r["bytes_per_step"],
        },
    }
    if not args.no_extras:
        extras = {}
        for name in CONFIGS:
            if name == args.workload:
                continue
            e = run(name)
            cfg = CONFIGS[name]
            if cfg["kind"] == "gemm":
                tflops = 2.0 * cfg["M"] * cfg["N"] * cfg["K"] / (e["ms_per_step"] * 1e-3) / 1e12
                extras[name] = {"desc": cfg["desc"], "tflops": round(tflops, 1),
                                "pct_of_fp16_dense_peak": round(100 * tflops / FP16_DENSE_PEAK_TFLOPS, 1),
                                "us_per_call": round(e["ms_per_step"] * 1e3, 2),
                                "note": "fp16 MFMA operands (weights dequantized with fp16 scales, x rounded "
                                        "to fp16), fp32 accumulate; includes the x-to-fp16 prepass"}
                continue
            extras[name] = {"desc": cfg["desc"], "gbs": round(e["gbs"], 1),
                            "pct_of_hbm_peak": round(100 * e["gbs"] / HBM_PEAK_GBS, 1),
                            "us_per_launch": round(e["ms_per_step"] * 1e3, 2)}
            if name in REF_PUBLISHED_GBS:
                extras[name]["ref_rtx6000d_gbs"] = REF_PUBLISHED_GBS[name]
        if not args.no_sweep:
            wl = SweepWorkload(hip, hiprt, qk, stream)
            ms = time_workload(hip, wl, args.sweep_steps, 2, stream)
            extras["c5"] = {"desc": f"decode-step sweep: {len(wl.mats)} matmuls at M=1 in {len(wl.launches)} "
                                    "grouped launches, "
                                    f"{wl.weight_bytes / 1e9:.2f} GB of weights (synthetic 64-layer stack)",
                            "gbs": round(wl.bytes_per_step / (ms * 1e-3) / 1e9, 1),
                            "pct_of_hbm_peak": round(100 * wl.bytes_per_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                            "ms_per_step": round(ms, 3)}
            wl.close()
        result["extras"] = extras
    if not args.no_cpu and not gemm:
        result["cpu_baseline"] = cpu_baseline(args.workload, main_cfg, r["y0"][0] if main_cfg["M"] == 1 else r["y0"],
                                              r["x"], args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    hip.stream_destroy(stream)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
