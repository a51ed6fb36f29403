#!/usr/bin/env python3
"""Benchmark of the MI355X Q4_K/Q6_K fused-dequant matmul (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2] [--no-cpu] [--no-extras]

A step is one pass of the hot path over one batch of synthetic input: one qk_matmul /
qk_gemv_group call through the C ABI (M=1..8: the int8 GEMV kernel alone, x converted inside;
M>=16: the GEMM kernel on fp16 x as the reference's GEMM takes it, or with fp32 x a rounding pass
first), or for c5 the 257 grouped launches of one decode step.  The K timed steps are captured
once into a HIP graph, replayed untimed until at least 0.2 s of GPU work has run and two replays
agree within 1 % (the steady state of a stream of calls), then replayed once more, timed; every step uses a different weight copy from a ring of copies totalling
>= 512 MiB, so the 256 MiB Infinity Cache cannot serve repeats.  Inputs are resident in HBM before
the timed region; timing uses HIP events on the launch stream.  Every GPU timing runs before any
CPU baseline, so that the GPU never starts a timing from minutes of idleness.

value = algorithmic bytes per step (GGUF weight bytes + fp32 x + fp32 y) / time per step for the
default workload c2 (Q6_K GEMV M=1 K=17408 N=5120).  Every BASELINE config
(c1, c2, c3a, c3b, c4, c5) gets a full measurement row under "configs": its own roofline (achieved
= algorithmic bytes or flops per call / mean call duration of the graph-timed run; traffic = HBM
bytes per launch from the committed rocprofv3 summary in profiles/) and its own cpu_baseline (the
reference's own AVX-512 matvec built from its headers into oracle/_ref, or the repository's CPU
restatement where that cannot run, on the host cores, over a bounded sample of the same workload).
The CPU figure is a reported baseline, not the target.  "extras" holds the other types of a Q4_K_M
file at their shapes, the two other shapes the reference reports, the output projection and the
token embedding, with their rooflines.  C1 and C2 also carry "ceiling_plain_read": a plain streaming
read of the same weight bytes (libqkprobe.so), the practical ceiling beside the 8 TB/s roofline.
"""
import argparse
import ctypes
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
ACT_F32, ACT_F16, ACT_F16_XPERM = 0, 1, 2  # include/qk.h QK_ACT_*
MALL_BYTES = 256 << 20

# BASELINE configs (BASELINE.json "configs"), GEMV family
CONFIGS = {
    "c1": dict(desc="Q4_K GEMV M=1 K=5120 N=17408 (ffn_gate)", kind="gemv", type=T_Q4_K, K=5120, N=17408, M=1, cid=1),
    "c2": dict(desc="Q6_K GEMV M=1 K=17408 N=5120 (ffn_down)", kind="gemv", type=T_Q6_K, K=17408, N=5120, M=1, cid=2),
    "c3a": dict(desc="Q4_K gate+up GLU M=4 K=5120 N=17408x2", kind="glu", type=T_Q4_K, K=5120, N=17408, M=4, cid=3),
    "c3b": dict(desc="Q4_K GEMV M=4 K=5120 N=5120", kind="gemv", type=T_Q4_K, K=5120, N=5120, M=4, cid=3),
    # the GEMMs take fp16 x as the reference's GEMM does (qwen_cuda/qwen.cpp:246): N(0,1) draws rounded to
    # fp16, the CPU baseline fed the same values
    "c4": dict(desc="Q4_K prefill GEMM M=512 K=5120 N=17408 (fp16 x)", kind="gemm", type=T_Q4_K, K=5120, N=17408,
               M=512, cid=4, xf16=True),
    # the same call with fp32 x (rounded to fp16 by k_gemm_cvt_x first)
    "c4_f32x": dict(desc="Q4_K prefill GEMM M=512 K=5120 N=17408 (fp32 x, rounded on the GPU)", kind="gemm",
                    type=T_Q4_K, K=5120, N=17408, M=512, cid=4),
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
    # the two other shapes the reference reports beside C1 / C2 (notes/parallel_decode_experiments.md:111, 116)
    "q4k_down": dict(desc="Q4_K GEMV M=1 K=17408 N=5120 (odd-layer ffn_down)", kind="gemv", type=T_Q4_K, K=17408,
                     N=5120, M=1, cid=12),
    "q6k_gate": dict(desc="Q6_K GEMV M=1 K=5120 N=17408", kind="gemv", type=T_Q6_K, K=5120, N=17408, M=1, cid=13),
    # batched decode below 16 tokens (the reference's GEMV for every T < 16 reads the weights once per
    # eight tokens, NT = 8 at qwen_cuda/kernels.cu:11, qwen.cpp:240-247): one pass here at M=8 and M=13
    "c1_m8": dict(desc="Q4_K matmul M=8 K=5120 N=17408 (C1 shape; qk_matmul's route from 5 tokens: the GEMM, one "
                       "weight pass)", kind="gemv", type=T_Q4_K,
                  K=5120, N=17408, M=8, cid=14),
    "c1_m13": dict(desc="Q4_K matmul M=13 K=5120 N=17408 (C1 shape; qk_matmul's route from 5 tokens: the GEMM, one "
                        "weight pass)", kind="gemv", type=T_Q4_K, K=5120, N=17408, M=13, cid=15),
    "c2_m8": dict(desc="Q6_K matmul M=8 K=17408 N=5120 (C2 shape; qk_matmul's route from 5 tokens: the GEMM, one "
                       "weight pass)", kind="gemv", type=T_Q6_K,
                  K=17408, N=5120, M=8, cid=16),
    "c2_m13": dict(desc="Q6_K matmul M=13 K=17408 N=5120 (C2 shape; qk_matmul's route from 5 tokens: the GEMM, one "
                        "weight pass)", kind="gemv", type=T_Q6_K, K=17408, N=5120, M=13, cid=17),
    # the same 13-token calls on the activations the reference's forward feeds for T < 16: fp16 in its
    # xperm layout (qwen_cuda/qwen.cpp:234), read by the GEMM where they lie
    "c1_m13x": dict(desc="Q4_K matmul M=13 K=5120 N=17408 (C1 shape, fp16 xperm x: the GEMM, one weight pass)",
                    kind="gemv", type=T_Q4_K, K=5120, N=17408, M=13, cid=18, xf16=True, xperm=True),
    "c2_m13x": dict(desc="Q6_K matmul M=13 K=17408 N=5120 (C2 shape, fp16 xperm x: the GEMM, one weight pass)",
                    kind="gemv", type=T_Q6_K, K=17408, N=5120, M=13, cid=19, xf16=True, xperm=True),
    # the decode FFN's gate/up launch at 13 tokens as the reference's forward issues it: fp16 xperm x in,
    # fp16 silu(g) u out at xperm(row) (qwen_cuda/qwen.cpp:264, kernels.cu:419-426); both matrices on the GEMM
    "c3a_m13x": dict(desc="Q4_K gate+up GLU M=13 K=5120 N=17408x2 (C3a shape, fp16 xperm x and output: the GEMM, "
                          "one weight pass)", kind="glu", type=T_Q4_K, K=5120, N=17408, M=13, cid=22, xf16=True,
                     xperm=True, yf16=True),
    "q5k_m512": dict(desc="Q5_K prefill GEMM M=512 K=17408 N=5120 (fp16 x)", kind="gemm", type=T_Q5_K, K=17408,
                     N=5120, M=512, cid=9, xf16=True),
    "q8_0_m512": dict(desc="Q8_0 prefill GEMM M=512 K=6144 N=5120 (fp16 x)", kind="gemm", type=T_Q8_0, K=6144,
                      N=5120, M=512, cid=10, xf16=True),
}
FP16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA headline
BASELINE_CONFIGS = ["c1", "c2", "c3a", "c3b", "c4", "c5"]
EXTRA_CONFIGS = ["q4k_down", "q6k_gate", "q5k", "q8_0", "q5k_m4", "lm_head", "c1_m8", "c1_m13", "c1_m13x", "c2_m8",
                 "c2_m13", "c2_m13x", "c3a_m13x", "c4_f32x", "q5k_m512", "q8_0_m512"]
# token embedding of the output-projection-sized Q6_K table (248320 x 5120, T16 as a GGUF upload
# places it): one decode token and one 1024-token prefill chunk per call
EMBED_CONFIGS = {"embed_m1": 1, "embed_m1024": 1024}
EMBED_K, EMBED_N, EMBED_TYPE = 5120, 248320, T_Q6_K
# the GEMV configs whose weight bytes also get a plain streaming read (the practical ceiling)
CEILING_CONFIGS = ["c1", "c2"]
READ_SHAPES = [(256, 8), (512, 8), (1024, 4), (1024, 8), (2048, 4)]  # (work-groups, loads in flight)
SWEEP_LAYERS = 64
# The reference's own published GEMV bandwidth for the same shapes on an RTX 6000D
# (notes/parallel_decode_experiments.md:111-116 of the reference).
REF_PUBLISHED_GBS = {"c1": 1192.0, "c2": 1214.0, "q4k_down": 1188.0, "q6k_gate": 1205.0}
KERNEL_SINGLE = "k_gemv1"  # M = 1..8 per launch: one kernel, x converted inside
GEMM_ROUTE_M = 5  # qk_matmul sends m >= 5 to the GEMM (include/qk.h)
KERNEL_GEMM = "k_gemm"
KERNEL_EMBED = "k_embed"


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def algorithmic_bytes(cfg, rb):
    nmat = 2 if cfg["kind"] == "glu" else 1
    xb = 2 if cfg.get("xf16") else 4
    yb = 2 if cfg.get("yf16") else 4
    return nmat * cfg["N"] * rb + cfg["M"] * cfg["K"] * xb + cfg["M"] * cfg["N"] * yb


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
        self.xf16 = bool(cfg.get("xf16"))
        if self.xf16:  # fp16 activations: the rounded values are the input, for the CPU side too
            self.x_host = self.x_host.astype(np.float16).astype(np.float32)
        xdev = self.x_host.astype(np.float16) if self.xf16 else self.x_host
        self.xperm = bool(cfg.get("xperm"))
        if self.xperm:  # the reference's decode layout: element i of a row at xperm_pos(i)
            i = np.arange(K)
            cols = (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7)
            xp = np.empty_like(xdev)
            xp[:, cols] = xdev
            xdev = xp
        self.x = hiprt.Buf.of(hip, xdev)
        self.y = hiprt.Buf(hip, M * N * 4)
        self.bytes_per_step = algorithmic_bytes(cfg, self.rb)

    def launch(self, i):
        ws = self.W[i % self.copies]
        if self.nmat == 2 and self.xf16:
            f = ACT_F16_XPERM if self.xperm else ACT_F16
            self.qk.gemv_group_act(ws, [self.y.ptr], True, self.x.ptr, f, self.cfg["M"],
                                   f if self.cfg.get("yf16") else ACT_F32, self.stream)
        elif self.nmat == 2:
            self.qk.gemv_group(ws, [self.y.ptr], True, self.x.ptr, self.cfg["M"], self.stream)
        elif self.xf16:
            self.qk.matmul_act(ws[0], self.x.ptr, ACT_F16_XPERM if self.xperm else ACT_F16, self.cfg["M"], self.y.ptr,
                               self.stream)
        else:
            self.qk.matmul(ws[0], self.x.ptr, self.cfg["M"], self.y.ptr, self.stream)

    def close(self):
        for b in self.bufs:
            b.close()
        self.x.close()
        self.y.close()


class ReadWorkload:
    """A plain streaming read of a GEMV workload's weight copies (the same bytes, the same ring):
    what a kernel that only reads them takes (libqkprobe.so, csrc/qk_probe.hip)."""

    def __init__(self, hip, hiprt, probe, gemv_wl, wgs, unroll, stream):
        self.probe, self.wl, self.wgs, self.unroll, self.stream = probe, gemv_wl, wgs, unroll, stream
        self.sink = hiprt.Buf(hip, 4 * wgs)
        self.bytes_per_step = gemv_wl.wbytes * gemv_wl.nmat

    def launch(self, i):
        w = self.wl.W[i % self.wl.copies][0]
        rc = self.probe.qkp_read(w.data, self.wl.wbytes, self.wgs, self.unroll, self.sink.ptr, self.stream)
        if rc != 0:
            raise RuntimeError("qkp_read failed")

    def close(self):
        self.sink.close()


class EmbedWorkload:
    """qk_embed of m tokens per call from a 248320 x 5120 Q6_K table (T16, as the GGUF upload places
    it); every call takes its own seeded random token ids, so rows come from HBM."""

    def __init__(self, hip, hiprt, qk, m, steps, stream):
        self.hip, self.qk, self.m, self.stream = hip, qk, m, stream
        rb = qk.row_bytes(EMBED_TYPE, EMBED_K)
        nb = EMBED_N * rb
        tmp = hiprt.Buf(hip, nb)
        self.table_buf = hiprt.Buf(hip, nb)
        qk.synth_fill(EMBED_TYPE, SEED_BASE | 14, 0, EMBED_N * (EMBED_K // 256), tmp.ptr)
        self.table = qk.repack(qk.weight_view(tmp.ptr, EMBED_TYPE, EMBED_K, EMBED_N, LAYOUT_GGUF), self.table_buf.ptr,
                               LAYOUT_T16)
        hip.sync()
        tmp.close()
        self.nsets = max(steps, 64)
        rng = np.random.default_rng(SEED_BASE | 14)
        self.tok_host = rng.integers(0, EMBED_N, size=(self.nsets, m), dtype=np.int32)
        self.tokens = hiprt.Buf.of(hip, self.tok_host)
        self.x = hiprt.Buf(hip, m * EMBED_K * 4)
        self.rb = rb
        self.bytes_per_step = m * (rb + 4 * EMBED_K + 4)  # rows read, fp32 rows written, token ids

    def launch(self, i):
        tok = self.tokens.ptr + (i % self.nsets) * self.m * 4
        self.qk.embed(self.table, tok, None, None, self.m, self.x.ptr, self.stream)

    def close(self):
        for b in (self.table_buf, self.tokens, self.x):
            b.close()


WARM_GPU_S = 0.2  # untimed GPU work before each timed replay


def warm_replays(hip, gexec, stream, warm_s):
    """Replays a captured graph untimed until at least warm_s seconds of GPU work have run and two
    consecutive timed batches agree within 1 % (at most 5 * warm_s): the clocks and the TLB are then
    in the state a steady stream of calls keeps them in.  Returns the GPU seconds spent."""
    e0, e1 = hip.event_create(), hip.event_create()
    spent, prev, batch = 0.0, None, 1
    while True:
        hip.event_record(e0, stream)
        for _ in range(batch):
            hip.graph_launch(gexec, stream)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        t = hip.elapsed_ms(e0, e1) * 1e-3
        spent += t
        per = t / batch
        if spent >= 5 * warm_s or (spent >= warm_s and prev is not None and abs(per - prev) <= 0.01 * prev):
            break
        prev = per
        if t < 0.02:  # batches of >= ~20 ms keep the GPU busy between the host's event waits
            batch = min(batch * 2, 1 << 12)
    hip.event_destroy(e0)
    hip.event_destroy(e1)
    return spent


def time_workload(hip, wl, steps, warmup, stream, warm_s=WARM_GPU_S):
    """Warmup eagerly, capture exactly `steps` launches into one graph, replay it untimed until the
    GPU is in steady state (warm_replays), then time exactly one replay (`steps` steps) with events on
    the launch stream, bracketed by device synchronisations.  Returns ms per step."""
    for i in range(warmup):
        wl.launch(i)
    hip.stream_sync(stream)
    hip.begin_capture(stream)
    for i in range(steps):
        wl.launch(i)
    graph, gexec = hip.end_capture(stream)
    warm_replays(hip, gexec, stream, warm_s)
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


def _cpu_runner():
    """The CPU matmul to time: the reference's own (oracle/_ref) where it runs, else the repository's
    restatement.  Returns (runner, oracle, kind, threads, host description)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib

    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    o = oracle_lib.Oracle()
    o.init(threads)
    runner, kind = o, "port"
    if oracle_lib.ref_available():
        runner, kind = oracle_lib.RefLib(), "reference"
        runner.init(threads)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    host = f"{model}; avx512={oracle_lib.cpu_has_avx512()}"
    return runner, o, kind, runner.threads, host


def _timed(runner, mats, xs, T, budget_s):
    """Seconds per pass over `mats`: one untimed pass, then passes until budget_s is spent (median of
    up to 7 batches)."""
    runner.time_seq(mats, xs, T, 1)
    one = max(runner.time_seq(mats, xs, T, 1), 1e-6)
    reps = max(1, int(budget_s / 7 / one))
    times = [runner.time_seq(mats, xs, T, reps) / reps for _ in range(7 if one * reps * 7 <= 2 * budget_s else 3)]
    return float(np.median(times)), reps * len(times)


def cpu_baseline(name, cfg, gpu, budget_s, cpu):
    """Times the CPU matmul for one BASELINE config on the host cores over a bounded sample of the
    same workload, in the unit of the GPU figure, and checks the GPU output against it on the same
    inputs."""
    runner, o, kind, threads, host = cpu
    out = {"unit": "GB/s", "cores": threads, "kind": kind}
    if cfg["kind"] in ("gemv", "glu"):
        typ, K, N, M = cfg["type"], cfg["K"], cfg["N"], cfg["M"]
        nmat = 2 if cfg["kind"] == "glu" else 1
        seed = SEED_BASE | cfg["cid"]
        nblk = N * (K // 256)
        ncop = 4  # 4 x >= 50 MB: beyond the host's last-level cache
        ws = [[o.fill(typ, seed, (c * nmat + j) * nblk, nblk) for j in range(nmat)] for c in range(ncop)]
        x = gpu["x"]
        ys = [runner.matmul(typ, ws[0][j], K, N, x) for j in range(nmat)]
        yc = ys[0] / (1.0 + np.exp(-ys[0].astype(np.float64))) * ys[1] if nmat == 2 else ys[0]
        mats = [(typ, ws[c][j], K, N) for c in range(ncop) for j in range(nmat)]
        t, calls = _timed(runner, mats, [x] * len(mats), M, budget_s)
        per_call = t / ncop
        nbytes = gpu["bytes_per_step"]
        out.update(value=round(nbytes / per_call / 1e9, 2),
                   sample=f"{calls * ncop} calls of {name} ({cfg['desc']}) cycling {ncop} weight copies, "
                          f"{per_call * 1e6:.0f} us per call (median of batches); {host}",
                   parity_gpu_vs_cpu_normwise=float(np.linalg.norm(gpu["y0"] - yc) / np.linalg.norm(yc)))
        return out
    if cfg["kind"] == "gemm":  # C4 on the CPU: the same weights and M=512 fp16-valued activations
        typ, K, N, M = cfg["type"], cfg["K"], cfg["N"], cfg["M"]
        w = o.fill(typ, SEED_BASE | cfg["cid"], 0, N * (K // 256))
        x = gpu["x"].astype(np.float16).astype(np.float32)
        y = runner.matmul(typ, w, K, N, x)
        t, calls = _timed(runner, [(typ, w, K, N)], [x], M, budget_s)
        out.update(value=round(2.0 * M * N * K / t / 1e12, 3), unit="TFLOP/s",
                   sample=f"{calls} calls of {name} ({cfg['desc']}), {t * 1e3:.1f} ms per call; {host}",
                   parity_gpu_vs_cpu_normwise=float(np.linalg.norm(gpu["y0"] - y) / np.linalg.norm(y)))
        return out
    # C5: layers 4..7 of the synthetic stack (three linear-attention layers, one full-attention layer
    # with a Q6_K attn_v; ffn_down Q6_K on the even ones) timed as a sequence, times 16, plus the output
    # projection timed on 1/8 of its rows, times 8
    mats = sweep_matrices()
    seed = SEED_BASE | 5
    sample = [m for m in mats if m[0].split(".")[0] in ("4", "5", "6", "7")]
    ws, xs = [], []
    for i, (_, typ, k, n) in enumerate(sample):
        ws.append((typ, o.fill(typ, seed ^ 0xC5, 10_000_000 * i, n * (k // 256)), k, n))
        xs.append(o.normal(seed + i, k).reshape(1, k))
    t_layers, calls = _timed(runner, ws, xs, 1, budget_s * 0.7)
    _, otyp, ok_, on = mats[-1]
    osub = on // 8
    ow = [(otyp, o.fill(otyp, seed ^ 0xC6, 0, osub * (ok_ // 256)), ok_, osub)]
    t_out, calls_o = _timed(runner, ow, [o.normal(seed + 99, ok_).reshape(1, ok_)], 1, budget_s * 0.3)
    step = 16 * t_layers + 8 * t_out
    out.update(value=round(gpu["bytes_per_step"] / step / 1e9, 2),
               sample=f"layers 4..7 ({len(sample)} matmuls, {calls} passes) x 16 + the output projection on "
                      f"{osub} of its {on} rows ({calls_o} passes) x 8 = {step * 1e3:.1f} ms per decode step; {host}")
    return out


def roofline(name, cfg, ms, nbytes, kernel):
    """The roofline object of one config: HBM-bound GEMVs in GB/s against 8 TB/s, the MFMA-bound
    GEMM in TFLOP/s against the 2.5 PFLOP/s dense fp16 peak."""
    if cfg["kind"] == "gemm":
        ach = 2.0 * cfg["M"] * cfg["N"] * cfg["K"] / (ms * 1e-3) / 1e12
        bound, peak, unit = "mfma", FP16_DENSE_PEAK_TFLOPS, "TFLOP/s"
    else:
        ach = nbytes / (ms * 1e-3) / 1e9
        bound, peak, unit = "hbm", HBM_PEAK_GBS, "GB/s"
    return {"bound": bound, "achieved": round(ach, 1), "peak": peak, "unit": unit, "frac": round(ach / peak, 4),
            "traffic": traffic_from_profiles(kernel, name), "kernel": kernel,
            "kernel_us": round(ms * 1e3, 2), "bytes_per_launch": nbytes}


GEMM_NOTE = ("one call = one k_gemm launch on fp16 x [m][k] read where it lies, the reference's GEMM input "
             "(qwen_cuda/qwen.cpp:246)")
GEMM_NOTE_F32 = ("one call = k_gemm_cvt_x (fp32 x rounded to fp16 [m][k]) + k_gemm; achieved divides by the whole "
                 "call")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(CONFIGS) + ["c5"] + sorted(EMBED_CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="time only --workload (profiling runs)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU timing budget per config (wall seconds)")
    ap.add_argument("--no-sweep", action="store_true", help="skip config 5 (allocates ~15.5 GB)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 16 device-to-device copies of 256 MiB (reference dispatches for the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE calibration) and exit")
    ap.add_argument("--sweep-steps", type=int, default=10)
    ap.add_argument("--tune", action="append", default=[], metavar="NAME=VALUE",
                    help="qk_set_tuning override for measurement sweeps (repeatable)")
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
    for t in args.tune:
        name, value = t.split("=", 1)
        qk.set_tuning(name, int(value))
    stream = hip.stream_create()
    qk.init_stream(stream)
    cpu = None if args.no_cpu else _cpu_runner()

    probe = None
    probe_path = os.path.join(PKG, "libqkprobe.so")
    if os.path.exists(probe_path):
        probe = ctypes.CDLL(probe_path)
        probe.qkp_read.restype = ctypes.c_int
        probe.qkp_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p]

    def run(name, with_events=False):
        """GPU timing of one config (no CPU work): ms per step and what its row needs."""
        if name == "c5":
            wl = SweepWorkload(hip, hiprt, qk, stream)
            ms = time_workload(hip, wl, args.sweep_steps, 2, stream)
            out = dict(ms_per_step=ms, bytes_per_step=wl.bytes_per_step, copies=1, launches=len(wl.launches),
                       matmuls=len(wl.mats), weight_bytes=wl.weight_bytes)
            wl.close()
            return out
        if name in EMBED_CONFIGS:
            wl = EmbedWorkload(hip, hiprt, qk, EMBED_CONFIGS[name], args.steps, stream)
            ms = time_workload(hip, wl, args.steps, args.warmup, stream)
            out = dict(ms_per_step=ms, bytes_per_step=wl.bytes_per_step, m=wl.m, row_bytes=wl.rb)
            wl.close()
            return out
        cfg = CONFIGS[name]
        wl = GemvWorkload(hip, hiprt, qk, cfg, stream)
        ms = time_workload(hip, wl, args.steps, args.warmup, stream)
        out = dict(ms_per_step=ms, bytes_per_step=wl.bytes_per_step, copies=wl.copies)
        if with_events:
            out["kernel_ms_mean"], out["kernel_ms_median"] = kernel_event_ms(hip, wl, 200, stream)
        if name in CEILING_CONFIGS and probe is not None:
            reads = []
            for wgs, unroll in READ_SHAPES:
                rw = ReadWorkload(hip, hiprt, probe, wl, wgs, unroll, stream)
                reads.append((time_workload(hip, rw, args.steps, args.warmup, stream, warm_s=0.05), wgs, unroll))
                rw.close()
            rms, wgs, unroll = min(reads)
            nbytes = wl.wbytes * wl.nmat
            out["ceiling"] = {
                "what": "plain streaming read of the same weight bytes and copies (libqkprobe.so k_read: "
                        "non-temporal 16-byte loads, contiguous per work-group), best of the read shapes",
                "bytes": nbytes, "us": round(rms * 1e3, 2), "gbs": round(nbytes / (rms * 1e-3) / 1e9, 1),
                "pct_of_hbm_peak": round(100 * nbytes / (rms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                "best_shape": {"work_groups": wgs, "loads_in_flight": unroll},
                "all_us": {f"{g}x{u}": round(t * 1e3, 2) for t, g, u in reads}}
        wl.launch(0)  # GPU output of copy 0 for the CPU-side check
        hip.stream_sync(stream)
        out["y0"] = wl.y.get(np.float32, (cfg["M"], cfg["N"]))
        out["x"] = wl.x_host
        wl.close()
        return out

    def row(name, r):
        """The measurement row of one config: value, roofline, cpu_baseline."""
        if name == "c5":
            ms = r["ms_per_step"]
            gbs = r["bytes_per_step"] / (ms * 1e-3) / 1e9
            rf = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(KERNEL_SINGLE, "c5"),
                  "kernel": f"{KERNEL_SINGLE} (every launch of the step)",
                  "kernel_us": round(ms * 1e3, 1), "bytes_per_launch": r["bytes_per_step"],
                  "timed_unit": f"one decode step = {r['launches']} grouped launches of {r['matmuls']} matmuls, "
                                "graph-replayed; traffic is per step"}
            d = {"desc": f"decode-step sweep: {r['matmuls']} matmuls at M=1 in {r['launches']} grouped launches, "
                         f"{r['weight_bytes'] / 1e9:.2f} GB of weights (synthetic 64-layer stack)",
                 "gbs": round(gbs, 1), "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                 "ms_per_step": round(ms, 3), "roofline": rf}
        elif name in EMBED_CONFIGS:
            ms = r["ms_per_step"]
            gbs = r["bytes_per_step"] / (ms * 1e-3) / 1e9
            rf = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(KERNEL_EMBED, name),
                  "kernel": KERNEL_EMBED, "kernel_us": round(ms * 1e3, 2), "bytes_per_launch": r["bytes_per_step"],
                  "timed_unit": f"one qk_embed call of {r['m']} tokens: {r['row_bytes']} B of Q6_K row read and "
                                f"{4 * EMBED_K} B of fp32 written per token"}
            d = {"desc": f"token embedding, {r['m']} token(s) per call from the {EMBED_N} x {EMBED_K} Q6_K table "
                         "(T16 layout, random ids)",
                 "gbs": round(gbs, 1), "us_per_call": round(ms * 1e3, 2), "roofline": rf}
        else:
            cfg = CONFIGS[name]
            routed = cfg["kind"] in ("gemv", "glu") and cfg["M"] >= GEMM_ROUTE_M  # the GEMM route
            kernel = KERNEL_GEMM if cfg["kind"] == "gemm" or routed else KERNEL_SINGLE
            rf = roofline(name, cfg, r["ms_per_step"], r["bytes_per_step"], kernel)
            d = {"desc": cfg["desc"]}
            if cfg["kind"] == "gemm":
                d.update(tflops=rf["achieved"], pct_of_fp16_dense_peak=round(100 * rf["frac"], 1),
                         us_per_call=rf["kernel_us"])
                rf["timed_unit"] = GEMM_NOTE if cfg.get("xf16") else GEMM_NOTE_F32
            else:
                d.update(gbs=rf["achieved"], pct_of_hbm_peak=round(100 * rf["frac"], 1), us_per_launch=rf["kernel_us"])
                rf["timed_unit"] = ("one call = one k_gemv1 launch (x converted into the int8 image inside)"
                                    if not routed else
                                    "one qk_gemv_group_act call of the gate/up pair on fp16 xperm x, which it "
                                    "sends to the GEMM from 5 tokens: both matrices in one k_gemm launch, then "
                                    "k_glu_sum adds the K-parts and writes fp16 silu(g) u at xperm(row); one "
                                    "weight pass"
                                    if cfg["kind"] == "glu" else
                                    "one qk_matmul_act call on fp16 x in the xperm layout, which it sends to the "
                                    "GEMM from 5 tokens: k_gemm reading x where it lies, in work-groups of one "
                                    "32-token block (+ the split-K sum), one weight pass"
                                    if cfg.get("xperm") else
                                    "one qk_matmul call, which sends m >= 5 to the GEMM: k_gemm_cvt_x (fp32 x "
                                    "rounded to fp16) + k_gemm in work-groups of one 32-token block (+ the split-K "
                                    "sum), one weight pass")
            if name in REF_PUBLISHED_GBS:
                d["ref_rtx6000d_gbs"] = REF_PUBLISHED_GBS[name]
            if "ceiling" in r:
                c = dict(r["ceiling"])
                c["gemv_frac_of_ceiling"] = round(r["ceiling"]["us"] / rf["kernel_us"], 3)
                d["ceiling_plain_read"] = c
            d["roofline"] = rf
        if cpu is not None and name in BASELINE_CONFIGS and (name != "c5" or not args.no_sweep):
            cfg = CONFIGS.get(name, {"kind": "sweep"})
            d["cpu_baseline"] = cpu_baseline(name, cfg, r, args.cpu_seconds, cpu)
        return d

    main_name = args.workload
    names = [main_name]
    if not args.no_extras:
        names += [n for n in BASELINE_CONFIGS if n != main_name and not (n == "c5" and args.no_sweep)]
        names += [n for n in EXTRA_CONFIGS + list(EMBED_CONFIGS) if n != main_name]
    # every GPU timing first, back to back; the CPU baselines (minutes of host work, GPU idle) after
    runs = {n: run(n, with_events=n == main_name and n != "c5" and n not in EMBED_CONFIGS) for n in names}
    rows = {n: row(n, runs[n]) for n in names}
    r, main_row = runs[main_name], rows[main_name]
    rf = dict(main_row["roofline"])
    if "kernel_ms_mean" in r:
        rf["single_launch_us_mean"] = round(r["kernel_ms_mean"] * 1e3, 2)
    cfgd = CONFIGS.get(main_name)
    gemm = cfgd is not None and cfgd["kind"] == "gemm"
    # dtype: the MFMA operand type of the path; numerics: what is computed in it
    if gemm:
        dtype, numerics = "f16", "f16 MFMA operands (weights dequantized with fp16 scales, x rounded to fp16), f32 accumulate"
    else:
        dtype, numerics = "i8", ("i8 MFMA on the quant ints and x as three int8 parts per super-block (each "
                                 "element within max|x|/16387064), i32 dot products, f32 scaling")
    if main_name in EMBED_CONFIGS:
        dtype, numerics = "f32", "bit-exact fp32 dequant of the quantized rows (qwen_cpu/quants.h dequant_row)"
    result = {
        "metric": "Q4_K/Q6_K GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOPS at M=512",
        "value": rf["achieved"],
        "unit": rf["unit"],
        "n_gpus": 1,
        "steps": args.steps if main_name != "c5" else args.sweep_steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(rf["achieved"] / REF_PUBLISHED_GBS[main_name], 3)
                        if main_name in REF_PUBLISHED_GBS else None),
        "dtype": dtype,
        "numerics": numerics,
        "data": "synthetic (splitmix64 GGUF blocks, N(0,1) fp32 activations)",
        "config": ({"workload": f"{main_name}: {cfgd['desc']}", "type": TYPE_NAME[cfgd["type"]], "M": cfgd["M"],
                    "K": cfgd["K"], "N": cfgd["N"], "weight_copies": r["copies"], "layout": "T16",
                    "timing": "hipGraph of K launches, hipEvents"} if cfgd else
                   {"workload": f"{main_name}: {main_row['desc']}", "timing": "hipGraph of K steps, hipEvents"}),
        "pct_of_peak": round(100 * rf["frac"], 1),
        "roofline": rf,
        "cpu_baseline": main_row.get("cpu_baseline"),
    }
    if "ceiling_plain_read" in main_row:
        result["ceiling_plain_read"] = main_row["ceiling_plain_read"]
    if not args.no_extras:
        # C1 beside C2 at the top: the metric names both M=1 types
        if "c1" in rows and main_name != "c1":
            result["c1"] = {k: rows["c1"][k] for k in ("gbs", "pct_of_hbm_peak", "us_per_launch")}
            result["c1"]["roofline_frac"] = rows["c1"]["roofline"]["frac"]
            if "ceiling_plain_read" in rows["c1"]:
                result["c1"]["ceiling_plain_read_us"] = rows["c1"]["ceiling_plain_read"]["us"]
        result["configs"] = {k: rows[k] for k in BASELINE_CONFIGS if k in rows}
        result["extras"] = {k: rows[k] for k in EXTRA_CONFIGS + list(EMBED_CONFIGS) if k in rows}
    hip.stream_destroy(stream)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
