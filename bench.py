#!/usr/bin/env python3
"""Benchmark of the MI355X AWA path on the 33-frame 256x256 DiT attention stack.

Workload: the AWA layer of all 32 DiT blocks at latent 9x16x16 (N = 2304
video tokens), window counts (3, 8, 8) -> 3x8x8 windows, 64 text tokens,
20 heads x 128. Blocks 0-8 compute in fp32, blocks 9-31 in bf16; even blocks
use unshifted windows (12 windows of 256 tokens), odd blocks shifted ones
(36 ragged windows of 80..256 tokens). Every block reads its own QKV (fp32 or
bf16, synthetic N(0,1) generated on the device and resident in HBM before
timing) and writes its own outputs. One step = the 32 layers on one stream,
including the fp32 -> bf16 conversion at block 9.

Prints one JSON line: the step's window-attention throughput (TFLOP/s over
the algorithmic FLOPs sum_w 4 L_w^2 d H), ms per step, the bf16 layers' share
of bf16 MFMA peak, the roofline entry of the dominant attention kernel (the
fp32 or bf16 instance with the larger share of the step, timed with HIP
events on the stack's stream; HBM-bound when its arithmetic intensity is
below the ridge point, MFMA-bound otherwise) and the CPU baseline (the
oracle's single-threaded restatement of the reference's CPU layer, on a
bounded sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "seedvr2-ncnn_amd"))

METRIC = "window-attn TFLOP/s & % bf16 MFMA peak; ms per 32-block DiT step, 33f 256²"
GRID = (9, 16, 16)
WINDOWS = (3, 8, 8)
TEXT = 64
HEADS = 20
HEAD_DIM = 128
BLOCKS = 32
FP32_PREFIX = 9
PEAK_BF16 = 2.5e15
PEAK_FP32 = 157.3e12
PEAK_HBM = 8.0e12
# MI355X peak engine clock and SIMDs (256 CUs x 4): the MFMA instruction roof
# of a kernel is its MFMA cycles spread evenly over the SIMDs at this clock.
PEAK_CLOCK_HZ = 2.4e9
SIMDS = 1024


def cpu_baseline(sample_layers: int) -> dict:
    """Single-threaded CPU restatement of the reference's CPU AWA forward
    (Pack -> MMRoPE -> WindowAttention -> Unpack in the reference's loop order)
    on one unshifted and one shifted layer of this workload, projected to the
    32-block step (16 layers of each)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.set_num_threads(1)
    times = []
    flops = []
    for shifted in (False, True)[:sample_layers]:
        g = O.Geometry(*GRID, *WINDOWS, TEXT, shifted)
        n = g.source_tokens * 3 * HEADS * HEAD_DIM
        video = O.fill_gaussian(n, 20260825, 0).reshape(g.source_tokens, 3, HEADS, HEAD_DIM)
        text = O.fill_gaussian(TEXT * 3 * HEADS * HEAD_DIM, 20260825, 1).reshape(TEXT, 3, HEADS, HEAD_DIM)
        cu = O.build_maps(g).cu_seqlens
        flops.append(float(sum(4.0 * (b - a) ** 2 * HEAD_DIM * HEADS for a, b in zip(cu[:-1], cu[1:]))))
        t0 = time.perf_counter()
        O.awa_layer(g, video, text, HEADS, HEAD_DIM, attention_order="cpu", text_order="cpu")
        times.append(time.perf_counter() - t0)
    step_s = 16.0 * sum(times) * (2 / len(times))
    step_flops = 16.0 * sum(flops) * (2 / len(flops))
    # The same layers with the oracle's (window, head) loops on every usable
    # host core: not the reference's single-threaded CPU layers.
    cores = len(os.sched_getaffinity(0))
    O.set_num_threads(cores)
    times_mt = []
    for shifted in (False, True)[:sample_layers]:
        g = O.Geometry(*GRID, *WINDOWS, TEXT, shifted)
        n = g.source_tokens * 3 * HEADS * HEAD_DIM
        video = O.fill_gaussian(n, 20260825, 0).reshape(g.source_tokens, 3, HEADS, HEAD_DIM)
        text = O.fill_gaussian(TEXT * 3 * HEADS * HEAD_DIM, 20260825, 1).reshape(TEXT, 3, HEADS, HEAD_DIM)
        t0 = time.perf_counter()
        O.awa_layer(g, video, text, HEADS, HEAD_DIM, attention_order="cpu", text_order="cpu")
        times_mt.append(time.perf_counter() - t0)
    O.set_num_threads(1)
    step_mt = 16.0 * sum(times_mt) * (2 / len(times_mt))
    return {
        "value": step_flops / step_s / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "host": host_cpu(),
        "kind": "port",
        "sample": (f"one unshifted and one shifted fp32 layer of this workload ({', '.join(f'{t:.2f}' for t in times)} s), "
                   f"single thread, reference CPU loop order; projected 32-block step {step_s * 1e3:.0f} ms"),
        "ms_per_step": step_s * 1e3,
        "all_cores": {
            "value": step_flops / step_mt / 1e12,
            "unit": "TFLOP/s",
            "cores": cores,
            "ms_per_step": step_mt * 1e3,
            "sample": (f"the same layers ({', '.join(f'{t:.2f}' for t in times_mt)} s) with the (window, head) loops "
                       f"on {cores} threads (OpenMP); not the reference's single-threaded layers"),
        },
    }


def qk_prologue(A, bufs, stream, iters: int = 20) -> dict:
    """The DiT block's QKV prologue at a bf16 block of the same workload (raw
    bf16 QKV projection, bf16 MFMA, bf16 outputs): q/k RMSNorm fused into the
    AWA gather (awa_forward_qknorm) against the reference's data flow, which
    normalises Q and K into an fp32 QKV, promotes V to it and runs the layer
    on that (DitRMSNorm x 4 + DitQKVConcat + AWA; here awa_rmsnorm x 4 +
    awa_cast x 2 + awa_forward). ms per layer, HIP events over `iters` layers."""
    t, h, w = GRID
    N = t * h * w
    row = HEADS * HEAD_DIM
    gam = [A.DeviceBuffer(HEAD_DIM * 4) for _ in range(4)]
    rng = np.random.RandomState(7)
    for g in gam:
        g.upload(rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32))
    norm = A.AwaQkNorm(*[g.ptr for g in gam], 1e-5)
    raw = {"video": (bufs[0].ptr, N), "text": (bufs[1].ptr, TEXT)}
    f32 = {k: A.DeviceBuffer(n * 3 * row * 4) for k, (_, n) in raw.items()}
    vo, to = bufs[2].ptr, bufs[3].ptr
    qkv = lambda ptr, n, es: A.mat(ptr, HEAD_DIM, 3 * HEADS, n, es)
    part = lambda ptr, n, es, k: A.mat(ptr + k * row * es, HEAD_DIM, HEADS, n, es, cstep=3 * row)
    out_v, out_t = A.mat(vo, HEAD_DIM, HEADS, N, 2), A.mat(to, HEAD_DIM, HEADS, TEXT, 2)
    res = {}
    for shifted in (False, True):
        plan = A.Plan(A.LayerParams(t, h, w, *WINDOWS, TEXT, shifted))
        plan.upload()

        def fused():
            plan.forward_qknorm(qkv(raw["video"][0], N, 2), qkv(raw["text"][0], TEXT, 2), norm, out_v, out_t,
                                A.COMPUTE_BF16, stream)

        def unfused():
            for key, (gq, gk) in (("video", (gam[0], gam[1])), ("text", (gam[2], gam[3]))):
                ptr, n = raw[key]
                dst = f32[key].ptr
                A.rmsnorm(part(ptr, n, 2, 0), gq.ptr, 1e-5, part(dst, n, 4, 0), stream)
                A.rmsnorm(part(ptr, n, 2, 1), gk.ptr, 1e-5, part(dst, n, 4, 1), stream)
                A.cast(part(ptr, n, 2, 2), part(dst, n, 4, 2), stream)
            plan.forward(qkv(f32["video"].ptr, N, 4), qkv(f32["text"].ptr, TEXT, 4), out_v, out_t,
                         A.COMPUTE_BF16, stream)

        times = {}
        for name, fn in (("fused_ms", fused), ("unfused_ms", unfused)):
            for _ in range(3):
                fn()
            e0, e1 = A.Event(), A.Event()
            e0.record(stream)
            for _ in range(iters):
                fn()
            e1.record(stream)
            stream.synchronize()
            times[name] = round(e0.elapsed_ms(e1) / iters, 5)
        times["speedup"] = round(times["unfused_ms"] / times["fused_ms"], 3)
        res["shifted" if shifted else "unshifted"] = times
        plan.destroy()
    res["data"] = "bf16 raw QKV projection of a bf16 block, gammas U(0.5, 1.5), eps 1e-5"
    return res


def host_cpu() -> dict:
    """The host the CPU baseline ran on: model name, logical CPUs, and the
    CPUs this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}


# The workloads the metric is quoted on: the 1-frame 256x256 fp32 image
# layer, a 5-frame bf16 clip (shifted), the 33-frame 256x256 mixed step, a
# 33-frame 512x512 bf16 clip and a 121-frame 256x256 bf16 clip. Each runs as
# a stack of attention layers with even layers unshifted and odd layers
# shifted: (latent t, h, w), window counts, arithmetic, the layers it is
# quoted on.
CONFIGS = {
    "fp32_image_1x16x16": ((1, 16, 16), (1, 8, 8), "fp32", ("unshifted",)),
    "bf16_shifted_clip_2x16x16": ((2, 16, 16), (1, 8, 8), "bf16", ("shifted",)),
    "mixed_step_9x16x16": ((9, 16, 16), (3, 8, 8), "mixed", ("unshifted", "shifted")),
    "bf16_clip_512_9x32x32": ((9, 32, 32), (3, 8, 8), "bf16", ("unshifted", "shifted")),
    "bf16_clip_121f_31x16x16": ((31, 16, 16), (8, 8, 8), "bf16", ("unshifted", "shifted")),
    # The production 256x256 image layer (windows (4, 3, 3): one 16 x 16
    # window of 256 + 64 rows, 20 units; the fp32 layer splits its keys).
    "fp32_production_256": ((1, 16, 16), (4, 3, 3), "fp32", ("unshifted",)),
    "bf16_production_256": ((1, 16, 16), (4, 3, 3), "bf16", ("unshifted",)),
}
MALL_BYTES = 256 * 1024 * 1024


def mfma_instruction_roof_ms(A, grid, windows, shifted: bool, label: str) -> float:
    """Time the layer's attention kernel needs for its MFMA instructions
    alone, at the peak clock with every SIMD busy. Each 32-row wave of a
    (window, head) unit covers all of the unit's keys; a 32x32x16 bf16 and a
    32x32x32 int8 MFMA each keep a SIMD busy 32 cycles. bf16 kernel: 32 MFMAs
    per wave and 64-key tile (16 for S^T = K Q^T, 16 for O^T += V^T P^T).
    Exact-score fp32 kernel: 88 per wave and 32-key tile (40 int8 for the
    score classes, 48 bf16 for the three-piece PV)."""
    plan = A.Plan(A.LayerParams(*grid, *windows, TEXT, shifted))
    wins = plan.windows()
    plan.destroy()
    mfmas = 0
    for t0, t1, h0, h1, w0, w1 in wins:
        L = (t1 - t0) * (h1 - h0) * (w1 - w0) + TEXT
        waves = -(-L // 32)
        mfmas += waves * (-(-L // 64) * 32 if label == "bf16" else -(-L // 32) * 88)
    return mfmas * HEADS * 32 / SIMDS / PEAK_CLOCK_HZ * 1e3


def key_segments(A, grid, windows, shifted: bool, label: str) -> int:
    """Key segments per (window, head) unit the layer's attention uses (1:
    one workgroup per query block; more: the keys split over workgroups and
    combined by a second kernel, which the layer time includes)."""
    plan = A.Plan(A.LayerParams(*grid, *windows, TEXT, shifted))
    plan.upload()
    s = plan.attention_split(HEADS, A.COMPUTE_F32 if label == "fp32" else A.COMPUTE_BF16)
    plan.destroy()
    return s


def config_measurements(A, stream, steps: int = 10, profile_steps: int = 5) -> dict:
    """Every workload above in two regimes. HBM-cold: every layer reads its
    own inputs and the stack's inputs and outputs total at least 1 GiB (four
    times the 256 MB Infinity Cache), so no layer finds its data cached.
    MALL-warm: every layer of the stack reads the same inputs, which stay in
    the Infinity Cache after the first. Per layer (median over the stack's
    unshifted or shifted layers, HIP events around each): the attention
    kernel and the whole layer (kernel + text mean), TFLOP/s, the share of
    the bf16 MFMA peak and the roofline fraction (F/t) / min(P, AI * 8 TB/s)
    with P the MFMA peak of the layer's arithmetic; and ms per 32-layer step."""
    out = {}
    for name, (grid, windows, arith, quoted) in CONFIGS.items():
        t, h, w = grid
        N = t * h * w
        per_block = lambda es: (N + TEXT) * HEADS * HEAD_DIM * 4 * es
        res = {"latent": list(grid), "window_counts": list(windows), "arithmetic": arith}
        for regime in ("hbm_cold", "mall_warm"):
            blocks = 32
            if regime == "hbm_cold" and arith != "mixed":
                need = -(-(4 * MALL_BYTES) // per_block(4 if arith == "fp32" else 2))
                blocks = max(32, need + (need & 1))
            prefix = {"fp32": blocks, "bf16": 0, "mixed": FP32_PREFIX}[arith]
            stack = A.AttentionStack(t, h, w, *windows, TEXT, blocks, prefix, HEADS, HEAD_DIM)
            keep, ptrs = [], [[], [], [], []]
            shared = {}
            for b in range(blocks):
                es = 4 if b < prefix else 2
                if regime == "mall_warm" and es in shared:
                    bufs = shared[es]
                else:
                    bufs = [A.DeviceBuffer(N * 3 * HEADS * HEAD_DIM * es), A.DeviceBuffer(TEXT * 3 * HEADS * HEAD_DIM * es),
                            A.DeviceBuffer(N * HEADS * HEAD_DIM * es), A.DeviceBuffer(TEXT * HEADS * HEAD_DIM * es)]
                    bufs[0].fill_normal(N * 3 * HEADS * HEAD_DIM, es, 7000 + 2 * b, stream)
                    bufs[1].fill_normal(TEXT * 3 * HEADS * HEAD_DIM, es, 7001 + 2 * b, stream)
                    keep.append(bufs)
                    shared[es] = bufs
                for i in range(4):
                    ptrs[i].append(bufs[i].ptr)
            stream.synchronize()
            for _ in range(3):
                stack.run(*ptrs, stream)
            e0, e1 = A.Event(), A.Event()
            e0.record(stream)
            for _ in range(steps):
                stack.run(*ptrs, stream)
            e1.record(stream)
            stream.synchronize()
            step_ms = e0.elapsed_ms(e1) / steps
            stack.set_profiling(True)
            att = np.zeros((profile_steps, blocks))
            lay = np.zeros((profile_steps, blocks))
            for s in range(profile_steps):
                stack.run(*ptrs, stream)
                stream.synchronize()
                att[s], lay[s] = stack.block_times()
            flops = stack.block_flops()
            stack.destroy()
            del keep, shared
            entry = {"layers_in_stack": blocks,
                     "ms_per_32_layers": round(step_ms * 32 / blocks, 4),
                     "step_input_mb": round(sum(per_block(4 if b < prefix else 2) for b in range(blocks)) / 1e6
                                            if regime == "hbm_cold" else 0.0, 1)}
            for kind in quoted:
                for label, precision in (("fp32", range(prefix)), ("bf16", range(prefix, blocks))):
                    idx = np.array([b for b in precision if (b & 1) == (kind == "shifted")], dtype=int)
                    if idx.size == 0:
                        continue
                    k_ms = float(np.median(att[:, idx]))
                    l_ms = float(np.median(lay[:, idx]))
                    fl = float(flops[idx].mean())
                    es = 4 if label == "fp32" else 2
                    alg = float(per_block(es))
                    peak = PEAK_FP32 if label == "fp32" else PEAK_BF16
                    roof = min(peak, fl / alg * PEAK_HBM)
                    key = kind if arith != "mixed" else f"{label}_{kind}"
                    entry[key] = {
                        "kernel_ms": round(k_ms, 5), "layer_ms": round(l_ms, 5),
                        "gflop": round(fl / 1e9, 3), "algorithmic_mb": round(alg / 1e6, 2),
                        "tflops": round(fl / (k_ms * 1e-3) / 1e12, 2),
                        "layer_tflops": round(fl / (l_ms * 1e-3) / 1e12, 2),
                        "pct_bf16_peak": round(100.0 * fl / (k_ms * 1e-3) / PEAK_BF16, 2),
                        "roofline_frac": round(fl / (k_ms * 1e-3) / roof, 4),
                        "layer_roofline_frac": round(fl / (l_ms * 1e-3) / roof, 4),
                        "roof": "hbm" if roof < peak else ("mfma_fp32" if label == "fp32" else "mfma_bf16"),
                        "key_segments": key_segments(A, grid, windows, kind == "shifted", label),
                    }
            res[regime] = entry
        out[name] = res
    return out


def cpu_baseline_image() -> dict:
    """The reference's CPU semantics on its CPU-runnable case, the fp32
    image layer (1x16x16, windows 1x8x8, 64 text tokens, 20 heads): the
    oracle's single-threaded restatement of the CPU forward, whole layer."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.set_num_threads(1)
    g = O.Geometry(1, 16, 16, 1, 8, 8, TEXT, False)
    video = O.fill_gaussian(g.source_tokens * 3 * HEADS * HEAD_DIM, 20260823, 0).reshape(g.source_tokens, 3, HEADS,
                                                                                      HEAD_DIM)
    text = O.fill_gaussian(TEXT * 3 * HEADS * HEAD_DIM, 20260823, 1).reshape(TEXT, 3, HEADS, HEAD_DIM)
    cu = O.build_maps(g).cu_seqlens
    flops = float(sum(4.0 * (b - a) ** 2 * HEAD_DIM * HEADS for a, b in zip(cu[:-1], cu[1:])))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        O.awa_layer(g, video, text, HEADS, HEAD_DIM, attention_order="cpu", text_order="cpu")
        times.append(time.perf_counter() - t0)
    s = float(np.median(times))
    return {"ms_per_layer": round(s * 1e3, 2), "tflops": flops / s / 1e12, "cores": 1, "kind": "port",
            "sample": "the whole fp32 image layer, median of 3 runs, single thread, reference CPU loop order",
            "host": host_cpu()}


MLP_HIDDEN = 6912  # SwiGLU hidden width for hidden 2560 (tools/reference/dit_block.py:195-197)


def dit_step(A, stream, steps: int, warmup: int = 2) -> dict:
    """The whole DiT step at the same workload: 32 full blocks (RMSNorm + Ada,
    QKV projection, AWA with the fused q/k norm, output projection, gate +
    residual, SwiGLU MLP, gate + residual; video and text branches; the last
    block video-only) with blocks 0-8 in fp32 and 9-31 in bf16. Random-init
    weights N(0, 0.02) (Ada vectors and gammas included), fp32 inputs N(0, 1),
    all resident on the device before timing. ms per step over `steps` steps
    (HIP events), per-block times from a profiled step, and the GEMM + attention
    FLOPs of the step."""
    t, h, w = GRID
    N = t * h * w
    hidden, hd, mh = HEADS * HEAD_DIM, HEADS * HEAD_DIM, MLP_HIDDEN
    stack = A.DitStack(t, h, w, *WINDOWS, TEXT, BLOCKS, FP32_PREFIX, HEADS, HEAD_DIM, hidden, mh)
    keep = []
    seed = [9000]

    def buf(count, es, stddev=0.02):
        b = A.DeviceBuffer(count * es)
        b.fill_normal(count, es, seed[0], stream, stddev)
        seed[0] += 1
        keep.append(b)
        return b.ptr

    wv, wt = [], []
    for b in range(BLOCKS):
        es = 4 if b < FP32_PREFIX else 2
        for lst in (wv, wt):
            # proj_in_gate and proj_in in one allocation, back to back (the
            # block then runs them as one GEMM).
            mlp_pair = buf(2 * mh * hidden, es)
            lst.append(A.AwaDitBranchWeights(
                buf(3 * hd * hidden, es), buf(hidden * hd, es), buf(hidden, 4), mlp_pair,
                mlp_pair + mh * hidden * es, buf(hidden * mh, es), buf(HEAD_DIM, 4), buf(HEAD_DIM, 4),
                buf(6 * hidden, 4)))
    video, text, emb = buf(N * hidden, 4, 1.0), buf(TEXT * hidden, 4, 1.0), buf(6 * hidden, 4, 1.0)
    vout, tout = buf(N * hidden, 2, 1.0), buf(TEXT * hidden, 2, 1.0)
    stream.synchronize()
    for _ in range(warmup):
        stack.run(wv, wt, video, text, emb, vout, tout, stream)
    e0, e1 = A.Event(), A.Event()
    e0.record(stream)
    for _ in range(steps):
        stack.run(wv, wt, video, text, emb, vout, tout, stream)
    e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    stack.set_profiling(True)
    stack.run(wv, wt, video, text, emb, vout, tout, stream)
    stream.synchronize()
    per_block = stack.block_times()
    stack.destroy()

    def gemm_flops(m, last_text=False):
        f = 2.0 * m * hidden * (3 * hd) + 2.0 * m * hd * hidden
        return f if last_text else f + 3 * 2.0 * m * hidden * mh

    att = A.AttentionStack(t, h, w, *WINDOWS, TEXT, BLOCKS, FP32_PREFIX, HEADS, HEAD_DIM)
    att_flops = float(att.block_flops().sum())
    att.destroy()
    flops = BLOCKS * gemm_flops(N) + (BLOCKS - 1) * gemm_flops(TEXT) + gemm_flops(TEXT, True) + att_flops
    return {
        "ms_per_step": round(ms, 3),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "step_gflop": round(flops / 1e9, 1),
        "fp32_block_ms": round(float(per_block[:FP32_PREFIX].mean()), 4),
        "bf16_block_ms": round(float(per_block[FP32_PREFIX:].mean()), 4),
        "steps": steps,
        "config": "32 blocks, hidden 2560, SwiGLU 6912, 20x128 heads, latent 9x16x16, windows 3x8x8, 64 text; "
                  "blocks 0-8 fp32, 9-31 bf16; GEMMs on hipBLASLt",
        "data": "random-init weights N(0, 0.02), inputs N(0, 1), synthetic",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--profile-steps", type=int, default=5, help="steps with per-block event timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dit-step", action="store_true", help="skip the full 32-block DiT step measurement")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-workload table (every quoted workload, HBM-cold and MALL-warm)")
    ap.add_argument("--dit-steps", type=int, default=5)
    ap.add_argument("--cpu-sample-layers", type=int, default=2, choices=(1, 2))
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "awa_attention_hbm_traffic.json"),
                    help="measured HBM bytes per launch of each attention kernel (rocprofv3 --pmc FETCH_SIZE and "
                         "WRITE_SIZE, scaled by the copy calibration)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 plain 64 MiB fp32 device copies (awa_cast), the known-size reference the "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by, and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import awa_hip as A

    A.init(0)
    if args.copy_calibration:
        n = 64 * 1024 * 1024 // 4
        src, dst = A.DeviceBuffer(n * 4), A.DeviceBuffer(n * 4)
        src.fill_normal(n, 4, 3)
        bi, bo = A.mat(src.ptr, 1024, 1024, 16, 4), A.mat(dst.ptr, 1024, 1024, 16, 4)
        for _ in range(5):
            A.cast(bi, bo)
        A.synchronize()
        print("copy calibration: 5 x 64 MiB fp32 device copies (read 64 MiB + write 64 MiB each)", flush=True)
        return 0
    t, h, w = GRID
    N = t * h * w
    row_qkv = 3 * HEADS * HEAD_DIM
    row_out = HEADS * HEAD_DIM
    buffers = []
    vq, tq, vo, to = [], [], [], []
    for b in range(BLOCKS):
        es = 4 if b < FP32_PREFIX else 2
        bufs = [A.DeviceBuffer(N * row_qkv * es), A.DeviceBuffer(TEXT * row_qkv * es),
                A.DeviceBuffer(N * row_out * es), A.DeviceBuffer(TEXT * row_out * es)]
        bufs[0].fill_normal(N * row_qkv, es, 20260825 * 64 + 2 * b)
        bufs[1].fill_normal(TEXT * row_qkv, es, 20260825 * 64 + 2 * b + 1)
        buffers.append(bufs)
        vq.append(bufs[0].ptr)
        tq.append(bufs[1].ptr)
        vo.append(bufs[2].ptr)
        to.append(bufs[3].ptr)
    stream = A.Stream()
    stack = A.AttentionStack(*GRID, *WINDOWS, TEXT, BLOCKS, FP32_PREFIX, HEADS, HEAD_DIM)
    A.synchronize()

    for _ in range(args.warmup):
        stack.run(vq, tq, vo, to, stream)
    stream.synchronize()
    start, stop = A.Event(), A.Event()
    wall0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        stack.run(vq, tq, vo, to, stream)
    stop.record(stream)
    stream.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = start.elapsed_ms(stop) / args.steps

    # Per-block kernel times (HIP events on the stack's stream around each attention kernel).
    stack.set_profiling(True)
    att = np.zeros(BLOCKS)
    blk = np.zeros(BLOCKS)
    for _ in range(args.profile_steps):
        stack.run(vq, tq, vo, to, stream)
        stream.synchronize()
        a, b_ = stack.block_times()
        att += a
        blk += b_
    att /= args.profile_steps
    blk /= args.profile_steps
    flops = stack.block_flops()
    step_flops = float(flops.sum())

    fp32_idx = np.arange(FP32_PREFIX)
    bf16_idx = np.arange(FP32_PREFIX, BLOCKS)
    # Dominant kernel by total time per step.
    fp32_total, bf16_total = att[fp32_idx].sum(), att[bf16_idx].sum()
    dom = fp32_idx if fp32_total >= bf16_total else bf16_idx
    dom_name = "window_attention_kernel<f32 MFMA>" if fp32_total >= bf16_total else "window_attention_kernel<bf16 MFMA>"
    avg_flops = float(flops[dom].mean())
    avg_ms = float(att[dom].mean())
    # Roofline of the dominant kernel: algorithmic bytes per launch are the QKV
    # rows read once and the outputs written once, (N + T_x) * H * d * (3 s_in + s_out).
    elem = 4 if dom is fp32_idx else 2
    alg_bytes = float((N + TEXT) * HEADS * HEAD_DIM * 4 * elem)
    mfma_peak = PEAK_FP32 if dom is fp32_idx else PEAK_BF16
    intensity = avg_flops / alg_bytes
    if intensity < mfma_peak / PEAK_HBM:
        bound, unit = "hbm", "GB/s"
        achieved = alg_bytes / (avg_ms * 1e-3) / 1e9
        peak = PEAK_HBM / 1e9
    else:
        bound, unit = "mfma", "TFLOP/s"
        achieved = avg_flops / (avg_ms * 1e-3) / 1e12
        peak = mfma_peak / 1e12
    traffic = None
    if args.traffic_json and os.path.exists(args.traffic_json):
        with open(args.traffic_json) as f:
            entry = json.load(f).get("kernels", {}).get("bf16" if dom is bf16_idx else "fp32")
        if entry is not None:
            traffic = entry.get("hbm_bytes_per_launch")

    def layer_stats(idx):
        ms = float(att[idx].mean())
        fl = float(flops[idx].mean())
        return {"kernel_ms": round(ms, 5), "layer_ms": round(float(blk[idx].mean()), 5),
                "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                "pct_bf16_peak": round(100.0 * fl / (ms * 1e-3) / PEAK_BF16, 2)}

    even = lambda idx: idx[idx % 2 == 0]
    odd = lambda idx: idx[idx % 2 == 1]
    def with_roof(stats, label, shifted):
        roof = mfma_instruction_roof_ms(A, GRID, WINDOWS, shifted, label)
        return {**stats, "mfma_instruction_roof_ms": round(roof, 5),
                "mfma_instruction_roof_frac": round(roof / stats["kernel_ms"], 4)}

    bf16_layers = {"unshifted": with_roof(layer_stats(even(bf16_idx)), "bf16", False),
                   "shifted": with_roof(layer_stats(odd(bf16_idx)), "bf16", True)}
    fp32_layers = {"unshifted": with_roof(layer_stats(even(fp32_idx)), "fp32", False),
                   "shifted": with_roof(layer_stats(odd(fp32_idx)), "fp32", True)}
    bf16_all_ms = float(att[bf16_idx].sum())
    bf16_pct = 100.0 * float(flops[bf16_idx].sum()) / (bf16_all_ms * 1e-3) / PEAK_BF16

    result = {
        "metric": METRIC,
        "value": round(step_flops / (ms_per_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+bf16",
        "data": "synthetic",
        "config": {
            "workload": "dit32_awa_attention_33f_256 (latent 9x16x16, windows 3x8x8, 64 text, 20x128 heads)",
            "latent": list(GRID), "window_counts": list(WINDOWS), "text_tokens": TEXT, "heads": HEADS,
            "head_dim": HEAD_DIM, "blocks": BLOCKS, "fp32_prefix_blocks": FP32_PREFIX,
            "step_gflop": round(step_flops / 1e9, 3), "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
        },
        "bf16_layers": {**bf16_layers, "pct_bf16_peak_all": round(bf16_pct, 2)},
        "fp32_layers": {k: {**v, "pct_fp32_peak": round(v["tflops"] * 1e12 / PEAK_FP32 * 100, 2)}
                        for k, v in fp32_layers.items()},
        "roofline": {
            "kernel": dom_name,
            "bound": bound,
            "achieved": round(achieved, 2),
            "peak": round(peak, 1),
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "flops_per_launch": avg_flops,
            "algorithmic_bytes_per_launch": alg_bytes,
            "arithmetic_intensity": round(intensity, 1),
            "tflops": round(avg_flops / (avg_ms * 1e-3) / 1e12, 2),
            "frac_of_mfma_peak": round(avg_flops / (avg_ms * 1e-3) / mfma_peak, 4),
            "avg_launch_ms": round(avg_ms, 5),
        },
    }
    result["qk_prologue"] = qk_prologue(A, buffers[FP32_PREFIX], stream)
    del buffers, vq, tq, vo, to
    if not args.no_configs:
        result["configs"] = config_measurements(A, stream)
    if not args.no_dit_step:
        result["dit_step"] = dit_step(A, stream, args.dit_steps)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_sample_layers)
        result["cpu_baseline_fp32_image"] = cpu_baseline_image()
    print(json.dumps(result), flush=True)
    stack.destroy()
    stream.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
