#!/usr/bin/env python3
"""Benchmark of the W4A16 G128 matrix path on one MI355X.

Headline (BASELINE.json metric "W4A16 GEMV GB/s (% HBM peak)"), workload
one step = the per-token decode projection set of one
Qwen2.5-1.5B layer, as src/engine.cu:361-431 issues it:
    rmsnorm_q8_1 -> QKV GEMV (1536->2048) -> O GEMV (1536->1536, +residual)
    -> rmsnorm_q8_1 -> gate+up SwiGLU GEMV (1536->2x8960) -> quantize(8960)
    -> down GEMV (8960->1536, +residual)
value = algorithmic GEMV bytes per step / step time.  Every step uses
another copy of the layer's weights; the copies span >= 512 MB (twice the
256 MB Infinity Cache) so the weights stream from HBM.  Steps are replayed
from one HIP graph (the reference decodes from a CUDA graph, engine.cu:453-470).

Also reported: per-kernel GB/s and roofline of the dominant kernel (gate+up),
configs[0] (W4A16 GEMV 1536->8960), configs[2] (LM head + argmax),
configs[3] (prefill dequant-GEMM TFLOP/s), and the oracle CPU baseline.
Inputs are synthetic (seeded), weights random in the packed layout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

H, I, V, NQ, NKV, HD = 1536, 8960, 151936, 12, 2, 128
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
POOL_BYTES = 512 << 20


def gemv_bytes(N, K, act="q8", out_n=None):
    """Algorithmic bytes of one GEMV: packed weights + fp16 scales + activation + output."""
    a = K * 2 if act == "f16" else K + K // 32 + K // 2
    return N * K // 2 + N * (K // 128) * 2 + a + (out_n if out_n is not None else N) * 2


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-step", action="store_true", help="headline step only (for profiling)")
    ap.add_argument("--only-roofline", action="store_true", help="dominant kernel's timing only (for profiling)")
    ap.add_argument("--only-prefill-gemm", type=int, default=0, metavar="M",
                    help="configs[3] gate/up GEMM at M tokens only, 20 launches (for profiling)")
    ap.add_argument("--only-decode", action="store_true",
                    help="configs[4] engine decode only: prompt 128, 64 graph tokens (for profiling)")
    ap.add_argument("--calib-read", action="store_true",
                    help="with --only-step: also stream-read 64 MiB 5 times (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the W4A16 path has no multi-GPU component; "
              "it would shard by weight rows, one all-reduce after O and down). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import qe_amd

    qe_amd.lib()
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def rand_w4(N, K, copies):
        qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (copies, N, K // 8), dtype=torch.int32, device=dev, generator=gen)
        sc = (torch.randn((copies, N, K // 128), device=dev, generator=gen).abs() * 0.02).half()
        return qw, sc

    def copies_for(nbytes):
        return max(2, -(-POOL_BYTES // nbytes))

    # one capture stream for every graph, holding a split-K workspace (the
    # prefill GEMMs split K only on streams that hold one); eager launches run
    # on the default stream, which holds one too
    cap_stream = torch.cuda.Stream()
    qe_amd.gemm_reserve_workspace(cap_stream)
    qe_amd.gemm_reserve_workspace()

    def graph_of(fn, reps):
        """Capture fn(i) for i in range(reps) into one graph."""
        s = cap_stream
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(min(reps, 3)):
                fn(i)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(reps):
                fn(i)
        return g

    def time_graph(g, replays, settle=False):
        g.replay()
        torch.cuda.synchronize()
        if settle:  # a first timed pass after idle time runs slow (clocks ramp); time a second one
            for _ in range(replays):
                g.replay()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / replays  # ms per graph

    if args.only_prefill_gemm:
        M = args.only_prefill_gemm
        qw, sc = rand_w4(2 * I, H, 1)
        A = torch.randn((M, H), device=dev, generator=gen).half()
        outp = torch.empty((M, I), dtype=torch.float16, device=dev)
        tw, ts = qe_amd.w4_tiled(qw[0], sc[0], 2 * I, H)
        for _ in range(20):
            qe_amd.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(qw[0], sc[0], A, outp, M, hidden_size=H,
                                                                 intermediate_size=I)
        for _ in range(20):
            qe_amd.launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(tw, ts, A, outp, M, hidden_size=H,
                                                                       intermediate_size=I)
        torch.cuda.synchronize()
        print(json.dumps({"only_prefill_gemm": {"M": M, "N": 2 * I, "K": H, "launches": "20 .qwenbin layout, "
                                                                                         "then 20 tiled"}}))
        return
    if args.only_decode:
        eng = qe_amd.Engine(qe_amd.default_config(), seed=2024)
        eng.prefill(np.random.default_rng(128).integers(0, V, 128).tolist())
        toks, step_ms = eng.decode(64, use_graph=True, timed=True)
        eng.close()
        print(json.dumps({"only_decode": {"tokens": 64, "itl_ms_p50": sorted(step_ms)[len(step_ms) // 2]}}))
        return

    # ---------------- activations / scratch ----------------------------------
    x = torch.randn(H, device=dev, generator=gen).half()
    hidden = x.clone()
    gamma = torch.ones(H, device=dev, dtype=torch.float16)
    q8 = torch.empty(I, dtype=torch.int8, device=dev)
    xs = torch.empty(I // 128, dtype=torch.float32, device=dev)
    s8 = torch.empty(I // 8, dtype=torch.int32, device=dev)
    dq = torch.empty(NQ * HD, dtype=torch.float16, device=dev)
    dk = torch.empty(NKV * HD, dtype=torch.float16, device=dev)
    dv = torch.empty(NKV * HD, dtype=torch.float16, device=dev)
    mlp = torch.empty(I, dtype=torch.float16, device=dev)

    # per-kernel timing: a graph of back-to-back launches over rotating weight copies
    def kernel_gbs(name, N, K, launch, nbytes, copies_bytes):
        C = copies_for(copies_bytes)
        qw, sc = rand_w4(N, K, C)
        g = graph_of(lambda i: launch(qw[i % C], sc[i % C]), C)
        ms = time_graph(g, 5) / C
        return {"kernel": name, "us": round(ms * 1e3, 3), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nbytes}

    if args.only_roofline:
        # the dominant kernel's measurement alone (profiled by rocprofv3 for the committed summary)
        qe_amd.launch_rmsnorm_q8_1(hidden, gamma, None, q8, xs, s8, hidden_size=H)
        gu = kernel_gbs("rmsnorm_gemv_dual_gate_up_swiglu_w4a16 1536->2x8960", 2 * I, H,
                        lambda w, s: qe_amd.launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(hidden, gamma, None, w, s,
                                                                                         mlp, H, I),
                        gemv_bytes(2 * I, H, act="f16", out_n=I) + H * 2, 2 * I * H // 2)
        print(json.dumps({"roofline_kernel": gu}))
        return

    # ---------------- headline: per-layer decode projection set --------------
    # Fused decode layer (this build's path, 4 launches):
    #   rmsnorm+Q8_1+QKV | O (Q8_1 in, +res) | rmsnorm+Q8_1+gate/up SwiGLU | down (fp16 in, quantized in-launch, +res)
    # Reference launch sequence (src/engine.cu:361-431, 7 launches) is timed too.
    b_qkv_f = gemv_bytes(NQ * HD + 2 * NKV * HD, H, act="f16") + H * 2      # + gamma
    b_o = gemv_bytes(H, H) + H * 2                                          # + fp16 residual read
    b_gu_f = gemv_bytes(2 * I, H, act="f16", out_n=I) + H * 2
    b_down_f = gemv_bytes(H, I, act="f16") + H * 2
    step_bytes = b_qkv_f + b_o + b_gu_f + b_down_f
    b_qkv = gemv_bytes(NQ * HD + 2 * NKV * HD, H)
    b_gu = gemv_bytes(2 * I, H, out_n=I)
    b_down = gemv_bytes(H, I) + H * 2
    ref_step_bytes = b_qkv + b_o + b_gu + b_down
    L = copies_for(step_bytes)
    wq, sq = rand_w4(NQ * HD, H, L)
    wk, sk = rand_w4(NKV * HD, H, L)
    wv, sv = rand_w4(NKV * HD, H, L)
    wo, so = rand_w4(H, H, L)
    wgu, sgu = rand_w4(2 * I, H, L)
    wd, sd = rand_w4(H, I, L)
    views = [qe_amd.make_qkv_view(wq[l], sq[l], dq, wk[l], sk[l], dk, wv[l], sv[l], dv) for l in range(L)]
    # attention sits between QKV and O and is outside this path: its Q8_1
    # output (K = 1536) is stood in by a fixed quantized vector.
    attn_q8 = torch.empty(H, dtype=torch.int8, device=dev)
    attn_xs = torch.empty(H // 128, dtype=torch.float32, device=dev)
    attn_s8 = torch.empty(H // 8, dtype=torch.int32, device=dev)
    qe_amd.launch_quantize_fp16_to_q8_1(x, attn_q8, attn_xs, attn_s8, H)

    def fused_step(i):
        l = i % L
        qe_amd.launch_rmsnorm_gemv_qkv_w4a16(hidden, gamma, None, views[l], hidden_size=H, num_q_heads=NQ,
                                             num_kv_heads=NKV, head_dim=HD)
        qe_amd.launch_gemv_w4a8(wo[l], so[l], attn_q8, attn_xs, attn_s8, hidden, hidden, H, H)
        qe_amd.launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(hidden, gamma, None, wgu[l], sgu[l], mlp, H, I)
        qe_amd.launch_gemv_w4a16(wd[l], sd[l], mlp, hidden, hidden, H, I)

    def reference_step(i):
        l = i % L
        qe_amd.launch_rmsnorm_q8_1(hidden, gamma, None, q8, xs, s8, hidden_size=H)
        qe_amd.launch_gemv_qkv_w4a8(views[l], q8, xs, s8, in_features=H, num_q_heads=NQ, num_kv_heads=NKV,
                                    head_dim=HD)
        qe_amd.launch_gemv_w4a8(wo[l], so[l], attn_q8, attn_xs, attn_s8, hidden, hidden, H, H)
        qe_amd.launch_rmsnorm_q8_1(hidden, gamma, None, q8, xs, s8, hidden_size=H)
        qe_amd.launch_gemv_dual_gate_up_swiglu_w4a8(wgu[l], sgu[l], q8, xs, s8, mlp, H, I)
        qe_amd.launch_quantize_fp16_to_q8_1(mlp, q8, xs, s8, I)
        qe_amd.launch_gemv_w4a8(wd[l], sd[l], q8, xs, s8, hidden, hidden, H, I)

    K_steps = max(args.steps, 1)

    def run_steps(step_fn):
        """W untimed warmup steps, then exactly K steps timed (one replay of a
        K-step graph between hipEvents, synchronized on both sides); ten more
        replays give the spread of the per-step time."""
        gk = graph_of(step_fn, K_steps)
        gk.replay()  # first replay of an instantiated graph carries one-time setup
        if args.warmup > 0:
            graph_of(step_fn, args.warmup).replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gk.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / K_steps
        spread = []
        for _ in range(10):
            e0.record()
            gk.replay()
            e1.record()
            torch.cuda.synchronize()
            spread.append(e0.elapsed_time(e1) / K_steps)
        spread.sort()
        return ms, {"p10_us": round(spread[1] * 1e3, 3), "p50_us": round(spread[5] * 1e3, 3),
                    "p90_us": round(spread[9] * 1e3, 3)}

    ms_per_step, step_spread = run_steps(fused_step)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    ms_ref, _ = run_steps(reference_step)

    result = {
        "metric": "W4A16 GEMV GB/s (% HBM peak); decode tok/s Qwen2.5-1.5B tg256",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x int4 -> int32 (sdot4), fp32 scale/accumulate, fp16 out",
        "data": "synthetic (seeded random packed int4 weights, |N(0,1)|*0.02 fp16 scales, N(0,1) fp16 x)",
        "config": {
            "workload": "configs[1]: one Qwen2.5-1.5B layer decode projection set, batch 1 "
                        "(QKV 1536->2048, O 1536->1536 +res, gate+up 1536->2x8960 SwiGLU, down 8960->1536 +res, "
                        "RMSNorm+Q8_1 fused into QKV and gate+up, down quantizes its fp16 input in-launch)",
            "bytes_per_step": step_bytes,
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "weight_copies": L,
            "timing": "the K-step HIP graph replayed once untimed (graph setup), W warmup steps, then one "
                      "replay of the graph of exactly K steps between hipEvents; weights rotated over >= 512 MB",
            "step_us_spread_10_more_replays": step_spread,
            "reference_launch_sequence": {
                "launches_per_step": 7, "us_per_step": round(ms_ref * 1e3, 3),
                "GB/s": round(ref_step_bytes / (ms_ref * 1e-3) / 1e9, 1)},
        },
    }
    if args.only_step:
        if args.calib_read:
            buf = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
            sink = torch.zeros(1 << 14, dtype=torch.int32, device=dev)
            for _ in range(5):
                qe_amd.stream_read(buf, buf.numel(), sink)
            torch.cuda.synchronize()
        print(json.dumps(result))
        return

    # ---------------- per-kernel GEMV roofline -------------------------------
    per = []
    qe_amd.launch_rmsnorm_q8_1(hidden, gamma, None, q8, xs, s8, hidden_size=H)
    torch.cuda.synchronize()
    per.append(kernel_gbs("gemv_w4a8 O 1536->1536", H, H,
                          lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, mlp, H, H),
                          gemv_bytes(H, H), H * H // 2))
    per.append(kernel_gbs("gemv_w4a8 QKV-shape 1536->2048", 2048, H,
                          lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, mlp, 2048, H),
                          gemv_bytes(2048, H), 2048 * H // 2))
    per.append(kernel_gbs("gemv_dual_gate_up_swiglu_w4a8 1536->2x8960", 2 * I, H,
                          lambda w, s: qe_amd.launch_gemv_dual_gate_up_swiglu_w4a8(w, s, q8, xs, s8, mlp, H, I),
                          b_gu, 2 * I * H // 2))
    gu = kernel_gbs("rmsnorm_gemv_dual_gate_up_swiglu_w4a16 1536->2x8960", 2 * I, H,
                    lambda w, s: qe_amd.launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(hidden, gamma, None, w, s,
                                                                                     mlp, H, I),
                    b_gu_f, 2 * I * H // 2)
    per.append(gu)
    per.append(kernel_gbs("gemv_w4a16 down 8960->1536 (+res)", H, I,
                          lambda w, s: qe_amd.launch_gemv_w4a16(w, s, mlp, hidden, hidden, H, I),
                          b_down_f, H * I // 2))
    qe_amd.launch_quantize_fp16_to_q8_1(mlp, q8, xs, s8, I)
    torch.cuda.synchronize()
    per.append(kernel_gbs("gemv_w4a8 down 8960->1536", H, I,
                          lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, hidden, H, I),
                          gemv_bytes(H, I), H * I // 2))
    qe_amd.launch_rmsnorm_q8_1(hidden, gamma, None, q8, xs, s8, hidden_size=H)
    torch.cuda.synchronize()
    logits = torch.empty(V, dtype=torch.float16, device=dev)
    lm = kernel_gbs("gemv_w4a8 LM head 1536->151936", V, H,
                    lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, logits, V, H),
                    gemv_bytes(V, H), V * H // 2)
    per.append(lm)
    c0 = kernel_gbs("gemv_w4a16 configs[0] 1536->8960", I, H,
                    lambda w, s: qe_amd.launch_gemv_w4a16(w, s, x, None, mlp, I, H),
                    gemv_bytes(I, H, act="f16"), I * H // 2)
    per.append(c0)

    # one GPU's share of a tensor-parallel decode layer at p = 8 (column shards
    # of QKV, gate/up and the LM head; row shards of O and down in whole
    # 128-groups): the kernels the sharded path would run, on one GPU
    P = 8
    shard = []
    kd = -(-(I // 128) // P) * 128   # down: ceil(70 / 8) = 9 groups -> K = 1152
    ko = 2 * HD                      # O: two of the 12 heads -> K = 256
    for name, N_, K_, launch_ in (
            (f"QKV column shard 1536->{(NQ * HD + 2 * NKV * HD) // P}", (NQ * HD + 2 * NKV * HD) // P, H,
             lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, mlp, (NQ * HD + 2 * NKV * HD) // P, H)),
            (f"gate/up column shard 1536->2x{I // P}", 2 * I // P, H,
             lambda w, s: qe_amd.launch_gemv_dual_gate_up_swiglu_w4a8(w, s, q8, xs, s8, mlp, H, I // P)),
            (f"down row shard {kd}->1536", H, kd,
             lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, hidden, H, kd)),
            (f"O row shard {ko}->1536", H, ko,
             lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, hidden, H, ko)),
            (f"LM head column shard 1536->{V // P}", V // P, H,
             lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8, xs, s8, None, logits, V // P, H))):
        nb = gemv_bytes(N_, K_, out_n=I // P if name.startswith("gate") else None)
        shard.append(kernel_gbs("gemv_w4a8 " + name, N_, K_, launch_, nb, N_ * K_ // 2))
    result["shard_tp8"] = shard

    # the same GEMV kernels on a matrix large enough to amortize the launch
    # (N = 65536, K = 16384: 536 MB of packed weights), beside the streaming
    # ceiling at that size: what the kernel reaches when it is not launch-bound
    KL, NL = 16384, 65536
    xl = torch.randn(KL, device=dev, generator=gen).half()
    q8l = torch.empty(KL, dtype=torch.int8, device=dev)
    xsl = torch.empty(KL // 128, dtype=torch.float32, device=dev)
    s8l = torch.empty(KL // 8, dtype=torch.int32, device=dev)
    outl = torch.empty(NL, dtype=torch.float16, device=dev)
    qe_amd.launch_quantize_fp16_to_q8_1(xl, q8l, xsl, s8l, KL)
    torch.cuda.synchronize()
    large = [kernel_gbs(f"gemv_w4a8 {KL}->{NL}", NL, KL,
                        lambda w, s: qe_amd.launch_gemv_w4a8(w, s, q8l, xsl, s8l, None, outl, NL, KL),
                        gemv_bytes(NL, KL), NL * KL // 2),
             kernel_gbs(f"gemv_w4a16 {KL}->{NL}", NL, KL,
                        lambda w, s: qe_amd.launch_gemv_w4a16(w, s, xl, None, outl, NL, KL),
                        gemv_bytes(NL, KL, act="f16"), NL * KL // 2)]
    result["gemv_large"] = large
    del xl, q8l, xsl, s8l, outl

    # achievable ceiling: a launch that only streams the same number of bytes
    sink = torch.zeros(1 << 14, dtype=torch.int32, device=dev)
    ceil = {}
    for nb in (gemv_bytes(H, H), b_gu_f, gemv_bytes(V, H), POOL_BYTES):
        nb16 = (nb + 4095) // 4096 * 4096
        C = copies_for(nb16) if nb16 < POOL_BYTES else 2
        pool = torch.empty((C, nb16), dtype=torch.uint8, device=dev)
        ms = time_graph(graph_of(lambda i: qe_amd.stream_read(pool[i % C], nb16, sink), C), 5) / C
        ceil[str(nb)] = {"us": round(ms * 1e3, 3), "GB/s": round(nb16 / (ms * 1e-3) / 1e9, 1)}
        del pool
    result["stream_read_ceiling"] = ceil
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "gemv_gate_up_traffic.txt")
    if os.path.exists(tfile):
        for line in open(tfile):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":", 1)[1]))
    result["roofline"] = {
        "kernel": gu["kernel"],
        "bound": "hbm",
        "achieved": gu["GB/s"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": gu["frac"],
        "traffic": traffic,
        "traffic_source": ("profiles/gemv_gate_up_traffic.txt: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of "
                           "this kernel (scaled by a known-size read), measured in an earlier run of this command, "
                           "not in this run") if traffic is not None else None,
        "bytes_per_launch": b_gu_f,
        "ceiling_same_bytes_GB/s": ceil[str(b_gu_f)]["GB/s"],
        "avg_launch_us": gu["us"],
    }
    result["kernels"] = per

    # ---------------- LM head + argmax ----------------------------
    val = torch.empty(256, dtype=torch.float32, device=dev)
    idx = torch.empty(256, dtype=torch.int32, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    C = copies_for(V * H // 2)
    wl, sl = rand_w4(V, H, C)

    def lm_argmax(i):
        qe_amd.launch_gemv_w4a8(wl[i % C], sl[i % C], q8, xs, s8, None, logits, V, H)
        qe_amd.launch_sample_and_advance(logits, val, idx, None, tok, vocab_size=V)

    ms = time_graph(graph_of(lm_argmax, C), 5) / C
    result["lm_head_argmax"] = {"us": round(ms * 1e3, 3), "GB/s": round(gemv_bytes(V, H) / (ms * 1e-3) / 1e9, 1),
                                "launches": 3}
    # fused: LM-head GEMV with the first sampling stage in its epilogue + stage 2 (2 launches, no logits)
    fval = torch.empty(qe_amd.LM_HEAD_SAMPLE_PARTS, dtype=torch.float32, device=dev)
    fidx = torch.empty(qe_amd.LM_HEAD_SAMPLE_PARTS, dtype=torch.int32, device=dev)

    def lm_fused(i):
        qe_amd.launch_gemv_lm_head_sample_w4a8(wl[i % C], sl[i % C], q8, xs, s8, None, fval, fidx, None, tok,
                                               vocab_size=V, in_features=H)

    ms = time_graph(graph_of(lm_fused, C), 5) / C
    result["lm_head_sample_fused"] = {"us": round(ms * 1e3, 3),
                                      "GB/s": round(gemv_bytes(V, H) / (ms * 1e-3) / 1e9, 1), "launches": 2}
    del wl, sl

    # ---------------- prefill dequant-GEMM -----------------------
    pre = []
    for M in (128, 512, 1024):
        A = torch.randn((M, I), device=dev, generator=gen).half()
        outp = torch.empty((M, 2 * I), dtype=torch.float16, device=dev)
        tot_flop, tot_ms, tot_ms_t = 0.0, 0.0, 0.0
        for (N, K, name) in ((2048, H, "qkv"), (H, H, "o"), (2 * I, H, "gate_up"), (H, I, "down")):
            C = max(2, min(64, copies_for(N * K // 2)))
            qw, sc = rand_w4(N, K, C)
            if name == "gate_up":
                fn = lambda i: qe_amd.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(
                    qw[i % C], sc[i % C], A, outp, M, hidden_size=K, intermediate_size=I)
            else:
                fn = lambda i: qe_amd.launch_gemm_prefill_w4a16(qw[i % C], sc[i % C], A, None, outp, M, N, K)
            ms = time_graph(graph_of(fn, C), 3, settle=True) / C
            # the same GEMM on the tiled load-time copy of the weights (what the engine's prefill runs)
            tl = [qe_amd.w4_tiled(qw[i], sc[i], N, K) for i in range(C)]
            if name == "gate_up":
                fnt = lambda i: qe_amd.launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(
                    tl[i % C][0], tl[i % C][1], A, outp, M, hidden_size=K, intermediate_size=I)
            else:
                fnt = lambda i: qe_amd.launch_gemm_prefill_w4a16_tiled(tl[i % C][0], tl[i % C][1], A, None, outp,
                                                                       M, N, K)
            mst = time_graph(graph_of(fnt, C), 3, settle=True) / C
            fl = 2.0 * M * N * K
            tot_flop += fl
            tot_ms += ms
            tot_ms_t += mst
            pre.append({"M": M, "shape": f"{name} {K}->{N}", "us": round(ms * 1e3, 2),
                        "TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 1), "tiled_us": round(mst * 1e3, 2),
                        "tiled_TFLOP/s": round(fl / (mst * 1e-3) / 1e12, 1)})
            del qw, sc, tl
        pre.append({"M": M, "shape": "layer total", "TFLOP/s": round(tot_flop / (tot_ms * 1e-3) / 1e12, 1),
                    "mfma_frac": round(tot_flop / (tot_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                    "tiled_TFLOP/s": round(tot_flop / (tot_ms_t * 1e-3) / 1e12, 1),
                    "tiled_mfma_frac": round(tot_flop / (tot_ms_t * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)})
        # int8-MFMA variant (W4A8: activation rows quantized to Q8_1 first, quantization included)
        q8p = torch.empty(M * I, dtype=torch.int8, device=dev)
        xsp = torch.empty(M * I // 128, dtype=torch.float32, device=dev)
        s8p = torch.empty(M * I // 8, dtype=torch.int32, device=dev)
        tot8 = 0.0
        for (N, K, name) in ((2048, H, "qkv"), (H, H, "o"), (2 * I, H, "gate_up"), (H, I, "down")):
            C = max(2, min(64, copies_for(N * K // 2)))
            qw, sc = rand_w4(N, K, C)

            def fn8(i, qw=qw, sc=sc, N=N, K=K, name=name):
                qe_amd.launch_quantize_fp16_to_q8_1(A, q8p, xsp, s8p, M * K)
                if name == "gate_up":
                    qe_amd.launch_gemm_prefill_dual_gate_up_swiglu_w4a8(qw[i % C], sc[i % C], q8p, xsp, s8p, outp, M,
                                                                        hidden_size=K, intermediate_size=I)
                else:
                    qe_amd.launch_gemm_prefill_w4a8(qw[i % C], sc[i % C], q8p, xsp, s8p, None, outp, M, N, K)

            tot8 += time_graph(graph_of(fn8, C), 3, settle=True) / C
            del qw, sc
        pre.append({"M": M, "shape": "layer total, int8 MFMA (W4A8, incl. Q8_1 quantization)",
                    "TFLOP/s": round(tot_flop / (tot8 * 1e-3) / 1e12, 1),
                    "mfma_frac_int8_peak": round(tot_flop / (tot8 * 1e-3) / 1e12 / (2 * MFMA_F16_PEAK_TFLOPS), 4)})
    result["prefill_gemm"] = pre
    # MFMA roofline of the dominant prefill kernel (gate/up SwiGLU, the largest GEMM of a layer) at M = 1024
    gu1024 = next(r for r in pre if r.get("M") == 1024 and r.get("shape", "").startswith("gate_up"))
    result["roofline_prefill"] = {
        "kernel": "gemm_prefill_dual_gate_up_swiglu_w4a16_tiled M=1024 1536->2x8960 (fp16 MFMA, tiled weights)",
        "bound": "mfma",
        "achieved": gu1024["tiled_TFLOP/s"],
        "peak": MFMA_F16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(gu1024["tiled_TFLOP/s"] / MFMA_F16_PEAK_TFLOPS, 4),
        "flop_per_launch": 2 * 1024 * 2 * I * H,
        "avg_launch_us": gu1024["tiled_us"],
        "qwenbin_layout_TFLOP/s": gu1024["TFLOP/s"],
    }

    # ---------------- end-to-end decode -------------------------
    # random-init Qwen2.5-1.5B in the packed layout, 128-token prompt of seeded
    # uniform ids, 256 greedy tokens from the captured decode graph.
    del wq, wk, wv, wo, wgu, wd
    torch.cuda.empty_cache()
    rng = np.random.default_rng(128)
    prompt = rng.integers(0, V, 128).tolist()
    eng = qe_amd.Engine(qe_amd.default_config(), seed=2024)
    t0 = time.perf_counter()
    eng.prefill(prompt)
    ttft_ms = (time.perf_counter() - t0) * 1e3
    eng.reset()
    t0 = time.perf_counter()
    eng.prefill(prompt)
    ttft_ms = min(ttft_ms, (time.perf_counter() - t0) * 1e3)
    toks, step_ms = eng.decode(256, use_graph=True, timed=True)
    prof = eng.profile_decode()
    eng.close()
    sm = sorted(step_ms)
    med = sm[len(sm) // 2]
    weight_bytes_per_token = 28 * (b_qkv + b_o + b_gu + b_down) + gemv_bytes(V, H)
    result["e2e_decode"] = {
        "workload": "configs[4]: 28 layers, random-init W4A16 G128, prompt 128 seeded uniform ids, greedy 256 tokens",
        "deviation": "group scales |N(0,1)|/sqrt(21.5*K) instead of the configs' |N(0,1)*0.02 (with 0.02 the "
                     "28-layer residual stream overflows fp16); the embedding/LM head keeps 0.02; timing does not "
                     "depend on the values",
        "decode_tok_s_median": round(1000.0 / med, 1),
        "decode_tok_s_mean": round(1000.0 * len(step_ms) / sum(step_ms), 1),
        "itl_ms_p50": round(med, 4), "itl_ms_p90": round(sm[int(len(sm) * 0.9)], 4),
        "ttft_ms_prefill128": round(ttft_ms, 3),
        "prefill_tok_s": round(128 / (ttft_ms * 1e-3), 1),
        "effective_GB/s": round(weight_bytes_per_token / (med * 1e-3) / 1e9, 1),
        "gemv_share_eager_profile": round(prof["gemv_ms"] / prof["total_ms"], 4),
        "profile_ms": {k: round(v, 4) for k, v in prof.items()},
        "first_tokens": toks[:8],
    }

    # ---------------- CPU baseline: the oracle (port of the CPU golden) ------
    if not args.no_cpu:
        import oracle
        qwc, scc = oracle.synth_w4(7, 2 * I, H)
        xv = oracle.synth_f16_normal(8, H)
        q8c, xsc, s8c = oracle.quantize_q8_1(xv)
        t0 = time.perf_counter()
        reps = 0
        while True:
            oracle.gemv_swiglu_w4a8(qwc, scc, q8c, xsc, s8c, H, I)
            reps += 1
            if time.perf_counter() - t0 > 10.0 or reps >= 2000:
                break
        dt = time.perf_counter() - t0
        # the same rows over the host cores this job may use (16 per GPU on the box)
        threads = max(1, min(os.cpu_count() or 1, 16))
        t1 = time.perf_counter()
        reps_mt = 0
        while True:
            oracle.gemv_swiglu_w4a8_mt(qwc, scc, q8c, xsc, s8c, H, I, threads)
            reps_mt += 1
            if time.perf_counter() - t1 > 5.0 or reps_mt >= 20000:
                break
        dt_mt = time.perf_counter() - t1
        result["cpu_baseline"] = {
            "value": round(b_gu * reps / dt / 1e9, 3),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"{reps} x gate+up SwiGLU GEMV 1536->2x8960 (configs[1]'s largest projection) with the "
                      f"scalar oracle (restated CPU golden, tests/test_kernels.cu:308-363), ~10 s, 1 thread; "
                      f"host nproc={os.cpu_count()}, CPU {cpu_model()}",
            "all_cores": {"value": round(b_gu * reps_mt / dt_mt / 1e9, 3), "unit": "GB/s", "cores": threads,
                          "sample": f"{reps_mt} x the same GEMV, rows split over {threads} threads, ~5 s"},
        }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
