#!/usr/bin/env python3
"""Benchmark of the quantized GEMV path on one MI355X.

Workload (the config the metric is quoted on):
Q6_K decode-FFN GEMV at batch 1 — per step, y1 = W1 x1 with W1 Q6_K
[14336 x 4096] and y2 = W2 x2 with W2 Q6_K [4096 x 14336]; fp32 x and y.
Weights are seeded synthetic GGUF blocks with the documented statistics,
converted once to the device layout, and replicated into enough distinct
copies (> 512 MB) that every launch streams its weights from HBM rather than
the 256 MB Infinity Cache; steps rotate through the copies.

value        = whole-job algorithmic bytes / wall time of the K timed steps
               (bytes = packed weight bytes + x + y, per launch)
roofline     = the same bytes per launch / mean duration of the dominant kernel
               (at batch 1 the whole drop-in call is one kernel, k_gemv1, which
               quantises x in LDS), measured with one HIP-event pair around a
               run of K back-to-back launches of one shape on the launch
               stream, vs 8 TB/s
cpu_baseline = the CPU oracle (a C restatement of the reference CPU path,
               one thread per token as the reference's rayon split gives at
               batch 1) timed on a bounded sample of the same GEMVs.
prefill      = BASELINE.json configs[4] (C4): Q4_K weight (out, in) =
               (14336, 4096) times bf16 activations [T x 4096], T = 512 and
               2048, fp32 output, on the MFMA path; TFLOP/s = 2 T in out / the
               event-timed mean of a run of back-to-back calls (activation
               pre-pass + GEMM), against the 2.5 PFLOP/s dense f16/bf16 MFMA
               peak, with its own bounded CPU-oracle sample.

`--gpus N` with N > 1 exits: this build targets one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0 = auto)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--extra", action="store_true", help="also time the other configs")
    ap.add_argument("--no-prefill", action="store_true", help="skip the C4 prefill leg")
    ap.add_argument("--prefill-iters", type=int, default=20)
    return ap.parse_args()


def bench_prefill(B, synth, G, dev, stream, iters, with_cpu, cpu_seconds):
    """C4: Q4_K (14336, 4096) x bf16 [T x 4096] on the MFMA path, T = 512, 2048."""
    import torch
    out_dim, in_dim = 14336, 4096
    w_host = synth.weight(G.Q4_K, out_dim, in_dim, seed=404)
    d_w = torch.from_numpy(w_host).to(dev)
    sptr = stream.cuda_stream
    res = {"workload": "C4 Q4_K prefill GEMM (out, in) = (14336, 4096), bf16 x [T x 4096]",
           "peak_tflops": MFMA_F16_PEAK_TFLOPS, "by_tokens": []}
    xs_host = {}
    for T in (512, 2048):
        xb = synth.bf16_activations(T, in_dim, seed=405).reshape(-1)
        xs_host[T] = xb
        d_x = torch.from_numpy(xb.view(np.int16)).to(dev)
        d_y = torch.empty(T * out_dim, dtype=torch.float32, device=dev)

        def call():
            B.matmul_q4k_bf16_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), d_w.numel(),
                                  d_x.data_ptr(), d_x.numel(), T, in_dim, out_dim, G.Q4_K, sptr)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(iters):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / iters
        tflops = 2.0 * T * in_dim * out_dim / (us * 1e-6) / 1e12
        entry = {"tokens": T, "us_per_op": round(us, 2), "tflops": round(tflops, 1),
                 "frac_of_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        if with_cpu and T == 512:
            # parity spot check on a spread of tokens
            sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
            from oracle import oracle as O
            toks = np.linspace(0, T - 1, 8).astype(int)
            xf = synth.bf16_bits_to_f32(xb.reshape(T, in_dim)[toks]).reshape(-1)
            rc, want = O.matmul_quant_f32(w_host, xf, len(toks), in_dim, out_dim, int(G.Q4_K))
            got = d_y.cpu().numpy().reshape(T, out_dim)[toks].reshape(-1)
            entry["check"] = {"max_rel_err_vs_oracle": float(np.abs(got - want).max() /
                                                             np.abs(want).max()),
                              "tokens_checked": len(toks), "tolerance": 1e-3}
        res["by_tokens"].append(entry)
        del d_x, d_y
    best = max(res["by_tokens"], key=lambda e: e["tflops"])
    res["roofline"] = {"bound": "mfma", "achieved": best["tflops"], "peak": MFMA_F16_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": best["frac_of_peak"],
                       "tokens": best["tokens"]}
    if with_cpu:
        # reference CPU path (oracle, all host threads = min(n_tok, cores) as
        # the rayon split gives) on a bounded token sample, scaled to TFLOP/s
        from oracle import oracle as O
        n_thr = O.lib().orc_num_cores()
        xb = xs_host[512]
        n_done, t_cpu = 0, 0.0
        while t_cpu < cpu_seconds / 2:
            toks = n_thr
            xf = synth.bf16_bits_to_f32(xb.reshape(512, in_dim)[:toks]).reshape(-1)
            t0 = time.perf_counter()
            O.matmul_quant_f32(w_host, xf, toks, in_dim, out_dim, int(G.Q4_K), n_threads=n_thr)
            t_cpu += time.perf_counter() - t0
            n_done += toks
        res["cpu_baseline"] = {
            "value": 2.0 * n_done * in_dim * out_dim / t_cpu / 1e12, "unit": "TFLOP/s",
            "cores": n_thr, "kind": "port",
            "sample": f"{n_done} tokens of C4 (Q4_K 14336x4096) in {t_cpu:.1f} s, oracle "
                      f"matmul_quant_f32 with one thread per token ({n_thr} threads)"}
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(sharding is described in DESIGN.md); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream

    dtype = G.Q6_K
    shapes = [(14336, 4096), (4096, 14336)]  # (out_dim, in_dim)
    n_tok = 1

    # ---- weights: one seeded matrix per shape, prepared, then replicated ----
    mats = []
    for si, (out_dim, in_dim) in enumerate(shapes):
        w_host = synth.weight(dtype, out_dim, in_dim, seed=100 + si)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, sptr)
        del raw
        mats.append((out_dim, in_dim, w_host, prep))
    step_wbytes = sum(m[3].numel() for m in mats)
    copies = args.copies or max(2, int(np.ceil(768e6 / step_wbytes)))
    reps = [[m[3] if c == 0 else m[3].clone() for m in mats] for c in range(copies)]

    xs, ys = [], []
    for si, (out_dim, in_dim, _, _) in enumerate(mats):
        xs.append(torch.from_numpy(synth.activations(n_tok, in_dim, seed=200 + si)).to(dev).reshape(-1))
        ys.append(torch.empty(n_tok * out_dim, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()

    def launch(si, c):
        out_dim, in_dim, _, _ = mats[si]
        w = reps[c][si]
        B.matmul_quant_f32_dev(ys[si].data_ptr(), ys[si].numel(), w.data_ptr(), w.numel(),
                               xs[si].data_ptr(), xs[si].numel(), n_tok, in_dim, out_dim, dtype,
                               sptr)

    def step(i):
        c = i % copies
        for si in range(len(mats)):
            launch(si, c)

    bytes_per_launch = [m[3].numel() + n_tok * (m[1] + m[0]) * 4 for m in mats]
    bytes_per_step = sum(bytes_per_launch)

    # ---- warmup ----
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps ----
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    t_start.record(stream)
    for i in range(args.steps):
        step(i)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - h0
    gpu_ms = t_start.elapsed_time(t_end)
    ms_per_step = gpu_ms / args.steps
    value = bytes_per_step * args.steps / (gpu_ms * 1e-3) / 1e9

    # ---- dominant kernel duration: at batch 1 each drop-in call is ONE
    # kernel (the fused GEMV, x quantised in LDS), timed as the
    # event-bracketed mean over a run of back-to-back launches of one shape
    # (one event pair per run, so event overhead is amortised over the run).
    per_kernel = []
    kern_us = []
    for si, (out_dim, in_dim, _, _) in enumerate(mats):
        def gemv_only(c):
            launch(si, c)
        for i in range(copies):
            gemv_only(i)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for i in range(args.steps):
            gemv_only(i % copies)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / args.steps
        kern_us.append(us)
        per_kernel.append({"shape": f"{out_dim}x{in_dim}", "bytes": bytes_per_launch[si],
                           "us_mean": round(us, 3),
                           "GBps": round(bytes_per_launch[si] / (us * 1e-6) / 1e9, 1)})
    dom = max(range(len(mats)), key=lambda s: kern_us[s])
    ach = bytes_per_launch[dom] / (kern_us[dom] * 1e-6) / 1e9

    # ---- correctness spot check of this run's outputs vs the oracle ----
    # (ys hold the last GEMV-only launch: same weights bytes, same x)
    check = None
    cpu_baseline = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import oracle as O
        y_gpu = [y.cpu().numpy() for y in ys]
        # last step used copy (K-1) % copies; all copies hold the same bytes
        errs = []
        for si, (out_dim, in_dim, w_host, _) in enumerate(mats):
            x_host = xs[si].cpu().numpy()
            t0 = time.perf_counter()
            rc, y_ref = O.matmul_quant_f32(w_host, x_host, n_tok, in_dim, out_dim, int(dtype),
                                           allow_q6k=True, n_threads=1)
            errs.append(float(np.abs(y_gpu[si] - y_ref).max() / np.abs(y_ref).max()))
        check = {"max_rel_err_vs_oracle": max(errs), "tolerance": 1e-3}
        # CPU baseline: bounded sample of whole GEMVs (reference threading:
        # one task per token, so batch 1 uses one core).
        n_ops, cpu_bytes, t_cpu = 0, 0, 0.0
        while t_cpu < args.cpu_seconds:
            si = n_ops % len(mats)
            out_dim, in_dim, w_host, _ = mats[si]
            x_host = xs[si].cpu().numpy()
            t0 = time.perf_counter()
            O.matmul_quant_f32(w_host, x_host, n_tok, in_dim, out_dim, int(dtype), allow_q6k=True,
                               n_threads=1)
            t_cpu += time.perf_counter() - t0
            cpu_bytes += bytes_per_launch[si]
            n_ops += 1
        cpu_baseline = {
            "value": cpu_bytes / t_cpu / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n_ops} whole Q6_K GEMVs (alternating 14336x4096 / 4096x14336, B=1) "
                      f"in {t_cpu:.1f} s; oracle/rsllm_oracle.c matmul_quant_f32 (reference "
                      f"algorithm; the reference's dtype guard rejects Q6_K), 1 thread = "
                      f"min(n_tok, cores); host has {os.cpu_count()} logical CPUs",
            "us_per_op": t_cpu / n_ops * 1e6,
        }

    prefill = None if args.no_prefill else bench_prefill(B, synth, G, dev, stream,
                                                          args.prefill_iters, not args.no_cpu,
                                                          args.cpu_seconds)

    line = {
        "metric": "Q4_K/Q6_K GEMV GB/s (% of HBM peak); Q4_K prefill GEMM TFLOP/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q6_k weights, f32 activations/accumulation",
        "data": "synthetic (seeded PCG64 GGUF Q6_K blocks with BASELINE.json C1 statistics; "
                "x ~ N(0,1) fp32)",
        "config": {
            "workload": "C1 Q6_K decode-FFN GEMV, batch 1: 14336x4096 then 4096x14336 per step",
            "bytes_per_step": bytes_per_step,
            "rotating_weight_copies": copies,
            "resident_weight_bytes": step_wbytes * copies,
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "wall_s_timed": round(wall_s, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(ach, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "rsllm_hip::k_gemv1<FQ6K, RT, NWV> (x quantised in LDS, one launch)",
            "kernel_shape": per_kernel[dom]["shape"],
            "kernel_us_mean": round(kern_us[dom], 3),
        },
        "per_kernel": per_kernel,
        "cpu_baseline": cpu_baseline,
        "check": check,
        "prefill": prefill,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
