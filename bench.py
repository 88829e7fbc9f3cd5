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
               (bytes = packed weight bytes + x + y, per launch); before the W
               warmup steps the GPU runs --spinup-ms (50) of 256 MB device
               copies, and every other timed region gets 20 ms of them, so
               timed regions of well under a millisecond measure the GPU's
               steady state rather than its wake-up after host-side idle
               time (on MI355X that ramp costs about 5% of a 20-step run)
roofline     = the same bytes per launch / mean duration of the dominant kernel
               (at batch 1 the whole drop-in call is one kernel, k_gemv1, which
               quantises x in LDS), measured with one HIP-event pair around a
               run of K back-to-back launches of one shape on the launch
               stream, vs 8 TB/s
cpu_baseline = the CPU oracle (a C restatement of the reference CPU path,
               one thread per token as the reference's rayon split gives at
               batch 1) timed on a bounded sample of the same GEMVs.
traffic      = HBM bytes per launch of the dominant kernel from two rocprofv3
               --pmc passes (FETCH_SIZE, WRITE_SIZE) over a child run of this
               script (--pmc-probe), each counter scaled by bytes / counter of a
               device copy of known size in the same pass
prefill      = BASELINE.json configs[4] (C4): Q4_K weight (out, in) =
               (14336, 4096) times bf16 activations [T x 4096], T = 512 and
               2048, fp32 output, on the MFMA path; TFLOP/s = 2 T in out / the
               event-timed mean of a run of back-to-back calls (activation
               pre-pass + GEMM), taken after 50 ms of the same call back to
               back (the clocks' warm-up under sustained matrix-core load,
               as a forward pass's back-to-back calls run), against the
               2.5 PFLOP/s dense f16/bf16 MFMA peak, with its own bounded
               CPU-oracle sample. The GEMM and pre-pass durations come from
               the same kernel-trace pass as the roofline (after 25 ms of
               warm-up calls), MFMA busy from one rocprofv3 --pmc pass.

Output: ONE compact JSON line on stdout. Every prefill figure is a flat
scalar member of "prefill"; the other configs are short rows in "extra".
`--detail-out FILE` writes the full per-case tables, traces and counter
details beside it.

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
    ap.add_argument("--spinup-ms", type=float, default=50.0,
                    help="device copies before the warmup steps, so the timed steps see the "
                         "GPU's steady state rather than its wake-up from idle")
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0 = auto)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the C0/C1-batched/C2/C3 legs and the copy-bandwidth probe")
    ap.add_argument("--extra-iters", type=int, default=100)
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure roofline.traffic")
    ap.add_argument("--gemv-probe", action="store_true",
                    help="internal: the batch-1 GEMVs run under rocprofv3 --kernel-trace")
    ap.add_argument("--batch-probe", action="store_true",
                    help="run only the batched decode calls (for rocprofv3 traces and counters)")
    ap.add_argument("--q8-probe", action="store_true",
                    help="run only the C2 int8-activation calls (quantize + matmul) for traces")
    ap.add_argument("--no-trace", action="store_true",
                    help="skip the kernel-trace pass (roofline from HIP events only)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="internal: the workload run under rocprofv3 --pmc (prints no JSON)")
    ap.add_argument("--prefill-probe", type=int, default=0, metavar="T",
                    help="internal: only run the C4 prefill call at T tokens 5 times (the "
                         "workload for rocprofv3 counter passes; prints no JSON)")
    ap.add_argument("--prefill-format", default="Q4_K", choices=("Q4_K", "Q6_K", "Q8_0"),
                    help="internal: weight format of --prefill-probe")
    ap.add_argument("--moe-probe", type=int, default=0, metavar="T",
                    help="internal: only run the C3 routed-expert call at T tokens 8 times "
                         "(for rocprofv3 kernel traces; prints no JSON)")
    ap.add_argument("--dsv4-probe", type=int, default=0, metavar="T",
                    help="internal: only run the DS-V4 routed-expert call (IQ2_XXS / Q2_K, 256 "
                         "experts, top-6) at T tokens 8 times after 25 ms of it (for rocprofv3 "
                         "kernel traces; prints no JSON)")
    ap.add_argument("--prefill-pmc-probe", action="store_true",
                    help="internal: the C4 prefill call at T = 512 and 2048, five times each, "
                         "for the MFMA-busy counter pass (prints no JSON)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the C4 prefill leg")
    ap.add_argument("--detail-out", default="",
                    help="also write the full per-case results (every leg's tables, traces and "
                         "counter details) as JSON to this file; stdout keeps the compact line")
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
        _sustain(lambda i: call(), SUSTAIN_MS)
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
    # The reference's own prefill call: matmul_quant_f32 with f32 x and n_tok
    # = T (engine_impl.rs:277 -> weight.rs:161-163 -> quant_matmul.rs:45),
    # through the drop-in device entry point (f32 -> scaled f16 pre-pass +
    # the same GEMM), beside the bf16 leg
    res["f32_x"] = []
    for T in (512, 2048):
        x_host = synth.activations(T, in_dim, seed=406).reshape(-1)
        d_x = torch.from_numpy(x_host).to(dev)
        d_y = torch.empty(T * out_dim, dtype=torch.float32, device=dev)

        def call_f32(i):
            B.matmul_quant_f32_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), d_w.numel(),
                                   d_x.data_ptr(), d_x.numel(), T, in_dim, out_dim, G.Q4_K, sptr)
        for i in range(3):
            call_f32(i)
        us = _time(call_f32, iters, stream, sustain_ms=SUSTAIN_MS)
        tflops = 2.0 * T * in_dim * out_dim / (us * 1e-6) / 1e12
        bf = next(e for e in res["by_tokens"] if e["tokens"] == T)
        entry = {"tokens": T, "us_per_op": round(us, 2), "tflops": round(tflops, 1),
                 "frac_of_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                 "vs_bf16_leg": round(bf["us_per_op"] / us, 3)}
        if with_cpu and T == 512:
            from oracle import oracle as O
            toks = np.linspace(0, T - 1, 8).astype(int)
            rc, want = O.matmul_quant_f32(w_host, x_host.reshape(T, in_dim)[toks].reshape(-1),
                                          len(toks), in_dim, out_dim, int(G.Q4_K))
            got = d_y.cpu().numpy().reshape(T, out_dim)[toks].reshape(-1)
            entry["check"] = {"max_rel_err_vs_oracle": float(np.abs(got - want).max() /
                                                             np.abs(want).max()),
                              "tokens_checked": len(toks), "tolerance": 1e-3}
        res["f32_x"].append(entry)
        del d_x, d_y
    # Grids under half the CUs (short prompts, few-row matrices): K split
    # across workgroups, partial sums added in split order. The FFN-down
    # shape (in 14336 -> out 4096) and C4 at T = 100, through the bf16 entry.
    res["k_split"] = []
    for (n_out, n_in, T, seed) in ((4096, 14336, 512, 407), (14336, 4096, 100, 408)):
        w_s = synth.weight(G.Q4_K, n_out, n_in, seed=seed) if n_out != out_dim else w_host
        d_ws = torch.from_numpy(w_s).to(dev) if n_out != out_dim else d_w
        xb = synth.bf16_activations(T, n_in, seed=seed + 1).reshape(-1)
        d_x = torch.from_numpy(xb.view(np.int16)).to(dev)
        d_y = torch.empty(T * n_out, dtype=torch.float32, device=dev)

        def call_s(i):
            B.matmul_q4k_bf16_dev(d_y.data_ptr(), d_y.numel(), d_ws.data_ptr(), d_ws.numel(),
                                  d_x.data_ptr(), d_x.numel(), T, n_in, n_out, G.Q4_K, sptr)
        for i in range(3):
            call_s(i)
        us = _time(call_s, iters, stream, sustain_ms=SUSTAIN_MS)
        tflops = 2.0 * T * n_in * n_out / (us * 1e-6) / 1e12
        entry = {"shape": f"{n_out}x{n_in}", "tokens": T, "us_per_op": round(us, 2),
                 "tflops": round(tflops, 1), "frac_of_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        if with_cpu:
            from oracle import oracle as O
            toks = np.linspace(0, T - 1, 6).astype(int)
            xf = synth.bf16_bits_to_f32(xb.reshape(T, n_in)[toks]).reshape(-1)
            rc, want = O.matmul_quant_f32(w_s, xf, len(toks), n_in, n_out, int(G.Q4_K))
            got = d_y.cpu().numpy().reshape(T, n_out)[toks].reshape(-1)
            entry["check"] = {"max_rel_err_vs_oracle": float(np.abs(got - want).max() /
                                                             np.abs(want).max()),
                              "tokens_checked": len(toks), "tolerance": 1e-3}
        res["k_split"].append(entry)
        del d_x, d_y, d_ws
    # The other formats on the same GEMM: Q6_K (C1's format) and Q8_0 (C2's)
    # at C4's shape, T = 512, through the reference's f32-x call on
    # weights in the device layout.
    res["formats"] = []
    T = 512
    for (dt, seed) in ((G.Q6_K, 409), (G.Q8_0, 410)):
        w_f = synth.weight(dt, out_dim, in_dim, seed=seed)
        raw = torch.from_numpy(w_f).to(dev)
        d_wf = torch.empty_like(raw)
        B.prepare_weights_dev(d_wf.data_ptr(), raw.data_ptr(), raw.numel(), dt, in_dim, sptr)
        del raw
        xf_all = synth.activations(T, in_dim, seed=seed + 1).reshape(-1)
        d_x = torch.from_numpy(xf_all).to(dev)
        d_y = torch.empty(T * out_dim, dtype=torch.float32, device=dev)

        def call_f(i):
            B.matmul_quant_f32_dev(d_y.data_ptr(), d_y.numel(), d_wf.data_ptr(), d_wf.numel(),
                                   d_x.data_ptr(), d_x.numel(), T, in_dim, out_dim, dt, sptr)
        for i in range(3):
            call_f(i)
        us = _time(call_f, iters, stream, sustain_ms=SUSTAIN_MS)
        tflops = 2.0 * T * in_dim * out_dim / (us * 1e-6) / 1e12
        entry = {"format": dt.name, "shape": f"{out_dim}x{in_dim}", "tokens": T,
                 "us_per_op": round(us, 2), "tflops": round(tflops, 1),
                 "frac_of_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        if with_cpu:
            from oracle import oracle as O
            toks = np.linspace(0, T - 1, 6).astype(int)
            xs = xf_all.reshape(T, in_dim)[toks].reshape(-1)
            rc, want = O.matmul_quant_f32(w_f, xs, len(toks), in_dim, out_dim, int(dt))
            got = d_y.cpu().numpy().reshape(T, out_dim)[toks].reshape(-1)
            entry["check"] = {"max_rel_err_vs_oracle": float(np.abs(got - want).max() /
                                                             np.abs(want).max()),
                              "tokens_checked": len(toks), "tolerance": 1e-3}
        res["formats"].append(entry)
        del d_x, d_y, d_wf
    res["mfma_ceiling"] = bench_mfma_ceiling(B, dev, stream)
    res["dense_f16_library"] = bench_dense_f16(dev, stream, out_dim, in_dim, iters)
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


def bench_mfma_ceiling(B, dev, stream, iters=200):
    """prefill.mfma_ceiling: the matrix-core issue rate the prefill GEMM is
    compared with (rsllm_hip_mfma_issue_dev): the GEMM's inner-loop shape,
    32 groups of four independent 16x16x32 f16 MFMAs per round, with 0, 4 or
    8 packed-f16 FMAs after each group, one or two 4-wavefront workgroups per
    CU on all 256 CUs."""
    import torch
    out = {"unit": "TFLOP/s", "mfma_per_wave": 128 * iters, "by_case": []}
    for valu in (0, 4, 8):
        for two in (False, True):
            n_wg = 512 if two else 256
            sink = torch.empty(n_wg * 256, dtype=torch.int32, device=dev)

            def call(i):
                B.mfma_issue_dev(sink.data_ptr(), sink.numel(), n_wg, iters, valu, two,
                                 stream.cuda_stream)
            call(0)
            us = _time(call, 5, stream)
            flops = 16384.0 * 128 * iters * 4 * n_wg
            tf = flops / (us * 1e-6) / 1e12
            out["by_case"].append({"valu_per_mfma": valu / 4, "waves_per_simd": 2 if two else 1,
                                   "us": round(us, 1), "tflops": round(tf, 1),
                                   "frac_of_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
    return out


def bench_dense_f16(dev, stream, out_dim, in_dim, iters):
    """prefill.dense_f16_library: the platform GEMM library (torch ->
    hipBLASLt) on the same shape with dense f16 weights and f16 output, no
    dequantisation, as a reference point for the fused Q4_K GEMM. The weight
    alternates between two copies."""
    import torch
    res = []
    ws = [torch.randn(out_dim, in_dim, device=dev, dtype=torch.float16) for _ in range(2)]
    for T in (512, 2048):
        x = torch.randn(T, in_dim, device=dev, dtype=torch.float16)

        def call(i):
            torch.nn.functional.linear(x, ws[i & 1])
        us = _time(call, iters, stream, sustain_ms=SUSTAIN_MS)
        tf = 2.0 * T * in_dim * out_dim / (us * 1e-6) / 1e12
        res.append({"tokens": T, "us_per_op": round(us, 2), "tflops": round(tf, 1),
                    "frac_of_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
        del x
    del ws
    return res


def _progress(msg):
    """One line per finished stage on stderr (the JSON line stays alone on
    stdout)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


SPINUP_COPY_BYTES = 256 << 20
_spin_bufs = []


def _spinup(ms):
    """Keep the GPU busy for `ms` milliseconds of 256 MB device copies (HBM
    traffic, outside any timed region), then wait for them. After the host
    has left the GPU idle (weight synthesis, oracle checks) its first
    milliseconds of work run slower than its steady state (measured on
    MI355X: the first 40 C1 GEMVs after 1 s idle took 254 us each, the next
    few hundred 11.9-12.3 us, against 11.4 us after a 20 ms copy spin); a
    timed region of well under a millisecond would measure that ramp."""
    import torch
    if ms <= 0:
        return
    if not _spin_bufs:
        a = torch.empty(SPINUP_COPY_BYTES, dtype=torch.uint8, device="cuda")
        _spin_bufs.extend([a, torch.empty_like(a)])
    a, b = _spin_bufs
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()


def _sustain(fn, ms):
    """Run `fn` back to back for `ms` milliseconds of wall time (outside any
    timed region), then wait for it. Under sustained matrix-core load the
    GPU's clocks settle some 10-20 ms after a spell of other work (measured
    on MI355X: the C4 prefill call at T = 2048 took 230-250 us over its first
    50 calls after a 20 ms copy spin-up, then 222-224 us; the C3 routed
    experts at T = 8 took 277 us per call over its first 16 calls, 241 us
    after 200); prefill and routed-expert calls come back to back in a
    forward pass, so those figures are taken after this warm-up on the timed
    call itself. The batched decode calls measured the same either way."""
    import torch
    t0, i = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()


SUSTAIN_MS = 50


def _time(fn, iters, stream, spin_ms=20, sustain_ms=0):
    """Mean microseconds per call over `iters` back-to-back calls, one HIP
    event pair on the launch stream around the whole run, after a spin-up
    of `spin_ms` (_spinup) or, with sustain_ms, `sustain_ms` of the call
    itself (_sustain)."""
    import torch
    if sustain_ms > 0:
        _sustain(fn, sustain_ms)
    else:
        _spinup(spin_ms)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for i in range(iters):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / iters


def _rotating(t, min_bytes=640e6):
    """Distinct device copies of `t` totalling >= min_bytes (> the 256 MB
    Infinity Cache), so every timed launch streams its weights from HBM."""
    n = max(2, int(np.ceil(min_bytes / (t.numel() * t.element_size()))))
    return [t] + [t.clone() for _ in range(n - 1)]


PMC_COPY_BYTES = 256 << 20
PMC_LAUNCHES = 24  # per C1 shape; the last 8 of each are counted


def pmc_probe():
    """Run under rocprofv3 --pmc by pmc_traffic(): three device copies of
    PMC_COPY_BYTES (the calibration kernel, bytes known) and then the dominant
    kernels of the bench line (C1 Q6_K batch-1 GEMV, 14336x4096 then
    4096x14336, one launch per call, PMC_LAUNCHES each) streaming their
    weights from HBM through rotating copies."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    dev = torch.device("cuda:0")
    sptr = torch.cuda.current_stream().cuda_stream
    a = torch.empty(PMC_COPY_BYTES, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    del a, b
    for si, (out_dim, in_dim) in enumerate(((14336, 4096), (4096, 14336))):
        w_host = synth.weight(G.Q6_K, out_dim, in_dim, seed=100 + si)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), G.Q6_K, in_dim, sptr)
        del raw
        reps = _rotating(prep)
        x = torch.from_numpy(synth.activations(1, in_dim, seed=200 + si)).to(dev).reshape(-1)
        y = torch.empty(out_dim, dtype=torch.float32, device=dev)
        for i in range(PMC_LAUNCHES):
            w = reps[i % len(reps)]
            B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                   x.numel(), 1, in_dim, out_dim, G.Q6_K, sptr)
        torch.cuda.synchronize()
        del reps, prep


def prefill_probe(T, fmt="Q4_K", warm=True):
    """The C4 prefill call (Q4_K 14336x4096 weights, bf16 x [T x 4096]) five
    times, for rocprofv3 runs that count MFMA and VALU work per dispatch;
    with fmt Q6_K or Q8_0, the same shape in that format through the f32-x
    call (weights in the device layout). With `warm`, PF_PROBE_WARM[T] calls
    (about 25 ms back to back, the clock warm-up of _sustain) come first:
    a kernel trace's last five calls of each kernel are the measured ones."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    out_dim, in_dim = 14336, 4096
    sptr = torch.cuda.current_stream().cuda_stream
    dt = G[fmt]
    n_warm = PF_PROBE_WARM.get(T, 0) if warm else 0
    w = torch.from_numpy(synth.weight(dt, out_dim, in_dim, seed=300)).cuda()
    y = torch.empty(T * out_dim, dtype=torch.float32, device="cuda")
    if dt == G.Q4_K:
        x = torch.from_numpy(synth.bf16_activations(T, in_dim, seed=301).reshape(-1)).cuda()
        for _ in range(5 + n_warm):
            B.matmul_q4k_bf16_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                  x.numel(), T, in_dim, out_dim, G.Q4_K, sptr)
    else:
        d = torch.empty_like(w)
        B.prepare_weights_dev(d.data_ptr(), w.data_ptr(), w.numel(), dt, in_dim, sptr)
        x = torch.from_numpy(synth.activations(T, in_dim, seed=301).reshape(-1)).cuda()
        for _ in range(5 + n_warm):
            B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), d.data_ptr(), d.numel(), x.data_ptr(),
                                   x.numel(), T, in_dim, out_dim, dt, sptr)
    torch.cuda.synchronize()


def moe_probe(T):
    """The C3 routed-expert call (64 experts, Q4_K gate/up 2048x7168, down
    7168x2048, top-8) at T tokens over 8 routings: 25 ms of calls back to
    back (the clock warm-up of _sustain), then 8 calls, one per routing; a
    kernel trace's last 8 calls are the measured ones."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    n_expert, n_embd, n_ff, k = 64, 7168, 2048, 8
    sptr = torch.cuda.current_stream().cuda_stream
    gate = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 600)
    up = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 601)
    down = synth.weight(G.Q4_K, n_expert * n_embd, n_ff, 602)
    d_g, d_u, d_d = (torch.from_numpy(a).cuda() for a in (gate, up, down))
    x = torch.from_numpy(synth.activations(T, n_embd, 610 + T).reshape(-1)).cuda()
    y = torch.zeros(T * n_embd, dtype=torch.float32, device="cuda")
    routs = []
    for r in range(8):
        routs.append(tuple(torch.from_numpy(a.reshape(-1)).cuda()
                           for a in synth.moe_routing(T, n_expert, k, 620 + T + 1000 * r)))

    def call(i):
        d_i, d_w = routs[i % 8]
        B.moe_routed_dev(y.data_ptr(), y.numel(), x.data_ptr(), x.numel(), d_g.data_ptr(),
                         d_u.data_ptr(), gate.nbytes, d_d.data_ptr(), down.nbytes, d_i.data_ptr(),
                         d_w.data_ptr(), d_i.numel(), T, n_embd, n_ff, n_expert, k, G.Q4_K,
                         G.Q4_K, 10.0, sptr)
    _sustain(call, 25)
    for r in range(8):
        call(r)
    torch.cuda.synchronize()


def dsv4_probe(T):
    """The DS-V4 routed-expert call (IQ2_XXS gate/up 2048x4096, Q2_K down
    4096x2048, 256 experts, top-6, weights in the device layout) at T tokens
    over 4 routings: 25 ms of calls back to back, then 8 calls; a kernel
    trace's last 8 calls are the measured ones."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    n_expert, n_embd, n_ff, k = 256, 4096, 2048, 6
    sptr = torch.cuda.current_stream().cuda_stream
    mats = []
    for seed, dt, rows, ind in ((650, G.IQ2_XXS, n_expert * n_ff, n_embd),
                                (651, G.IQ2_XXS, n_expert * n_ff, n_embd),
                                (652, G.Q2_K, n_expert * n_embd, n_ff)):
        raw = torch.from_numpy(synth.weight(dt, rows, ind, seed)).cuda()
        d = torch.empty_like(raw)
        B.prepare_weights_dev(d.data_ptr(), raw.data_ptr(), raw.numel(), dt, ind, sptr)
        mats.append(d)
        del raw
    d_g, d_u, d_d = mats
    x = torch.from_numpy(synth.activations(T, n_embd, 660 + T).reshape(-1)).cuda()
    y = torch.zeros(T * n_embd, dtype=torch.float32, device="cuda")
    routs = [tuple(torch.from_numpy(a.reshape(-1)).cuda()
                   for a in synth.moe_routing(T, n_expert, k, 670 + T + 1000 * r)) for r in range(4)]

    def call(i):
        d_i, d_w = routs[i % 4]
        B.moe_routed_dev(y.data_ptr(), y.numel(), x.data_ptr(), x.numel(), d_g.data_ptr(),
                         d_u.data_ptr(), d_g.numel(), d_d.data_ptr(), d_d.numel(), d_i.data_ptr(),
                         d_w.data_ptr(), d_i.numel(), T, n_embd, n_ff, n_expert, k, G.IQ2_XXS,
                         G.Q2_K, 10.0, sptr)
    _sustain(call, 25)
    for r in range(8):
        call(r)
    torch.cuda.synchronize()


TRACE_LAUNCHES = 64
# (tag, dtype name, out_dim, in_dim) of the batch-1 GEMVs --gemv-probe runs,
# in launch order: C1 both orientations (the bench line), then C0
PROBE_GEMVS = [("C1", "Q6_K", 14336, 4096), ("C1", "Q6_K", 4096, 14336), ("C0", "Q4_K", 4096, 4096)]


# (tag, dtype name, out_dim, in_dim, tokens) of the batched decode calls
# --batch-probe runs (C1 at 4 and 8 tokens, C2 Q8_0 at 8 and 32)
PROBE_BATCHED = [("C1", "Q6_K", 14336, 4096, 4), ("C1", "Q6_K", 4096, 14336, 4),
                 ("C1", "Q6_K", 14336, 4096, 8), ("C1", "Q6_K", 4096, 14336, 8),
                 ("C2", "Q8_0", 4096, 4096, 8), ("C2", "Q8_0", 4096, 4096, 16),
                 ("C2", "Q8_0", 4096, 4096, 32), ("C2", "Q8_0", 1024, 4096, 16),
                 ("C2", "Q8_0", 1024, 4096, 32)]


def batch_probe():
    """Run under rocprofv3 (kernel trace, counters): the batched decode calls
    of PROBE_BATCHED through matmul_quant_f32_dev, TRACE_LAUNCHES each, every
    call reading a different weight copy so the weights stream from HBM."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    dev = torch.device("cuda:0")
    sptr = torch.cuda.current_stream().cuda_stream
    for si, (_, dname, out_dim, in_dim, n_tok) in enumerate(PROBE_BATCHED):
        dtype = G[dname]
        w_host = synth.weight(dtype, out_dim, in_dim, seed=100 + si)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, sptr)
        del raw
        reps = _rotating(prep)
        x = torch.from_numpy(synth.activations(n_tok, in_dim, seed=200 + si)).to(dev).reshape(-1)
        y = torch.empty(n_tok * out_dim, dtype=torch.float32, device=dev)
        _spinup(20)
        for i in range(TRACE_LAUNCHES):
            w = reps[i % len(reps)]
            B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                   x.numel(), n_tok, in_dim, out_dim, dtype, sptr)
        torch.cuda.synchronize()
        del reps, prep


def q8_probe():
    """Run under rocprofv3 --kernel-trace: C2 (4096x4096, 1024x4096) through
    the int8-activation path at 1..32 tokens, TRACE_LAUNCHES calls of
    quantize_q8_0_batch_dev + matmul_q8_0_batch_dev each after 20 ms of
    copies, every matmul reading a different weight copy."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    dev = torch.device("cuda:0")
    sptr = torch.cuda.current_stream().cuda_stream
    for (o, i_) in ((4096, 4096), (1024, 4096)):
        raw = torch.from_numpy(synth.weight(G.Q8_0, o, i_, 540 + o // 1024)).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), G.Q8_0, i_, sptr)
        del raw
        reps = _rotating(prep)
        blocks = i_ // 32
        for n_tok in (1, 2, 4, 8, 16, 32):
            x = torch.from_numpy(synth.activations(n_tok, i_, 550 + n_tok).reshape(-1)).to(dev)
            xq = torch.empty(n_tok * blocks * 32, dtype=torch.int8, device=dev)
            xs = torch.empty(n_tok * blocks, dtype=torch.float32, device=dev)
            y = torch.empty(n_tok * o, dtype=torch.float32, device=dev)
            _spinup(20)
            for i in range(TRACE_LAUNCHES):
                w = reps[i % len(reps)]
                B.quantize_q8_0_batch_dev(x.data_ptr(), x.numel(), xq.data_ptr(), xq.numel(),
                                          xs.data_ptr(), xs.numel(), n_tok, i_, 0, sptr)
                B.matmul_q8_0_batch_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(),
                                        xq.data_ptr(), xq.numel(), xs.data_ptr(), xs.numel(),
                                        n_tok, i_, o, sptr)
            torch.cuda.synchronize()
        del reps, prep


# C4 prefill calls the trace child runs after the batch-1 GEMVs: (T, calls,
# skipped): the first `skipped` calls of each T (about 25 ms of back-to-back
# calls, the clock warm-up of _sustain) are dropped
PF_TRACE = [(512, 480, 380), (2048, 150, 110)]
PF_PROBE_WARM = {512: 380, 2048: 110}


def gemv_probe():
    """Run under rocprofv3 --kernel-trace by kernel_trace(): the batch-1
    GEMVs of PROBE_GEMVS, TRACE_LAUNCHES launches each through
    matmul_quant_f32_dev (one kernel per call at batch 1), every launch
    reading a different weight copy (> 640 MB of copies per shape) so the
    weights stream from HBM; then the C4 prefill call (Q4_K 14336x4096,
    bf16 x) at the token counts of PF_TRACE."""
    import torch
    from rsllm_amd import backend as B
    from rsllm_amd import synth
    from rsllm_amd.ggml import GgmlType as G
    dev = torch.device("cuda:0")
    sptr = torch.cuda.current_stream().cuda_stream
    for si, (_, dname, out_dim, in_dim) in enumerate(PROBE_GEMVS):
        dtype = G[dname]
        w_host = synth.weight(dtype, out_dim, in_dim, seed=100 + si)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, sptr)
        del raw
        reps = _rotating(prep)
        x = torch.from_numpy(synth.activations(1, in_dim, seed=200 + si)).to(dev).reshape(-1)
        y = torch.empty(out_dim, dtype=torch.float32, device=dev)
        _spinup(20)
        for i in range(TRACE_LAUNCHES):
            w = reps[i % len(reps)]
            B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                   x.numel(), 1, in_dim, out_dim, dtype, sptr)
        torch.cuda.synchronize()
        del reps, prep
    out_dim, in_dim = 14336, 4096
    w = torch.from_numpy(synth.weight(G.Q4_K, out_dim, in_dim, seed=404)).to(dev)
    for T, calls, _ in PF_TRACE:
        x = torch.from_numpy(synth.bf16_activations(T, in_dim, seed=405).reshape(-1)).to(dev)
        y = torch.empty(T * out_dim, dtype=torch.float32, device=dev)
        _spinup(20)
        for _ in range(calls):
            B.matmul_q4k_bf16_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                  x.numel(), T, in_dim, out_dim, G.Q4_K, sptr)
        torch.cuda.synchronize()
        del x, y


def _summary(us):
    us = np.asarray(us, dtype=np.float64)
    return {"n": int(us.size), "us_mean": round(float(us.mean()), 3),
            "us_median": round(float(np.median(us)), 3),
            "us_p10": round(float(np.percentile(us, 10)), 3),
            "us_p90": round(float(np.percentile(us, 90)), 3)}


def kernel_trace():
    """Kernel-trace durations of the batch-1 GEMVs: one rocprofv3
    --kernel-trace pass over a child run of gemv_probe(). The k_gemv1
    dispatches come in PROBE_GEMVS order, TRACE_LAUNCHES per shape; the first
    8 of each shape are dropped (warm-up). Returns a list of per-shape
    summaries (mean / median / p10 / p90 in microseconds) or an error dict."""
    import shutil
    import sqlite3
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return {"error": "rocprofv3 not found"}
    here = os.path.abspath(__file__)
    env = dict(os.environ, TMPDIR="/tmp")
    d = tempfile.mkdtemp(prefix="rsllm_kt_", dir="/tmp")
    cmd = ["timeout", "-s", "KILL", "150", exe, "--kernel-trace", "-d", d, "-o", "p", "--",
           sys.executable, here, "--gemv-probe"]
    try:
        r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=180)
    except subprocess.TimeoutExpired:
        return {"error": "kernel-trace pass timed out"}
    dbs = [os.path.join(root, f) for root, _, fs in os.walk(d) for f in fs if f.endswith(".db")]
    if not dbs:
        return {"error": f"kernel-trace pass failed (rc {r.returncode})",
                "stderr_tail": r.stderr[-400:]}
    rows = sqlite3.connect(dbs[0]).execute(
        "select name, duration from kernels order by dispatch_id").fetchall()
    shutil.rmtree(d, ignore_errors=True)
    durs = [(n, v) for n, v in rows if "k_gemv1" in n]
    if len(durs) != TRACE_LAUNCHES * len(PROBE_GEMVS):
        return {"error": f"expected {TRACE_LAUNCHES * len(PROBE_GEMVS)} k_gemv1 dispatches, "
                         f"found {len(durs)}"}
    gemv = []
    for si, (tag, dname, out_dim, in_dim) in enumerate(PROBE_GEMVS):
        part = durs[si * TRACE_LAUNCHES:(si + 1) * TRACE_LAUNCHES][8:]
        gemv.append({"config": tag, "dtype": dname, "shape": f"{out_dim}x{in_dim}",
                     "kernel": part[0][0].split("(")[0],
                     **_summary([v / 1e3 for _, v in part])})
    # prefill: per call one pre-pass (k_prefill_x), one GEMM (k_prefill_q4k_w8)
    # and, where the GEMM splits K, the partial-sum kernel (k_prefill_sum*),
    # counted with the GEMM
    calls_seen = []  # [pre-pass, GEMM, partial sums] in ns per call
    for n, v in rows:
        if "k_prefill_x" in n:
            calls_seen.append([v, 0, 0])
        elif calls_seen and "k_prefill_q4k_w8" in n:
            calls_seen[-1][1] += v
        elif calls_seen and "k_prefill_sum" in n:
            calls_seen[-1][2] += v
    n_calls = sum(c for _, c, _ in PF_TRACE)
    prefill = []
    if len(calls_seen) == n_calls and all(c[1] > 0 for c in calls_seen):
        o = 0
        for T, calls, skip in PF_TRACE:
            sl = calls_seen[o + skip:o + calls]
            prefill.append({"tokens": T, "gemm": _summary([(c[1] + c[2]) / 1e3 for c in sl]),
                            "partial_sums": _summary([c[2] / 1e3 for c in sl]),
                            "prepass": _summary([c[0] / 1e3 for c in sl])})
            o += calls
    else:
        prefill = {"error": f"expected {n_calls} prefill calls, found {len(calls_seen)}"}
    return {"gemv": gemv, "prefill": prefill}


def prefill_pmc_probe():
    """Run under rocprofv3 --pmc by prefill_mfma_busy(): the C4 prefill call
    (Q4_K 14336x4096, bf16 x) five times at T = 512, then five times at
    T = 2048."""
    prefill_probe(512, warm=False)
    prefill_probe(2048, warm=False)


# MI355X: 256 CUs of 4 SIMDs in 8 XCDs (GRBM_GUI_ACTIVE is summed over the XCDs)
N_SIMDS, N_XCDS = 1024, 8


def prefill_mfma_busy():
    """MFMA utilisation of the C4 prefill GEMM: one rocprofv3 --pmc pass
    (SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_MFMA, SQ_INSTS_VALU, GRBM_GUI_ACTIVE)
    over a child run of prefill_pmc_probe(). Busy fraction = matrix-pipe busy
    cycles per SIMD / the kernel's GPU cycles (GRBM_GUI_ACTIVE per XCD), the
    median over the five dispatches of each T."""
    import shutil
    import sqlite3
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return {"error": "rocprofv3 not found"}
    here = os.path.abspath(__file__)
    env = dict(os.environ, TMPDIR="/tmp")
    d = tempfile.mkdtemp(prefix="rsllm_pfpmc_", dir="/tmp")
    ctrs = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "GRBM_GUI_ACTIVE"]
    cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", *ctrs, "-d", d, "-o", "p", "--",
           sys.executable, here, "--prefill-pmc-probe"]
    try:
        r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=150)
    except subprocess.TimeoutExpired:
        return {"error": "prefill counter pass timed out"}
    dbs = [os.path.join(root, f) for root, _, fs in os.walk(d) for f in fs if f.endswith(".db")]
    if r.returncode != 0 or not dbs:
        return {"error": f"prefill counter pass failed (rc {r.returncode})",
                "stderr_tail": r.stderr[-400:]}
    rows = sqlite3.connect(dbs[0]).execute(
        "select dispatch_id, name, counter_name, counter_value from pmc_events "
        "order by dispatch_id").fetchall()
    shutil.rmtree(d, ignore_errors=True)
    per = {}
    for did, name, cn, v in rows:
        if "k_prefill_q4k_w8" in name:
            per.setdefault(did, {})[cn] = per.get(did, {}).get(cn, 0.0) + float(v)
    disp = [per[k] for k in sorted(per)]
    if len(disp) != 10:
        return {"error": f"expected 10 GEMM dispatches, found {len(disp)}"}
    out = {"counters": ctrs, "simds": N_SIMDS, "xcds": N_XCDS}
    for j, T in enumerate((512, 2048)):
        busy = [c["SQ_VALU_MFMA_BUSY_CYCLES"] / N_SIMDS / (c["GRBM_GUI_ACTIVE"] / N_XCDS)
                for c in disp[5 * j:5 * j + 5]]
        valu = [(c["SQ_INSTS_VALU"] - c["SQ_INSTS_MFMA"]) / c["SQ_INSTS_MFMA"]
                for c in disp[5 * j:5 * j + 5]]
        out[f"t{T}"] = {"mfma_busy": round(float(np.median(busy)), 4),
                        "valu_per_mfma": round(float(np.median(valu)), 3)}
    return out


def bench_stream_read(B, dev, stream, iters):
    """extra.stream_read: the streaming-read ceiling for the byte counts of the
    batch-1 GEMVs (C1 48.2 MB, C0 9.47 MB): rsllm_hip_stream_read_dev over
    rotating buffers (> 640 MB), swept over grid size, workgroup size, loads
    in flight and access order; the best configuration per size and its
    GB/s."""
    import torch
    sptr = stream.cuda_stream
    res = []
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for tag, nbytes in (("C1", 48242688), ("C0", 9469952)):
        nbytes = nbytes // 16 * 16
        reps = _rotating(torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1))
        sink = torch.empty(4 * cus * 1024, dtype=torch.int32, device=dev)
        best = None
        for n_wg in (cus, 2 * cus, 4 * cus):
            for threads in (256, 512, 1024):
                for unroll in (2, 4, 8):
                    for contiguous in (1, 0):
                        def call(i):
                            B.stream_read_dev(reps[i % len(reps)].data_ptr(), nbytes,
                                              sink.data_ptr(), sink.numel(), n_wg, threads,
                                              unroll, contiguous, sptr)
                        for i in range(len(reps)):
                            call(i)
                        us = _time(call, iters, stream)
                        if best is None or us < best["us"]:
                            best = {"config": tag, "bytes": nbytes, "us": round(us, 3),
                                    "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                                    "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                    "n_wg": n_wg, "threads": threads, "unroll": unroll,
                                    "contiguous": bool(contiguous)}
        res.append(best)
        del reps, sink
    return res


def pmc_traffic():
    """roofline.traffic: HBM bytes per launch of the dominant kernel from two
    rocprofv3 --pmc passes over a child run of pmc_probe() (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch). Each counter is scaled by bytes / counter of
    the calibration copy in the same pass, whose read and write sizes are
    known. Returns ({shape: bytes} or None, details)."""
    import shutil
    import sqlite3
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return None, {"error": "rocprofv3 not found"}
    here = os.path.abspath(__file__)
    env = dict(os.environ, TMPDIR="/tmp")
    det = {"calibration": f"device copy of {PMC_COPY_BYTES} bytes (read {PMC_COPY_BYTES}, "
                          f"write {PMC_COPY_BYTES})"}
    totals = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="rsllm_pmc_", dir="/tmp")
        cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", ctr, "-d", d, "-o", "p", "--",
               sys.executable, here, "--pmc-probe"]
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=150)
        except subprocess.TimeoutExpired:
            return None, {"error": f"{ctr} pass timed out"}
        dbs = [os.path.join(root, f) for root, _, fs in os.walk(d) for f in fs if f.endswith(".db")]
        if r.returncode != 0 or not dbs:
            return None, {"error": f"{ctr} pass failed (rc {r.returncode})",
                          "stderr_tail": r.stderr[-400:]}
        rows = sqlite3.connect(dbs[0]).execute(
            "select name, counter_value from pmc_events where counter_name = ? "
            "order by dispatch_id", (ctr,)).fetchall()
        shutil.rmtree(d, ignore_errors=True)
        # the calibration copies are the probe's first three copy dispatches
        # (later ones are weight uploads and clones of other sizes)
        copy = [v for n, v in rows if "copyBuffer" in n][:3]
        gemv = [v for n, v in rows if "k_gemv1" in n]
        if not copy or len(gemv) != 2 * PMC_LAUNCHES:
            return None, {"error": f"{ctr}: kernels not found in the pass"}
        factor = PMC_COPY_BYTES / (float(np.median(copy)) * 1024.0)
        per_shape = []
        for si, shape in enumerate(("14336x4096", "4096x14336")):
            kib = float(np.median(gemv[(si + 1) * PMC_LAUNCHES - 8:(si + 1) * PMC_LAUNCHES]))
            per_shape.append({"shape": shape, "gemv_kib_per_dispatch": round(kib, 1),
                              "bytes_per_launch": round(kib * 1024.0 * factor)})
            totals[shape] = totals.get(shape, 0.0) + kib * 1024.0 * factor
        det[ctr] = {"copy_kib_per_dispatch": round(float(np.median(copy)), 1),
                    "factor_bytes_per_counted_byte": round(factor, 4), "per_shape": per_shape}
    return {k: round(v) for k, v in totals.items()}, det


def bench_extra(B, synth, G, dev, stream, iters, with_cpu):
    """The other configs: device copy bandwidth, C0, C1 at B = 4 / 8, C2 (f32-x
    path and the bit-exact int8-activation path), C3 routed experts."""
    import torch
    sptr = stream.cuda_stream
    out = {}
    # ---- measured device copy bandwidth (read + write) ----
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    us = _time(lambda i: dst.copy_(src), 20, stream)
    out["device_copy"] = {"bytes_moved": 2 * src.numel(), "us": round(us, 1),
                          "GBps": round(2 * src.numel() / (us * 1e-6) / 1e9, 1),
                          "what": "torch copy_ of 1 GiB device -> device (read + write)"}
    del src, dst

    # ---- GEMV configs through matmul_quant_f32_dev ----
    def gemv_case(tag, dtype, out_dim, in_dim, n_tok, seed):
        w_host = synth.weight(dtype, out_dim, in_dim, seed)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, sptr)
        del raw
        reps = _rotating(prep)
        x_host = synth.activations(n_tok, in_dim, seed + 1).reshape(-1)
        x = torch.from_numpy(x_host).to(dev)
        y = torch.empty(n_tok * out_dim, dtype=torch.float32, device=dev)

        def call(i):
            w = reps[i % len(reps)]
            B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                   x.numel(), n_tok, in_dim, out_dim, dtype, sptr)
        for i in range(len(reps)):
            call(i)
        us = _time(call, iters, stream)
        nbytes = prep.numel() + n_tok * (in_dim + out_dim) * 4
        e = {"config": tag, "dtype": dtype.name, "shape": f"{out_dim}x{in_dim}", "batch": n_tok,
             "bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if with_cpu:
            sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
            from oracle import oracle as O
            rc, want = O.matmul_quant_f32(w_host, x_host, n_tok, in_dim, out_dim, int(dtype),
                                          allow_q6k=True)
            got = y.cpu().numpy()
            e["max_rel_err_vs_oracle"] = float(np.abs(got - want).max() / np.abs(want).max())
        del reps, prep
        return e

    rows = [gemv_case("C0", G.Q4_K, 4096, 4096, 1, 500)]
    for n_tok in (4, 8):
        rows.append(gemv_case("C1", G.Q6_K, 14336, 4096, n_tok, 510))
        rows.append(gemv_case("C1", G.Q6_K, 4096, 14336, n_tok, 520))
    for (o, i_) in ((4096, 4096), (1024, 4096)):
        for n_tok in (1, 2, 4, 8, 16, 32):
            rows.append(gemv_case("C2", G.Q8_0, o, i_, n_tok, 530 + o // 1024))
    out["gemv"] = rows
    _progress("extra: gemv done")
    out["stream_read"] = bench_stream_read(B, dev, stream, iters)
    _progress("extra: stream_read done")

    # ---- C2 through the int8-activation path (quantize + matmul, bit-exact) ----
    q8 = []
    for (o, i_) in ((4096, 4096), (1024, 4096)):
        w_host = synth.weight(G.Q8_0, o, i_, 540 + o // 1024)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), G.Q8_0, i_, sptr)
        del raw
        reps = _rotating(prep)
        blocks = i_ // 32
        for n_tok in (1, 2, 4, 8, 16, 32):
            x_host = synth.activations(n_tok, i_, 550 + n_tok).reshape(-1)
            x = torch.from_numpy(x_host).to(dev)
            xq = torch.empty(n_tok * blocks * 32, dtype=torch.int8, device=dev)
            xs = torch.empty(n_tok * blocks, dtype=torch.float32, device=dev)
            y = torch.empty(n_tok * o, dtype=torch.float32, device=dev)

            def quant(i):
                B.quantize_q8_0_batch_dev(x.data_ptr(), x.numel(), xq.data_ptr(), xq.numel(),
                                          xs.data_ptr(), xs.numel(), n_tok, i_, 0, sptr)

            def mm(i):
                w = reps[i % len(reps)]
                B.matmul_q8_0_batch_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(),
                                        xq.data_ptr(), xq.numel(), xs.data_ptr(), xs.numel(),
                                        n_tok, i_, o, sptr)
            quant(0)
            for i in range(len(reps)):
                mm(i)
            us_q = _time(quant, iters, stream)
            us_m = _time(mm, iters, stream)
            nbytes = prep.numel() + n_tok * blocks * 36 + n_tok * o * 4
            e = {"shape": f"{o}x{i_}", "batch": n_tok, "quantize_us": round(us_q, 3),
                 "matmul_us": round(us_m, 3), "matmul_bytes": nbytes,
                 "matmul_GBps": round(nbytes / (us_m * 1e-6) / 1e9, 1),
                 "frac_hbm": round(nbytes / (us_m * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
            if with_cpu and n_tok in (1, 32):
                from oracle import oracle as O
                rc, oq, os_ = O.quantize_q8_0_batch(x_host, n_tok, i_)
                rc, want = O.matmul_q8_0_batch(w_host, oq, os_, n_tok, i_, o)
                e["bit_exact_vs_oracle"] = bool(
                    np.array_equal(xq.cpu().numpy(), oq) and
                    np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)))
            q8.append(e)
        del reps, prep
    out["q8_int8"] = q8
    _progress("extra: q8_int8 done")

    # ---- caller chain at DS-V4 Flash shapes (weight.rs:113-266, moe.rs:422-502) ----
    chain = []
    # matmul_grouped_lora_down: attn_output_a, 8 groups of [1024 x 4096] Q8_0
    n_g, g_dim, rank = 8, 4096, 1024
    w_host = synth.weight(G.Q8_0, n_g * rank, g_dim, 700)
    raw = torch.from_numpy(w_host).to(dev)
    prep = torch.empty_like(raw)
    B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), G.Q8_0, g_dim, sptr)
    del raw
    reps = _rotating(prep)
    for n_tok in (1, 2, 4, 8, 16):
        x = torch.from_numpy(synth.activations(n_tok, n_g * g_dim, 701).reshape(-1)).to(dev)
        y = torch.empty(n_tok * n_g * rank, dtype=torch.float32, device=dev)

        def lora(i):
            w = reps[i % len(reps)]
            B.matmul_grouped_lora_down_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(),
                                           x.data_ptr(), x.numel(), n_tok, n_g, g_dim, rank,
                                           G.Q8_0, sptr)
        for i in range(len(reps)):
            lora(i)
        us = _time(lora, iters, stream)
        nbytes = prep.numel() + n_tok * n_g * (g_dim + rank) * 4
        chain.append({"op": "matmul_grouped_lora_down", "dtype": "Q8_0",
                      "shape": f"{n_g} x [{rank}x{g_dim}]", "batch": n_tok, "bytes": nbytes,
                      "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                      "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    del reps, prep
    # apply_shared_expert: gate/up [2048 x 4096], down [4096 x 2048], Q8_0
    e_dim, f_dim = 4096, 2048
    blobs = []
    for j, (r_, c_) in enumerate(((f_dim, e_dim), (f_dim, e_dim), (e_dim, f_dim))):
        raw = torch.from_numpy(synth.weight(G.Q8_0, r_, c_, 710 + j)).to(dev)
        p_ = torch.empty_like(raw)
        B.prepare_weights_dev(p_.data_ptr(), raw.data_ptr(), raw.numel(), G.Q8_0, c_, sptr)
        blobs.append(p_)
        del raw
    shared_bytes = sum(b_.numel() for b_ in blobs)
    n_copies = max(2, int(640e6 // shared_bytes) + 1)
    copies = [blobs] + [[b_.clone() for b_ in blobs] for _ in range(n_copies - 1)]
    for n_tok in (1, 4, 8, 16):
        x = torch.from_numpy(synth.activations(n_tok, e_dim, 720).reshape(-1)).to(dev)
        y = torch.empty(n_tok * e_dim, dtype=torch.float32, device=dev)

        def shared(i):
            g_, u_, d_ = copies[i % len(copies)]
            B.apply_shared_expert_dev(y.data_ptr(), y.numel(), x.data_ptr(), x.numel(),
                                      g_.data_ptr(), g_.numel(), G.Q8_0, u_.data_ptr(),
                                      u_.numel(), G.Q8_0, d_.data_ptr(), d_.numel(), G.Q8_0,
                                      n_tok, e_dim, f_dim, 10.0, sptr)
        for i in range(len(copies)):
            shared(i)
        us = _time(shared, iters, stream)
        nbytes = shared_bytes + 2 * n_tok * e_dim * 4
        chain.append({"op": "apply_shared_expert", "dtype": "Q8_0",
                      "shape": f"gate/up {f_dim}x{e_dim}, down {e_dim}x{f_dim}", "batch": n_tok,
                      "bytes": nbytes, "us": round(us, 3),
                      "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                      "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    del copies, blobs
    # matmul_weight_f32, F32 arm: 4096 x 4096 f32 weights
    wf = torch.randn(4096 * 4096, dtype=torch.float32, device=dev)
    reps = _rotating(wf)
    for n_tok in (1, 4):
        x = torch.randn(n_tok * 4096, dtype=torch.float32, device=dev)
        y = torch.empty(n_tok * 4096, dtype=torch.float32, device=dev)

        def wf32(i):
            w = reps[i % len(reps)]
            B.matmul_weight_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel() * 4,
                                    x.data_ptr(), x.numel(), n_tok, 4096, 4096, G.F32, sptr)
        for i in range(len(reps)):
            wf32(i)
        us = _time(wf32, iters, stream)
        nbytes = wf.numel() * 4 + n_tok * 8192 * 4
        chain.append({"op": "matmul_weight_f32", "dtype": "F32", "shape": "4096x4096",
                      "batch": n_tok, "bytes": nbytes, "us": round(us, 3),
                      "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                      "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    del reps, wf
    out["caller_chain"] = chain

    # ---- whole-model upload (GGUF mapping -> device arena, device layout) ----
    n_each, rows_q6, rows_q4 = 8, 40000, 58000
    base = np.random.default_rng(800).integers(0, 256, 16 << 20, dtype=np.uint8)
    tensors = []
    for j in range(n_each):
        for dt, rows, rb in ((G.Q6_K, rows_q6, 3360), (G.Q4_K, rows_q4, 2304)):
            n = rows * rb
            a = np.resize(base, n) ^ np.uint8(j * 2 + (dt == G.Q6_K))
            tensors.append((f"blk.{j}.{dt.name.lower()}.weight", a, dt, 4096))
    total = sum(t[1].size for t in tensors)
    runs = []
    for r in range(3):
        fp = bytes([r]) * 32
        t0 = time.perf_counter()
        mid = B.model_upload(fp, tensors)
        wall = time.perf_counter() - t0
        info = B.model_info(mid)
        B.model_release(mid)
        runs.append((wall, info["upload_seconds"]))
    best = min(runs)
    out["model_upload"] = {
        "bytes": total, "tensors": len(tensors),
        "what": "16 tensors of 134 MB (8 Q6_K converted to the device layout, 8 Q4_K copied) "
                "from host memory into one device arena; best of 3 uploads",
        "seconds": round(best[0], 4), "GBps": round(total / best[0] / 1e9, 2),
        "library_seconds": round(best[1], 4),
        "all_runs_s": [round(w, 4) for w, _ in runs]}
    del tensors, base

    # ---- C3 routed experts (64 experts, Q4_K gate/up 2048x7168, down 7168x2048, top-8) ----
    # Two device copies of the expert stacks and 8 routings per T: call i
    # uses copy i % 2 and routing (i // 2) % 8, so consecutive calls never
    # share weight bytes and a call's experts (198 MB at T = 1) are not in
    # the 256 MB Infinity Cache from the call before.
    n_expert, n_embd, n_ff, k = 64, 7168, 2048, 8
    gate = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 600)
    up = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 601)
    down = synth.weight(G.Q4_K, n_expert * n_embd, n_ff, 602)
    wcopies = []
    for c in range(2):
        t3 = tuple(torch.from_numpy(a).to(dev) for a in (gate, up, down))
        wcopies.append(t3)
    per_expert = (gate.nbytes + up.nbytes + down.nbytes) // n_expert
    n_rout = 8
    moe = []
    for T in (1, 2, 4, 8, 16, 32):
        x_host = synth.activations(T, n_embd, 610 + T).reshape(-1)
        routs = [synth.moe_routing(T, n_expert, k, 620 + T + 1000 * r) for r in range(n_rout)]
        ids, wts = routs[0]
        x = torch.from_numpy(x_host).to(dev)
        d_rout = [(torch.from_numpy(i_.reshape(-1)).to(dev), torch.from_numpy(w_.reshape(-1)).to(dev))
                  for i_, w_ in routs]
        y = torch.zeros(T * n_embd, dtype=torch.float32, device=dev)

        def call(i):
            d_g, d_u, d_d = wcopies[i % 2]
            d_ids, d_w = d_rout[(i // 2) % n_rout]
            B.moe_routed_dev(y.data_ptr(), y.numel(), x.data_ptr(), x.numel(), d_g.data_ptr(),
                             d_u.data_ptr(), gate.nbytes, d_d.data_ptr(), down.nbytes,
                             d_ids.data_ptr(), d_w.data_ptr(), ids.size, T, n_embd, n_ff, n_expert,
                             k, G.Q4_K, G.Q4_K, 10.0, sptr)
        for i in range(4):
            call(i)
        n_it = 2 * n_rout * max(1, iters // 64)
        us = _time(call, n_it, stream, sustain_ms=SUSTAIN_MS)
        n_act = float(np.mean([len(np.unique(i_)) for i_, _ in routs]))
        nbytes = int(n_act * per_expert + 2 * T * n_embd * 4)
        e = {"tokens": T, "active_experts": n_act, "bytes": nbytes, "us": round(us, 2),
             "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if with_cpu and T == 1:
            from oracle import oracle as O
            y.zero_()
            call(0)  # copy 0, routing 0
            torch.cuda.synchronize()
            want = np.zeros(T * n_embd, np.float32)
            t0 = time.perf_counter()
            rc = O.moe_routed(want, x_host, T, n_embd, n_ff, gate, up, down, int(G.Q4_K),
                              int(G.Q4_K), n_expert, ids, wts, k, 10.0)
            t_cpu = time.perf_counter() - t0
            got = y.cpu().numpy()
            e["max_rel_err_vs_oracle"] = float(np.abs(got - want).max() / np.abs(want).max())
            e["cpu_baseline"] = {"value": nbytes / t_cpu / 1e9, "unit": "GB/s", "cores": 1,
                                 "kind": "port",
                                 "sample": f"1 token, {k} experts x 3 GEMVs in {t_cpu:.2f} s, "
                                           "oracle moe_routed (accumulate_moe_outputs "
                                           "composition of matmul_quant_f32)"}
        moe.append(e)
    out["moe"] = {"workload": "C3 64 experts, Q4_K gate/up (2048, 7168), down (7168, 2048), "
                              "top-8, softmax weights", "by_tokens": moe,
                  "timing": "back-to-back calls alternating two weight copies and cycling 8 "
                            "routings (active_experts and bytes are their means)"}
    del wcopies
    _progress("extra: moe done")
    out["dsv4"] = bench_dsv4(B, synth, G, dev, stream, iters, with_cpu)
    return out


def bench_dsv4(B, synth, G, dev, stream, iters, with_cpu):
    """extra.dsv4: the DS-V4-Flash expert formats (IQ2_XXS gate/up, Q2_K
    down) at the reference's expert shapes (n_embd 4096, n_ff 2048): one
    expert matrix of each format through matmul_quant_f32_dev at 8 and 32
    tokens (decode batches) and at 512 (a prefill call), and the routed
    experts (256 experts, top-6, moe_routed_dev) from 1 to 2048 tokens. Every
    figure is taken after 50 ms of the same call back to back; the oracle
    checks 4 tokens of each dense case and of the 32-token MoE call."""
    import torch
    sptr = stream.cuda_stream
    if with_cpu:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import oracle as O
    res = {"dense": [], "moe": []}
    for (dt, o, i_, seed) in ((G.Q2_K, 4096, 2048, 640), (G.IQ2_XXS, 2048, 4096, 641)):
        w_host = synth.weight(dt, o, i_, seed)
        raw = torch.from_numpy(w_host).to(dev)
        prep = torch.empty_like(raw)
        B.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dt, i_, sptr)
        del raw
        reps = _rotating(prep)
        for T in (8, 32, 512):
            x_host = synth.activations(T, i_, seed + T).reshape(-1)
            x = torch.from_numpy(x_host).to(dev)
            y = torch.empty(T * o, dtype=torch.float32, device=dev)

            def call(i):
                w = reps[i % len(reps)]
                B.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(),
                                       x.data_ptr(), x.numel(), T, i_, o, dt, sptr)
            us = _time(call, iters, stream, sustain_ms=SUSTAIN_MS)
            nbytes = prep.numel() + T * (i_ + o) * 4
            e = {"dtype": dt.name, "shape": f"{o}x{i_}", "tokens": T, "us": round(us, 3),
                 "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "tflops": round(2.0 * T * o * i_ / (us * 1e-6) / 1e12, 2)}
            if with_cpu:
                toks = np.unique(np.linspace(0, T - 1, 4).astype(int))
                xs = x_host.reshape(T, i_)[toks].reshape(-1)
                rc, want = O.matmul_quant_f32(w_host, xs, len(toks), i_, o, int(dt))
                got = y.cpu().numpy().reshape(T, o)[toks].reshape(-1)
                e["max_rel_err_vs_oracle"] = float(np.abs(got - want).max() / np.abs(want).max())
            res["dense"].append(e)
            del x, y
        del reps, prep
    n_expert, n_embd, n_ff, k = 256, 4096, 2048, 6
    gate = synth.weight(G.IQ2_XXS, n_expert * n_ff, n_embd, 650)
    up = synth.weight(G.IQ2_XXS, n_expert * n_ff, n_embd, 651)
    down = synth.weight(G.Q2_K, n_expert * n_embd, n_ff, 652)
    # the device layout of both formats (8-block super-tiles; each expert's
    # matrix holds a whole number of them)
    dev_w = []
    for a, dt, ind in ((gate, G.IQ2_XXS, n_embd), (up, G.IQ2_XXS, n_embd), (down, G.Q2_K, n_ff)):
        raw = torch.from_numpy(a).to(dev)
        d = torch.empty_like(raw)
        B.prepare_weights_dev(d.data_ptr(), raw.data_ptr(), raw.numel(), dt, ind, sptr)
        dev_w.append(d)
        del raw
    d_g, d_u, d_d = dev_w
    per_expert = (gate.nbytes + up.nbytes + down.nbytes) // n_expert
    for T in (1, 8, 32, 512, 2048):
        x_host = synth.activations(T, n_embd, 660 + T).reshape(-1)
        routs = [synth.moe_routing(T, n_expert, k, 670 + T + 1000 * r) for r in range(4)]
        x = torch.from_numpy(x_host).to(dev)
        d_rout = [tuple(torch.from_numpy(a.reshape(-1)).to(dev) for a in rw) for rw in routs]
        y = torch.zeros(T * n_embd, dtype=torch.float32, device=dev)

        def call(i):
            d_ids, d_w = d_rout[i % 4]
            B.moe_routed_dev(y.data_ptr(), y.numel(), x.data_ptr(), x.numel(), d_g.data_ptr(),
                             d_u.data_ptr(), gate.nbytes, d_d.data_ptr(), down.nbytes,
                             d_ids.data_ptr(), d_w.data_ptr(), T * k, T, n_embd, n_ff, n_expert,
                             k, G.IQ2_XXS, G.Q2_K, 10.0, sptr)
        us = _time(call, 8 if T >= 512 else 16, stream, sustain_ms=SUSTAIN_MS)
        n_act = float(np.mean([len(np.unique(i_)) for i_, _ in routs]))
        nbytes = n_act * per_expert + 2 * T * n_embd * 4
        e = {"tokens": T, "active_experts": n_act, "us": round(us, 2),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
             "tflops": round(2.0 * T * k * 3 * n_embd * n_ff / (us * 1e-6) / 1e12, 2)}
        if with_cpu and T == 32:
            ids, wts = routs[0]
            y.zero_()
            call(0)
            torch.cuda.synchronize()
            toks = np.array([0, 11, 22, 31])
            want = np.zeros(len(toks) * n_embd, np.float32)
            rc = O.moe_routed(want, x_host.reshape(T, n_embd)[toks].reshape(-1), len(toks),
                              n_embd, n_ff, gate, up, down, int(G.IQ2_XXS), int(G.Q2_K), n_expert,
                              ids[toks], wts[toks], k, 10.0)
            got = y.cpu().numpy().reshape(T, n_embd)[toks].reshape(-1)
            e["max_rel_err_vs_oracle"] = float(np.abs(got - want).max() / np.abs(want).max())
        res["moe"].append(e)
        del x, y, d_rout
    del d_g, d_u, d_d, dev_w
    res["workload"] = ("DS-V4 expert formats: IQ2_XXS gate/up (2048, 4096), Q2_K down (4096, "
                       "2048); routed experts 256 x (gate, up, down), top-6")
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(sharding is described in DESIGN.md); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.pmc_probe:
        pmc_probe()
        return
    if args.prefill_pmc_probe:
        prefill_pmc_probe()
        return
    if args.gemv_probe:
        gemv_probe()
        return
    if args.q8_probe:
        q8_probe()
        return
    if args.batch_probe:
        batch_probe()
        return
    if args.prefill_probe:
        prefill_probe(args.prefill_probe, args.prefill_format)
        return
    if args.moe_probe:
        moe_probe(args.moe_probe)
        return
    if args.dsv4_probe:
        dsv4_probe(args.dsv4_probe)
        return
    # the counter passes run first, in child processes, before this process
    # touches the GPU
    traffic, traffic_detail = (None, {"skipped": True}) if args.no_traffic else pmc_traffic()
    _progress("counter passes done")
    trace = {"skipped": True} if args.no_trace else kernel_trace()
    _progress("kernel-trace pass done")
    pf_busy = {"skipped": True} if (args.no_trace or args.no_prefill) else prefill_mfma_busy()
    _progress("prefill counter pass done")

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

    # ---- spin-up (device copies, not steps), then warmup ----
    _spinup(args.spinup_ms)
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
    ach_events = bytes_per_launch[dom] / (kern_us[dom] * 1e-6) / 1e9
    # roofline from the kernel trace of the same launches when the trace pass
    # ran (its per-dispatch durations exclude launch gaps); the event mean
    # stays beside it
    trace_ok = isinstance(trace.get("gemv"), list)
    if trace_ok:
        tr_us = [trace["gemv"][si]["us_mean"] for si in range(len(mats))]
        dom = max(range(len(mats)), key=lambda s: tr_us[s])
        dom_us = tr_us[dom]
    else:
        dom_us = kern_us[dom]
    ach = bytes_per_launch[dom] / (dom_us * 1e-6) / 1e9

    _progress("bench line timed")
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

    _progress("check and CPU baseline done")
    prefill = None if args.no_prefill else bench_prefill(B, synth, G, dev, stream,
                                                          args.prefill_iters, not args.no_cpu,
                                                          args.cpu_seconds)

    _progress("prefill leg done")
    extra = None if args.no_extra else bench_extra(B, synth, G, dev, stream, args.extra_iters,
                                                    not args.no_cpu)

    line = {
        "metric": "Q4_K/Q6_K GEMV GB/s (% of HBM peak); Q4_K prefill GEMM TFLOP/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "spinup_ms": args.spinup_ms,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q6_k weights; x re-expressed per 16-element group as two int8 limbs "
                 "(about 16 significant bits); exact int32 dots, fp32 scaling and sums",
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
            "traffic": traffic.get(per_kernel[dom]["shape"]) if traffic else None,
            "kernel": "rsllm_hip::k_gemv1<FQ6K, NW, PD, GPT> (x quantised in LDS, one launch)",
            "kernel_shape": per_kernel[dom]["shape"],
            "kernel_us_mean": round(dom_us, 3),
            "kernel_us_from": "rocprofv3 kernel trace" if trace_ok else "HIP events",
            "kernel_us_events": round(kern_us[dom], 3),
            "achieved_events": round(ach_events, 2),
        },
        "cpu_baseline": cpu_baseline,
        "check": check,
    }
    if trace_ok:
        for e in trace["gemv"]:
            key = f"trace_{e['dtype']}_{e['shape']}_us"
            line["roofline"][key] = e["us_mean"]
    if traffic:
        for shape, nb in traffic.items():
            line["roofline"][f"traffic_{shape}"] = nb
    line["prefill"] = prefill_scalars(prefill, trace.get("prefill"), pf_busy)
    line["extra"] = extra_compact(extra)
    detail = {"per_kernel": per_kernel, "trace": trace, "traffic_by_shape": traffic,
              "traffic_detail": traffic_detail, "prefill_mfma_busy": pf_busy,
              "prefill": prefill, "extra": extra}
    if args.detail_out:
        with open(args.detail_out, "w") as f:
            json.dump({"line": line, "detail": detail}, f, indent=1)
    print(json.dumps(line))


def prefill_scalars(pf, pf_trace, pf_busy):
    """The C4 prefill results as flat scalar members (whole call by HIP
    events, GEMM and pre-pass by kernel trace, MFMA busy by counters, the CPU
    baseline), so every figure survives a reader that keeps scalars only."""
    if pf is None:
        return None
    peak = MFMA_F16_PEAK_TFLOPS
    out = {"workload": pf["workload"], "peak_tflops": peak, "unit": "TFLOP/s"}
    for e in pf["by_tokens"]:
        t = e["tokens"]
        out[f"t{t}_us"] = e["us_per_op"]
        out[f"t{t}_tflops"] = e["tflops"]
        out[f"t{t}_frac"] = e["frac_of_peak"]
        if "check" in e:
            out[f"t{t}_max_rel_err_vs_oracle"] = e["check"]["max_rel_err_vs_oracle"]
    for e in pf.get("f32_x", []):
        t = e["tokens"]
        out[f"t{t}_f32x_us"] = e["us_per_op"]
        out[f"t{t}_f32x_frac"] = e["frac_of_peak"]
        if "check" in e:
            out[f"t{t}_f32x_max_rel_err_vs_oracle"] = e["check"]["max_rel_err_vs_oracle"]
    if isinstance(pf_trace, list):
        out["kernel_us_from"] = ("rocprofv3 kernel trace (k_prefill_q4k_w8 plus its partial-sum "
                                 "kernel where K is split, k_prefill_x)")
        for e in pf_trace:
            t = e["tokens"]
            us = e["gemm"]["us_mean"]
            out[f"t{t}_kernel_us"] = us
            out[f"t{t}_kernel_frac"] = round(2.0 * t * 4096 * 14336 / (us * 1e-6) / 1e12 / peak, 4)
            out[f"t{t}_partial_sums_us"] = e["partial_sums"]["us_mean"]
            out[f"t{t}_prepass_us"] = e["prepass"]["us_mean"]
    elif pf_trace is not None:
        out["kernel_trace_error"] = str(pf_trace)[:120]
    if isinstance(pf_busy, dict) and "t512" in pf_busy:
        out["mfma_busy_from"] = ("rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / "
                                 "(GRBM_GUI_ACTIVE / 8 XCDs), this run")
        for t in (512, 2048):
            out[f"t{t}_mfma_busy"] = pf_busy[f"t{t}"]["mfma_busy"]
            out[f"t{t}_valu_per_mfma"] = pf_busy[f"t{t}"]["valu_per_mfma"]
    elif pf_busy is not None and not pf_busy.get("skipped"):
        out["mfma_busy_error"] = str(pf_busy)[:120]
    for e in pf.get("formats", []):
        out[f"{e['format'].lower()}_t{e['tokens']}_us"] = e["us_per_op"]
        out[f"{e['format'].lower()}_t{e['tokens']}_frac"] = e["frac_of_peak"]
    for e in pf.get("k_split", []):
        out[f"ksplit_{e['shape']}_t{e['tokens']}_us"] = e["us_per_op"]
        out[f"ksplit_{e['shape']}_t{e['tokens']}_frac"] = e["frac_of_peak"]
    for e in pf.get("dense_f16_library", []):
        out[f"dense_f16_library_t{e['tokens']}_frac"] = e["frac_of_peak"]
    cases = pf.get("mfma_ceiling", {}).get("by_case", [])
    for e in cases:
        if e["valu_per_mfma"] in (0.0, 2.0) and e["waves_per_simd"] == 2:
            out[f"mfma_issue_ceiling_{int(e['valu_per_mfma'])}valu_frac"] = e["frac_of_peak"]
    cb = pf.get("cpu_baseline")
    if cb:
        out["cpu_baseline_tflops"] = cb["value"]
        out["cpu_baseline_cores"] = cb["cores"]
        out["cpu_baseline_kind"] = cb["kind"]
        out["cpu_baseline_sample"] = cb["sample"]
    return out


def extra_compact(ex):
    """The other configs as short rows (the full tables go to --detail-out):
    gemv [config dtype shape B, us, frac of 8 TB/s, max rel err vs oracle];
    q8_int8 [shape B, quantize us, matmul us, frac, bit-exact];
    moe [T, us, frac, active experts]; caller_chain [op shape B, us, frac];
    stream_read [config, us, frac]; dsv4_dense [format shape T, us, frac,
    TFLOP/s, max rel err]; dsv4_moe [T, us, frac, TFLOP/s, active experts,
    max rel err]."""
    if ex is None:
        return None

    def r(v, n=4):
        return None if v is None else round(v, n)
    out = {"device_copy_GBps": ex["device_copy"]["GBps"]}
    out["gemv"] = [[f"{e['config']} {e['dtype']} {e['shape']} B={e['batch']}", e["us"],
                    e["frac_hbm"], r(e.get("max_rel_err_vs_oracle"), 7)] for e in ex["gemv"]]
    out["stream_read"] = [[e["config"], e["us"], e["frac_hbm"]] for e in ex["stream_read"]]
    out["q8_int8"] = [[f"{e['shape']} B={e['batch']}", e["quantize_us"], e["matmul_us"],
                       e["frac_hbm"], e.get("bit_exact_vs_oracle")] for e in ex["q8_int8"]]
    out["caller_chain"] = [[f"{e['op']} {e['dtype']} B={e['batch']}", e["us"], e["frac_hbm"]]
                           for e in ex["caller_chain"]]
    out["model_upload_GBps"] = ex["model_upload"]["GBps"]
    out["moe_workload"] = ex["moe"]["workload"]
    out["moe"] = [[e["tokens"], e["us"], e["frac_hbm"], e["active_experts"]]
                  for e in ex["moe"]["by_tokens"]]
    m1 = ex["moe"]["by_tokens"][0]
    if "max_rel_err_vs_oracle" in m1:
        out["moe_t1_max_rel_err_vs_oracle"] = r(m1["max_rel_err_vs_oracle"], 7)
        out["moe_t1_cpu_baseline"] = m1["cpu_baseline"]
    ds = ex.get("dsv4")
    if ds:
        out["dsv4_workload"] = ds["workload"]
        out["dsv4_dense"] = [[f"{e['dtype']} {e['shape']} T={e['tokens']}", e["us"],
                              e["frac_hbm"], e["tflops"], r(e.get("max_rel_err_vs_oracle"), 7)]
                             for e in ds["dense"]]
        out["dsv4_moe"] = [[e["tokens"], e["us"], e["frac_hbm"], e["tflops"], e["active_experts"],
                            r(e.get("max_rel_err_vs_oracle"), 7)] for e in ds["moe"]]
    return out


if __name__ == "__main__":
    main()
