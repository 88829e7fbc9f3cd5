"""The library called from many host threads at once, as the reference's
CpuBackend may be (a stateless Send + Sync handle, backend-cpu/src/lib.rs:42-45,
its kernels on the rayon pool, parallel.rs:37-54):

* 4 threads call the host-pointer matmul_quant_f32 and moe_routed
  concurrently on different weights; every result is checked against the
  oracle;
* 2 threads enqueue device-pointer calls that use the kernels' workspace
  (batched GEMV, routed experts) on streams of their own; results are
  bit-identical to the same calls made one at a time;
* one thread registers and releases a tensor over and over while others run
  host-pointer matmuls on it: every result matches (registered copy or
  per-call upload, the same bytes through the same kernels);
* rsllm_hip_stream_release frees a stream's workspace and a later call on
  the stream still works;
* 2 threads enqueue the same workspace-using calls on hipStreamPerThread (one
  handle value, a different stream in each thread): each thread gets a
  workspace set of its own, and results are bit-identical to serial calls.
ctypes releases the GIL around each library call, so the calls overlap."""
import threading

import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

ITERS = 6


def _run_threads(fns):
    errors = []

    def wrap(f):
        try:
            f()
        except BaseException as e:  # noqa: BLE001 - reported to the main thread
            errors.append(e)
    ts = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a worker thread did not finish"
    if errors:
        raise errors[0]


def test_host_matmul_and_moe_from_four_threads(hip, oracle):
    hip.init(0)
    # (dtype, out_dim, in_dim, n_tok): batch 1, the batched int8-limb kernel,
    # the matrix-core GEMV (workspace) and the pre-pass GEMV (workspace)
    mm_cases = [(G.Q4_K, 1024, 2048, 1), (G.Q6_K, 1536, 1024, 3), (G.Q8_0, 2048, 1024, 12),
                (G.Q2_K, 512, 1024, 20)]
    mm = []
    for i, (dt, o, n, t) in enumerate(mm_cases):
        w = synth.weight(dt, o, n, 1300 + i)
        x = synth.activations(t, n, 1310 + i).reshape(-1)
        rc, want = oracle.matmul_quant_f32(w, x, t, n, o, int(dt))
        assert rc == 0
        mm.append((dt, o, n, t, w, x, want))
    n_embd, n_ff, n_expert, k = 512, 256, 8, 2
    moe = []
    for j, n_tok in enumerate((2, 9)):
        gate = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 1320 + 3 * j)
        up = synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 1321 + 3 * j)
        down = synth.weight(G.Q4_K, n_expert * n_embd, n_ff, 1322 + 3 * j)
        x = synth.activations(n_tok, n_embd, 1330 + j)
        ids, w = synth.moe_routing(n_tok, n_expert, k, 1340 + j)
        want = np.zeros(n_tok * n_embd, np.float32)
        assert oracle.moe_routed(want, x, n_tok, n_embd, n_ff, gate, up, down, int(G.Q4_K),
                                 int(G.Q4_K), n_expert, ids, w, k, 10.0) == 0
        moe.append((gate, up, down, x, ids, w, n_tok, want))

    def mm_worker(case):
        dt, o, n, t, w, x, want = case

        def run():
            for _ in range(ITERS):
                got = np.empty(t * o, np.float32)
                hip.matmul_quant_f32(got, w, x, t, n, o, dt)
                assert rel_err(got, want) <= REL_TOL, f"{dt.name} {o}x{n} T={t}"
        return run

    def moe_worker(case):
        gate, up, down, x, ids, w, n_tok, want = case

        def run():
            for _ in range(ITERS):
                got = np.zeros(n_tok * n_embd, np.float32)
                hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff,
                               n_expert, k, G.Q4_K, G.Q4_K, 10.0)
                assert rel_err(got, want) <= REL_TOL, f"moe T={n_tok}"
        return run

    # six threads: four matmul workers and two MoE workers, all at once
    _run_threads([mm_worker(c) for c in mm] + [moe_worker(c) for c in moe])


def test_dev_calls_on_own_streams_from_two_threads(hip):
    import torch
    hip.init(0)
    # workspace users: matrix-core GEMV (16 tokens) and routed experts
    # (grouped matrix-core route, 12 tokens x top-4)
    o, n, t = 2048, 2048, 16
    w_host = synth.weight(G.Q4_K, o, n, 1400)
    w = torch.from_numpy(w_host).cuda()
    xs = [torch.from_numpy(synth.activations(t, n, 1401 + i).reshape(-1)).cuda() for i in range(2)]
    n_embd, n_ff, n_expert, k, mt = 1024, 1024, 8, 4, 12
    gate = torch.from_numpy(synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 1410)).cuda()
    up = torch.from_numpy(synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 1411)).cuda()
    down = torch.from_numpy(synth.weight(G.Q4_K, n_expert * n_embd, n_ff, 1412)).cuda()
    mx = [torch.from_numpy(synth.activations(mt, n_embd, 1413 + i).reshape(-1)).cuda()
          for i in range(2)]
    routes = [synth.moe_routing(mt, n_expert, k, 1420 + i) for i in range(2)]
    ids = [torch.from_numpy(r[0].reshape(-1)).cuda() for r in routes]
    wts = [torch.from_numpy(r[1].reshape(-1)).cuda() for r in routes]

    def calls(i, stream):
        y = torch.empty(t * o, dtype=torch.float32, device="cuda")
        hip.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), xs[i].data_ptr(),
                                 xs[i].numel(), t, n, o, G.Q4_K, stream)
        m = torch.zeros(mt * n_embd, dtype=torch.float32, device="cuda")
        hip.moe_routed_dev(m.data_ptr(), m.numel(), mx[i].data_ptr(), mx[i].numel(),
                           gate.data_ptr(), up.data_ptr(), gate.numel(), down.data_ptr(),
                           down.numel(), ids[i].data_ptr(), wts[i].data_ptr(), mt * k, mt, n_embd,
                           n_ff, n_expert, k, G.Q4_K, G.Q4_K, 10.0, stream)
        return y, m

    # one at a time on the default stream
    ref = []
    for i in range(2):
        y, m = calls(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref.append((y.cpu().numpy(), m.cpu().numpy()))
    torch.cuda.synchronize()

    def worker(i):
        def run():
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(ITERS):
                    y, m = calls(i, s.cuda_stream)
                    s.synchronize()
                    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref[i][0].view(np.uint32))
                    assert np.array_equal(m.cpu().numpy().view(np.uint32), ref[i][1].view(np.uint32))
            s.synchronize()
            hip.stream_release(s.cuda_stream)
        return run

    _run_threads([worker(0), worker(1)])


def test_register_release_race_with_host_calls(hip):
    hip.init(0)
    o, n = 1024, 2048
    w = synth.weight(G.Q6_K, o, n, 1500)
    cases = [(t, synth.activations(t, n, 1501 + t).reshape(-1)) for t in (1, 6)]
    ref = {}
    for t, x in cases:
        y = np.empty(t * o, np.float32)
        hip.matmul_quant_f32(y, w, x, t, n, o, G.Q6_K)  # per-call upload
        ref[t] = y
    stop = threading.Event()

    def churn():
        while not stop.is_set():
            hip.register_weights(w, G.Q6_K, n)
            hip.release_weights()

    def caller(t, x):
        def run():
            for _ in range(4 * ITERS):
                y = np.empty(t * o, np.float32)
                hip.matmul_quant_f32(y, w, x, t, n, o, G.Q6_K)
                assert np.array_equal(y.view(np.uint32), ref[t].view(np.uint32))
        return run

    ch = threading.Thread(target=churn)
    ch.start()
    try:
        _run_threads([caller(t, x) for t, x in cases])
    finally:
        stop.set()
        ch.join(timeout=60)
    assert not ch.is_alive()
    hip.release_weights()


def test_stream_release_then_reuse(hip):
    import torch
    hip.init(0)
    o, n, t = 1024, 1024, 12
    w_host = synth.weight(G.Q8_0, o, n, 1600)
    raw = torch.from_numpy(w_host).cuda()
    w = torch.empty_like(raw)
    hip.prepare_weights_dev(w.data_ptr(), raw.data_ptr(), raw.numel(), G.Q8_0, n, 0)
    x = torch.from_numpy(synth.activations(t, n, 1601).reshape(-1)).cuda()
    s = torch.cuda.Stream()
    outs = []
    for _ in range(2):
        y = torch.empty(t * o, dtype=torch.float32, device="cuda")
        hip.matmul_quant_f32_dev(y.data_ptr(), y.numel(), w.data_ptr(), w.numel(), x.data_ptr(),
                                 x.numel(), t, n, o, G.Q8_0, s.cuda_stream)
        s.synchronize()
        outs.append(y.cpu().numpy())
        hip.stream_release(s.cuda_stream)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


HIP_STREAM_PER_THREAD = 2  # the value of hipStreamPerThread in hip_runtime_api.h


def test_dev_calls_on_stream_per_thread_from_two_threads(hip):
    """Batched GEMVs whose K is split across workgroups (activation image
    and partial sums in the workspace: Q8_0 1024 x 4096 at 32 tokens, Q6_K
    4096 x 8192 at 8), from two threads on hipStreamPerThread. Sharing one
    workspace set between the two real streams would race on the activation
    images and the partial sums."""
    import torch
    hip.init(0)
    cases = [(G.Q8_0, 1024, 4096, 32), (G.Q6_K, 4096, 8192, 8)]
    ws = []
    for j, (dt, o, n, t) in enumerate(cases):
        raw = torch.from_numpy(synth.weight(dt, o, n, 1700 + j)).cuda()
        d = torch.empty_like(raw)
        hip.prepare_weights_dev(d.data_ptr(), raw.data_ptr(), raw.numel(), dt, n, 0)
        ws.append(d)
    xs = [[torch.from_numpy(synth.activations(t, n, 1710 + 2 * j + i).reshape(-1)).cuda()
           for i in range(2)] for j, (_, _, n, t) in enumerate(cases)]
    torch.cuda.synchronize()

    def calls(i, stream):
        ys = []
        for j, (dt, o, n, t) in enumerate(cases):
            y = torch.empty(t * o, dtype=torch.float32, device="cuda")
            hip.matmul_quant_f32_dev(y.data_ptr(), y.numel(), ws[j].data_ptr(), ws[j].numel(),
                                     xs[j][i].data_ptr(), xs[j][i].numel(), t, n, o, dt, stream)
            ys.append(y)
        return ys

    ref = []
    for i in range(2):
        ys = calls(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref.append([y.cpu().numpy() for y in ys])

    def worker(i):
        def run():
            for _ in range(ITERS):
                ys = calls(i, HIP_STREAM_PER_THREAD)
                torch.cuda.synchronize()
                for y, r in zip(ys, ref[i]):
                    assert np.array_equal(y.cpu().numpy().view(np.uint32), r.view(np.uint32))
            hip.stream_release(HIP_STREAM_PER_THREAD)
        return run

    _run_threads([worker(0), worker(1)])
