"""rsllm_hip_matmul_quant_f32_dev_noalloc: the same results as
rsllm_hip_matmul_quant_f32_dev (it runs the same kernels, with the static
per-GPU workspace in place of the library-allocated one), on calls that use
that workspace, twice in a row with the second call smaller; that those
calls make no device allocation (the library's allocation counter does not
move, on a stream no call has used before; the allocating entry point on
another new stream does move it); and the rejection of a call whose
workspace would exceed the static maximum."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

# (dtype, out_dim, in_dim, n_tok): each takes a kernel path that uses the
# workspace: the matrix-core batched GEMV (f16 activation image) for 5..32
# tokens of >= 1024 rows, the activation pre-pass + GEMV otherwise, and
# above 32 tokens the prefill GEMM (f16 image, per-token scales and, on
# small grids, the partial sums of its K splits: 8 and 4 splits here; on a
# grid of 272 tiles, the compact partial sums of its last 16 tiles' 2 splits)
CALLS = [
    [(G.Q4_K, 4096, 4096, 24), (G.Q6_K, 1024, 2048, 12)],   # matrix cores, then smaller
    [(G.Q8_0, 512, 4096, 20), (G.Q4_K, 256, 1024, 11)],     # pre-pass path, then smaller
    [(G.Q6_K, 2048, 4096, 32), (G.Q2_K, 300, 512, 13)],     # mixed paths, then smaller
    [(G.Q6_K, 1024, 4096, 300), (G.Q8_0, 512, 2048, 40)],   # prefill GEMMs, then smaller
    [(G.Q4_K, 4000, 1024, 2049), (G.Q8_0, 3000, 2048, 1100)],  # tail split, then K split
]


def _run(hip, torch, fn, w_dev, x_dev, n_tok, in_dim, out_dim, dtype):
    y = torch.full((n_tok * out_dim,), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    fn(y.data_ptr(), y.numel(), w_dev.data_ptr(), w_dev.numel(), x_dev.data_ptr(), x_dev.numel(),
       n_tok, in_dim, out_dim, dtype, s)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("calls", CALLS)
def test_noalloc_matches_dev_entry(hip, oracle, calls):
    import torch
    hip.init(0)
    s = torch.cuda.current_stream().cuda_stream
    for i, (dtype, out_dim, in_dim, n_tok) in enumerate(calls):
        print(f"noalloc call {i}: {dtype.name} {out_dim}x{in_dim} T={n_tok}", flush=True)
        w = synth.weight(dtype, out_dim, in_dim, seed=900 + i)
        raw = torch.from_numpy(w).cuda()
        prep = torch.empty_like(raw)
        hip.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, s)
        x = synth.activations(n_tok, in_dim, seed=910 + i).reshape(-1)
        xd = torch.from_numpy(x).cuda()
        got = _run(hip, torch, hip.matmul_quant_f32_dev_noalloc, prep, xd, n_tok, in_dim, out_dim,
                   dtype)
        ref = _run(hip, torch, hip.matmul_quant_f32_dev, prep, xd, n_tok, in_dim, out_dim, dtype)
        # the same kernels on the same inputs: bit for bit
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
        assert rc == 0
        assert rel_err(got, want) <= REL_TOL


@pytest.mark.gpu
def test_noalloc_allocates_nothing(hip):
    """Every path of CALLS on a fresh stream: rsllm_hip_device_allocations
    is unchanged across the no-allocation calls (inputs and outputs are made
    before the first count), and grows when the allocating _dev entry point
    runs the same call on another fresh stream (a workspace set of its own)."""
    import torch
    hip.init(0)
    s0 = torch.cuda.current_stream().cuda_stream
    bufs = []
    for i, (dtype, out_dim, in_dim, n_tok) in enumerate(c for calls in CALLS for c in calls):
        raw = torch.from_numpy(synth.weight(dtype, out_dim, in_dim, seed=950 + i)).cuda()
        prep = torch.empty_like(raw)
        hip.prepare_weights_dev(prep.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim, s0)
        x = torch.from_numpy(synth.activations(n_tok, in_dim, seed=960 + i).reshape(-1)).cuda()
        y = torch.empty(n_tok * out_dim, dtype=torch.float32, device="cuda")
        bufs.append((dtype, out_dim, in_dim, n_tok, prep, x, y))
    torch.cuda.synchronize()
    fresh = torch.cuda.Stream()
    before = hip.device_allocations()
    for dtype, out_dim, in_dim, n_tok, prep, x, y in bufs:
        hip.matmul_quant_f32_dev_noalloc(y.data_ptr(), y.numel(), prep.data_ptr(), prep.numel(),
                                         x.data_ptr(), x.numel(), n_tok, in_dim, out_dim, dtype,
                                         fresh.cuda_stream)
    fresh.synchronize()
    assert hip.device_allocations() == before
    other = torch.cuda.Stream()
    dtype, out_dim, in_dim, n_tok, prep, x, y = bufs[0]
    hip.matmul_quant_f32_dev(y.data_ptr(), y.numel(), prep.data_ptr(), prep.numel(), x.data_ptr(),
                             x.numel(), n_tok, in_dim, out_dim, dtype, other.cuda_stream)
    other.synchronize()
    assert hip.device_allocations() > before
    hip.stream_release(other.cuda_stream)


def test_noalloc_rejects_workspace_above_the_maximum(hip):
    # 32 tokens of a 1M-element Q8_0 row need a 64 MB f16 activation image;
    # validation and the size check run before any device work (placeholder
    # addresses, never dereferenced)
    in_dim, out_dim, n_tok = 1_000_192, 1024, 32
    w_len = out_dim * (in_dim // 32) * 34
    fake = 1 << 40
    with pytest.raises(hip.InvalidArgument, match="workspace"):
        hip.matmul_quant_f32_dev_noalloc(fake, n_tok * out_dim, fake, w_len, fake, n_tok * in_dim,
                                         n_tok, in_dim, out_dim, G.Q8_0, 0)
