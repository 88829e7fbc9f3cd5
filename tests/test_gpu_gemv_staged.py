"""The matrix-core GEMV with its weights staged through LDS (k_gemv_mfs):
5..32 tokens of Q4_K / Q8_0 matrices with in_dim a multiple of 1024 and of
Q6_K matrices with in_dim a multiple of 2048, against the oracle's
matmul_quant_f32 (rsllm-backend-cpu/src/ops/quant_matmul.rs:45-119).

32-row workgroups and 1024-element chunks; matrices with few rows split K
over 2..8 workgroups per 32 rows and add the partials in split order.
Cases cross the 32-row tile edge (1, 31, 33, ragged tails), the
16-token tile edge (16 / 17 tokens), uneven split runs (5 and 7 chunks over
2, 4 or 8 splits) and Q6_K scales over the whole int8 range. The weights
reach the matrix cores exact and x as hi + lo f16 planes, so the bound is
fp32-level (2e-5; an f16 rounding of weights or activations gives 1e-4 and
up). A weights pointer off 16-byte alignment takes the unstaged kernel and
must agree to the same bound; repeated calls are bit-identical (the split
sums run in a fixed order)."""
import numpy as np
import pytest

from conftest import rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

EXACT_TOL = 2e-5


def _prepared(torch, hip, dtype, w, in_dim, offset=0):
    """Device copy of w in the device layout, starting `offset` bytes into
    its buffer."""
    s = torch.cuda.current_stream().cuda_stream
    raw = torch.zeros(w.size + offset, dtype=torch.uint8, device="cuda")
    raw[offset:] = torch.from_numpy(w).cuda()
    if dtype == G.Q4_K:
        return raw
    d = torch.zeros_like(raw)
    hip.prepare_weights_dev(d.data_ptr() + offset, raw.data_ptr() + offset, w.size, dtype, in_dim, s)
    return d


def _run(torch, hip, dtype, w, x, n_tok, in_dim, out_dim, offset=0):
    s = torch.cuda.current_stream().cuda_stream
    d_w = _prepared(torch, hip, dtype, w, in_dim, offset)
    d_x = torch.from_numpy(x).cuda()
    d_y = torch.full((n_tok * out_dim,), float("nan"), device="cuda")
    hip.matmul_quant_f32_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr() + offset, w.size,
                             d_x.data_ptr(), x.size, n_tok, in_dim, out_dim, dtype, s)
    torch.cuda.synchronize()
    return d_y.cpu().numpy()


CASES = [
    # (dtype, out_dim, in_dim, n_tok)
    (G.Q4_K, 1, 4096, 5), (G.Q4_K, 31, 1024, 16), (G.Q4_K, 33, 5120, 17), (G.Q4_K, 1000, 5120, 32),
    (G.Q4_K, 4097, 2048, 9), (G.Q4_K, 14336, 1024, 8),
    (G.Q8_0, 7, 1024, 9), (G.Q8_0, 100, 5120, 12), (G.Q8_0, 1024, 4096, 32), (G.Q8_0, 3001, 3072, 24),
    (G.Q6_K, 16, 14336, 5), (G.Q6_K, 65, 2048, 16), (G.Q6_K, 999, 6144, 20), (G.Q6_K, 4096, 2048, 32),
    (G.Q6_K, 9000, 2048, 8),
]


@pytest.mark.parametrize("dtype,out_dim,in_dim,n_tok", CASES)
def test_staged_gemv_vs_oracle(oracle, hip, dtype, out_dim, in_dim, n_tok):
    import torch
    w = synth.weight(dtype, out_dim, in_dim, 2500 + out_dim + n_tok)
    if dtype == G.Q6_K:
        w = synth.q6k_full_scales(w, 2600 + n_tok)
    x = synth.activations(n_tok, in_dim, 2700 + n_tok)
    # token scales 1e-3 .. 1e3, one token zero: each token is scaled on its own
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 7) - 3)).astype(np.float32)[:, None]
    x[n_tok // 2] = 0.0
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    got = _run(torch, hip, dtype, w, x, n_tok, in_dim, out_dim)
    assert not np.isnan(got).any()
    g, wv = got.reshape(n_tok, out_dim), want.reshape(n_tok, out_dim)
    assert np.all(g[n_tok // 2] == 0.0)
    for t in range(n_tok):
        if np.abs(wv[t]).max() > 0:
            assert rel_err(g[t], wv[t]) <= EXACT_TOL, f"token {t}"
    print(f"staged {dtype.name} {out_dim}x{in_dim} T={n_tok}: rel err {rel_err(g, wv):.3e}")
    again = _run(torch, hip, dtype, w, x, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0])
def test_unaligned_weights_take_the_unstaged_kernel(oracle, hip, dtype):
    import torch
    out_dim, in_dim, n_tok = 300, 4096, 12
    w = synth.weight(dtype, out_dim, in_dim, 2800 + int(dtype))
    x = synth.activations(n_tok, in_dim, 2801).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    for offset in (0, 4):
        got = _run(torch, hip, dtype, w, x, n_tok, in_dim, out_dim, offset)
        assert rel_err(got, want) <= EXACT_TOL, f"offset {offset}"
