"""GEMV / matmul_quant_f32 on the GPU against the oracle (the reference's
matmul_quant_f32, backend-cpu/src/ops/quant_matmul.rs:45-119): max|Δ|/max|y|
<= 1e-3 (REL_TOL) on seeded inputs, ragged shapes, every benchmark shape."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu


def run_both(oracle, hip, dtype, out_dim, in_dim, n_tok, seed):
    w = synth.weight(dtype, out_dim, in_dim, seed)
    x = synth.activations(n_tok, in_dim, seed + 1).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype), allow_q6k=True)
    assert rc == 0
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    return got, want


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q4_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim,in_dim", [(1, 256), (7, 512), (33, 768), (100, 2048), (257, 1280)])
@pytest.mark.parametrize("n_tok", [1, 2, 3, 5, 8, 13])
def test_gemv_ragged_shapes(oracle, hip, dtype, out_dim, in_dim, n_tok):
    got, want = run_both(oracle, hip, dtype, out_dim, in_dim, n_tok, seed=out_dim * 31 + n_tok)
    assert not np.isnan(got).any()
    assert rel_err(got, want) <= REL_TOL


# The matrix-core path (5..32 tokens of Q4_K / Q6_K / Q2_K / IQ2_XXS, 9..32
# of Q8_0): one and two 16-token tiles, partial tiles, row counts off the
# 16-row tile, few K steps per wavefront (in 256) and many (in 7168), token
# scales far apart. Q2_K and IQ2_XXS (the DS-V4 expert formats) run
# mf_rows (or, Q2_K, the fused LDS kernel) at these in_dim, which are not
# multiples of 2048.
@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim,in_dim", [(1024, 256), (1030, 1024), (2000, 7168), (4097, 512)])
@pytest.mark.parametrize("n_tok", [5, 9, 15, 16, 17, 31, 32])
def test_gemv_mfma_batches(oracle, hip, dtype, out_dim, in_dim, n_tok):
    w = synth.weight(dtype, out_dim, in_dim, 7 + n_tok)
    x = synth.activations(n_tok, in_dim, 8 + n_tok)
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 7) - 3)).astype(np.float32)[:, None]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    got = np.empty(n_tok * out_dim, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    # per token: each token's outputs against that token's own maximum
    g = got.reshape(n_tok, out_dim)
    wv = want.reshape(n_tok, out_dim)
    for t in range(n_tok):
        if np.abs(wv[t]).max() > 0:
            assert rel_err(g[t], wv[t]) <= REL_TOL, f"token {t}"


# The one-pass kernel (k_gemv_mfo: Q8_0 / Q4_K, 9..32 tokens, 192..512
# workgroups of 128 or 64 rows x a 512- or 256-element K slice): one slice
# (y written directly), a partial last row block at both row counts, many
# slices, token scales far apart.
@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q8_0])
@pytest.mark.parametrize("out_dim,in_dim", [(24576, 512), (3000, 4096), (1000, 4096)])
@pytest.mark.parametrize("n_tok", [9, 17, 32])
def test_gemv_one_pass_shapes(oracle, hip, dtype, out_dim, in_dim, n_tok):
    w = synth.weight(dtype, out_dim, in_dim, 70 + n_tok)
    x = synth.activations(n_tok, in_dim, 71 + n_tok)
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 9) - 4)).astype(np.float32)[:, None]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    assert not np.isnan(got).any()
    g = got.reshape(n_tok, out_dim)
    wv = want.reshape(n_tok, out_dim)
    for t in range(n_tok):
        assert rel_err(g[t], wv[t]) <= 1e-5, f"token {t}"


# Exact weights and two-plane (hi + lo f16) activations on the matrix cores:
# matrices of a few rows (where a maximum over few outputs is most
# sensitive, and f16-rounded weights reached 1.2e-3 on 16 rows) within an
# fp32-level bound (about 1e-6 measured; one f16 rounding gives 2e-4 and up).
@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim", [1, 7, 16, 33, 100])
@pytest.mark.parametrize("n_tok", [9, 16, 32])
def test_gemv_mfma_exact_weights_few_rows(oracle, hip, dtype, out_dim, n_tok):
    in_dim = 4096
    w = synth.weight(dtype, out_dim, in_dim, 1700 + out_dim + n_tok)
    x = synth.activations(n_tok, in_dim, 1800 + n_tok).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    got = np.empty(n_tok * out_dim, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    err = rel_err(got, want)
    print(f"mfma exact {dtype.name} {out_dim}x{in_dim} T={n_tok}: rel err {err:.3e}")
    assert err <= 2e-5


# IQ2_XXS rows of whole 8-block super-tiles (in_dim a multiple of 2048) take
# the staged kernel above 16 tokens (weights copied through LDS in half
# super-tiles, qs and the d run; K split over workgroups for matrices of few
# rows, 64 x 8192) and the unstaged kernel up to 16; dense Q2_K calls keep
# the unstaged kernel (the grouped MoE route stages both formats in its
# 8-slot batches: test_gpu_moe). Ragged last row blocks, 1 to 4 super-tiles
# per row, within the exact-route bound.
@pytest.mark.parametrize("dtype", [G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim,in_dim", [(1030, 4096), (4097, 2048), (64, 8192), (300, 6144)])
@pytest.mark.parametrize("n_tok", [5, 8, 16, 32])
def test_gemv_mfma_staged_dsv4_formats(oracle, hip, dtype, out_dim, in_dim, n_tok):
    w = synth.weight(dtype, out_dim, in_dim, 2100 + out_dim + n_tok)
    x = synth.activations(n_tok, in_dim, 2200 + n_tok)
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 5) - 2)).astype(np.float32)[:, None]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    g = got.reshape(n_tok, out_dim)
    wv = want.reshape(n_tok, out_dim)
    assert not np.isnan(g).any()
    for t in range(n_tok):
        assert rel_err(g[t], wv[t]) <= 2e-5, f"token {t}"


# Q8_0 takes the matrix cores from 3 tokens on matrices of 8192 or more
# columns, from 5 on 8192 or more rows, from 9 otherwise; each side of each
# threshold against the oracle, per token: within 2e-5 on the matrix cores
# (exact weights, hi + lo activations), REL_TOL on the int8-limb route
@pytest.mark.parametrize("out_dim,in_dim,n_tok,mfma", [
    (96, 8192, 2, False), (96, 8192, 3, True), (40, 14336, 4, True), (8200, 512, 4, False),
    (8200, 512, 5, True), (8192, 1024, 8, True), (300, 4096, 8, False), (300, 4096, 9, True)])
def test_gemv_q8_0_matrix_core_thresholds(oracle, hip, out_dim, in_dim, n_tok, mfma):
    w = synth.weight(G.Q8_0, out_dim, in_dim, 2300 + out_dim + n_tok)
    x = synth.activations(n_tok, in_dim, 2400 + n_tok).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(G.Q8_0))
    assert rc == 0
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, G.Q8_0)
    g, wv = got.reshape(n_tok, out_dim), want.reshape(n_tok, out_dim)
    tol = 2e-5 if mfma else REL_TOL
    for t in range(n_tok):
        assert rel_err(g[t], wv[t]) <= tol, f"token {t}"


# GGUF Q6_K scales use the whole int8 range (-128..127); |sc (q - 32)| then
# reaches 4096, past the integers f16 holds exactly (2048). Every route —
# the int8-limb GEMVs (1..4 tokens), the matrix-core GEMV (5..32), its fused
# LDS kernel (5..8 tokens of tall matrices) and the 32-token chunks above 32
# — stays at its bound with every block holding sc = -128 and 127 (an
# f16-rounded sc (q - 32) gives 1e-4 and up). Above 32 tokens with in_dim a
# multiple of 2048 the prefill GEMM (f16 weights and activations) takes the
# call, within REL_TOL at these scales too.
@pytest.mark.parametrize("out_dim,in_dim,n_tok", [
    (16, 4096, 1), (100, 2048, 3), (33, 4096, 5), (16, 4096, 9), (257, 2048, 12),
    (1000, 1024, 16), (64, 4096, 32), (8200, 1024, 6), (300, 1280, 40), (300, 2048, 40)])
def test_gemv_q6k_full_range_scales(oracle, hip, out_dim, in_dim, n_tok):
    w = synth.q6k_full_scales(synth.weight(G.Q6_K, out_dim, in_dim, 1900 + n_tok), 1950 + n_tok)
    x = synth.activations(n_tok, in_dim, 1960 + n_tok).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(G.Q6_K))
    assert rc == 0
    got = np.empty(n_tok * out_dim, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, G.Q6_K)
    err = rel_err(got, want)
    print(f"q6k full-range scales {out_dim}x{in_dim} T={n_tok}: rel err {err:.3e}")
    exact = 5 <= n_tok <= 32 or (n_tok > 32 and in_dim % 2048 != 0)
    assert err <= (2e-5 if exact else REL_TOL)


# The fused matrix-core kernel (5..8 tokens, out_dim >= 8192, f16 x in LDS):
# row counts off the 16-row block, K steps fewer than wavefronts (256 -> 2
# steps over 16 wavefronts) and many, token scales far apart, one token
# zero. (Q8_0 takes the matrix cores below 9 tokens from 8192 rows, where
# these shapes are.)
@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim,in_dim", [(8192, 256), (8200, 1024), (9001, 3072)])
@pytest.mark.parametrize("n_tok", [5, 6, 8])
def test_gemv_mfma_fused_lds(oracle, hip, dtype, out_dim, in_dim, n_tok):
    w = synth.weight(dtype, out_dim, in_dim, 70 + n_tok)
    x = synth.activations(n_tok, in_dim, 80 + n_tok)
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 7) - 3)).astype(np.float32)[:, None]
    x[1] = 0.0
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_quant_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    g = got.reshape(n_tok, out_dim)
    wv = want.reshape(n_tok, out_dim)
    assert not np.isnan(g).any()
    assert np.all(g[1] == 0.0)
    for t in range(n_tok):
        if np.abs(wv[t]).max() > 0:
            assert rel_err(g[t], wv[t]) <= REL_TOL, f"token {t}"


# Benchmark shapes at full size (BASELINE configs C0-C2).
@pytest.mark.parametrize("dtype,out_dim,in_dim,n_tok", [
    (G.Q4_K, 4096, 4096, 1),
    (G.Q6_K, 14336, 4096, 1), (G.Q6_K, 14336, 4096, 4), (G.Q6_K, 14336, 4096, 8),
    (G.Q6_K, 4096, 14336, 1), (G.Q6_K, 4096, 14336, 4), (G.Q6_K, 4096, 14336, 8),
    (G.Q6_K, 14336, 4096, 32), (G.Q4_K, 4096, 4096, 16),
    (G.Q8_0, 4096, 4096, 1), (G.Q8_0, 4096, 4096, 2), (G.Q8_0, 4096, 4096, 4),
    (G.Q8_0, 4096, 4096, 8), (G.Q8_0, 4096, 4096, 16), (G.Q8_0, 4096, 4096, 32),
    (G.Q8_0, 1024, 4096, 1), (G.Q8_0, 1024, 4096, 2), (G.Q8_0, 1024, 4096, 4),
    (G.Q8_0, 1024, 4096, 8), (G.Q8_0, 1024, 4096, 16), (G.Q8_0, 1024, 4096, 32),
    (G.Q2_K, 7168, 2048, 1), (G.Q2_K, 7168, 2048, 8), (G.Q2_K, 7168, 2048, 32),
    (G.IQ2_XXS, 2048, 7168, 1), (G.IQ2_XXS, 2048, 7168, 8), (G.IQ2_XXS, 2048, 7168, 32),
])
def test_gemv_config_shapes(oracle, hip, dtype, out_dim, in_dim, n_tok):
    got, want = run_both(oracle, hip, dtype, out_dim, in_dim, n_tok, seed=11)
    err = rel_err(got, want)
    print(f"{dtype.name} {out_dim}x{in_dim} B={n_tok}: rel err {err:.3e}")
    assert err <= REL_TOL


def test_registered_weights_path(oracle, hip):
    dtype, out_dim, in_dim = G.Q6_K, 300, 1024
    w = synth.weight(dtype, out_dim, in_dim, 3)
    x = synth.activations(2, in_dim, 4).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, 2, in_dim, out_dim, int(dtype))
    hip.register_weights(w, dtype, in_dim)
    try:
        got = np.empty(2 * out_dim, np.float32)
        hip.matmul_quant_f32(got, w, x, 2, in_dim, out_dim, dtype)
        assert rel_err(got, want) <= REL_TOL
    finally:
        hip.release_weights()


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0])
def test_dev_entry_point_matches_host(oracle, hip, dtype):
    import torch
    out_dim, in_dim, n_tok = 129, 2048, 3
    w = synth.weight(dtype, out_dim, in_dim, 9)
    x = synth.activations(n_tok, in_dim, 10).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    d_raw = torch.from_numpy(w).cuda()
    d_w = torch.empty_like(d_raw)
    d_x = torch.from_numpy(x).cuda()
    d_y = torch.full((n_tok * out_dim,), float("nan"), device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    hip.prepare_weights_dev(d_w.data_ptr(), d_raw.data_ptr(), w.size, dtype, in_dim, s)
    hip.matmul_quant_f32_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), w.size, d_x.data_ptr(),
                             x.size, n_tok, in_dim, out_dim, dtype, s)
    torch.cuda.synchronize()
    assert rel_err(d_y.cpu().numpy(), want) <= REL_TOL


def test_in_dim_zero_gives_zeros(hip):
    out = np.full(6, np.nan, np.float32)
    hip.matmul_quant_f32(out, np.zeros(0, np.uint8), np.zeros(0, np.float32), 2, 0, 3, G.Q4_K)
    assert np.array_equal(out, np.zeros(6, np.float32))


def test_n_tok_zero_is_noop(hip):
    w = synth.weight(G.Q8_0, 4, 64, 1)
    out = np.zeros(0, np.float32)
    hip.matmul_quant_f32(out, w, np.zeros(0, np.float32), 0, 64, 4, G.Q8_0)


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q4_0])
def test_prequant_entry_points_match_one_shot(oracle, hip, dtype):
    """quantize_x_dev + matmul_prequant_dev is the same product as
    matmul_quant_f32_dev (same activation limbs; the one-shot call may sum in
    another order): agreement to 1e-6 of max|y|, both within tolerance of
    the oracle."""
    import torch
    out_dim, in_dim, n_tok = 77, 1280, 2
    w = synth.weight(dtype, out_dim, in_dim, 21)
    x = synth.activations(n_tok, in_dim, 22).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    s = torch.cuda.current_stream().cuda_stream
    d_raw = torch.from_numpy(w).cuda()
    d_w = torch.empty_like(d_raw)
    hip.prepare_weights_dev(d_w.data_ptr(), d_raw.data_ptr(), w.size, dtype, in_dim, s)
    d_x = torch.from_numpy(x).cuda()
    y1 = torch.empty(n_tok * out_dim, device="cuda")
    y2 = torch.empty(n_tok * out_dim, device="cuda")
    hip.matmul_quant_f32_dev(y1.data_ptr(), y1.numel(), d_w.data_ptr(), w.size, d_x.data_ptr(),
                             x.size, n_tok, in_dim, out_dim, dtype, s)
    nb = hip.xq_bytes(dtype, n_tok, in_dim)
    xq = torch.empty(nb, dtype=torch.uint8, device="cuda")
    hip.quantize_x_dev(dtype, d_x.data_ptr(), x.size, n_tok, in_dim, xq.data_ptr(), nb, s)
    hip.matmul_prequant_dev(y2.data_ptr(), y2.numel(), d_w.data_ptr(), w.size, xq.data_ptr(), nb,
                            n_tok, in_dim, out_dim, dtype, s)
    torch.cuda.synchronize()
    a, b = y1.cpu().numpy(), y2.cpu().numpy()
    assert np.abs(a - b).max() <= 1e-6 * np.abs(b).max()
    assert rel_err(a, want) <= REL_TOL
    assert rel_err(b, want) <= REL_TOL
