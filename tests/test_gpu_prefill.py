"""Prefill GEMM (Q4_K weights x bf16 activations, MFMA) against the oracle:
the reference's matmul_quant_f32 (backend-cpu/src/ops/quant_matmul.rs:45-119)
on f32(bf16 x). Two bars on every call:
* every output of every checked token within the derived bound of
  prefill_bound.py (the f16 weight and activation roundings and the fp32
  sums, relative to sum_i |w_i x_i|), whatever the token's magnitude or
  number of outputs;
* max|d|/max|y| <= 1e-3 (REL_TOL) over the whole output, the north star's
  metric.
Weights enter the matrix cores as f16 (d*sc, dmin*m rounded to f16, one f16
fma per weight), which puts the measured error at about 3e-4."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from prefill_bound import assert_within_bound
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu


def run_prefill(hip, w, xb, n_tok, in_dim, out_dim):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    d_w = torch.from_numpy(w).cuda()
    d_x = torch.from_numpy(xb.view(np.int16)).cuda()
    d_y = torch.full((n_tok * out_dim,), float("nan"), device="cuda")
    hip.matmul_q4k_bf16_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), w.size, d_x.data_ptr(),
                            xb.size, n_tok, in_dim, out_dim, G.Q4_K, s)
    torch.cuda.synchronize()
    return d_y.cpu().numpy()


def check(oracle, got, w, xb, tokens, n_tok, in_dim, out_dim):
    """Compare rows `tokens` of the GPU output with the oracle on those
    tokens: every output within the derived bound, and the whole within
    REL_TOL."""
    xf = synth.bf16_bits_to_f32(xb.reshape(n_tok, in_dim)[tokens]).reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, xf, len(tokens), in_dim, out_dim, int(G.Q4_K))
    assert rc == 0
    g = got.reshape(n_tok, out_dim)[tokens]
    want = want.reshape(len(tokens), out_dim)
    assert not np.isnan(g).any()
    err = rel_err(g, want)
    ratio = assert_within_bound(G.Q4_K, w, xf.reshape(len(tokens), in_dim), g, want, out_dim,
                                in_dim, f"prefill {out_dim}x{in_dim} T={n_tok}")
    print(f"prefill {out_dim}x{in_dim} T={n_tok}: rel err {err:.3e}, worst |d|/bound {ratio:.3f}")
    assert err <= REL_TOL, f"rel err {err:.3e}"
    return err


@pytest.mark.parametrize("out_dim,in_dim", [(1, 256), (17, 512), (256, 256), (300, 768),
                                            (1000, 2048)])
@pytest.mark.parametrize("n_tok", [1, 5, 128, 129, 300])
def test_prefill_ragged_shapes(oracle, hip, out_dim, in_dim, n_tok):
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=out_dim + 7 * n_tok)
    xb = synth.bf16_activations(n_tok, in_dim, seed=in_dim + n_tok).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    check(oracle, got, w, xb, np.arange(n_tok), n_tok, in_dim, out_dim)


@pytest.mark.parametrize("in_dim", [16384, 16640])
def test_prefill_long_rows(oracle, hip, in_dim):
    """Rows at and past the activation pre-pass's register cache (16384
    elements per token): the longer row is read twice instead of once."""
    out_dim, n_tok = 64, 3
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=in_dim)
    xb = synth.bf16_activations(n_tok, in_dim, seed=in_dim + 1).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    check(oracle, got, w, xb, np.arange(n_tok), n_tok, in_dim, out_dim)


def test_prefill_token_scales(oracle, hip):
    """Tokens spanning 60 binades (1e-18 .. 1e18), a zero token, and one
    token with a single nonzero element: every output within the bound,
    which scales with the token's own activations."""
    out_dim, in_dim, n_tok = 1024, 1024, 9
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=5)
    x = synth.activations(n_tok, in_dim, seed=6)
    for t, sc in enumerate([1e-18, 1e-9, 1e-3, 1.0, 1e3, 1e9, 1e18]):
        x[t] *= sc
    x[7] = 0.0
    x[8] = 0.0
    x[8, 300] = -2.5
    xb = synth.f32_to_bf16_bits(x).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    yz = got.reshape(n_tok, out_dim)[7]
    assert np.array_equal(yz, np.zeros(out_dim, np.float32))
    check(oracle, got, w, xb, np.array([0, 1, 2, 3, 4, 5, 6, 8]), n_tok, in_dim, out_dim)


def test_prefill_special_blocks(oracle, hip):
    """Weight blocks with subnormal / zero d and dmin, and extreme scales."""
    out_dim, in_dim, n_tok = 64, 512, 33
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=8).reshape(-1, 144).copy()
    g = np.random.default_rng(9)
    idx = g.choice(w.shape[0], size=w.shape[0] // 3, replace=False)
    choices = np.array([0x0000, 0x0001, 0x03FF, 0x0400, 0x1400, 0x2000], np.uint16)
    d = g.choice(choices, size=(len(idx), 2))
    w[idx, 0:4] = d.view(np.uint8).reshape(len(idx), 4)
    w = w.reshape(-1)
    xb = synth.bf16_activations(n_tok, in_dim, seed=10).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    check(oracle, got, w, xb, np.arange(n_tok), n_tok, in_dim, out_dim)


def test_prefill_many_tiles_ragged(oracle, hip):
    """16 row tiles (the last of 160 rows) x 11 token tiles (the last of one
    token), an odd number of super-blocks per row (3: the K loop's tail of a
    single super-block): tokens on both sides of every token-tile edge and the
    last one are checked against the oracle."""
    out_dim, in_dim, n_tok = 4000, 768, 1281
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=4000)
    xb = synth.bf16_activations(n_tok, in_dim, seed=4001).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    edges = np.arange(128, n_tok, 128)
    tokens = np.unique(np.concatenate([[0, 1, n_tok - 1], edges - 1, edges]))
    check(oracle, got, w, xb, tokens, n_tok, in_dim, out_dim)


@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(4096, 14336, 300), (700, 2304, 40),
                                                  (2048, 4096, 200), (1023, 4096, 33),
                                                  (1, 2048, 35)])
def test_prefill_k_split(oracle, hip, out_dim, in_dim, n_tok):
    """Grids of fewer than 128 workgroups split K across workgroups and add
    the partial sums in split order: the FFN-down shape (4096 rows, K =
    14336: 5 splits of 11 or 12 super-blocks), 9 super-blocks in 4 uneven
    splits with a ragged last row tile, 2048 x 4096 (8 splits of 2
    super-blocks), and outputs whose count is not a multiple of 4 (33 x
    1023, 35 x 1), which the split sum adds element by element.
    Results are deterministic: a second call gives the same bits."""
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=out_dim + in_dim)
    xb = synth.bf16_activations(n_tok, in_dim, seed=n_tok + 3).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    again = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    tokens = np.unique(np.concatenate([np.arange(0, 4), np.linspace(0, n_tok - 1, 12).astype(int),
                                       [127, 128, n_tok - 1]]))
    tokens = tokens[tokens < n_tok]
    check(oracle, got, w, xb, tokens, n_tok, in_dim, out_dim)


@pytest.mark.parametrize("n_tok", [100, 512, 2048])
def test_prefill_config_shape(oracle, hip, n_tok):
    """Config C4: Q4_K (out, in) = (14336, 4096), T in {512, 2048}, and T = 100
    (one partial 128-token tile). The oracle runs on a spread subset of
    tokens (every token's output is independent), both sides of the 64- and
    128-token boundaries included."""
    out_dim, in_dim = 14336, 4096
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=404)
    xb = synth.bf16_activations(n_tok, in_dim, seed=405).reshape(-1)
    got = run_prefill(hip, w, xb, n_tok, in_dim, out_dim)
    tokens = np.unique(np.concatenate([np.arange(0, 8), np.arange(62, 67), np.arange(125, 131),
                                       np.linspace(0, n_tok - 1, 24).astype(int)]))
    tokens = tokens[tokens < n_tok]
    err = check(oracle, got, w, xb, tokens, n_tok, in_dim, out_dim)
    print(f"C4 T={n_tok}: rel err {err:.3e} over {len(tokens)} tokens")


def test_prefill_validation(hip):
    import torch
    w = synth.weight(G.Q4_K, 4, 256, seed=1)
    d_w = torch.from_numpy(w).cuda()
    d_x = torch.zeros(2 * 256, dtype=torch.int16, device="cuda")
    d_y = torch.zeros(2 * 4, device="cuda")
    w8 = synth.weight(G.Q8_0, 4, 256, seed=1)
    d_w8 = torch.from_numpy(w8).cuda()
    with pytest.raises(hip.Unimplemented):
        hip.matmul_q4k_bf16_dev(d_y.data_ptr(), 8, d_w8.data_ptr(), w8.size, d_x.data_ptr(), 512,
                                2, 256, 4, G.Q8_0)
    with pytest.raises(hip.NotBlockAligned):
        hip.matmul_q4k_bf16_dev(d_y.data_ptr(), 8, d_w.data_ptr(), w.size, d_x.data_ptr(), 512, 2,
                                100, 4, G.Q4_K)
    with pytest.raises(hip.ShapeMismatch):
        hip.matmul_q4k_bf16_dev(d_y.data_ptr(), 8, d_w.data_ptr(), w.size, d_x.data_ptr(), 511, 2,
                                256, 4, G.Q4_K)
    # n_tok = 0 is a no-op; in_dim = 0 gives zeros
    hip.matmul_q4k_bf16_dev(None, 0, d_w.data_ptr(), w.size, None, 0, 0, 256, 4, G.Q4_K)
    d_y.fill_(float("nan"))
    hip.matmul_q4k_bf16_dev(d_y.data_ptr(), 8, None, 0, None, 0, 2, 0, 4, G.Q4_K)
    torch.cuda.synchronize()
    assert torch.equal(d_y.cpu(), torch.zeros(8))
