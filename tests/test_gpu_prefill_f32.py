"""The reference's own prefill call on the GPU: matmul_quant_f32 with f32
activations and n_tok = T (rsllm-models/src/engine_impl.rs:277 ->
dsv4/weight.rs:161-163 -> backend-cpu/src/ops/quant_matmul.rs:45-119),
through the drop-in entry points, against the oracle.

Routes above 32 tokens:
* Q4_K, Q8_0, and Q6_K with in_dim a multiple of 2048 (rows of whole
  8-block super-tiles): the prefill GEMM on the matrix cores (f32 x scaled
  per token by 2^e and rounded once to f16; weights f16(d*sc)*q -
  f16(dmin*m) for Q4_K, f16(d*q) for Q8_0, f16(d*sc)*(q-32) for Q6_K):
  every output of every checked token within the derived bound of
  prefill_bound.py, and the whole within the north star's 1e-3 (REL_TOL),
  about 3e-4 measured;
* other Q6_K rows, and Q2_K and IQ2_XXS (the DS-V4 expert formats): the
  exact matrix-core GEMV (integer weights, hi + lo f16 activations) over
  32-token chunks, a short tail included: an fp32-level bound (2e-5) on
  every token;
* other formats: the int8-limb GEMV (REL_TOL).
A device pointer that is not 16-byte aligned keeps the call off the GEMM
(its global->LDS copies move 16-byte pieces) and must still be right."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from prefill_bound import assert_within_bound
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

EXACT_TOL = 2e-5


def prepared(torch, hip, dtype, w, in_dim):
    raw = torch.from_numpy(w).cuda()
    if dtype == G.Q4_K:
        return raw
    d = torch.empty_like(raw)
    hip.prepare_weights_dev(d.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim,
                            torch.cuda.current_stream().cuda_stream)
    return d


def run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim, x_offset=0):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    d_w = prepared(torch, hip, dtype, w, in_dim)
    # x_offset floats of padding in front: an x pointer off 16-byte alignment
    d_x = torch.from_numpy(np.concatenate([np.zeros(x_offset, np.float32), x])).cuda()
    d_y = torch.full((n_tok * out_dim,), float("nan"), device="cuda")
    hip.matmul_quant_f32_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), w.size,
                             d_x.data_ptr() + 4 * x_offset, x.size, n_tok, in_dim, out_dim, dtype,
                             s)
    torch.cuda.synchronize()
    return d_y.cpu().numpy()


def check(oracle, got, w, x, tokens, dtype, n_tok, in_dim, out_dim, tol, route):
    """Rows `tokens` of the GPU output against the oracle. route "gemm" (the
    prefill GEMM): every output within the derived bound and the whole
    within tol; "chunks" (exact matrix-core chunks) and "limb" (int8-limb
    GEMV): every token within tol of its own outputs."""
    xs = x.reshape(n_tok, in_dim)[tokens].reshape(-1)
    rc, want = oracle.matmul_quant_f32(w, xs, len(tokens), in_dim, out_dim, int(dtype))
    assert rc == 0
    g = got.reshape(n_tok, out_dim)[tokens]
    want = want.reshape(len(tokens), out_dim)
    assert not np.isnan(g).any()
    err = rel_err(g, want)
    print(f"prefill f32 {dtype.name} {out_dim}x{in_dim} T={n_tok} ({route}): rel err {err:.3e}")
    assert err <= tol
    if route == "gemm":
        assert_within_bound(dtype, w, xs.reshape(len(tokens), in_dim), g, want, out_dim, in_dim,
                            f"prefill f32 {dtype.name} {out_dim}x{in_dim} T={n_tok}")
    else:
        for i in range(len(tokens)):
            if np.abs(want[i]).max() > 0:
                assert rel_err(g[i], want[i]) <= tol, f"token {tokens[i]}"
    return err


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("out_dim,in_dim", [(300, 768), (1000, 2048), (4097, 256)])
@pytest.mark.parametrize("n_tok", [33, 40, 100, 129])
def test_prefill_f32_ragged(oracle, hip, dtype, out_dim, in_dim, n_tok):
    w = synth.weight(dtype, out_dim, in_dim, seed=2000 + out_dim + n_tok)
    x = synth.activations(n_tok, in_dim, seed=2100 + n_tok)
    # token scales 1e-3 .. 1e3: each token is scaled on its own
    x *= (np.float32(10.0) ** ((np.arange(n_tok) % 7) - 3)).astype(np.float32)[:, None]
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    gemm = dtype in (G.Q4_K, G.Q8_0) or (dtype == G.Q6_K and in_dim % 2048 == 0)
    route = "gemm" if gemm else "chunks"
    tol = EXACT_TOL if route == "chunks" else REL_TOL
    check(oracle, got, w, x, np.arange(n_tok), dtype, n_tok, in_dim, out_dim, tol, route)


@pytest.mark.parametrize("n_tok", [512, 2048])
def test_prefill_f32_c4(oracle, hip, n_tok):
    """C4's weights (Q4_K 14336 x 4096) at T = 512 and 2048 with f32 x, the
    call the reference's prefill makes; oracle on a spread subset of tokens,
    including both sides of the 128-token tile edges."""
    out_dim, in_dim = 14336, 4096
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=404)
    x = synth.activations(n_tok, in_dim, seed=2205).reshape(-1)
    got = run_dev(hip, G.Q4_K, w, x, n_tok, in_dim, out_dim)
    tokens = np.unique(np.concatenate([np.arange(0, 4), np.arange(126, 130),
                                       np.linspace(0, n_tok - 1, 12).astype(int)]))
    check(oracle, got, w, x, tokens, G.Q4_K, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("dtype", [G.Q6_K, G.Q8_0])
def test_prefill_f32_c1_shape(oracle, hip, dtype):
    """A decode-FFN shape (14336 x 4096) with 200 tokens on the GEMM (a
    partial second 128-token tile), every token within 1e-3."""
    out_dim, in_dim, n_tok = 14336, 4096, 200
    w = synth.weight(dtype, out_dim, in_dim, seed=2300)
    x = synth.activations(n_tok, in_dim, seed=2301).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    tokens = np.array([0, 31, 32, 100, 127, 128, 191, 192, 199])
    check(oracle, got, w, x, tokens, dtype, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(4096, 4096, 512), (1024, 4096, 512),
                                                  (4000, 768, 1281), (700, 2304, 40),
                                                  (3, 2048, 35)])
def test_prefill_f32_q8_0_gemm(oracle, hip, out_dim, in_dim, n_tok):
    """Q8_0 on the prefill GEMM: config C2's attention shapes at T = 512
    (4096 x 4096 splits K 4 ways, 1024 x 4096 16 ways), 16 x 11 tiles with
    ragged last row and token tiles and 3 super-tiles per row, and 9
    super-tiles in 4 uneven splits with 40 tokens. Repeated calls are
    bit-identical."""
    w = synth.weight(G.Q8_0, out_dim, in_dim, seed=2500 + out_dim)
    x = synth.activations(n_tok, in_dim, seed=2501 + n_tok).reshape(-1)
    got = run_dev(hip, G.Q8_0, w, x, n_tok, in_dim, out_dim)
    again = run_dev(hip, G.Q8_0, w, x, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    edges = np.arange(128, n_tok, 128)
    tokens = np.unique(np.concatenate([[0, 1, n_tok - 1], edges - 1, edges,
                                       np.linspace(0, n_tok - 1, 8).astype(int)]))
    check(oracle, got, w, x, tokens, G.Q8_0, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(14336, 4096, 512), (4096, 14336, 512),
                                                  (4000, 2048, 1281), (700, 4096, 40),
                                                  (1, 2048, 33), (17, 6144, 200)])
def test_prefill_f32_q6_k_gemm(oracle, hip, out_dim, in_dim, n_tok):
    """Q6_K on the prefill GEMM: the C1 FFN shapes at T = 512 (14336 x 4096
    unsplit; 4096 x 14336 splits K 4 ways, 14 blocks each, so splits start
    inside a super-tile), 16 x 11 tiles with a ragged last row tile (4000
    rows) and a 1-token last token tile, 16 blocks in 8 splits with 40
    tokens, a one-row matrix of one super-tile (every copy of the tile's
    other rows repeats row 0), and 17 rows of three super-tiles. Repeated
    calls are bit-identical."""
    w = synth.weight(G.Q6_K, out_dim, in_dim, seed=2700 + out_dim)
    x = synth.activations(n_tok, in_dim, seed=2701 + n_tok).reshape(-1)
    got = run_dev(hip, G.Q6_K, w, x, n_tok, in_dim, out_dim)
    again = run_dev(hip, G.Q6_K, w, x, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    edges = np.arange(128, n_tok, 128)
    tokens = np.unique(np.concatenate([[0, 1, n_tok - 1], edges - 1, edges,
                                       np.linspace(0, n_tok - 1, 8).astype(int)]))
    check(oracle, got, w, x, tokens, G.Q6_K, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q8_0, G.Q6_K])
@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(4000, 2048, 2100), (2500, 2048, 4400)])
def test_prefill_f32_tail_split(oracle, hip, dtype, out_dim, in_dim, n_tok):
    """Grids of more than one round of 256 tiles whose last round holds at
    most 128 tiles split those tiles' K (the others one workgroup each) and
    add the compact partial sums in split order: 16 x 17 tiles (the last 16,
    token tile 16 of 52 tokens on every row tile, the last row tile of 160
    rows: 4 splits of 2 blocks), and 10 x 35 tiles (the last 94, from row
    tile 6 of token tile 25 on, a 196-row last row tile, a 48-token last
    token tile: 2 splits of 4 blocks). Repeated calls are bit-identical; the
    checked tokens take both sides of every token-tile edge."""
    w = synth.weight(dtype, out_dim, in_dim, seed=2900 + out_dim + int(dtype))
    x = synth.activations(n_tok, in_dim, seed=2901 + n_tok).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    again = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    edges = np.arange(128, n_tok, 128)
    tokens = np.unique(np.concatenate([[0, 1, n_tok - 1], edges - 1, edges,
                                       np.linspace(0, n_tok - 1, 8).astype(int)]))
    check(oracle, got, w, x, tokens, dtype, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("dtype", [G.Q6_K, G.Q8_0])
def test_prefill_f32_special_blocks(oracle, hip, dtype):
    """The Q6_K and Q8_0 GEMMs on blocks with zero, subnormal and small
    normal d (a third of the blocks), and for Q6_K int8 scales of -128 and
    127 in another third, 64 x 2048 with 33 tokens (K split 4 ways)."""
    out_dim, in_dim, n_tok = 64, 2048, 33
    bb, d_at = (210, 208) if dtype == G.Q6_K else (34, 0)
    w = synth.weight(dtype, out_dim, in_dim, seed=2800).reshape(-1, bb).copy()
    g = np.random.default_rng(2801)
    idx = g.choice(w.shape[0], size=w.shape[0] // 3, replace=False)
    choices = np.array([0x0000, 0x0001, 0x03FF, 0x0400, 0x1400, 0x2000], np.uint16)
    w[idx, d_at:d_at + 2] = g.choice(choices, size=len(idx)).view(np.uint8).reshape(-1, 2)
    if dtype == G.Q6_K:
        rest = np.setdiff1d(np.arange(w.shape[0]), idx)[: w.shape[0] // 3]
        sc = g.choice(np.array([-128, 127], np.int8), size=(len(rest), 16))
        w[rest, 192:208] = sc.view(np.uint8)
    w = w.reshape(-1)
    x = synth.activations(n_tok, in_dim, seed=2802).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    check(oracle, got, w, x, np.arange(n_tok), dtype, n_tok, in_dim, out_dim, REL_TOL, "gemm")


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q8_0, G.Q6_K])
def test_prefill_f32_unaligned_large_grid(oracle, hip, dtype):
    """x off 16-byte alignment on a grid that does not split K (56 x 3
    workgroups): the int8-limb route then needs a larger workspace than the
    GEMM would (2.5 or 3 bytes per element of x against 2), and the call
    sizes it for either route."""
    out_dim, in_dim, n_tok = 14336, 4096, 300
    w = synth.weight(dtype, out_dim, in_dim, seed=2600)
    x = synth.activations(n_tok, in_dim, seed=2601).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim, x_offset=1)
    tokens = np.array([0, 1, 150, 298, 299])
    check(oracle, got, w, x, tokens, dtype, n_tok, in_dim, out_dim, REL_TOL, "limb")


def test_prefill_f32_unaligned_x_and_host_form(oracle, hip):
    """x off 16-byte alignment (the int8-limb route), and the synchronous
    host-pointer form (the GEMM), on the same call."""
    out_dim, in_dim, n_tok = 1000, 2048, 70
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=2400)
    x = synth.activations(n_tok, in_dim, seed=2401).reshape(-1)
    got = run_dev(hip, G.Q4_K, w, x, n_tok, in_dim, out_dim, x_offset=1)
    check(oracle, got, w, x, np.arange(n_tok), G.Q4_K, n_tok, in_dim, out_dim, REL_TOL, "limb")
    host = np.empty(n_tok * out_dim, np.float32)
    hip.matmul_quant_f32(host, w, x, n_tok, in_dim, out_dim, G.Q4_K)
    check(oracle, host, w, x, np.arange(n_tok), G.Q4_K, n_tok, in_dim, out_dim, REL_TOL, "gemm")


# (block bytes, offset of d) in the GGUF layouts
_D_AT = {G.Q4_K: (144, 0), G.Q6_K: (210, 208), G.Q8_0: (34, 0)}
# scales whose f16 weights pass 65504 (Q4_K: d and dmin; Q6_K: d with |sc|
# up to 64 and |q - 32| up to 32; Q8_0: d with |q| up to 127) and f16
# subnormal scales (every weight then below 2^-14)
_BIG = {G.Q4_K: (0x5C00, 0x5C00), G.Q6_K: (0x5800, None), G.Q8_0: (0x6400, None)}
_TINY = {G.Q4_K: (0x0010, 0x0008), G.Q6_K: (0x0003, None), G.Q8_0: (0x0021, None)}


def _set_scales(w, dtype, in_dim, rows, blocks, pair):
    bb, d_at = _D_AT[dtype]
    per_row = in_dim // (32 if dtype == G.Q8_0 else 256)
    w = w.reshape(-1, bb)
    for r in rows:
        for b in blocks:
            w[r * per_row + b, d_at:d_at + 2] = np.array([pair[0]], np.uint16).view(np.uint8)
            if pair[1] is not None:
                w[r * per_row + b, 2:4] = np.array([pair[1]], np.uint16).view(np.uint8)


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0])
@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(600, 4096, 300), (700, 4096, 40)])
def test_prefill_f32_scale_range(oracle, hip, dtype, out_dim, in_dim, n_tok):
    """The range guard. Rows with scales whose f16 weights pass 65504
    (Q4_K d = dmin = 256, Q6_K d = 128, Q8_0 d = 1024), in every block of
    some rows and in one block of others, send their workgroups through the
    second pass with per-row power-of-two exponents; rows whose scales are
    all f16-subnormal stay exact-scaled. Both shapes run 3 row tiles; the
    second splits K (40 tokens). Every output within the derived bound, and
    every one of those rows within 1e-3 of its own outputs; repeated calls
    bit-identical."""
    per_row = in_dim // (32 if dtype == G.Q8_0 else 256)
    w = synth.weight(dtype, out_dim, in_dim, seed=2900 + out_dim).copy()
    big_all, big_one, tiny = [0, 5, 300], [7, 511, out_dim - 1], [9, 260, 520]
    _set_scales(w, dtype, in_dim, big_all, range(per_row), _BIG[dtype])
    _set_scales(w, dtype, in_dim, big_one, [per_row // 2], _BIG[dtype])
    _set_scales(w, dtype, in_dim, tiny, range(per_row), _TINY[dtype])
    x = synth.activations(n_tok, in_dim, seed=2901).reshape(-1)
    got = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    again = run_dev(hip, dtype, w, x, n_tok, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    assert np.isfinite(got).all()
    tokens = np.unique(np.concatenate([[0, 1, n_tok - 1], np.linspace(0, n_tok - 1, 7).astype(int)]))
    check(oracle, got, w, x, tokens, dtype, n_tok, in_dim, out_dim, REL_TOL, "gemm")
    rc, want = oracle.matmul_quant_f32(w, x.reshape(n_tok, in_dim)[tokens].reshape(-1),
                                       len(tokens), in_dim, out_dim, int(dtype))
    g = got.reshape(n_tok, out_dim)[tokens]
    want = want.reshape(len(tokens), out_dim)
    for r in big_all + big_one + tiny + [1, 8, 299]:
        assert rel_err(g[:, r], want[:, r]) <= REL_TOL, f"row {r}"


def test_prefill_bf16_scale_range(oracle, hip):
    """The range guard on the bf16 entry point: Q4_K rows with d = dmin = 256
    in every block among normal rows, C4's row length."""
    out_dim, in_dim, n_tok = 512, 4096, 130
    w = synth.weight(G.Q4_K, out_dim, in_dim, seed=2950).copy()
    rows = [3, 200, 511]
    _set_scales(w, G.Q4_K, in_dim, rows, range(16), _BIG[G.Q4_K])
    xb = synth.bf16_activations(n_tok, in_dim, seed=2951).reshape(-1)
    import torch
    s = torch.cuda.current_stream().cuda_stream
    d_w = torch.from_numpy(w).cuda()
    d_x = torch.from_numpy(xb.view(np.int16)).cuda()
    d_y = torch.full((n_tok * out_dim,), float("nan"), device="cuda")
    hip.matmul_q4k_bf16_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), w.size, d_x.data_ptr(),
                            xb.size, n_tok, in_dim, out_dim, G.Q4_K, s)
    torch.cuda.synchronize()
    got = d_y.cpu().numpy()
    assert np.isfinite(got).all()
    tokens = np.array([0, 64, 127, 128, 129])
    xf = synth.bf16_bits_to_f32(xb.reshape(n_tok, in_dim)[tokens])
    rc, want = oracle.matmul_quant_f32(w, xf.reshape(-1), len(tokens), in_dim, out_dim, int(G.Q4_K))
    g = got.reshape(n_tok, out_dim)[tokens]
    want = want.reshape(len(tokens), out_dim)
    assert_within_bound(G.Q4_K, w, xf, g, want, out_dim, in_dim, "bf16 scale range")
    for r in rows + [0, 4, 510]:
        assert rel_err(g[:, r], want[:, r]) <= REL_TOL, f"row {r}"
