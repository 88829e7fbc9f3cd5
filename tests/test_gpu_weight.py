"""matmul_weight_f32 and matmul_grouped_lora_down (rsllm-models/src/dsv4/
weight.rs:113-266) on the GPU against the oracle: max|Δ|/max|y| <= 1e-3
(REL_TOL) for both arms, every one-launch / per-group / gathered path of the
grouped form (DS-V4's attn_output_a shape: 8 groups of [1024 x 4096] Q8_0),
ragged shapes, and the device-pointer forms."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu


def f32_weights(out_dim, in_dim, seed):
    return np.random.default_rng(seed).standard_normal(out_dim * in_dim).astype(np.float32)


@pytest.mark.parametrize("n_tok,in_dim,out_dim", [(1, 1, 1), (2, 4, 3), (3, 37, 5), (1, 256, 130),
                                                  (5, 1000, 64), (8, 4096, 300), (17, 300, 7)])
def test_weight_f32_f32_arm(oracle, hip, n_tok, in_dim, out_dim):
    w = f32_weights(out_dim, in_dim, in_dim + out_dim)
    x = synth.activations(n_tok, in_dim, 3).reshape(-1)
    rc, want = oracle.matmul_weight_f32(w, x, n_tok, in_dim, out_dim, oracle.F32)
    assert rc == 0
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_weight_f32(got, w, x, n_tok, in_dim, out_dim, G.F32)
    err = rel_err(got, want)
    print(f"weight_f32 F32 T={n_tok} {out_dim}x{in_dim}: rel err {err:.3e}")
    assert err <= REL_TOL


def test_weight_f32_hand_dot(hip):
    # weight.rs:329-354, exact in any summation order
    w = np.array([1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 1], np.float32)
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    out = np.full(6, np.nan, np.float32)
    hip.matmul_weight_f32(out, w, x, 2, 4, 3, G.F32)
    assert out.tolist() == [1.0, 2.0, 7.0, 5.0, 6.0, 15.0]


def test_weight_f32_zero_in_dim_gives_zeros(hip):
    out = np.full(6, np.nan, np.float32)
    hip.matmul_weight_f32(out, np.zeros(0, np.float32), np.zeros(0, np.float32), 2, 0, 3, G.F32)
    assert np.array_equal(out, np.zeros(6, np.float32))


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q4_0, G.Q2_K, G.IQ2_XXS])
@pytest.mark.parametrize("n_tok", [1, 3, 12])
def test_weight_f32_quant_arm(oracle, hip, dtype, n_tok):
    out_dim, in_dim = 77, 1024
    w = synth.weight(dtype, out_dim, in_dim, 5)
    x = synth.activations(n_tok, in_dim, 6).reshape(-1)
    rc, want = oracle.matmul_weight_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    got = np.full(n_tok * out_dim, np.nan, np.float32)
    hip.matmul_weight_f32(got, w, x, n_tok, in_dim, out_dim, dtype)
    assert rel_err(got, want) <= REL_TOL


def grouped_case(dtype, n_tok, n_groups, group_dim, rank, seed):
    if dtype == G.F32:
        w = f32_weights(n_groups * rank, group_dim, seed)
    else:
        w = synth.weight(dtype, n_groups * rank, group_dim, seed)
    x = synth.activations(n_tok, n_groups * group_dim, seed + 1)
    return w, x


def oracle_grouped(oracle, w, x, toks, n_groups, group_dim, rank, dtype):
    """The oracle on a subset of tokens (tokens are independent)."""
    rc, want = oracle.matmul_grouped_lora_down(w, x[toks], len(toks), n_groups, group_dim, rank,
                                               int(dtype))
    assert rc == 0
    return want.reshape(len(toks), n_groups * rank)


@pytest.mark.parametrize("dtype,n_groups,group_dim,rank", [
    (G.F32, 2, 3, 2), (G.F32, 3, 300, 17), (G.F32, 4, 1024, 64),
    (G.Q8_0, 3, 256, 5),
    (G.Q8_0, 3, 96, 5),      # 15 blocks per group: not whole 8-block super-tiles
    (G.Q6_K, 2, 256, 3),     # 3 blocks per group
    (G.Q8_0, 4, 1024, 16),
    (G.Q4_K, 3, 512, 7),
    (G.Q6_K, 4, 2048, 8),
    (G.Q2_K, 2, 2048, 24),
    (G.IQ2_XXS, 2, 4096, 8),
    (G.Q4_0, 5, 512, 16),
])
@pytest.mark.parametrize("n_tok", [1, 2, 5, 8])
def test_grouped_lora_down_small(oracle, hip, dtype, n_groups, group_dim, rank, n_tok):
    w, x = grouped_case(dtype, n_tok, n_groups, group_dim, rank, 40 + n_tok)
    want = oracle_grouped(oracle, w, x, np.arange(n_tok), n_groups, group_dim, rank, dtype)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, dtype)
    err = rel_err(got.reshape(n_tok, -1), want)
    print(f"lora_down {G(dtype).name} T={n_tok} {n_groups}x[{rank}x{group_dim}]: rel err {err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("dtype,n_groups,group_dim,rank", [
    (G.F32, 3, 300, 17), (G.Q8_0, 4, 1024, 16), (G.Q4_K, 3, 512, 7), (G.Q6_K, 4, 2048, 8),
])
@pytest.mark.parametrize("n_tok", [9, 20])
def test_grouped_lora_down_many_tokens(oracle, hip, dtype, n_groups, group_dim, rank, n_tok):
    """More than 8 tokens: one launch per chunk of up to 8 tokens."""
    w, x = grouped_case(dtype, n_tok, n_groups, group_dim, rank, 70 + n_tok)
    toks = np.array([0, 3, n_tok - 1])
    want = oracle_grouped(oracle, w, x, toks, n_groups, group_dim, rank, dtype)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, dtype)
    assert not np.isnan(got).any()
    assert rel_err(got.reshape(n_tok, -1)[toks], want) <= REL_TOL


def lora_dev(hip, w, x, n_tok, n_groups, group_dim, rank, dtype):
    """The device form on a whole-matrix device layout; returns the output
    (NaN where nothing was written) or raises."""
    import torch
    s = torch.cuda.current_stream().cuda_stream
    d_raw = torch.from_numpy(w).cuda()
    d_w = torch.empty_like(d_raw)
    hip.prepare_weights_dev(d_w.data_ptr(), d_raw.data_ptr(), w.size, dtype, group_dim, s)
    d_x = torch.from_numpy(x.reshape(-1).copy()).cuda()
    d_y = torch.full((n_tok * n_groups * rank,), float("nan"), device="cuda")
    try:
        hip.matmul_grouped_lora_down_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), w.size,
                                         d_x.data_ptr(), d_x.numel(), n_tok, n_groups, group_dim,
                                         rank, dtype, s)
    finally:
        torch.cuda.synchronize()
    return d_y.cpu().numpy()


@pytest.mark.parametrize("dtype,group_dim,rank", [(G.Q8_0, 96, 5), (G.Q6_K, 256, 3)])
@pytest.mark.parametrize("n_tok", [3, 9, 17])
def test_grouped_lora_down_unaligned_groups(oracle, hip, dtype, group_dim, rank, n_tok):
    """Groups that are not whole 8-block super-tiles of the device layout run
    as one launch per chunk of up to 8 tokens on the whole matrix's layout,
    host and device forms alike."""
    n_groups = 3
    w, x = grouped_case(dtype, n_tok, n_groups, group_dim, rank, 3)
    want = oracle_grouped(oracle, w, x, np.arange(n_tok), n_groups, group_dim, rank, dtype)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, dtype)
    assert rel_err(got.reshape(n_tok, -1), want) <= REL_TOL
    got = lora_dev(hip, w, x, n_tok, n_groups, group_dim, rank, dtype)
    assert rel_err(got.reshape(n_tok, -1), want) <= REL_TOL


@pytest.mark.parametrize("rank", [8, 3])
def test_grouped_lora_down_groups_too_long_for_lds(oracle, hip, rank):
    """A Q8_0 group of 32800 elements (more than one token's x fits in LDS)
    runs per group on gathered x. With rank 8 the groups are whole
    super-tiles (8 x 1025 blocks) and both forms compute; with rank 3 they
    are not: the host form converts each group on its own, the device form
    reports Unimplemented and writes nothing."""
    n_tok, n_groups, group_dim = 2, 2, 32800
    w, x = grouped_case(G.Q8_0, n_tok, n_groups, group_dim, rank, 8)
    want = oracle_grouped(oracle, w, x, np.arange(n_tok), n_groups, group_dim, rank, G.Q8_0)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, G.Q8_0)
    assert rel_err(got.reshape(n_tok, -1), want) <= REL_TOL
    if rank == 8:
        got = lora_dev(hip, w, x, n_tok, n_groups, group_dim, rank, G.Q8_0)
        assert rel_err(got.reshape(n_tok, -1), want) <= REL_TOL
    else:
        with pytest.raises(hip.Unimplemented):
            lora_dev(hip, w, x, n_tok, n_groups, group_dim, rank, G.Q8_0)


@pytest.mark.parametrize("n_tok", [1, 2, 5, 9, 16, 33])
def test_grouped_lora_down_dsv4_attn_output_a(oracle, hip, n_tok):
    """DS-V4 Flash attn_output_a: 8 groups of [1024 x 4096] Q8_0 (weight.rs:
    171-182); up to 8 tokens one launch of the int8-limb kernel, from 9 the
    matrix cores in chunks of 16 tokens (33: the last chunk has one)."""
    n_groups, group_dim, rank = 8, 4096, 1024
    w, x = grouped_case(G.Q8_0, n_tok, n_groups, group_dim, rank, 900)
    toks = np.unique(np.array([0, n_tok // 2, n_tok - 1]))
    want = oracle_grouped(oracle, w, x, toks, n_groups, group_dim, rank, G.Q8_0)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.register_weights(w, G.Q8_0, group_dim)
    try:
        hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank,
                                     G.Q8_0)
    finally:
        hip.release_weights()
    assert not np.isnan(got).any()
    err = rel_err(got.reshape(n_tok, -1)[toks], want)
    print(f"lora_down DS-V4 T={n_tok}: rel err {err:.3e}")
    assert err <= REL_TOL


def test_grouped_lora_down_longer_blob(oracle, hip):
    """The blob may extend past the last group (weight.rs:313-319 only checks
    that each slice ends inside it); the extra rows are ignored."""
    n_tok, n_groups, group_dim, rank = 3, 3, 512, 8
    w, x = grouped_case(G.Q6_K, n_tok, n_groups + 1, group_dim, rank, 12)
    x = np.ascontiguousarray(x[:, : n_groups * group_dim])
    want = oracle_grouped(oracle, w, x, np.arange(n_tok), n_groups, group_dim, rank, G.Q6_K)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, G.Q6_K)
    assert rel_err(got.reshape(n_tok, -1), want) <= REL_TOL


@pytest.mark.parametrize("dtype", [G.F32, G.Q8_0, G.Q6_K, G.Q4_K])
@pytest.mark.parametrize("n_tok", [2, 11])
def test_device_forms(oracle, hip, dtype, n_tok):
    import torch
    n_groups, group_dim, rank = 4, 1024, 32
    w, x = grouped_case(dtype, n_tok, n_groups, group_dim, rank, 21)
    s = torch.cuda.current_stream().cuda_stream
    wb = w.view(np.uint8)
    d_raw = torch.from_numpy(wb.copy()).cuda()
    if dtype == G.F32:
        d_w = d_raw
    else:
        d_w = torch.empty_like(d_raw)
        hip.prepare_weights_dev(d_w.data_ptr(), d_raw.data_ptr(), wb.size, dtype, group_dim, s)
    d_x = torch.from_numpy(x.reshape(-1).copy()).cuda()
    # grouped form
    d_y = torch.full((n_tok * n_groups * rank,), float("nan"), device="cuda")
    hip.matmul_grouped_lora_down_dev(d_y.data_ptr(), d_y.numel(), d_w.data_ptr(), wb.size,
                                     d_x.data_ptr(), d_x.numel(), n_tok, n_groups, group_dim,
                                     rank, dtype, s)
    # matmul_weight_f32 on the whole stacked matrix with group 0's x repeated
    # is a plain [n_groups * rank x group_dim] product
    x0 = np.ascontiguousarray(x[:, :group_dim])
    d_x0 = torch.from_numpy(x0.reshape(-1).copy()).cuda()
    d_z = torch.full((n_tok * n_groups * rank,), float("nan"), device="cuda")
    hip.matmul_weight_f32_dev(d_z.data_ptr(), d_z.numel(), d_w.data_ptr(), wb.size,
                              d_x0.data_ptr(), d_x0.numel(), n_tok, group_dim, n_groups * rank,
                              dtype, s)
    torch.cuda.synchronize()
    want = oracle_grouped(oracle, w, x, np.arange(n_tok), n_groups, group_dim, rank, dtype)
    assert rel_err(d_y.cpu().numpy().reshape(n_tok, -1), want) <= REL_TOL
    rc, want_z = oracle.matmul_weight_f32(w, x0, n_tok, group_dim, n_groups * rank, int(dtype))
    assert rc == 0
    assert rel_err(d_z.cpu().numpy(), want_z) <= REL_TOL


@pytest.mark.parametrize("dtype,n_groups,group_dim,rank", [
    (G.Q4_K, 2, 1024, 512), (G.Q6_K, 4, 2048, 256), (G.Q8_0, 3, 512, 384),
])
@pytest.mark.parametrize("n_tok", [9, 20, 40])
def test_grouped_lora_down_matrix_cores(oracle, hip, dtype, n_groups, group_dim, rank, n_tok):
    """9 or more tokens with ranks that are multiples of 64 and at least 1024
    outputs per token: the matrix-core path (one pass over the stacked matrix
    per 16 tokens; a workgroup's 64 rows belong to one group)."""
    w, x = grouped_case(dtype, n_tok, n_groups, group_dim, rank, 300 + n_tok)
    toks = np.unique(np.minimum(np.array([0, 15, 16, n_tok - 1]), n_tok - 1))
    want = oracle_grouped(oracle, w, x, toks, n_groups, group_dim, rank, dtype)
    got = np.full(n_tok * n_groups * rank, np.nan, np.float32)
    hip.matmul_grouped_lora_down(got, w, x.reshape(-1), n_tok, n_groups, group_dim, rank, dtype)
    assert not np.isnan(got).any()
    err = rel_err(got.reshape(n_tok, -1)[toks], want)
    print(f"lora_down mfma {G(dtype).name} T={n_tok} {n_groups}x[{rank}x{group_dim}]: rel err {err:.3e}")
    assert err <= REL_TOL
