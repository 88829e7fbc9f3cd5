"""Routed-expert MoE on the GPU against the oracle (accumulate_moe_outputs,
rsllm-models/src/dsv4/moe.rs:648-707 with apply_expert_swiglu :479-502 and
apply_swiglu_clamp :515-531, every matmul as matmul_quant_f32):
max|Δ|/max|y| <= 1e-3 over the accumulated output, on small shapes with
every format pairing, duplicated experts, skipped (w = 0) slots, engaged
clamps, and on C3 shapes (64 experts of gate/up 2048x7168, down 7168x2048,
Q4_K, top-8) with the oracle on a subset of tokens."""
import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

# Bound for the matrix-core routes: the weights reach the MFMA as exact
# integers with their scales applied in fp32, and every activation as two
# f16 planes (hi + lo, about 2^-22 relative), so the error is fp32-level
# (about 1e-6 of max |y| measured); 2e-5 leaves a wide margin and still
# fails a single f16 rounding of weights or activations (2e-4 and up).
MFMA_TOL = 2e-5


def make_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d, seed):
    gate = synth.weight(dt_gu, n_expert * n_ff, n_embd, seed)
    up = synth.weight(dt_gu, n_expert * n_ff, n_embd, seed + 1)
    down = synth.weight(dt_d, n_expert * n_embd, n_ff, seed + 2)
    x = synth.activations(n_tok, n_embd, seed + 3)
    ids, w = synth.moe_routing(n_tok, n_expert, k, seed + 4)
    return gate, up, down, x, ids, w


def run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k, dt_gu,
               dt_d, clamp=10.0):
    out = base.copy()
    rc = oracle.moe_routed(out, x, n_tok, n_embd, n_ff, gate, up, down, int(dt_gu), int(dt_d),
                           n_expert, ids, w, k, clamp)
    assert rc == 0
    return out


@pytest.mark.parametrize("dt_gu,dt_d", [(G.IQ2_XXS, G.Q2_K), (G.Q4_K, G.Q2_K),
                                        (G.Q4_K, G.Q4_K), (G.Q4_K, G.Q6_K), (G.Q8_0, G.Q8_0),
                                        (G.Q6_K, G.Q4_0)])
@pytest.mark.parametrize("n_tok,k", [(1, 2), (3, 3), (8, 4)])
def test_moe_small(oracle, hip, dt_gu, dt_d, n_tok, k):
    n_embd, n_ff, n_expert = 512, 256, 6
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d,
                                          17 * n_tok + k)
    if n_tok > 1:
        w[1, k - 1] = 0.0  # skipped slot
    base = synth.activations(n_tok, n_embd, 5).reshape(-1)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      dt_gu, dt_d)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   dt_gu, dt_d, 10.0)
    err = rel_err(got - base, want - base)
    print(f"moe {dt_gu.name}/{dt_d.name} T={n_tok} k={k}: rel err {err:.3e}")
    assert err <= REL_TOL


def test_moe_clamp_engaged_and_all_tokens_on_one_expert(oracle, hip):
    n_tok, n_embd, n_ff, n_expert, k = 9, 256, 512, 4, 2
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 31)
    x = (x * 300.0).astype(np.float32)     # gate/up far past the clamp
    ids[:, 0] = 2                          # 9 tokens on expert 2: batches of 4, 4, 1
    ids[:, 1] = np.where(ids[:, 1] == 2, 3, ids[:, 1])
    base = np.zeros(n_tok * n_embd, np.float32)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      G.Q4_K, G.Q4_K)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_K, 10.0)
    assert rel_err(got, want) <= REL_TOL


def test_moe_zero_weights_and_clamp_off(oracle, hip):
    n_tok, n_embd, n_ff, n_expert, k = 4, 256, 256, 5, 3
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 41)
    w[0, :] = 0.0
    base = synth.activations(n_tok, n_embd, 42).reshape(-1)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      G.Q4_K, G.Q4_K, clamp=0.0)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_K, 0.0)
    assert np.array_equal(got[:n_embd], base[:n_embd])  # token 0: every slot skipped
    assert rel_err(got - base, want - base) <= REL_TOL


def test_moe_validation(hip):
    n_tok, n_embd, n_ff, n_expert, k = 2, 256, 256, 3, 2
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 61)
    out = np.zeros(n_tok * n_embd, np.float32)
    bad = ids.copy()
    bad[1, 0] = n_expert
    with pytest.raises(hip.InvalidArgument):
        hip.moe_routed(out, x.reshape(-1), gate, up, down, bad, w, n_tok, n_embd, n_ff, n_expert,
                       k, G.Q4_K, G.Q4_K, 10.0)
    with pytest.raises(hip.NotBlockAligned):
        hip.moe_routed(out, x.reshape(-1), gate, up, down, ids, w, n_tok, 200, n_ff, n_expert, k,
                       G.Q4_K, G.Q4_K, 10.0)
    with pytest.raises(hip.ShapeMismatch):
        hip.moe_routed(out, x.reshape(-1), gate, up, down[:-144], ids, w, n_tok, n_embd, n_ff,
                       n_expert, k, G.Q4_K, G.Q4_K, 10.0)


@pytest.mark.parametrize("n_tok", [1, 2, 3, 8, 32])
def test_moe_c3_shapes(oracle, hip, n_tok):
    """C3 shapes with 16 experts (every expert's kernel path is the same as
    with 64); the oracle runs on up to 6 tokens (tokens are independent)."""
    n_embd, n_ff, n_expert, k = 7168, 2048, 16, 8
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 300)
    base = np.zeros(n_tok * n_embd, np.float32)
    got = base.copy()
    hip.register_weights(gate, G.Q4_K, n_embd)
    hip.register_weights(up, G.Q4_K, n_embd)
    hip.register_weights(down, G.Q4_K, n_ff)
    try:
        hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                       G.Q4_K, G.Q4_K, 10.0)
    finally:
        hip.release_weights()
    toks = np.unique(np.linspace(0, n_tok - 1, min(n_tok, 6)).astype(int))
    want = run_oracle(oracle, np.zeros(len(toks) * n_embd, np.float32), x[toks], gate, up, down,
                      ids[toks], w[toks], len(toks), n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K)
    err = rel_err(got.reshape(n_tok, n_embd)[toks], want.reshape(len(toks), n_embd))
    print(f"moe C3 T={n_tok}: rel err {err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("n_tok,k,dup", [(4, 7, False), (4, 7, True), (4, 8, True), (2, 5, True),
                                         (6, 4, True)])
def test_moe_fused_boundary_and_duplicates(oracle, hip, n_tok, k, dup):
    """n_tok * k pairs up to 32 with all slots in LDS take the two-launch
    fused path (routing in every workgroup, SwiGLU and the weighted sum in
    the GEMV epilogues); (4, 8) at n_ff 256 needs more LDS than allowed and
    takes the multi-launch path. `dup` makes a token pick one expert twice
    and puts six pairs on expert 0 (more slots than one pass of 4). The
    Q4_0 down projection has no matrix-core route, so calls of more than 16
    pairs stay on the fused pair here."""
    n_embd, n_ff, n_expert = 512, 256, 9
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_0,
                                          91 + n_tok + k)
    if dup:
        ids[0, 1] = ids[0, 0]
        flat = ids.reshape(-1)
        flat[: min(6, flat.size)] = 0
    w[n_tok - 1, 0] = 0.0
    base = synth.activations(n_tok, n_embd, 8).reshape(-1)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      G.Q4_K, G.Q4_0)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_0, 10.0)
    err = rel_err(got - base, want - base)
    print(f"moe fused boundary T={n_tok} k={k} dup={dup}: rel err {err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("dt_gu,dt_d", [(G.Q8_0, G.Q8_0), (G.Q6_K, G.Q4_0), (G.Q4_K, G.Q8_0)])
@pytest.mark.parametrize("n_embd,n_ff", [(4096, 512), (2048, 512), (1024, 2048), (4096, 2048)])
@pytest.mark.parametrize("n_tok,k", [(1, 1), (2, 1), (2, 3)])
def test_moe_fused_rows_spanning_columns(oracle, hip, dt_gu, dt_d, n_embd, n_ff, n_tok, k):
    """Fused path with in_dim over several 8-unit x columns and few rows per
    workgroup, so wavefront runs would end inside a row if they were not
    whole (chunk, row) pairs."""
    n_expert = 3
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d,
                                          7 * n_tok + k)
    base = np.zeros(n_tok * n_embd, np.float32)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      dt_gu, dt_d)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   dt_gu, dt_d, 10.0)
    assert rel_err(got, want) <= REL_TOL


@pytest.mark.parametrize("dt_gu,dt_d", [(G.Q4_K, G.Q4_K), (G.Q4_K, G.Q6_K), (G.Q8_0, G.Q4_K),
                                        (G.Q6_K, G.Q8_0), (G.Q2_K, G.Q4_0)])
@pytest.mark.parametrize("n_tok,k", [(40, 2), (5, 8), (9, 8)])
def test_moe_grouped_many_tokens(oracle, hip, dt_gu, dt_d, n_tok, k):
    """Calls the fused pair does not take in one go run grouped by expert:
    on the matrix cores for Q4_K, Q6_K and Q8_0 experts (each expert's slots
    in batches of up to 8 or 16), through the fused pair over token chunks or
    the int8-limb grouped GEMV otherwise. Every token's first pick is expert
    0 (40 slots: three batches, the last partial), token 1 picks one expert
    twice and one slot has weight 0."""
    n_embd, n_ff, n_expert = 1024, 1024, 9
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d,
                                          500 + n_tok + k)
    ids[:, 0] = 0
    ids[1, 1] = ids[1, 0]
    w[3, 1] = 0.0
    base = synth.activations(n_tok, n_embd, 9).reshape(-1)
    want = run_oracle(oracle, base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                      dt_gu, dt_d)
    got = base.copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   dt_gu, dt_d, 10.0)
    err = rel_err(got - base, want - base)
    print(f"moe grouped {dt_gu.name}/{dt_d.name} T={n_tok} k={k}: rel err {err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("dt", [G.Q8_0, G.Q6_K, G.Q4_K])
@pytest.mark.parametrize("n_tok", [9, 16, 32])
def test_moe_grouped_dsv4_like_shapes(oracle, hip, dt, n_tok):
    """DS-V4-like expert shapes (n_embd 4096, n_ff 2048), all three matrices
    in one format, checked on up to 6 tokens. All three formats take the
    matrix-core route from 8 tokens; its weights are exact and x and the
    SwiGLU output reach it as hi + lo f16 planes, so the chained error is
    held to MFMA_TOL (f16-rounded weights and activations reached 1.2e-3 for
    Q6_K and 9.3e-4 for Q8_0 here)."""
    n_embd, n_ff, n_expert, k = 4096, 2048, 16, 6
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, dt, dt,
                                          700 + n_tok + int(dt))
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   dt, dt, 10.0)
    toks = np.unique(np.linspace(0, n_tok - 1, min(n_tok, 6)).astype(int))
    want = run_oracle(oracle, np.zeros(len(toks) * n_embd, np.float32), x[toks], gate, up, down,
                      ids[toks], w[toks], len(toks), n_embd, n_ff, n_expert, k, dt, dt)
    err = rel_err(got.reshape(n_tok, n_embd)[toks], want.reshape(len(toks), n_embd))
    print(f"moe dsv4-like {dt.name} T={n_tok}: rel err {err:.3e}")
    assert err <= MFMA_TOL


@pytest.mark.parametrize("n_tok", [3, 9, 32])
def test_moe_grouped_dsv4_formats(oracle, hip, n_tok):
    """The DS-V4-Flash expert formats (IQ2_XXS gate/up, Q2_K down) at DS-V4
    expert shapes (n_embd 4096, n_ff 2048, top-6 of 16) on the grouped
    matrix-core route (calls past the fused pair's 16 pairs): exact codebook
    and 2-bit weights with their scales in fp32, hi + lo activations, so the
    chained error is held to MFMA_TOL. Checked on up to 6 tokens."""
    n_embd, n_ff, n_expert, k = 4096, 2048, 16, 6
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.IQ2_XXS, G.Q2_K,
                                          740 + n_tok)
    w[0, 1] = 0.0  # a skipped slot
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.IQ2_XXS, G.Q2_K, 10.0)
    toks = np.unique(np.linspace(0, n_tok - 1, min(n_tok, 6)).astype(int))
    want = run_oracle(oracle, np.zeros(len(toks) * n_embd, np.float32), x[toks], gate, up, down,
                      ids[toks], w[toks], len(toks), n_embd, n_ff, n_expert, k, G.IQ2_XXS, G.Q2_K)
    err = rel_err(got.reshape(n_tok, n_embd)[toks], want.reshape(len(toks), n_embd))
    print(f"moe dsv4 formats T={n_tok}: rel err {err:.3e}")
    assert err <= MFMA_TOL


def test_moe_grouped_q6k_full_range_scales(oracle, hip):
    """Q6_K experts whose scales span the whole int8 range (sc (q - 32) up to
    4096, past f16's exact integers) on the grouped matrix-core route: the
    split f16 + remainder weights keep the chained error at MFMA_TOL."""
    n_embd, n_ff, n_expert, k, n_tok = 2048, 1024, 8, 4, 16
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q6_K, G.Q6_K, 770)
    gate, up, down = (synth.q6k_full_scales(m, 780 + i) for i, m in enumerate((gate, up, down)))
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q6_K, G.Q6_K, 10.0)
    want = run_oracle(oracle, np.zeros(n_tok * n_embd, np.float32), x, gate, up, down, ids, w,
                      n_tok, n_embd, n_ff, n_expert, k, G.Q6_K, G.Q6_K)
    err = rel_err(got, want)
    print(f"moe grouped q6k full-range scales T={n_tok}: rel err {err:.3e}")
    assert err <= MFMA_TOL


# ---- prefill-sized calls: every token of a forward pass (moe.rs:281,346) ----

def _subset_check(oracle, got, x, gate, up, down, ids, w, toks, n_embd, n_ff, n_expert, k, dt_gu,
                  dt_d, base=None):
    n_tok = x.shape[0]
    b = np.zeros(len(toks) * n_embd, np.float32) if base is None else base[toks].reshape(-1).copy()
    want = run_oracle(oracle, b, x[toks], gate, up, down, ids[toks], w[toks], len(toks), n_embd,
                      n_ff, n_expert, k, dt_gu, dt_d)
    g = got.reshape(n_tok, n_embd)[toks]
    if base is not None:
        g = g - base[toks]
        want = want.reshape(len(toks), n_embd) - base[toks]
    return rel_err(g, want.reshape(len(toks), n_embd))


def test_moe_prefill_2048_tokens_top6_256_experts(oracle, hip):
    """DS-V4 routing at prefill size: 2048 tokens, top-6 of 256 experts
    (12288 pairs, past the 4096 the first build refused; two token chunks of
    the 8192-pair pass), Q4_K experts on the matrix-core route, checked on
    tokens from both chunks and at the chunk edge."""
    n_tok, n_embd, n_ff, n_expert, k = 2048, 1024, 1024, 256, 6
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 4100)
    w[5, 2] = 0.0   # skipped slots
    w[1700, 0] = 0.0
    base = synth.activations(n_tok, n_embd, 4101)
    got = base.reshape(-1).copy()
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_K, 10.0)
    toks = np.array([0, 5, 700, 1364, 1365, 1700, 2047])
    err = _subset_check(oracle, got, x, gate, up, down, ids, w, toks, n_embd, n_ff, n_expert, k,
                        G.Q4_K, G.Q4_K, base=base)
    print(f"moe prefill T={n_tok} k={k} E={n_expert}: rel err {err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("dt_d,tol", [(G.Q2_K, MFMA_TOL), (G.Q4_0, REL_TOL)])
def test_moe_prefill_iq2xxs_1500_tokens(oracle, hip, dt_d, tol):
    """IQ2_XXS gate/up at 1500 tokens x top-6 (9000 pairs: two chunks): with
    Q2_K down (the real DS-V4-Flash pairing) on the grouped matrix-core
    route, within MFMA_TOL; with Q4_0 down (no matrix-core form) through the
    int8-limb grouped GEMVs of the multi-launch route."""
    n_tok, n_embd, n_ff, n_expert, k = 1500, 512, 256, 64, 6
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.IQ2_XXS, dt_d,
                                          4200)
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.IQ2_XXS, dt_d, 10.0)
    toks = np.array([0, 1, 681, 1364, 1365, 1366, 1499])
    err = _subset_check(oracle, got, x, gate, up, down, ids, w, toks, n_embd, n_ff, n_expert, k,
                        G.IQ2_XXS, dt_d)
    print(f"moe prefill IQ2_XXS/{dt_d.name} T={n_tok}: rel err {err:.3e}")
    assert err <= tol


def test_moe_many_pairs_one_expert_and_device_form(oracle, hip):
    """Every pair on one expert (one long slot run across 40 routing blocks of
    256 pairs) through the device-pointer form, against the host form."""
    import torch
    n_tok, n_embd, n_ff, n_expert, k = 2560, 256, 512, 4, 4
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 4300)
    ids[:] = 2
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_K, 10.0)
    toks = np.array([0, 2047, 2048, 2559])
    err = _subset_check(oracle, got, x, gate, up, down, ids, w, toks, n_embd, n_ff, n_expert, k,
                        G.Q4_K, G.Q4_K)
    assert err <= REL_TOL
    s = torch.cuda.current_stream().cuda_stream
    d = [torch.from_numpy(np.ascontiguousarray(a)).cuda()
         for a in (gate, up, down, x.reshape(-1), ids.reshape(-1), w.reshape(-1))]
    y = torch.zeros(n_tok * n_embd, dtype=torch.float32, device="cuda")
    hip.moe_routed_dev(y.data_ptr(), y.numel(), d[3].data_ptr(), d[3].numel(), d[0].data_ptr(),
                       d[1].data_ptr(), gate.nbytes, d[2].data_ptr(), down.nbytes,
                       d[4].data_ptr(), d[5].data_ptr(), ids.size, n_tok, n_embd, n_ff, n_expert,
                       k, G.Q4_K, G.Q4_K, 10.0, s)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("n_tok", [40, 65])
def test_moe_dev_skips_out_of_range_ids_and_unaligned_out(oracle, hip, n_tok):
    """The device entry point skips slots whose expert id is out of range
    (it cannot inspect ids), as it skips w = 0 slots: the result equals the
    oracle's with those slots' weights zeroed. Q4_K experts from 8 tokens
    take the matrix-core route; 40 x 8 pairs route in one launch, 65 x 8
    (past 512) in three. A second call accumulates into an `out` 4 bytes off
    16-byte alignment (the one-output-per-thread accumulate): the same bits."""
    import torch
    n_embd, n_ff, n_expert, k = 1024, 1024, 9, 8
    gate, up, down, x, ids, w = make_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K,
                                          4500 + n_tok)
    bad = [(0, 1, -1), (3, 0, n_expert), (n_tok - 1, 7, 1 << 20), (n_tok // 2, 4, -7)]
    for t, i, e in bad:
        ids[t, i] = e
    w[2, 3] = 0.0
    ids_ok, w_ok = ids.copy(), w.copy()
    for t, i, _ in bad:
        ids_ok[t, i], w_ok[t, i] = 0, 0.0
    base = synth.activations(n_tok, n_embd, 4600 + n_tok).reshape(-1)
    want = run_oracle(oracle, base, x, gate, up, down, ids_ok, w_ok, n_tok, n_embd, n_ff, n_expert,
                      k, G.Q4_K, G.Q4_K)
    s = torch.cuda.current_stream().cuda_stream
    d = [torch.from_numpy(np.ascontiguousarray(a)).cuda()
         for a in (gate, up, down, x.reshape(-1), ids.reshape(-1).astype(np.int32), w.reshape(-1))]
    outs = []
    for off in (0, 1):
        y = torch.zeros(n_tok * n_embd + 4, dtype=torch.float32, device="cuda")
        yv = y[off:off + n_tok * n_embd]
        yv.copy_(torch.from_numpy(base).cuda())
        assert (yv.data_ptr() % 16 == 0) == (off == 0)
        hip.moe_routed_dev(yv.data_ptr(), yv.numel(), d[3].data_ptr(), d[3].numel(),
                           d[0].data_ptr(), d[1].data_ptr(), gate.nbytes, d[2].data_ptr(),
                           down.nbytes, d[4].data_ptr(), d[5].data_ptr(), ids.size, n_tok, n_embd,
                           n_ff, n_expert, k, G.Q4_K, G.Q4_K, 10.0, s)
        torch.cuda.synchronize()
        outs.append(yv.cpu().numpy().copy())
    err = rel_err(outs[0] - base, want - base)
    print(f"moe dev out-of-range ids T={n_tok}: rel err {err:.3e}")
    assert err <= MFMA_TOL
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


# ---- C3 at its real expert count (64 experts) ------

@pytest.fixture(scope="module")
def c3_experts():
    n_expert, n_embd, n_ff = 64, 7168, 2048
    return (synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 4400),
            synth.weight(G.Q4_K, n_expert * n_ff, n_embd, 4401),
            synth.weight(G.Q4_K, n_expert * n_embd, n_ff, 4402))


@pytest.mark.parametrize("n_tok", [1, 2, 4, 8, 16, 32])
def test_moe_c3_64_experts(oracle, hip, c3_experts, n_tok):
    """C3 as configured: 64 experts, Q4_K gate/up (2048, 7168) and down
    (7168, 2048), top-8 with softmax weights, T = 1, 2, 4, 8, 16 and 32 (the
    sweep of BASELINE.json configs[3]), checked on up to 6 tokens against
    the oracle (accumulate_moe_outputs, moe.rs:648-707): the matrix-core
    route from 8 tokens within MFMA_TOL, the fused int8-limb kernels below
    it within REL_TOL."""
    n_expert, n_embd, n_ff, k = 64, 7168, 2048, 8
    gate, up, down = c3_experts
    x = synth.activations(n_tok, n_embd, 4410 + n_tok)
    ids, w = synth.moe_routing(n_tok, n_expert, k, 4420 + n_tok)
    got = np.zeros(n_tok * n_embd, np.float32)
    hip.moe_routed(got, x.reshape(-1), gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k,
                   G.Q4_K, G.Q4_K, 10.0)
    toks = np.unique(np.linspace(0, n_tok - 1, 6).astype(int))
    err = _subset_check(oracle, got, x, gate, up, down, ids, w, toks, n_embd, n_ff, n_expert, k,
                        G.Q4_K, G.Q4_K)
    print(f"moe C3 64 experts T={n_tok}: rel err {err:.3e}")
    assert err <= (MFMA_TOL if n_tok >= 8 else REL_TOL)
