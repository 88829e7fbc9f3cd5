"""Pins the oracle's routed-expert restatement (orc_moe_routed, restating
accumulate_moe_outputs / apply_expert_swiglu / apply_swiglu_clamp,
rsllm-models/src/dsv4/moe.rs:479-531,648-707):
- the reference's clamp KATs (moe.rs:791-833) and sigmoid KATs
  (rsllm-backend-cpu/src/ops/scalar.rs:222-240);
- an independent float64 numpy composition built from the numpy dequant
  restatement (a dropped clamp, a swapped gate/up, a wrong expert stride or
  a missing routing weight each fail it);
- the invariants w = 0 => slot skipped, and out accumulates."""
import numpy as np
import pytest

from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G


def test_swiglu_clamp_kats(oracle):
    # swiglu_clamp_bounds_gate_above_and_up_both_sides (moe.rs:791-800)
    g, u = oracle.swiglu_clamp([-15.0, -5.0, 0.0, 5.0, 15.0], [-15.0, -5.0, 0.0, 5.0, 15.0], 10.0)
    assert g.tolist() == [-15.0, -5.0, 0.0, 5.0, 10.0]
    assert u.tolist() == [-10.0, -5.0, 0.0, 5.0, 10.0]
    # swiglu_clamp_disabled_when_threshold_tiny (:802-811)
    g, u = oracle.swiglu_clamp([1e6, -1e6], [1e6, -1e6], 0.0)
    assert g.tolist() == [1e6, -1e6] and u.tolist() == [1e6, -1e6]
    # swiglu_clamp_threshold_boundary_at_1e_minus_6 (:813-833)
    g, u = oracle.swiglu_clamp([100.0], [100.0], 1e-6)
    assert g.tolist() == [100.0] and u.tolist() == [100.0]
    g, u = oracle.swiglu_clamp([100.0], [100.0], 1.000001e-6)
    assert g[0] < 1e-5 and u[0] < 1e-5
    # NaN passes through (moe.rs:508-513)
    g, u = oracle.swiglu_clamp([np.nan], [np.nan], 10.0)
    assert np.isnan(g[0]) and np.isnan(u[0])


def test_sigmoid_kats(oracle):
    # sigmoid_matches_reference (scalar.rs:222-230)
    assert abs(oracle.sigmoid(0.0) - 0.5) < 1e-6
    assert abs(oracle.sigmoid(2.0) - 0.880797) < 1e-4
    assert abs(oracle.sigmoid(-2.0) - 0.119203) < 1e-4
    assert abs(oracle.sigmoid(20.0) - 1.0) < 1e-6
    assert abs(oracle.sigmoid(-20.0)) < 1e-6
    # no overflow for large negative inputs (:232-240)
    assert oracle.sigmoid(-100.0) >= 0.0 and np.isfinite(oracle.sigmoid(-100.0))
    assert oracle.silu(3.0) == pytest.approx(3.0 / (1.0 + np.exp(-3.0)), rel=1e-6)


def moe_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d, seed):
    gate = synth.weight(dt_gu, n_expert * n_ff, n_embd, seed)
    up = synth.weight(dt_gu, n_expert * n_ff, n_embd, seed + 1)
    down = synth.weight(dt_d, n_expert * n_embd, n_ff, seed + 2)
    x = synth.activations(n_tok, n_embd, seed + 3)
    ids, w = synth.moe_routing(n_tok, n_expert, k, seed + 4)
    return gate, up, down, x, ids, w


def np_moe(out, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d, c,
           oracle):
    """float64 composition from the numpy dequant restatement."""
    Wg = oracle.NP_DEQUANT[dt_gu](gate).astype(np.float64).reshape(n_expert, n_ff, n_embd)
    Wu = oracle.NP_DEQUANT[dt_gu](up).astype(np.float64).reshape(n_expert, n_ff, n_embd)
    Wd = oracle.NP_DEQUANT[dt_d](down).astype(np.float64).reshape(n_expert, n_embd, n_ff)
    res = out.astype(np.float64).reshape(n_tok, n_embd).copy()
    for t in range(n_tok):
        for i in range(k):
            e, we = int(ids[t, i]), float(w[t, i])
            if we == 0.0:
                continue
            g = Wg[e] @ x[t].astype(np.float64)
            u = Wu[e] @ x[t].astype(np.float64)
            if c > 1e-6:
                g = np.minimum(g, c)
                u = np.clip(u, -c, c)
            with np.errstate(over="ignore"):
                a = g / (1.0 + np.exp(-g)) * u
            res[t] += we * (Wd[e] @ a)
    return res.reshape(-1)


@pytest.mark.parametrize("dt_gu,dt_d", [(G.Q4_K, G.Q4_K), (G.Q4_K, G.Q6_K), (G.Q8_0, G.Q8_0)])
def test_moe_oracle_vs_float64_composition(oracle, dt_gu, dt_d):
    n_tok, n_embd, n_ff, n_expert, k = 3, 512, 256, 6, 3
    gate, up, down, x, ids, w = moe_case(n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d, 50)
    w[1, 2] = 0.0  # skipped slot
    base = synth.activations(n_tok, n_embd, 99).reshape(-1)
    out = base.copy()
    rc = oracle.moe_routed(out, x, n_tok, n_embd, n_ff, gate, up, down, int(dt_gu), int(dt_d),
                           n_expert, ids, w, k, 10.0)
    assert rc == 0
    want = np_moe(base, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k, dt_gu, dt_d,
                  10.0, oracle)
    assert np.abs(out - want).max() <= 1e-4 * np.abs(want).max()


def test_moe_oracle_clamp_engages(oracle):
    """Scaled-up activations push gate/up past the clamp: the clamped float64
    composition matches, the unclamped one does not."""
    n_tok, n_embd, n_ff, n_expert, k = 2, 256, 256, 4, 2
    gate, up, down, x, ids, w = moe_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 70)
    x = (x * 400.0).astype(np.float32)
    out = np.zeros(n_tok * n_embd, np.float32)
    assert oracle.moe_routed(out, x, n_tok, n_embd, n_ff, gate, up, down, int(G.Q4_K), int(G.Q4_K),
                             n_expert, ids, w, k, 10.0) == 0
    zero = np.zeros_like(out)
    clamped = np_moe(zero, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k, G.Q4_K,
                     G.Q4_K, 10.0, oracle)
    unclamped = np_moe(zero, x, gate, up, down, ids, w, n_tok, n_embd, n_ff, n_expert, k, G.Q4_K,
                       G.Q4_K, 0.0, oracle)
    assert np.abs(out - clamped).max() <= 1e-4 * np.abs(clamped).max()
    assert np.abs(out - unclamped).max() > 1e-2 * np.abs(unclamped).max()


def test_moe_oracle_zero_weights_leave_out_unchanged(oracle):
    n_tok, n_embd, n_ff, n_expert, k = 2, 256, 256, 3, 2
    gate, up, down, x, ids, w = moe_case(n_tok, n_embd, n_ff, n_expert, k, G.Q4_K, G.Q4_K, 80)
    w[:] = 0.0
    base = synth.activations(n_tok, n_embd, 81).reshape(-1)
    out = base.copy()
    assert oracle.moe_routed(out, x, n_tok, n_embd, n_ff, gate, up, down, int(G.Q4_K), int(G.Q4_K),
                             n_expert, ids, w, k, 10.0) == 0
    assert np.array_equal(out, base)
