"""The oracle's apply_shared_expert (rsllm-models/src/dsv4/moe.rs:422-455,
apply_expert_swiglu :479-502) pinned by the reference's own test of it
(apply_shared_expert_applies_swiglu_clamp, moe.rs:743-789, at DS-V4's
shapes n_embd 4096, n_ff 2048, shape.rs:25,152), by a float64 recompute of
the F32 form and by equality with the routed-expert oracle on one expert of
weight 1 (moe.rs:648-707 adds w * y, so with w = 1 onto zeros it is y)."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

N_EMBD, N_FF, CLAMP = 4096, 2048, 10.0


def identity_weights(rows, cols):
    w = np.zeros((rows, cols), np.float32)
    n = min(rows, cols)
    w[np.arange(n), np.arange(n)] = 1.0
    return w.reshape(-1)


def f64_swiglu(g, u, c):
    if c > 1e-6:
        g = np.minimum(g, c)
        u = np.clip(u, -c, c)
    return g / (1.0 + np.exp(-g)) * u


def test_reference_clamp_test():
    # moe.rs:743-789: identity-truncation gate/up/down, x[0] = 1e3
    gate = identity_weights(N_FF, N_EMBD)
    up = identity_weights(N_FF, N_EMBD)
    down = identity_weights(N_EMBD, N_FF)
    x = np.zeros(N_EMBD, np.float32)
    x[0] = 1e3
    rc, out = O.apply_shared_expert(x, gate, O.F32, up, O.F32, down, O.F32, 1, N_EMBD, N_FF,
                                    CLAMP)
    assert rc == O.OK
    assert 90.0 < out[0] < 110.0                       # the reference's assertion
    assert abs(out[0] - 10.0 / (1.0 + math.exp(-10.0)) * 10.0) < 1e-4
    assert not out[1:].any()
    # clamp off (the reference's None): silu(1000) * 1000 = 1e6
    rc, out = O.apply_shared_expert(x, gate, O.F32, up, O.F32, down, O.F32, 1, N_EMBD, N_FF, 0.0)
    assert rc == O.OK and out[0] == 1e6


@pytest.mark.parametrize("clamp", [0.0, 1.5])
def test_f32_form_matches_float64(clamp):
    rng = np.random.default_rng(3)
    n_tok, n_embd, n_ff = 3, 96, 40
    gate = rng.standard_normal(n_ff * n_embd).astype(np.float32) * 0.3
    up = rng.standard_normal(n_ff * n_embd).astype(np.float32) * 0.3
    down = rng.standard_normal(n_embd * n_ff).astype(np.float32) * 0.3
    x = rng.standard_normal(n_tok * n_embd).astype(np.float32)
    rc, out = O.apply_shared_expert(x, gate, O.F32, up, O.F32, down, O.F32, n_tok, n_embd, n_ff,
                                    clamp)
    assert rc == O.OK
    X = x.reshape(n_tok, n_embd).astype(np.float64)
    hg = X @ gate.reshape(n_ff, n_embd).astype(np.float64).T
    hu = X @ up.reshape(n_ff, n_embd).astype(np.float64).T
    want = f64_swiglu(hg, hu, clamp) @ down.reshape(n_embd, n_ff).astype(np.float64).T
    assert np.abs(out.reshape(n_tok, n_embd) - want).max() <= 1e-5 * np.abs(want).max()
    if clamp:
        assert (hg > clamp).any() and (np.abs(hu) > clamp).any()   # the clamp engages


@pytest.mark.parametrize("dt_gu,dt_d", [(G.Q4_K, G.Q6_K), (G.Q8_0, G.Q8_0), (G.IQ2_XXS, G.Q2_K)])
def test_quant_form_is_one_routed_expert_of_weight_one(dt_gu, dt_d):
    n_tok, n_embd, n_ff = 3, 512, 256
    gate = synth.weight(dt_gu, n_ff, n_embd, 1)
    up = synth.weight(dt_gu, n_ff, n_embd, 2)
    down = synth.weight(dt_d, n_embd, n_ff, 3)
    x = synth.activations(n_tok, n_embd, 4)
    rc, out = O.apply_shared_expert(x, gate, int(dt_gu), up, int(dt_gu), down, int(dt_d), n_tok,
                                    n_embd, n_ff, CLAMP)
    assert rc == O.OK
    want = np.zeros(n_tok * n_embd, np.float32)
    ids = np.zeros((n_tok, 1), np.int32)
    w = np.ones((n_tok, 1), np.float32)
    assert O.moe_routed(want, x, n_tok, n_embd, n_ff, gate, up, down, int(dt_gu), int(dt_d), 1,
                        ids, w, 1, CLAMP) == O.OK
    np.testing.assert_array_equal(out, want)


def test_errors_in_order():
    n_embd, n_ff = 64, 32
    g = np.zeros(n_ff * n_embd, np.float32)
    d = np.zeros(n_embd * n_ff, np.float32)
    x = np.zeros(2 * n_embd, np.float32)
    call = O.apply_shared_expert
    assert call(x[:-1], g, O.F32, g, O.F32, d, O.F32, 2, n_embd, n_ff, 10.0)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 30
    assert call(x, g, O.F32, g, O.F32, d, O.F32, 2, n_embd, n_ff, 10.0,
                out_len=3)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 31
    assert call(x, g[:-1], O.F32, g, O.F32, d, O.F32, 2, n_embd, n_ff, 10.0)[0] == O.SHAPE_MISMATCH
    assert O.last_detail() == (12, 0)
    q = np.zeros(n_ff * 2 * 34, np.uint8)   # Q8_0 [n_ff x 64]
    assert call(x, g, O.F32, q[:-1], O.Q8_0, d, O.F32, 2, n_embd, n_ff,
                10.0)[0] == O.SHAPE_MISMATCH
    assert O.last_detail() == (13, 1)
    assert call(x, g, O.F32, q, O.Q8_0, d[:-1], O.F32, 2, n_embd, n_ff,
                10.0)[0] == O.SHAPE_MISMATCH
    assert O.last_detail() == (12, 2)
    # no tokens: no matmul runs, so bad weights pass
    rc, out = call(np.zeros(0, np.float32), g[:-1], O.F32, g, O.F32, d, O.F32, 0, n_embd, n_ff,
                   10.0)
    assert rc == O.OK and out.size == 0
