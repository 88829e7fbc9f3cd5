"""The prefill GEMMs' error bound (prefill_bound.py) pinned on the CPU.

A numpy model of the GEMM's roundings (f16 weight scales and weights, per
token power-of-two scaled f16 activations, exact products, float64 sums)
must stay within the bound of the oracle's matmul_quant_f32 on every output,
also on blocks with f16-subnormal and zero scales; and the bound must catch
plausible mistakes planted in that model (a neighbouring sub-block's scale,
the min term dropped, q - 31 for q - 32, an activation scale off by one
binade), so it is not vacuous."""
import numpy as np
import pytest

from oracle import oracle as O
from prefill_bound import prefill_bound, weight_terms
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G


def _f16(v):
    return np.asarray(v, dtype=np.float64).astype(np.float16).astype(np.float64)


def model_weights(dtype, w, out_dim, in_dim, mistake=None):
    """f16 weights [out_dim, in_dim] as the GEMM forms them."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    if dtype == G.Q4_K:
        b = w.reshape(-1, 144)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64)
        dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)
        sc, m = O.np_scale_min(b[:, 4:16])
        if mistake == "neighbour_scale":
            sc = sc[:, [1, 0, 3, 2, 5, 4, 7, 6]]
        qs = b[:, 16:].reshape(-1, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float64)
        a = _f16(d * sc)
        bb = _f16(dmin * m)
        if mistake == "no_min":
            bb = bb * 0.0
        wt = _f16(a[:, :, None] * q - bb[:, :, None])
    elif dtype == G.Q6_K:
        b = w.reshape(-1, 210)
        d = b[:, 208:210].copy().view(np.float16).astype(np.float64)
        q, sc = O.np_q6k_values(b)
        if mistake == "q_minus_31":
            q = q + 1
        a = _f16(d * sc.astype(np.float64))
        wt = _f16(a * q)
    else:
        b = w.reshape(-1, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64)
        wt = _f16(d * b[:, 2:].view(np.int8).astype(np.float64))
    return wt.reshape(out_dim, in_dim)


def model_gemm(dtype, w, x, out_dim, in_dim, mistake=None):
    x = np.asarray(x, dtype=np.float32).reshape(-1, in_dim).astype(np.float64)
    amax = np.abs(x).max(axis=1)
    e = np.zeros(len(x), np.int64)
    nz = amax > 0
    e[nz] = np.minimum(14 - np.floor(np.log2(amax[nz])).astype(np.int64), 120)
    if mistake == "act_binade":
        e = e + 1
    xt = _f16(x * np.ldexp(1.0, e)[:, None])
    y = xt @ model_weights(dtype, w, out_dim, in_dim, mistake).T
    if mistake == "act_binade":
        e = e - 1
    return y * np.ldexp(1.0, -e)[:, None]


def _weights(dtype, out_dim, in_dim, seed, special):
    w = synth.weight(dtype, out_dim, in_dim, seed=seed)
    if not special:
        return w
    bb, d_at = {G.Q4_K: (144, 0), G.Q6_K: (210, 208), G.Q8_0: (34, 0)}[dtype]
    w = w.reshape(-1, bb).copy()
    g = np.random.default_rng(seed + 1)
    idx = g.choice(w.shape[0], size=w.shape[0] // 2, replace=False)
    choices = np.array([0x0000, 0x0001, 0x0007, 0x03FF, 0x0400, 0x0401, 0x2000], np.uint16)
    w[idx, d_at:d_at + 2] = g.choice(choices, size=len(idx)).view(np.uint8).reshape(-1, 2)
    if dtype == G.Q4_K:
        w[idx, 2:4] = g.choice(choices, size=len(idx)).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0])
@pytest.mark.parametrize("special", [False, True])
def test_model_within_bound(dtype, special):
    out_dim, in_dim, n_tok = 48, 1024, 6
    w = _weights(dtype, out_dim, in_dim, 3100 + int(dtype), special)
    x = synth.activations(n_tok, in_dim, seed=3101)
    x[1] *= 1e-12
    x[2] *= 1e12
    rc, want = O.matmul_quant_f32(w, x.reshape(-1), n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    want = want.reshape(n_tok, out_dim).astype(np.float64)
    B = prefill_bound(dtype, w, x, out_dim, in_dim)
    err = np.abs(model_gemm(dtype, w, x, out_dim, in_dim) - want)
    assert (err <= B).all(), f"max |d|/bound {np.max(err / B):.3f}"
    # the bound is far above the rounding actually seen, but within two
    # orders of magnitude of sum_i |w_i x_i| 2^-11
    A, _ = weight_terms(dtype, w, out_dim, in_dim)
    S = np.abs(x.astype(np.float64)) @ A.T
    assert (B <= 0.01 * S + 1e-30).all()


@pytest.mark.parametrize("dtype,mistake", [(G.Q4_K, "neighbour_scale"), (G.Q4_K, "no_min"),
                                           (G.Q6_K, "q_minus_31"), (G.Q8_0, "act_binade"),
                                           (G.Q4_K, "act_binade")])
def test_bound_catches_planted_mistakes(dtype, mistake):
    out_dim, in_dim, n_tok = 48, 1024, 6
    w = synth.weight(dtype, out_dim, in_dim, seed=3200 + int(dtype))
    x = synth.activations(n_tok, in_dim, seed=3201)
    rc, want = O.matmul_quant_f32(w, x.reshape(-1), n_tok, in_dim, out_dim, int(dtype))
    want = want.reshape(n_tok, out_dim).astype(np.float64)
    B = prefill_bound(dtype, w, x, out_dim, in_dim)
    err = np.abs(model_gemm(dtype, w, x, out_dim, in_dim, mistake) - want)
    assert (err > B).any(), f"{mistake} not caught: max |d|/bound {np.max(err / B):.3f}"


def test_small_scales_exact():
    """f16 represents every multiple of 2^-24 below 2^-13 exactly, and every
    intermediate of a weight's dequantisation is such a multiple: with the
    smallest subnormal scale (d = dmin = 2^-24) all of them stay below 2^-13,
    and the model's f16 weights equal the oracle's dequantisation bit for
    bit."""
    for dtype, bb, d_at in ((G.Q4_K, 144, 0), (G.Q6_K, 210, 208), (G.Q8_0, 34, 0)):
        w = synth.weight(dtype, 16, 1024, seed=3300).reshape(-1, bb).copy()
        w[:, d_at:d_at + 2] = np.array([0x0001], np.uint16).view(np.uint8)
        if dtype == G.Q4_K:
            w[:, 2:4] = np.array([0x0001], np.uint16).view(np.uint8)
        w = w.reshape(-1)
        rc, ref = O.dequant(int(dtype), w, 16 * 1024)
        assert rc == 0
        model = model_weights(dtype, w, 16, 1024).reshape(-1)
        assert np.abs(model).max() <= 2.0 ** -13
        assert np.array_equal(model, ref.astype(np.float64)), dtype.name
