"""Per-output error bound of the prefill GEMMs (k_prefill_q4k_w8,
k_prefill_q8_w8, k_prefill_q6_w8) against the reference's matmul_quant_f32
(backend-cpu/src/ops/quant_matmul.rs:45-119), computed from the GGUF blocks
and the activations alone.

What the GEMM rounds, for output (t, o) = sum_i w_i x_i over K = in_dim terms:

* Weights. Q4_K: a = f16(d sc_j), b = f16(dmin m_j), w~ = f16(a q - b);
  Q6_K: a = f16(d sc), w~ = f16(a (q - 32)); Q8_0: w~ = f16(d q). d, dmin
  are f16 and sc, m, q integers, so each exact intermediate is a multiple of
  2^-24: its f16 rounding is exact below 2^-13 (f16 holds every multiple of
  2^-24 there) and within 2^-11 relative everywhere. With A_i = |d sc q| + |dmin m| (Q4_K) or |w_i| (Q6_K, Q8_0):
  |w~_i - w_i| <= (2 + 2^-11) 2^-11 A_i, and the reference's own w_i (one
  f32 rounding of the Q4_K subtraction) adds 2^-24 A_i.
  A workgroup that met an f16 overflow recomputes with row r's weights
  scaled by 2^-E_r, 2^E_r <= 2^-13 N_r, where N_r bounds the row's weights
  (945 |d| + 63 |dmin| per Q4_K block, 4096 |d| per Q6_K block, 128 |d| per
  Q8_0 block, the largest over the row). Its roundings are then no longer
  exact in the subnormal range: at most c_q 2^(E_r - 25) <= c_q 2^-38 N_r
  more per weight (c_q = 17, 33, 129: the rounded scale times the largest
  integer factor, plus the final rounding).
* Activations. Token t is scaled by 2^e_t (max |x_t| 2^e_t in [2^14, 2^15),
  e_t <= 120) and rounded to f16: within 2^-11 relative, or 2^(-25 - e_t)
  absolute, and 2^-e_t <= max(2^-14 max|x_t|, 2^-120).
* Products of two f16 values are exact in fp32. The GPU's sums (MFMA
  accumulation in any order, the two K groups, K-split partials) and the
  reference's sequential f32 sum each round at most K + 32 times:
  (2 K + 64) 2^-24 relative to sum_i |w_i x_i| between them (any summation
  order of n terms is within (n - 1) 2^-24 (1 + o(1)) of the exact sum).
  The final power-of-two scalings are exact unless the result is
  subnormal (2^-149).

So with S_to = sum_i A_oi |x_ti|:

  |y_gpu - y_ref| <= (3.002 2^-11 + (2 K + 64) 2^-24) (1 + 2^-9) S_to
                     + c_q 2^-38 N_o sum_i |x_ti|
                     + 2^-25 max(2^-14 max|x_t|, 2^-120) (1 + 2^-9) sum_i A_oi
                     + 2^-140

(3.002 = two weight roundings and one activation rounding, with their
cross terms.) The bound holds for every output, however few outputs a token
has; the whole-output metric max|d|/max|y| <= 1e-3 is checked beside it.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from rsllm_amd.ggml import GgmlType as G

C_Q = {G.Q4_K: 17.0, G.Q6_K: 33.0, G.Q8_0: 129.0}


def _f16_64(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float64).reshape(-1)


def weight_terms(dtype, w: np.ndarray, out_dim: int, in_dim: int):
    """(A [out_dim, in_dim], N [out_dim]) in float64 from GGUF blocks: A the
    magnitude sum of each weight's dequantisation terms, N the row's largest
    block bound (non-finite scales ignored)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    if dtype == G.Q4_K:
        b = w.reshape(-1, 144)
        d = np.abs(_f16_64(b[:, 0:2]))
        dmin = np.abs(_f16_64(b[:, 2:4]))
        sc, m = O.np_scale_min(b[:, 4:16])
        qs = b[:, 16:].reshape(-1, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float64)
        A = d[:, None, None] * sc[:, :, None] * q + (dmin[:, None] * m)[:, :, None]
        nblk = 945.0 * d + 63.0 * dmin
        per_row = in_dim // 256
    elif dtype == G.Q6_K:
        b = w.reshape(-1, 210)
        d = np.abs(_f16_64(b[:, 208:210]))
        q, sc = O.np_q6k_values(b)
        A = d[:, None] * np.abs(sc.astype(np.float64) * q)
        nblk = 4096.0 * d
        per_row = in_dim // 256
    elif dtype == G.Q8_0:
        b = w.reshape(-1, 34)
        d = np.abs(_f16_64(b[:, 0:2]))
        A = d[:, None] * np.abs(b[:, 2:].view(np.int8).astype(np.float64))
        nblk = 128.0 * d
        per_row = in_dim // 32
    else:
        raise ValueError(dtype)
    A = A.reshape(out_dim, in_dim)
    nblk = np.where(np.isfinite(nblk), nblk, 0.0).reshape(out_dim, per_row)
    return A, nblk.max(axis=1)


def prefill_bound(dtype, w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    """[T, out_dim] bound on |y_gpu - y_ref| for activations x [T, in_dim]
    (the values the GEMM is given: f32, or f32 of the bf16 input)."""
    A, N = weight_terms(dtype, w, out_dim, in_dim)
    ax = np.abs(np.asarray(x, dtype=np.float64).reshape(-1, in_dim))
    S = ax @ A.T
    K = float(in_dim)
    rel = (3.002 * 2.0 ** -11 + (2 * K + 64) * 2.0 ** -24) * (1 + 2.0 ** -9)
    amax = ax.max(axis=1)
    x_abs = 2.0 ** -25 * np.maximum(2.0 ** -14 * amax, 2.0 ** -120) * (1 + 2.0 ** -9)
    return (rel * S + C_Q[dtype] * 2.0 ** -38 * N[None, :] * ax.sum(axis=1)[:, None] +
            x_abs[:, None] * A.sum(axis=1)[None, :] + 2.0 ** -140)


def assert_within_bound(dtype, w, x, got, want, out_dim, in_dim, what=""):
    """Every output of every token within prefill_bound; returns the largest
    ratio |d| / bound."""
    B = prefill_bound(dtype, w, x, out_dim, in_dim)
    g = np.asarray(got, dtype=np.float64).reshape(B.shape)
    r = np.asarray(want, dtype=np.float64).reshape(B.shape)
    assert np.array_equal(np.isfinite(g), np.isfinite(r)), f"{what}: non-finite outputs differ"
    fin = np.isfinite(r)
    err = np.abs(g - r)
    ratio = np.where(fin, err / B, 0.0)
    worst = np.unravel_index(int(np.argmax(ratio)), ratio.shape)
    assert ratio.max() <= 1.0, (f"{what}: token {worst[0]} output {worst[1]}: |d| = "
                                f"{err[worst]:.3e} > bound {B[worst]:.3e}")
    return float(ratio.max())
