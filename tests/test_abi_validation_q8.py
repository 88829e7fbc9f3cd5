"""Argument validation of the Q8_0 int8-activation entry points, in the
reference's order and with its error classes (q8_0.rs:101-118 for
quantize_q8_0_batch, :229-252 for matmul_q8_0_batch, parallel.rs:44 and
rayon's zero chunk size for the panicking shapes). Validation runs before
any device work, so these run without a GPU."""
import numpy as np
import pytest


def q(hip, x_len, xq_len, s_len, n_tok, in_dim):
    hip.quantize_q8_0_batch(np.zeros(x_len, np.float32), np.zeros(xq_len, np.int8),
                            np.zeros(s_len, np.float32), n_tok, in_dim)


def m(hip, out_len, w_len, xq_len, xs_len, n_tok, in_dim, out_dim):
    hip.matmul_q8_0_batch(np.zeros(out_len, np.float32), np.zeros(w_len, np.uint8),
                          np.zeros(xq_len, np.int8), np.zeros(xs_len, np.float32), n_tok, in_dim,
                          out_dim)


@pytest.mark.parametrize("args,msg", [
    ((63, 64, 2, 1, 64), "x must be"),
    ((64, 63, 3, 1, 64), "xq must be"),        # xq checked before scale
    ((64, 64, 3, 1, 64), "scale must be"),
    ((40, 32, 2, 2, 20), "xq must be"),        # 2 tokens of 20: one padded block each
])
def test_quantize_shape_errors_in_order(hip, args, msg):
    with pytest.raises(hip.ShapeMismatch, match=msg):
        q(hip, *args)


def test_quantize_zero_in_dim_panics_in_reference(hip):
    with pytest.raises(hip.InvalidArgument):
        q(hip, 0, 0, 0, 3, 0)


@pytest.mark.parametrize("args,msg", [
    ((4, 0, 0, 0, 1, 32, 4), "weights must be"),      # matmul_rejects_shape_mismatch (:454-459)
    ((4, 4 * 34, 31, 1, 1, 32, 4), "xq must be"),
    ((4, 4 * 34, 32, 2, 1, 32, 4), "xscale must be"),
    ((5, 4 * 34, 32, 1, 1, 32, 4), "out must be"),
    ((8, 4 * 2 * 34, 64, 2, 1, 40, 4), "out must be"),  # in_dim 40 -> 2 blocks per row
])
def test_matmul_shape_errors_in_order(hip, args, msg):
    with pytest.raises(hip.ShapeMismatch, match=msg):
        m(hip, *args)


def test_matmul_zero_out_dim_panics_in_reference(hip):
    with pytest.raises(hip.InvalidArgument):
        m(hip, 0, 0, 32, 1, 1, 32, 0)
