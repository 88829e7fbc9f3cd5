"""Pins the oracle's Q8_0 int8-activation restatement (orc_quantize_q8_0_*,
orc_dot_q8_0_row_scalar, orc_matmul_q8_0_batch; backend-cpu/src/ops/
q8_0.rs:42-263) before it is the GPU's parity reference:
- the reference's own tests in q8_0.rs:323-545 (tests/kats.py, shared with
  the GPU tests);
- closed forms that a plausible mistake fails: round half to even, the
  saturating cast of +-inf / NaN, exact integer sums with power-of-two
  scales, left-to-right block order, (ws * xs) * dot association, no FMA;
- invariants over seeded data: |q| <= 127 and the block maximum maps to
  +-127, reconstruction error <= d / 2, and the reference's validation
  order."""
import numpy as np
import pytest

import kats


def o_quantize(oracle):
    def q(x, n_tok, in_dim):
        return oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    return q


def o_matmul(oracle):
    def m(w, xq, xs, n_tok, in_dim, out_dim):
        return oracle.matmul_q8_0_batch(w, xq, xs, n_tok, in_dim, out_dim)
    return m


@pytest.mark.parametrize("kat", kats.q8_kats(), ids=lambda k: k[0])
def test_q8_kats(oracle, kat):
    kat[1](o_quantize(oracle), o_matmul(oracle))


def test_quantize_invariants(oracle):
    rng = np.random.default_rng(3)
    n_tok, in_dim = 4, 1000
    x = (rng.standard_normal(n_tok * in_dim) * rng.choice([1e-3, 1.0, 1e4], n_tok * in_dim)
         ).astype(np.float32)
    rc, q, s = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert rc == 0
    blocks = (in_dim + 31) // 32
    xp = np.zeros((n_tok, blocks * 32), np.float32)
    xp[:, :in_dim] = x.reshape(n_tok, in_dim)
    xb = xp.reshape(n_tok, blocks, 32)
    qb = q.reshape(n_tok, blocks, 32).astype(np.int32)
    sb = s.reshape(n_tok, blocks)
    amax = np.abs(xb).max(axis=2)
    assert np.array_equal(sb, (amax / np.float32(127.0)).astype(np.float32))
    assert np.all(np.abs(qb) <= 127)
    # the element of largest magnitude maps to +-127
    idx = np.abs(xb).argmax(axis=2)
    top = np.take_along_axis(qb, idx[..., None], axis=2)[..., 0]
    assert np.all(np.abs(top) == 127)
    err = np.abs(qb * sb[..., None].astype(np.float64) - xb)
    assert np.all(err <= sb[..., None] * (0.5 + 1e-5))
    # the zero-padded tail of the partial last block
    assert np.all(qb[:, -1, in_dim % 32:] == 0)


def test_quantize_validation_order(oracle):
    L = oracle.lib()
    x = np.zeros(64, np.float32)
    q = np.zeros(64, np.int8)
    s = np.zeros(2, np.float32)
    P = oracle._p
    assert L.orc_quantize_q8_0_batch(P(x), 63, P(q), 64, P(s), 2, 1, 64) == kats.SHAPE_MISMATCH
    assert oracle.last_detail()[0] == 1
    assert L.orc_quantize_q8_0_batch(P(x), 64, P(q), 63, P(s), 2, 1, 64) == kats.SHAPE_MISMATCH
    assert oracle.last_detail()[0] == 2
    assert L.orc_quantize_q8_0_batch(P(x), 64, P(q), 64, P(s), 3, 1, 64) == kats.SHAPE_MISMATCH
    assert oracle.last_detail()[0] == 3


def test_matmul_validation_order(oracle):
    L = oracle.lib()
    P = oracle._p
    w = np.zeros(2 * 2 * 34, np.uint8)
    xq = np.zeros(64, np.int8)
    xs = np.zeros(2, np.float32)
    out = np.zeros(2, np.float32)
    args = [P(out), 2, P(w), w.size, P(xq), 64, P(xs), 2, 1, 64, 2, 1]
    assert L.orc_matmul_q8_0_batch(*args) == 0
    for pos, bad, code in ((3, w.size - 1, 1), (5, 63, 2), (7, 1, 3), (1, 3, 4)):
        a = list(args)
        a[pos] = bad
        assert L.orc_matmul_q8_0_batch(*a) == kats.SHAPE_MISMATCH
        assert oracle.last_detail()[0] == code


def test_matmul_equals_dequantised_float64_within_order_error(oracle):
    """Against float64 over the same quantised operands: the only difference
    is f32 rounding of the products and the running sum."""
    rng = np.random.default_rng(11)
    n_tok, in_dim, out_dim = 3, 200, 7
    blocks = (in_dim + 31) // 32
    w = np.zeros(out_dim * blocks * 34, np.uint8)
    wq = rng.integers(-128, 128, (out_dim, blocks, 32)).astype(np.int8)
    ws = (rng.random((out_dim, blocks)) * 0.01).astype(np.float16)
    for o in range(out_dim):
        for b in range(blocks):
            w[(o * blocks + b) * 34:(o * blocks + b + 1) * 34] = kats.pack_q8_0(float(ws[o, b]), wq[o, b])
    x = rng.standard_normal(n_tok * in_dim).astype(np.float32)
    rc, xq, xs = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert rc == 0
    rc, out = oracle.matmul_q8_0_batch(w, xq, xs, n_tok, in_dim, out_dim)
    assert rc == 0
    xqb = xq.reshape(n_tok, blocks, 32).astype(np.float64)
    xqb[:, -1, in_dim % 32:] = 0
    want = np.einsum("tbk,obk,ob,tb->to", xqb, wq.astype(np.float64), ws.astype(np.float64),
                     xs.reshape(n_tok, blocks).astype(np.float64))
    assert np.abs(out.reshape(n_tok, out_dim) - want).max() <= 1e-6 * np.abs(want).max()
