"""The Q8_0 int8-activation path on the GPU (quantize_q8_0_batch,
matmul_q8_0_batch; backend-cpu/src/ops/q8_0.rs:95-129, :217-263) against the
oracle: BIT-EXACT (float32 bit patterns compared) for the quantiser's int8
codes and scales and for the matmul's outputs (same int32 block dots, same
(ws * xs) * dot products, same left-to-right f32 block sum), on the
reference's own tests, closed-form cases, ragged shapes (partial last block,
odd row and token counts), scale edge cases (non-finite, subnormal f16
scales, activations with subnormal block scales) and the attention
projection shapes 4096x4096 / 1024x4096 at batch 1..32."""
import numpy as np
import pytest

import kats
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu


def h_quantize(hip):
    def q(x, n_tok, in_dim):
        blocks = (in_dim + 31) // 32
        xq = np.full(n_tok * blocks * 32, 99, np.int8)
        sc = np.zeros(n_tok * blocks, np.float32)
        try:
            hip.quantize_q8_0_batch(np.ascontiguousarray(x, np.float32), xq, sc, n_tok, in_dim)
        except hip.Error as e:
            return e.status, xq, sc
        return 0, xq, sc
    return q


def h_matmul(hip):
    def m(w, xq, xs, n_tok, in_dim, out_dim):
        out = np.full(n_tok * out_dim, np.nan, np.float32)
        try:
            hip.matmul_q8_0_batch(out, np.ascontiguousarray(w, np.uint8),
                                  np.ascontiguousarray(xq, np.int8),
                                  np.ascontiguousarray(xs, np.float32), n_tok, in_dim, out_dim)
        except hip.Error as e:
            return e.status, out
        return 0, out
    return m


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("kat", kats.q8_kats(), ids=lambda k: k[0])
def test_q8_kats_on_gpu(hip, kat):
    kat[1](h_quantize(hip), h_matmul(hip))


def ragged_activations(n_tok, in_dim, seed):
    """~N(0,1) rows with some blocks scaled far down (subnormal block
    scales, overflowing inverses), up (1e30) and zeroed."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((n_tok, in_dim)).astype(np.float32)
    blocks = (in_dim + 31) // 32
    for t in range(n_tok):
        for b in range(blocks):
            r = g.random()
            sl = slice(32 * b, min(32 * b + 32, in_dim))
            if r < 0.05:
                x[t, sl] *= np.float32(1e-37)
            elif r < 0.10:
                x[t, sl] *= np.float32(1e-41)
            elif r < 0.13:
                x[t, sl] *= np.float32(1e30)
            elif r < 0.16:
                x[t, sl] = 0.0
    return x.reshape(-1)


@pytest.mark.parametrize("n_tok,in_dim", [(1, 32), (1, 20), (3, 100), (5, 4096), (32, 1000),
                                          (7, 7168), (2, 16416)])
def test_quantize_bit_exact(oracle, hip, n_tok, in_dim):
    x = ragged_activations(n_tok, in_dim, 100 + in_dim + n_tok)
    rc, want_q, want_s = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert rc == 0
    rc, got_q, got_s = h_quantize(hip)(x, n_tok, in_dim)
    assert rc == 0
    assert np.array_equal(got_q, want_q)
    assert same_bits(got_s, want_s)


def test_quantize_non_finite_in_one_token(hip):
    x = synth.activations(4, 256, 3).reshape(-1).copy()
    x[2 * 256 + 77] = np.inf
    with pytest.raises(hip.NonFiniteInput):
        hip.quantize_q8_0_batch(x, np.zeros(4 * 256, np.int8), np.zeros(32, np.float32), 4, 256)
    # the next call on the same thread starts clean
    x[2 * 256 + 77] = 0.5
    hip.quantize_q8_0_batch(x, np.zeros(4 * 256, np.int8), np.zeros(32, np.float32), 4, 256)


def q8_weights(out_dim, in_dim, seed, specials=False):
    """GGUF Q8_0 rows of the attention-projection statistics; partial last
    blocks carry garbage quant bytes past in_dim (ignored by the reference)."""
    g = np.random.default_rng(seed)
    blocks = (in_dim + 31) // 32
    w = synth.q8_0_blocks(g, out_dim * blocks)
    if specials:
        n = w.shape[0]
        pick = g.choice(n, size=min(n, max(4, n // 50)), replace=False)
        bits = g.choice(np.array([0x7E00, 0x7C00, 0xFC00, 0x0001, 0x8001, 0x0000, 0x7BFF, 0x03FF],
                                 np.uint16), size=pick.size)
        w[pick, 0] = bits & 0xFF
        w[pick, 1] = bits >> 8
    return w.reshape(-1)


@pytest.mark.parametrize("n_tok,in_dim,out_dim", [
    (1, 32, 1), (1, 64, 17), (2, 100, 3), (3, 4096, 33), (4, 1000, 16), (5, 7168, 48),
    (8, 256, 100), (9, 2048, 31), (16, 4096, 64), (32, 520, 129), (33, 4096, 20),
    (12, 14336, 40), (20, 100, 9), (64, 4096, 130), (17, 2080, 257), (7, 1500, 1025),
    (1, 14336, 4100), (1, 4000, 8200), (1, 1000, 4097)])
def test_matmul_bit_exact(oracle, hip, n_tok, in_dim, out_dim):
    w = q8_weights(out_dim, in_dim, 7 * in_dim + out_dim, specials=True)
    x = ragged_activations(n_tok, in_dim, in_dim + n_tok)
    rc, xq, xs = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert rc == 0
    xq = xq.copy()
    blocks = (in_dim + 31) // 32
    if in_dim % 32:
        # nonzero tails in the activation codes are ignored as well (:183-187)
        xq.reshape(n_tok, blocks, 32)[:, -1, in_dim % 32:] = 5
    rc, want = oracle.matmul_q8_0_batch(w, xq, xs, n_tok, in_dim, out_dim)
    assert rc == 0
    rc, got = h_matmul(hip)(w, xq, xs, n_tok, in_dim, out_dim)
    assert rc == 0
    assert same_bits(got, want), f"max diff {np.abs(got - want).max()}"


@pytest.mark.parametrize("out_dim", [4096, 1024])
@pytest.mark.parametrize("n_tok", [1, 2, 4, 8, 16, 32])
def test_attention_projection_shapes(oracle, hip, n_tok, out_dim):
    """Config C2 (Q8_0 attention projections, in_dim 4096, batch 1..32) end to
    end: quantise on the GPU, matmul on the GPU, both bit-exact."""
    in_dim = 4096
    w = q8_weights(out_dim, in_dim, 900 + out_dim)
    x = synth.activations(n_tok, in_dim, 40 + n_tok).reshape(-1)
    rc, gq, gs = h_quantize(hip)(x, n_tok, in_dim)
    assert rc == 0
    rc, oq, os_ = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert rc == 0 and np.array_equal(gq, oq) and same_bits(gs, os_)
    rc, got = h_matmul(hip)(w, gq, gs, n_tok, in_dim, out_dim)
    assert rc == 0
    rc, want = oracle.matmul_q8_0_batch(w, oq, os_, n_tok, in_dim, out_dim)
    assert rc == 0
    assert same_bits(got, want)


def test_device_entry_points_match_host(oracle, hip):
    import torch
    n_tok, in_dim, out_dim = 6, 1000, 70
    w = q8_weights(out_dim, in_dim, 5)
    x = ragged_activations(n_tok, in_dim, 6)
    blocks = (in_dim + 31) // 32
    dev = torch.device("cuda:0")
    dx = torch.from_numpy(x).to(dev)
    dq = torch.empty(n_tok * blocks * 32, dtype=torch.int8, device=dev)
    ds = torch.empty(n_tok * blocks, dtype=torch.float32, device=dev)
    st = torch.full((1,), 7, dtype=torch.int32, device=dev)
    dw_raw = torch.from_numpy(w).to(dev)
    dw = torch.empty_like(dw_raw)
    dout = torch.empty(n_tok * out_dim, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    # the device layout of the rows, in_dim rounded up to whole blocks
    hip.prepare_weights_dev(dw.data_ptr(), dw_raw.data_ptr(), w.size, G.Q8_0, blocks * 32, stream)
    hip.quantize_q8_0_batch_dev(dx.data_ptr(), dx.numel(), dq.data_ptr(), dq.numel(),
                                ds.data_ptr(), ds.numel(), n_tok, in_dim, st.data_ptr(), stream)
    hip.matmul_q8_0_batch_dev(dout.data_ptr(), dout.numel(), dw.data_ptr(), dw.numel(),
                              dq.data_ptr(), dq.numel(), ds.data_ptr(), ds.numel(), n_tok, in_dim,
                              out_dim, stream)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    rc, oq, os_ = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    assert np.array_equal(dq.cpu().numpy(), oq) and same_bits(ds.cpu().numpy(), os_)
    rc, want = oracle.matmul_q8_0_batch(w, oq, os_, n_tok, in_dim, out_dim)
    assert same_bits(dout.cpu().numpy(), want)
    # a non-finite input sets the status word
    dx[3 * in_dim + 5] = float("nan")
    hip.quantize_q8_0_batch_dev(dx.data_ptr(), dx.numel(), dq.data_ptr(), dq.numel(),
                                ds.data_ptr(), ds.numel(), n_tok, in_dim, st.data_ptr(), stream)
    torch.cuda.synchronize()
    assert int(st.item()) == 1


def test_registered_weights_are_used(oracle, hip):
    """A Q8_0 tensor registered for matmul_quant_f32 serves matmul_q8_0_batch
    from its resident device copy, with the same bit-exact result."""
    n_tok, in_dim, out_dim = 4, 2048, 96
    w = q8_weights(out_dim, in_dim, 77, specials=True)
    x = synth.activations(n_tok, in_dim, 78).reshape(-1)
    rc, xq, xs = oracle.quantize_q8_0_batch(x, n_tok, in_dim)
    rc, want = oracle.matmul_q8_0_batch(w, xq, xs, n_tok, in_dim, out_dim)
    hip.register_weights(w, G.Q8_0, in_dim)
    try:
        rc, got = h_matmul(hip)(w, xq, xs, n_tok, in_dim, out_dim)
        assert rc == 0 and same_bits(got, want)
    finally:
        hip.release_weights()


def test_zero_sized_calls(hip):
    # n_tok == 0: nothing to do; in_dim == 0 (matmul): zero blocks, out = 0.0
    hip.matmul_q8_0_batch(np.zeros(0, np.float32), np.zeros(4 * 2 * 34, np.uint8),
                          np.zeros(0, np.int8), np.zeros(0, np.float32), 0, 64, 4)
    out = np.full(6, 3.0, np.float32)
    hip.matmul_q8_0_batch(out, np.zeros(0, np.uint8), np.zeros(0, np.int8),
                          np.zeros(0, np.float32), 2, 0, 3)
    assert np.all(out == 0.0)
    hip.quantize_q8_0_batch(np.zeros(0, np.float32), np.zeros(0, np.int8),
                            np.zeros(0, np.float32), 0, 64)
