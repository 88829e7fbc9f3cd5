"""Pins the CPU oracle before it is trusted as the parity reference.

Each check is chosen so that a plausible transcription mistake (a swapped
nibble, a wrong scale index, a dropped min term, a reassociated sum) fails:
the reference's own known-answer tests, brute force over every scale pattern
and every f16 bit pattern, an independent numpy restatement over every block
of seeded data, float64 recomputation, and invariants of the algorithm.
"""
import numpy as np
import pytest

import kats
from conftest import rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G


@pytest.mark.parametrize("kat", kats.dequant_kats(), ids=lambda k: k[0])
def test_reference_dequant_kats(oracle, kat):
    name, dtype, src, n, check = kat
    rc, got = oracle.dequant(dtype, src, n)
    check(rc, got)


def test_size_mismatch_details(oracle):
    # q8_0.rs:149-163 asserts src_bytes = 33, expected_bytes = 34.
    rc, _ = oracle.dequant(kats.Q8_0, np.zeros(33, np.uint8), 32)
    assert rc == oracle.DEQUANT_SIZE_MISMATCH
    assert oracle.last_detail() == (33, 34)
    # q4_k.rs:36-41: a partial block reports ceil(n/256)*144.
    rc, _ = oracle.dequant(kats.Q4_K, np.zeros(144, np.uint8), 128)
    assert oracle.last_detail() == (144, 144)


def test_f16_widening_all_bit_patterns(oracle):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    # NaN: quiet bit set, payload kept, sign kept.
    nan_bits = got[~fin].view(np.uint32)
    hb = h[~fin].astype(np.uint32)
    assert np.array_equal(nan_bits, ((hb >> 15) << 31) | 0x7FC00000 | ((hb & 0x3FF) << 13))


def test_q4k_scale_min_brute_force(oracle):
    # Every (sc, m) pair of 6-bit values in every sub-block position j,
    # packed by the reference's inverse packer (q4_k.rs:100-124).
    vals = np.arange(64)
    for j in range(8):
        for sc in vals:
            base_sc = [(j + 5 * i) % 64 for i in range(8)]
            base_m = [(3 * j + 7 * i) % 64 for i in range(8)]
            for m in (0, 1, 31, 32, 63, int(sc)):
                s, mm = list(base_sc), list(base_m)
                s[j], mm[j] = int(sc), m
                q = kats.pack_scales(s, mm)
                for jj in range(8):
                    assert oracle.q4k_scale_min(jj, q) == (s[jj], mm[jj])


def test_np_scale_min_matches_oracle_all_12bit_pairs(oracle):
    # The numpy unpacker (used by the independent restatement) against the
    # oracle on random 12-byte patterns covering every byte value.
    g = synth.rng(2)
    q = g.integers(0, 256, size=(4096, 12), dtype=np.uint8)
    sc, m = oracle.np_scale_min(q)
    for i in range(0, 4096, 37):
        for j in range(8):
            assert oracle.q4k_scale_min(j, q[i]) == (sc[i, j], m[i, j])


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS, G.Q4_1, G.Q5_K,
                                   G.Q8_K])
def test_oracle_matches_independent_numpy_restatement(oracle, dtype):
    w = synth.weight(dtype, 512, 4096, seed=int(dtype))
    n = 512 * 4096
    rc, got = oracle.dequant(int(dtype), w, n)
    assert rc == 0
    want = oracle.NP_DEQUANT[int(dtype)](w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4k_closed_form_invariants(oracle):
    g = synth.rng(9)
    blocks = synth.q4k_blocks(g, 64)
    # dmin = 0 => value = d*sc*q exactly; q = 0 => value = -dmin*m.
    b0 = blocks.copy()
    b0[:, 2:4] = 0
    rc, v = oracle.dequant(kats.Q4_K, b0.reshape(-1), 64 * 256)
    d = b0[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1, 1)
    sc, m = oracle.np_scale_min(b0[:, 4:16])
    qs = b0[:, 16:].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float64)
    assert np.array_equal(v.reshape(-1, 8, 32).astype(np.float64), d * sc[:, :, None] * q)
    b1 = blocks.copy()
    b1[:, 16:] = 0
    rc, v = oracle.dequant(kats.Q4_K, b1.reshape(-1), 64 * 256)
    dmin = b1[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1, 1, 1)
    sc, m = oracle.np_scale_min(b1[:, 4:16])
    assert np.array_equal(v.reshape(-1, 8, 32).astype(np.float64),
                          np.broadcast_to(-(dmin * m[:, :, None]), (64, 8, 32)))


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q4_0, G.Q2_K, G.IQ2_XXS])
def test_matmul_equals_dequant_then_float64_dot(oracle, dtype):
    out_dim, in_dim, n_tok = 37, 1024, 3
    if dtype == G.Q4_0:
        g = synth.rng(4)
        w = g.integers(0, 256, size=(out_dim * in_dim // 32, 18), dtype=np.uint8)
        w[:, 0:2] = np.abs(g.normal(0, 1e-2, (w.shape[0], 1))).astype(np.float16).view(np.uint8)
        w = w.reshape(-1)
    else:
        w = synth.weight(dtype, out_dim, in_dim, 4)
    x = synth.activations(n_tok, in_dim, 5)
    rc, out = oracle.matmul_quant_f32(w, x, n_tok, in_dim, out_dim, int(dtype))
    assert rc == 0
    rc, wd = oracle.dequant(int(dtype), w, out_dim * in_dim)
    ref = x.astype(np.float64) @ wd.reshape(out_dim, in_dim).astype(np.float64).T
    # A sequential fp32 dot of 1024 terms: error ~ n * eps * sum|w x|.
    bound = in_dim * 2 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(wd.reshape(out_dim, in_dim)).T)
    assert np.all(np.abs(out.reshape(n_tok, out_dim) - ref) <= bound)
    assert rel_err(out, ref.reshape(-1)) < 1e-5


def test_matmul_is_sequential_f32_dot(oracle):
    # Bit-for-bit the reference's loop: dot += w[i] * x[i], in i order, no FMA.
    w = synth.weight(G.Q8_0, 5, 256, 6)
    x = synth.activations(2, 256, 7)
    rc, out = oracle.matmul_quant_f32(w, x, 2, 256, 5, kats.Q8_0)
    rc, wd = oracle.dequant(kats.Q8_0, w, 5 * 256)
    wd = wd.reshape(5, 256)
    for t in range(2):
        for o in range(5):
            acc = np.float32(0)
            for i in range(256):
                acc = np.float32(acc + np.float32(wd[o, i] * x[t, i]))
            assert out[t * 5 + o] == acc


def test_matmul_thread_count_invariant(oracle):
    w = synth.weight(G.Q4_K, 64, 512, 8)
    x = synth.activations(7, 512, 9)
    outs = [oracle.matmul_quant_f32(w, x, 7, 512, 64, kats.Q4_K, n_threads=t)[1] for t in (1, 2, 7)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_matmul_error_order(oracle):
    # quant_matmul.rs:57-92: dtype, in_dim % block, weights, x, out; then the
    # row_len > 0 assertion of parallel.rs:44.
    O = oracle
    rc, _ = O.matmul_quant_f32(np.zeros(0, np.uint8), np.zeros(0, np.float32), 1, 32, 4, kats.F16, allow_q6k=False, out_len=4)
    assert rc == O.SHAPE_MISMATCH  # rejects_unsupported_dtype (:156-170)
    rc, _ = O.matmul_quant_f32(np.zeros(0, np.uint8), np.zeros(0, np.float32), 1, 30, 4, kats.Q4_0, out_len=4)
    assert rc == O.NOT_BLOCK_ALIGNED and O.last_detail() == (30, 32)  # rejects_unaligned_in_dim
    rc, _ = O.matmul_quant_f32(np.zeros(0, np.uint8), np.zeros(0, np.float32), 1, 256, 4, kats.Q6_K, allow_q6k=False, out_len=4)
    assert rc == O.SHAPE_MISMATCH  # Q6_K is outside the reference's guard
    rc, _ = O.matmul_quant_f32(np.zeros(10, np.uint8), np.zeros(32, np.float32), 1, 32, 4, kats.Q8_0, out_len=4)
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 1
    rc, _ = O.matmul_quant_f32(np.zeros(136, np.uint8), np.zeros(31, np.float32), 1, 32, 4, kats.Q8_0, out_len=4)
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 2
    rc, _ = O.matmul_quant_f32(np.zeros(136, np.uint8), np.zeros(32, np.float32), 1, 32, 4, kats.Q8_0, out_len=3)
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 3
    rc, _ = O.matmul_quant_f32(np.zeros(0, np.uint8), np.zeros(32, np.float32), 1, 32, 0, kats.Q8_0, out_len=0)
    assert rc == O.PANIC


def test_reference_q4_0_matmul_kat(oracle):
    # quant_matmul.rs:189-248 q4_0_matmul_matches_naive_within_tolerance.
    wq, x, n_tok, in_dim, out_dim = kats.q4_0_matmul_case()
    rc, out = oracle.matmul_quant_f32(wq, x, n_tok, in_dim, out_dim, kats.Q4_0)
    assert rc == 0
    rc, wd = oracle.dequant(kats.Q4_0, wq, out_dim * in_dim)
    wd = wd.reshape(out_dim, in_dim)
    for t in range(n_tok):
        for o in range(out_dim):
            want = np.float32(0)
            for i in range(in_dim):
                want = np.float32(want + np.float32(wd[o, i] * x[t * in_dim + i]))
            got = out[t * out_dim + o]
            assert abs(got - want) < 1e-4 * max(abs(want), 1.0)


def test_iq2xxs_codebook(oracle):
    """The IQ2_XXS grid (iq2_xxs/tables.rs) against the reference's own
    assertions (iq2_xxs.rs:165-186 and the decoded entries 0-4 quoted in its
    tests, :248-389), plus invariants a transcription slip would break: 256
    distinct entries, every byte in {8, 25, 43}, ascending as u64."""
    g = [oracle.lib().orc_iq2xxs_grid(i) for i in range(256)]
    assert g[0] == 0x0808080808080808
    assert g[1] == 0x080808080808082B
    assert g[2] == 0x0808080808081919
    assert g[3] == 0x0808080808082B08
    assert g[4] == 0x0808080808082B2B
    assert g[255] == 0x2B2B2B1908081908
    assert len(set(g)) == 256
    assert all(g[i] < g[i + 1] for i in range(255))
    b = np.array(g, np.uint64).view(np.uint8)
    assert set(b.tolist()) <= {8, 25, 43}


def test_q2k_closed_form_invariants(oracle):
    """dmin = 0 => (d * sc) * q exactly; all codes 0 => -(dmin * m)."""
    g = synth.rng(21)
    blocks = synth.q2k_blocks(g, 32)
    b0 = blocks.copy()
    b0[:, 82:84] = 0
    rc, v = oracle.dequant(kats.Q2_K, b0.reshape(-1), 32 * 256)
    assert rc == 0
    d = b0[:, 80:82].copy().view(np.float16).astype(np.float64)
    e = np.arange(256)
    sc = (b0[:, e // 16] & 15).astype(np.float64)
    q = ((b0[:, 16 + 32 * (e // 128) + e % 32] >> (2 * ((e % 128) // 32))) & 3).astype(np.float64)
    assert np.array_equal(v.reshape(32, 256).astype(np.float64), d * sc * q)
    b1 = blocks.copy()
    b1[:, 16:80] = 0
    rc, v = oracle.dequant(kats.Q2_K, b1.reshape(-1), 32 * 256)
    dmin = b1[:, 82:84].copy().view(np.float16).astype(np.float64)
    m = (b1[:, e // 16] >> 4).astype(np.float64)
    assert np.array_equal(v.reshape(32, 256).astype(np.float64), -(dmin * m) + 0.0)
