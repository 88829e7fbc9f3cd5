"""Dequantisation on the GPU is bit-exact with the oracle (the reference's
dequant_to_f32, rsllm-gguf/src/dequant/mod.rs:69-85) — on every block of the
benchmark configs and on blocks with special f16 scales."""
import numpy as np
import pytest

import kats
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

# Special f16 scale patterns: zero, -0, smallest subnormal, largest
# subnormal, smallest normal, 1.0, max finite, -max, +inf, -inf, qNaN.
SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00,
               0x7E00]


def assert_bits_equal(got: np.ndarray, want: np.ndarray):
    assert got.shape == want.shape
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), "NaN positions differ"
    g, w = got[~gn].view(np.uint32), want[~wn].view(np.uint32)
    bad = np.nonzero(g != w)[0]
    assert bad.size == 0, f"{bad.size} elements differ, first at {bad[:5]}: {got[~gn][bad[:5]]} vs {want[~wn][bad[:5]]}"


# Special f32 scale patterns (Q8_K's d): zero, -0, smallest subnormal,
# smallest normal, 1.0, max finite, +inf, -inf, qNaN, and a value whose
# products with int8 codes round.
SPECIAL_F32 = [0x00000000, 0x80000000, 0x00000001, 0x00800000, 0x3F800000, 0x7F7FFFFF,
               0x7F800000, 0xFF800000, 0x7FC00000, 0x3DCCCCCD]


def special_blocks(dtype, n_per=4, seed=7):
    be, bb = {G.Q4_K: (256, 144), G.Q6_K: (256, 210), G.Q8_0: (32, 34), G.Q2_K: (256, 84),
              G.IQ2_XXS: (256, 66), G.Q4_1: (32, 20), G.Q5_K: (256, 176),
              G.Q8_K: (256, 292)}[dtype]
    if dtype == G.Q8_K:
        blocks = synth.weight(dtype, len(SPECIAL_F32) * n_per, be, seed).reshape(-1, bb).copy()
        for i, pat in enumerate(SPECIAL_F32):
            for r in range(n_per):
                blocks[i * n_per + r, 0:4] = np.frombuffer(np.uint32(pat).tobytes(), np.uint8)
        return blocks.reshape(-1)
    blocks = synth.weight(dtype, len(SPECIAL_F16) * n_per, be, seed).reshape(-1, bb).copy()
    for i, pat in enumerate(SPECIAL_F16):
        for r in range(n_per):
            row = blocks[i * n_per + r]
            lo, hi = pat & 0xFF, pat >> 8
            if dtype in (G.Q4_K, G.Q4_1, G.Q5_K):
                row[0], row[1] = lo, hi                          # d
                p2 = SPECIAL_F16[(i + r + 1) % len(SPECIAL_F16)]
                row[2], row[3] = p2 & 0xFF, p2 >> 8              # dmin / m
            elif dtype == G.Q6_K:
                row[208], row[209] = lo, hi
            elif dtype == G.Q2_K:
                row[80], row[81] = lo, hi                        # d
                p2 = SPECIAL_F16[(i + r + 1) % len(SPECIAL_F16)]
                row[82], row[83] = p2 & 0xFF, p2 >> 8            # dmin
            else:
                row[0], row[1] = lo, hi
    return blocks.reshape(-1)


@pytest.mark.parametrize("dtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K, G.IQ2_XXS, G.Q4_1, G.Q5_K,
                                   G.Q8_K])
def test_dequant_special_scales_bit_exact(oracle, hip, dtype):
    src = special_blocks(dtype)
    n = src.size // dtype.block_bytes() * dtype.block_elements()
    rc, want = oracle.dequant(int(dtype), src, n)
    assert rc == 0
    got = np.empty(n, np.float32)
    hip.dequant_to_f32(dtype, src, got)
    assert_bits_equal(got, want)


# (dtype, out_dim, in_dim) of every benchmark weight matrix.
CONFIG_MATRICES = [
    (G.Q4_K, 4096, 4096),     # C0
    (G.Q6_K, 14336, 4096),    # C1
    (G.Q6_K, 4096, 14336),    # C1
    (G.Q8_0, 4096, 4096),     # C2 Q/O
    (G.Q8_0, 1024, 4096),     # C2 K/V
    (G.Q4_K, 2048, 7168),     # C3 gate/up (one expert)
    (G.Q4_K, 7168, 2048),     # C3 down (one expert)
    (G.Q4_K, 14336, 4096),    # C4
    (G.Q2_K, 7168, 2048),     # a DS-V4-Flash-style routed down expert
    (G.IQ2_XXS, 2048, 7168),  # a DS-V4-Flash-style routed gate/up expert
]


@pytest.mark.parametrize("dtype,out_dim,in_dim", CONFIG_MATRICES)
def test_dequant_config_matrix_bit_exact(oracle, hip, dtype, out_dim, in_dim):
    src = synth.weight(dtype, out_dim, in_dim, seed=1000 + out_dim + in_dim)
    n = out_dim * in_dim
    rc, want = oracle.dequant(int(dtype), src, n)
    assert rc == 0
    got = np.empty(n, np.float32)
    hip.dequant_to_f32(dtype, src, got)
    assert_bits_equal(got, want)
    # f16-subnormal scales are present in this data (about 5% of blocks).
    if dtype in (G.Q4_K, G.Q6_K):
        off = 0 if dtype == G.Q4_K else 208
        d = src.reshape(-1, dtype.block_bytes())[:, off:off + 2].copy().view(np.uint16).reshape(-1)
        assert ((d & 0x7C00) == 0).mean() > 0.01


@pytest.mark.parametrize("dtype,n", [(G.Q4_1, 7168 * 64), (G.Q5_K, 7168 * 256),
                                     (G.Q8_K, 4096 * 256)])
def test_dequant_remaining_k_arms_bit_exact(oracle, hip, dtype, n):
    """Q4_1, Q5_K and Q8_K (dequant/mod.rs:76,78,82; off the matmul path:
    q4_0.rs:66-87, q5_k.rs:34-94, q8_k.rs:32-70) over seeded blocks."""
    src = synth.weight(dtype, n // 4096, 4096, seed=1200 + int(dtype))
    rc, want = oracle.dequant(int(dtype), src, n)
    assert rc == 0
    got = np.empty(n, np.float32)
    hip.dequant_to_f32(dtype, src, got)
    assert_bits_equal(got, want)


@pytest.mark.parametrize("dtype", [G.F32, G.F16, G.BF16, G.Q4_0])
def test_dequant_other_arms_bit_exact(oracle, hip, dtype):
    g = synth.rng(5)
    n = 4096
    src = g.integers(0, 256, size=dtype.byte_size(n), dtype=np.uint8)
    rc, want = oracle.dequant(int(dtype), src, n)
    assert rc == 0
    got = np.empty(n, np.float32)
    hip.dequant_to_f32(dtype, src, got)
    assert_bits_equal(got, want)


def test_dequant_dev_entry_point(oracle, hip):
    import torch
    src = synth.weight(G.Q6_K, 64, 512, seed=3)
    n = 64 * 512
    rc, want = oracle.dequant(int(G.Q6_K), src, n)
    d_src = torch.from_numpy(src).cuda()
    d_dst = torch.empty(n, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    hip.dequant_to_f32_dev(G.Q6_K, d_src.data_ptr(), src.size, d_dst.data_ptr(), n, stream)
    torch.cuda.synchronize()
    assert_bits_equal(d_dst.cpu().numpy(), want)


@pytest.mark.parametrize("kat", [k for k in kats.dequant_kats()
                                 if k[1] in (kats.Q2_K, kats.IQ2_XXS, kats.Q4_1, kats.Q5_K, kats.Q8_K)],
                         ids=lambda k: k[0])
def test_reference_q2k_iq2xxs_kats_on_gpu(hip, kat):
    """The reference's Q2_K / IQ2_XXS / Q4_1 / Q5_K / Q8_K dequant tests
    (q2_k.rs:171-272, iq2_xxs.rs:188-399, q4_0.rs:184-213, q5_k.rs:166-228,
    q8_k.rs:94-163, dequant/mod.rs:165-304) through librsllm_hip.so."""
    name, dtype, src, n, check = kat
    got = np.empty(n, np.float32)
    try:
        hip.dequant_to_f32(dtype, src, got)
        rc = 0
    except hip.Error as e:
        rc = e.status
    check(rc, got)
