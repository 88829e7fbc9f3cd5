"""Seeded synthetic GGUF tensors and activations for the benchmark configs.

Block statistics follow the workload definitions the benchmark is quoted on:

* Q4_K (256 elements / 144 B): ``d``, ``dmin`` = f16(|N(0, 1e-3)|); 8 scales
  and 8 mins uniform 0..63 packed into 12 bytes by the inverse of
  ``q4_k_scale_min`` (rsllm-gguf/src/dequant/mod.rs:48-58; the reference's own
  inverse is ``pack_scales``, q4_k.rs:100-124); 128 uniform random ``qs`` bytes.
* Q6_K (256 / 210 B): ``ql``/``qh`` uniform random bytes; 16 int8 scales
  uniform -64..63; ``d`` = f16(|N(0, 1e-3)|) at byte 208.
* Q8_0 (32 / 34 B): ``d`` = f16(|N(0, 1e-2)|); 32 int8 uniform -127..127.
* activations fp32 N(0, 1); prefill activations bf16(N(0, 1)).

Everything derives from ``numpy.random.Generator(PCG64(seed))`` so a seed
reproduces the same bytes on every host.
"""
from __future__ import annotations

import numpy as np

from .ggml import GgmlType


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _f16_abs_normal(g: np.random.Generator, n: int, sigma: float) -> np.ndarray:
    return np.abs(g.normal(0.0, sigma, n)).astype(np.float16)


def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack [n, 8] 6-bit scales and mins into [n, 12] bytes.

    Inverse of ``q4_k_scale_min``: j < 4 keeps sc/m in the low 6 bits of
    bytes j / j+4; j >= 4 puts the low nibbles in byte j+4 and the top two
    bits in bits 6-7 of bytes j-4 (scale) and j (min).
    """
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    q = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    q[:, 0:4] = sc[:, 0:4]
    q[:, 4:8] = m[:, 0:4]
    q[:, 8:12] = (m[:, 4:8] & 0x0F) << 4 | (sc[:, 4:8] & 0x0F)
    q[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    q[:, 4:8] |= (m[:, 4:8] >> 4) << 6
    return q


def q4k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 144] uint8 Q4_K super-blocks with the documented statistics."""
    out = np.empty((n_blocks, 144), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    sc = g.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    mn = g.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    out[:, 4:16] = pack_q4k_scales(sc, mn)
    out[:, 16:144] = g.integers(0, 256, size=(n_blocks, 128), dtype=np.uint8)
    return out


def q6k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 210] uint8 Q6_K super-blocks with the documented statistics."""
    out = np.empty((n_blocks, 210), dtype=np.uint8)
    out[:, 0:192] = g.integers(0, 256, size=(n_blocks, 192), dtype=np.uint8)
    out[:, 192:208] = g.integers(-64, 64, size=(n_blocks, 16), dtype=np.int8).view(np.uint8)
    out[:, 208:210] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    return out


def q8_0_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 34] uint8 Q8_0 blocks with the documented statistics."""
    out = np.empty((n_blocks, 34), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-2).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:34] = g.integers(-127, 128, size=(n_blocks, 32), dtype=np.int8).view(np.uint8)
    return out


def q4_0_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 18] uint8 Q4_0 blocks: d = f16(|N(0, 1e-2)|), 16 random qs bytes."""
    out = np.empty((n_blocks, 18), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-2).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:18] = g.integers(0, 256, size=(n_blocks, 16), dtype=np.uint8)
    return out


def q2k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 84] uint8 Q2_K blocks: 16 scale bytes (4-bit scale, 4-bit
    min) and 64 qs bytes uniform; d, dmin = f16(|N(0, 1e-3)|)."""
    out = g.integers(0, 256, size=(n_blocks, 84), dtype=np.uint8)
    out[:, 80:82] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    out[:, 82:84] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    return out


def iq2xxs_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 66] uint8 IQ2_XXS blocks: d = f16(|N(0, 1e-3)|), grid
    indices, 7-bit sign indices and 4-bit extras uniform."""
    out = g.integers(0, 256, size=(n_blocks, 66), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    return out


def q4_1_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 20] uint8 Q4_1 blocks: d = f16(|N(0, 1e-2)|), m = f16(N(0,
    1e-2)), 16 random code bytes."""
    out = g.integers(0, 256, size=(n_blocks, 20), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-2).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = (g.standard_normal(n_blocks) * 1e-2).astype(np.float16).view(np.uint8).reshape(n_blocks, 2)
    return out


def q5k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 176] uint8 Q5_K blocks: d, dmin = f16(|N(0, 1e-3)|), scale
    bytes, qh and qs uniform."""
    out = g.integers(0, 256, size=(n_blocks, 176), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = _f16_abs_normal(g, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    return out


def q8k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    """[n_blocks, 292] uint8 Q8_K blocks: d = f32(|N(0, 1e-2)|), qs and bsums
    uniform."""
    out = g.integers(0, 256, size=(n_blocks, 292), dtype=np.uint8)
    out[:, 0:4] = np.abs(g.standard_normal(n_blocks) * 1e-2).astype(np.float32).view(np.uint8).reshape(n_blocks, 4)
    return out


_BLOCKS = {GgmlType.Q4_K: q4k_blocks, GgmlType.Q6_K: q6k_blocks, GgmlType.Q8_0: q8_0_blocks,
           GgmlType.Q4_0: q4_0_blocks, GgmlType.Q2_K: q2k_blocks, GgmlType.IQ2_XXS: iq2xxs_blocks,
           GgmlType.Q4_1: q4_1_blocks, GgmlType.Q5_K: q5k_blocks, GgmlType.Q8_K: q8k_blocks}


def weight(dtype: GgmlType, out_dim: int, in_dim: int, seed: int) -> np.ndarray:
    """Row-major GGUF weight [out_dim x in_dim] as a flat uint8 array."""
    dtype = GgmlType(dtype)
    be = dtype.block_elements()
    if in_dim % be:
        raise ValueError(f"in_dim {in_dim} is not a multiple of {be}")
    n_blocks = out_dim * (in_dim // be)
    return _BLOCKS[dtype](rng(seed), n_blocks).reshape(-1)


def q6k_full_scales(w: np.ndarray, seed: int) -> np.ndarray:
    """A copy of a Q6_K weight with its 16 int8 scales per block redrawn from
    the full int8 range -128..127 (what GGUF files hold; the benchmark's
    statistics stop at -64..63), sc = -128 and 127 present in every block."""
    b = np.array(w, dtype=np.uint8).reshape(-1, 210)
    sc = rng(seed).integers(-128, 128, size=(b.shape[0], 16), dtype=np.int16).astype(np.int8)
    sc[:, 0], sc[:, 15] = -128, 127
    b[:, 192:208] = sc.view(np.uint8)
    return b.reshape(-1)


def activations(n_tok: int, dim: int, seed: int) -> np.ndarray:
    """fp32 N(0, 1) activations [n_tok x dim]."""
    return rng(seed).standard_normal((n_tok, dim), dtype=np.float32)


def bf16_activations(n_tok: int, dim: int, seed: int) -> np.ndarray:
    """bf16(N(0, 1)) activations [n_tok x dim] as uint16 bit patterns (RNE)."""
    x = activations(n_tok, dim, seed)
    return f32_to_bf16_bits(x)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bits (no NaNs expected)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = b + 0x7FFF + ((b >> 16) & 1)
    return (rounded >> 16).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def moe_routing(n_tok: int, n_expert: int, k: int, seed: int):
    """Top-k expert ids drawn uniformly without replacement per token, and
    softmax-normalised fp32 weights over k N(0, 1) logits."""
    g = rng(seed)
    ids = np.stack([g.choice(n_expert, size=k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    logits = g.standard_normal((n_tok, k)).astype(np.float32)
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    w = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.reshape(n_tok, k), w.reshape(n_tok, k)
