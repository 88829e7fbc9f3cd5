"""The reference's known-answer tests for this path, as data.

Each KAT builds its input with a block packer (the inverse of the decoder,
as the reference's own tests do) and states the expected values in closed
form, exactly as the cited reference test does. The same KATs run against
the oracle (CPU) and against librsllm_hip.so (GPU), so both are pinned to
the reference's own expectations.

A ``dequant`` callable has the signature ``dequant(dtype, src_bytes, n) ->
(status, float32[n])``.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q6_K, F32, F16, BF16, Q3_K = 2, 8, 12, 14, 0, 1, 30, 11
DEQUANT_SIZE_MISMATCH, UNSUPPORTED_DEQUANT = 5, 6


def f16_bytes(v: float) -> bytes:
    return np.float16(v).tobytes()  # round-to-nearest-even, as half::f16::from_f32


# --- packers (inverses of the decoders) -------------------------------------

def pack_scales(sc, m) -> np.ndarray:
    """Inverse of q4_k_scale_min (the reference's pack_scales, q4_k.rs:100-124)."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = sc[j]
        q[j + 4] = m[j]
    for j in range(4, 8):
        q[j + 4] = ((m[j] & 15) << 4) | (sc[j] & 15)
        q[j - 4] |= ((sc[j] >> 4) & 3) << 6
        q[j] |= ((m[j] >> 4) & 3) << 6
    return q


def pack_q4k(d, dmin, sc, m, nibbles) -> np.ndarray:
    """One Q4_K block: low nibble of qs[32k + l] = element 64k + l, high
    nibble = element 64k + 32 + l (q4_k.rs:127-146)."""
    nib = np.asarray(nibbles, np.uint8).reshape(4, 2, 32)
    qs = (nib[:, 1, :] << 4) | (nib[:, 0, :] & 15)
    return np.concatenate([np.frombuffer(f16_bytes(d) + f16_bytes(dmin), np.uint8),
                           pack_scales(sc, m), qs.reshape(-1).astype(np.uint8)])


def pack_q6k(q6, scales, d) -> np.ndarray:
    """One Q6_K block from 256 6-bit values (q6_k.rs:112-155)."""
    q6 = np.asarray(q6, np.uint8)
    out = np.zeros(210, np.uint8)
    for h in range(2):
        for l in range(32):
            v1, v2, v3, v4 = (int(q6[h * 128 + l + 32 * i]) for i in range(4))
            out[h * 64 + l] = (v1 & 15) | ((v3 & 15) << 4)
            out[h * 64 + l + 32] = (v2 & 15) | ((v4 & 15) << 4)
            out[128 + h * 32 + l] = ((v1 >> 4) & 3) | (((v2 >> 4) & 3) << 2) | \
                (((v3 >> 4) & 3) << 4) | (((v4 >> 4) & 3) << 6)
    out[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    out[208:210] = np.frombuffer(f16_bytes(d), np.uint8)
    return out


def pack_q8_0(d, qs) -> np.ndarray:
    return np.concatenate([np.frombuffer(f16_bytes(d), np.uint8),
                           np.asarray(qs, np.int8).view(np.uint8)])


def pack_q4_0(d, nibbles) -> np.ndarray:
    nib = np.asarray(nibbles, np.uint8)
    qs = ((nib[16:32] & 15) << 4) | (nib[0:16] & 15)
    return np.concatenate([np.frombuffer(f16_bytes(d), np.uint8), qs.astype(np.uint8)])


def pack_q4_0_row(x: np.ndarray) -> np.ndarray:
    """The reference's Q4_0 row quantizer used by its matmul test
    (quant_matmul.rs:130-153): d = amax / -8, q = clamp(floor(x/d + 8.5))."""
    x = np.asarray(x, np.float32)
    out = []
    for b in range(x.size // 32):
        blk = x[b * 32:(b + 1) * 32]
        amax = np.float32(np.abs(blk).max())
        d = np.float32(amax / np.float32(-8.0))
        idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        q = np.clip(np.floor(blk * idv + np.float32(8.5)).astype(np.int32), 0, 15).astype(np.uint8)
        out.append(np.concatenate([np.frombuffer(f16_bytes(d), np.uint8),
                                   (q[0:16] | (q[16:32] << 4)).astype(np.uint8)]))
    return np.concatenate(out)


# --- dequant KATs: (name, dtype, src, n, check) -------------------------------
# check(status, values) raises AssertionError on mismatch.

def _close(want, tol):
    want = np.asarray(want, np.float32)

    def check(rc, got):
        assert rc == 0, f"status {rc}"
        assert np.all(np.abs(got - want) < tol), f"max diff {np.abs(got - want).max()}"
    return check


def _status(code):
    def check(rc, got):
        assert rc == code, f"status {rc}, want {code}"
    return check


def dequant_kats():
    k = []
    # q4_k.rs:167-188 zero_quants_yields_minus_min_per_subblock
    m = list(range(1, 9))
    k.append(("q4k_zero_quants_minus_min", Q4_K, pack_q4k(1.0, 1.0, [0] * 8, m, [0] * 256), 256,
              _close(np.repeat(-np.array(m, np.float32), 32), 1e-3)))
    # q4_k.rs:190-209 distinct_sub_block_scales
    sc = list(range(1, 9))
    k.append(("q4k_distinct_sub_block_scales", Q4_K, pack_q4k(1.0, 0.0, sc, [0] * 8, [1] * 256),
              256, _close(np.repeat(np.array(sc, np.float32), 32), 1e-2)))
    # q4_k.rs:211-230 linear_with_offset_combined
    nib = [i % 16 for i in range(256)]
    k.append(("q4k_linear_with_offset", Q4_K, pack_q4k(0.5, 0.25, [4] * 8, [2] * 8, nib), 256,
              _close(2.0 * np.array(nib, np.float32) - 0.5, 1e-2)))
    # q4_k.rs:232-250 size errors
    k.append(("q4k_wrong_src_size", Q4_K, np.zeros(143, np.uint8), 256, _status(DEQUANT_SIZE_MISMATCH)))
    k.append(("q4k_partial_block_dst", Q4_K, np.zeros(144, np.uint8), 128, _status(DEQUANT_SIZE_MISMATCH)))
    # q6_k.rs:163-172 zero_quants_yields_zero
    k.append(("q6k_zero_quants", Q6_K, pack_q6k([32] * 256, [5] * 16, 1.0), 256,
              _close(np.zeros(256), 1e-3)))
    # q6_k.rs:174-192 unit_scale_centered_dequant
    q6 = [i % 64 for i in range(256)]
    k.append(("q6k_unit_scale_centered", Q6_K, pack_q6k(q6, [1] * 16, 1.0), 256,
              _close(np.array(q6, np.float32) - 32.0, 1e-3)))
    # q6_k.rs:194-203 negative_scales_invert_sign
    k.append(("q6k_negative_scales", Q6_K, pack_q6k([33] * 256, [-1] * 16, 1.0), 256,
              _close(-np.ones(256), 1e-3)))
    # q6_k.rs:205-228 distinct_per_sub_block_scales
    k.append(("q6k_distinct_scales", Q6_K, pack_q6k([33] * 256, list(range(1, 17)), 1.0), 256,
              _close(np.repeat(np.arange(1, 17, dtype=np.float32), 16), 1e-3)))
    # q6_k.rs:230-254 distinct_per_sub_block_quants
    q6 = [2 * (i // 16) for i in range(256)]
    k.append(("q6k_distinct_quants", Q6_K, pack_q6k(q6, [1] * 16, 1.0), 256,
              _close(np.array(q6, np.float32) - 32.0, 1e-3)))
    # q6_k.rs:256-264 wrong_src_size_errors
    k.append(("q6k_wrong_src_size", Q6_K, np.zeros(209, np.uint8), 256, _status(DEQUANT_SIZE_MISMATCH)))
    # q8_0.rs:82-92 single_block_identity_scale
    qs = [i - 16 for i in range(32)]
    k.append(("q8_identity_scale", Q8_0, pack_q8_0(1.0, qs), 32, _close(np.array(qs), 1e-4)))
    # q8_0.rs:94-104 single_block_scaled
    qs = [i + 1 for i in range(32)]
    k.append(("q8_scaled", Q8_0, pack_q8_0(2.0, qs), 32, _close(2.0 * np.array(qs), 1e-4)))
    # q8_0.rs:106-120 negative_scale_and_values
    pat = [-128, -64, -1, 0, 1, 64, 127, 0]
    qs = [pat[i % 8] for i in range(32)]
    k.append(("q8_negative_scale", Q8_0, pack_q8_0(-0.5, qs), 32, _close(-0.5 * np.array(qs), 1e-3)))
    # q8_0.rs:122-136 multiple_blocks
    q1, q2 = list(range(32)), [-i for i in range(32)]
    k.append(("q8_multiple_blocks", Q8_0, np.concatenate([pack_q8_0(1.0, q1), pack_q8_0(2.0, q2)]), 64,
              _close(np.concatenate([np.array(q1), 2.0 * np.array(q2)]), 1e-4)))
    # q8_0.rs:138-163 size errors, :165-170 empty buffers
    k.append(("q8_partial_block_dst", Q8_0, np.zeros(34, np.uint8), 16, _status(DEQUANT_SIZE_MISMATCH)))
    k.append(("q8_wrong_src_size", Q8_0, np.zeros(33, np.uint8), 32, _status(DEQUANT_SIZE_MISMATCH)))
    k.append(("q8_empty", Q8_0, np.zeros(0, np.uint8), 0, _status(0)))
    # dequant/mod.rs:98-108 unsupported_dtype_reports_error (Q3_K)
    k.append(("unsupported_q3_k", Q3_K, np.zeros(110, np.uint8), 256, _status(UNSUPPORTED_DEQUANT)))
    # dequant/mod.rs:110-141 float arms
    k.append(("f32_roundtrip", F32, np.array([1.0, -2.5, 1.5, 0.0], np.float32).view(np.uint8), 4,
              _close([1.0, -2.5, 1.5, 0.0], 1e-12)))
    k.append(("f16_roundtrip", F16, np.array([1.0, -1.0, 2.0, 0.0], np.float16).view(np.uint8), 4,
              _close([1.0, -1.0, 2.0, 0.0], 1e-12)))
    bf = (np.array([1.0, -1.0, 2.0, 0.0], np.float32).view(np.uint32) >> 16).astype(np.uint16)
    k.append(("bf16_roundtrip", BF16, bf.view(np.uint8), 4, _close([1.0, -1.0, 2.0, 0.0], 1e-12)))
    # dequant/mod.rs:152-163, 180-190, 223-234, 256-270 dispatch arms
    k.append(("q4_0_arm", Q4_0, pack_q4_0(2.0, [8] * 32), 32, _close(np.zeros(32), 1e-3)))
    k.append(("q8_0_arm", Q8_0, pack_q8_0(1.0, [5] * 32), 32, _close(5 * np.ones(32), 1e-3)))
    k.append(("q4_k_arm", Q4_K, pack_q4k(1.0, 0.0, [2] * 8, [0] * 8, [3] * 256), 256,
              _close(6 * np.ones(256), 1e-2)))
    q6blk = np.concatenate([np.zeros(192, np.uint8), np.ones(16, np.uint8),
                            np.frombuffer(f16_bytes(1.0), np.uint8)])
    k.append(("q6_k_arm", Q6_K, q6blk, 256, _close(-32 * np.ones(256), 1e-2)))
    # rsllm-gguf/tests/fake_llama_end_to_end.rs:232-255: Q8_0 (scale 2, quants
    # alternating +-1) and Q4_0 (scale 1, nibbles cycling 0..15)
    k.append(("fake_llama_q8_0", Q8_0, pack_q8_0(2.0, [1 if i % 2 == 0 else -1 for i in range(32)]), 32,
              _close([2.0 if i % 2 == 0 else -2.0 for i in range(32)], 1e-3)))
    k.append(("fake_llama_q4_0", Q4_0, pack_q4_0(1.0, [i % 16 for i in range(32)]), 32,
              _close([(i % 16) - 8.0 for i in range(32)], 1e-3)))
    return k


def q4_0_matmul_case():
    """quant_matmul.rs:189-248: in 64, out 3, 2 tokens, sin/cos data, Q4_0 via
    the reference's row packer; checked against dequant-then-naive at 1e-4."""
    in_dim, out_dim, n_tok = 64, 3, 2
    i = np.arange(out_dim * in_dim, dtype=np.float32)
    w = (np.sin(i * np.float32(0.05)) * np.float32(4.0)).astype(np.float32)
    x = np.cos(np.arange(n_tok * in_dim, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    wq = np.concatenate([pack_q4_0_row(w[o * in_dim:(o + 1) * in_dim]) for o in range(out_dim)])
    return wq, x, n_tok, in_dim, out_dim
