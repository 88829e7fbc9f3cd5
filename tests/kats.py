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
Q2_K, IQ2_XXS = 10, 16
Q4_1, Q5_K, Q8_K = 3, 13, 15
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


def pack_q2k(d, dmin, sc, m, q2) -> np.ndarray:
    """Inverse of the Q2_K decoder (the reference's pack_block, q2_k.rs:111-162):
    scales[j] = m_j << 4 | sc_j; element e = 128h + 32k + l (l < 32) is the
    2-bit field at shift 2k of qs[32h + l]; d, dmin at bytes 80, 82."""
    out = np.zeros(84, np.uint8)
    for j in range(16):
        out[j] = ((m[j] & 15) << 4) | (sc[j] & 15)
    for e in range(256):
        h, k, l = e // 128, (e % 128) // 32, e % 32
        out[16 + 32 * h + l] |= (int(q2[e]) & 3) << (2 * k)
    out[80:82] = np.frombuffer(f16_bytes(d), np.uint8)
    out[82:84] = np.frombuffer(f16_bytes(dmin), np.uint8)
    return out


def pack_iq2xxs(d, grids, signs, extras) -> np.ndarray:
    """Inverse of the IQ2_XXS decoder (the reference's pack_block,
    iq2_xxs.rs:131-157): per sub-group, u32 of 4 grid indices, then u32 of
    4 7-bit sign indices (bits 7l..7l+6) and the 4-bit extra in bits 28-31."""
    out = [np.frombuffer(f16_bytes(d), np.uint8)]
    for g in range(8):
        a0 = sum(int(grids[g][l]) << (8 * l) for l in range(4))
        a1 = sum(int(signs[g][l]) << (7 * l) for l in range(4)) | (int(extras[g]) << 28)
        out.append(np.frombuffer(np.array([a0, a1], np.uint32).tobytes(), np.uint8))
    return np.concatenate(out)


# --- dequant KATs: (name, dtype, src, n, check) -------------------------------
# check(status, values) raises AssertionError on mismatch.

def pack_q4_1(d, m, nibbles) -> np.ndarray:
    """q4_0.rs:123-133 pack_q4_1: f16 d, f16 m, byte j = nibble j | nibble j + 16 << 4."""
    nb = np.asarray(nibbles, np.uint8) & 15
    qs = nb[:16] | (nb[16:] << 4)
    return np.concatenate([np.frombuffer(f16_bytes(d) + f16_bytes(m), np.uint8), qs.astype(np.uint8)])


def pack_q5k(d, dmin, sc, m, q5) -> np.ndarray:
    """q5_k.rs:122-156 pack_block: f16 d, dmin, the Q4_K scale packing, qh bit
    (2k) / (2k + 1) of byte l for elements 64k + l / 64k + 32 + l at or above
    16, qs[32k + l] = low nibble of element 64k + l | that of 64k + 32 + l << 4."""
    q5 = np.asarray(q5, np.uint8)
    qh = np.zeros(32, np.uint8)
    qs = np.zeros(128, np.uint8)
    for k in range(4):
        for l in range(32):
            lo, hi = q5[64 * k + l], q5[64 * k + 32 + l]
            if lo >= 16:
                qh[l] |= 1 << (2 * k)
            if hi >= 16:
                qh[l] |= 1 << (2 * k + 1)
            qs[32 * k + l] = (lo & 15) | ((hi & 15) << 4)
    return np.concatenate([np.frombuffer(f16_bytes(d) + f16_bytes(dmin), np.uint8),
                           pack_scales(sc, m), qh, qs])


def pack_q8k(d, qs) -> np.ndarray:
    """q8_k.rs:78-86 pack_block: f32 d, 256 int8 codes, 32 zero bsum bytes."""
    return np.concatenate([np.frombuffer(np.float32(d).tobytes(), np.uint8),
                           np.asarray(qs, np.int8).view(np.uint8), np.zeros(32, np.uint8)])


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
    # q2_k.rs:171-189 zero_quants_yields_minus_min_per_sub_block
    m16 = list(range(16))
    k.append(("q2k_zero_quants_minus_min", Q2_K, pack_q2k(1.0, 1.0, [0] * 16, m16, [0] * 256), 256,
              _close(np.repeat(-np.array(m16, np.float32), 16), 1e-3)))
    # q2_k.rs:192-211 distinct_per_sub_block_scales
    k.append(("q2k_distinct_sub_block_scales", Q2_K, pack_q2k(1.0, 0.0, m16, [0] * 16, [1] * 256),
              256, _close(np.repeat(np.array(m16, np.float32), 16), 1e-2)))
    # q2_k.rs:214-232 full_2bit_range_with_offset
    q2 = [i % 4 for i in range(256)]
    k.append(("q2k_full_2bit_range_with_offset", Q2_K, pack_q2k(0.5, 0.25, [4] * 16, [2] * 16, q2),
              256, _close(2.0 * np.array(q2, np.float32) - 0.5, 1e-2)))
    # q2_k.rs:235-262 distinct_sc_and_m_combined
    sc = [(j % 4) + 1 for j in range(16)]
    mm = [((15 - j) % 4) + 1 for j in range(16)]
    k.append(("q2k_distinct_sc_and_m_combined", Q2_K, pack_q2k(1.0, 1.0, sc, mm, [2] * 256), 256,
              _close(np.repeat(2.0 * np.array(sc, np.float32) - np.array(mm, np.float32), 16),
                     1e-3)))
    # q2_k.rs:265-272 wrong_src_size_errors; dequant/mod.rs:273-289 dispatch arm
    k.append(("q2k_wrong_src_size", Q2_K, np.zeros(83, np.uint8), 256,
              _status(DEQUANT_SIZE_MISMATCH)))
    blk = np.concatenate([np.full(16, 3, np.uint8), np.full(64, 0x55, np.uint8),
                          np.frombuffer(f16_bytes(1.0) + f16_bytes(0.0), np.uint8)])
    k.append(("q2k_dispatch_arm", Q2_K, blk, 256, _close(np.full(256, 3.0), 1e-2)))
    # iq2_xxs.rs:188-198 zero_grid_yields_zero
    z4 = [[0] * 4 for _ in range(8)]
    k.append(("iq2xxs_zero_d", IQ2_XXS, pack_iq2xxs(0.0, z4, z4, [0] * 8), 256,
              _close(np.zeros(256), 1e-3)))
    # iq2_xxs.rs:200-212 uniform_pattern_uniform_output
    k.append(("iq2xxs_uniform", IQ2_XXS, pack_iq2xxs(1.0, z4, z4, [0] * 8), 256,
              _close(np.ones(256), 1e-3)))
    # iq2_xxs.rs:214-233 extras_scale_subgroups_independently
    k.append(("iq2xxs_extras", IQ2_XXS, pack_iq2xxs(1.0, z4, z4, list(range(8))), 256,
              _close(np.repeat(1.0 + 2.0 * np.arange(8), 32), 1e-3)))
    # iq2_xxs.rs:235-246 signs_flip_negate_elements
    k.append(("iq2xxs_all_signs", IQ2_XXS, pack_iq2xxs(1.0, z4, [[127] * 4] * 8, [0] * 8), 256,
              _close(-np.ones(256), 1e-3)))
    # iq2_xxs.rs:248-329 distinct_l_slots_within_one_subgroup
    g = [[0, 1, 2, 3]] + [[0] * 4] * 7
    want = np.ones(256, np.float32)
    want[0:8] = 1.0
    want[8:16] = [-5.375, 1, 1, 1, 1, 1, 1, -1.0]
    want[16:24] = [3.125, -3.125, 1, 1, 1, 1, 1, -1.0]
    want[24:32] = [-1.0, -5.375, 1, 1, 1, 1, 1, 1]
    k.append(("iq2xxs_distinct_l_slots", IQ2_XXS, pack_iq2xxs(1.0, g, g, [0] * 8), 256,
              _close(want, 1e-3)))
    # iq2_xxs.rs:331-389 distinct_subgroups_with_distinct_grids_and_extras
    want = np.ones(256, np.float32)
    for l in range(4):
        want[32 + 8 * l:32 + 8 * l + 8] = [16.125] + [3.0] * 7
        want[128 + 8 * l:128 + 8 * l + 8] = [48.375, 48.375] + [9.0] * 6
    grid_idx = [[i] * 4 for i in range(8)]
    dst_check = want.copy()

    def check_subgroups(rc, got, w=dst_check):
        assert rc == 0, f"status {rc}"
        for sl in (slice(0, 32), slice(32, 64), slice(128, 160)):
            assert np.all(np.abs(got[sl] - w[sl]) < 1e-3)
    k.append(("iq2xxs_distinct_subgroups", IQ2_XXS, pack_iq2xxs(1.0, grid_idx, z4, list(range(8))),
              256, check_subgroups))
    # iq2_xxs.rs:391-399 wrong_src_size_errors; dequant/mod.rs iq2_xxs dispatch arm
    k.append(("iq2xxs_wrong_src_size", IQ2_XXS, np.zeros(65, np.uint8), 256,
              _status(DEQUANT_SIZE_MISMATCH)))
    # q4_0.rs:184-193 q4_1_min_only_offset
    k.append(("q4_1_min_only_offset", Q4_1, pack_q4_1(0.0, 3.5, [7] * 32), 32,
              _close(np.full(32, 3.5), 1e-3)))
    # q4_0.rs:195-213 q4_1_linear_with_offset
    nib = [i % 16 for i in range(32)]
    k.append(("q4_1_linear_with_offset", Q4_1, pack_q4_1(0.5, 1.0, nib), 32,
              _close(0.5 * np.array(nib, np.float32) + 1.0, 1e-3)))
    # dequant/mod.rs:165-178 q4_1_dispatch_routes_to_q4_1_arm (d 0, m 7, zero codes)
    k.append(("q4_1_arm", Q4_1, pack_q4_1(0.0, 7.0, [0] * 32), 32, _close(np.full(32, 7.0), 1e-3)))
    # q5_k.rs:166-184 five_bit_range_zero_min
    q5 = [i % 32 for i in range(256)]
    k.append(("q5k_five_bit_range_zero_min", Q5_K, pack_q5k(1.0, 0.0, [1] * 8, [0] * 8, q5), 256,
              _close(np.array(q5, np.float32), 1e-2)))
    # q5_k.rs:185-195 full_range_with_offset
    k.append(("q5k_full_range_with_offset", Q5_K, pack_q5k(0.5, 0.5, [2] * 8, [1] * 8, [31] * 256),
              256, _close(np.full(256, 30.5), 1e-2)))
    # q5_k.rs:197-218 distinct_per_sub_block_scales_and_mins
    sc8 = list(range(1, 9))
    k.append(("q5k_distinct_scales_and_mins", Q5_K, pack_q5k(1.0, 1.0, sc8, sc8, [0] * 256), 256,
              _close(np.repeat(-np.array(sc8, np.float32), 32), 1e-2)))
    # q5_k.rs:220-228 wrong_src_size_errors
    k.append(("q5k_wrong_src_size", Q5_K, np.zeros(175, np.uint8), 256,
              _status(DEQUANT_SIZE_MISMATCH)))
    # dequant/mod.rs:236-255 q5_k_dispatch_routes_to_q5_k_arm (sc 2, qh 0, codes 1)
    blk = np.concatenate([np.frombuffer(f16_bytes(1.0) + f16_bytes(0.0), np.uint8),
                          pack_scales([2] * 8, [0] * 8), np.zeros(32, np.uint8),
                          np.full(128, 0x11, np.uint8)])
    k.append(("q5k_dispatch_arm", Q5_K, blk, 256, _close(np.full(256, 2.0), 1e-2)))
    # q8_k.rs:94-109 unit_scale_passes_through_qs
    qs = [i % 127 for i in range(256)]
    k.append(("q8k_unit_scale", Q8_K, pack_q8k(1.0, qs), 256, _close(np.array(qs, np.float32), 1e-4)))
    # q8_k.rs:110-120 negative_scale_inverts_sign
    k.append(("q8k_negative_scale", Q8_K, pack_q8k(-0.5, [5] * 256), 256,
              _close(np.full(256, -2.5), 1e-4)))
    # q8_k.rs:121-136 boundary_quant_values
    qs = [0] * 256
    qs[0], qs[1], qs[2], qs[3] = -128, 127, 0, -1
    want = np.float32(0.01) * np.array(qs, np.float32)
    k.append(("q8k_boundary_values", Q8_K, pack_q8k(0.01, qs), 256, _close(want, 1e-4)))
    # q8_k.rs:137-146 wrong_src_size_errors
    k.append(("q8k_wrong_src_size", Q8_K, np.zeros(291, np.uint8), 256,
              _status(DEQUANT_SIZE_MISMATCH)))
    # q8_k.rs:147-163 multi_block_decode (wrapping int8 patterns)
    qa = np.arange(256).astype(np.uint8).view(np.int8)
    qb = (-qa.astype(np.int16)).astype(np.int8)
    want = np.concatenate([2.0 * qa.astype(np.float32), -qb.astype(np.float32)])
    k.append(("q8k_multi_block", Q8_K, np.concatenate([pack_q8k(2.0, qa), pack_q8k(-1.0, qb)]), 512,
              _close(want, 1e-4)))
    # dequant/mod.rs:291-303 q8_k_dispatch_routes_to_q8_k_arm (d 2, codes 3)
    k.append(("q8k_dispatch_arm", Q8_K, pack_q8k(2.0, [3] * 256), 256, _close(np.full(256, 6.0), 1e-3)))
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


# --- Q8_0 int8-activation path (backend-cpu/src/ops/q8_0.rs) -----------------
# An implementation is a pair of callables:
#   quantize(x_flat, n_tok, in_dim) -> (status, int8[n_tok*blocks*32], f32[n_tok*blocks])
#   matmul(w, xq, xscale, n_tok, in_dim, out_dim) -> (status, f32[n_tok*out_dim])
# KATs are (name, run(quantize, matmul)) and raise AssertionError on mismatch.
NON_FINITE_INPUT, SHAPE_MISMATCH = 3, 1


def pack_q8_0_row_with(quantize, w) -> np.ndarray:
    """The reference test helper pack_q8_0_row (q8_0.rs:302-320): quantize the
    row as an activation, then store f16(scale) and the 32 quants per block."""
    w = np.asarray(w, np.float32)
    rc, q, s = quantize(w, 1, w.size)
    assert rc == 0
    out = []
    for b in range(s.size):
        out.append(np.frombuffer(f16_bytes(float(s[b])), np.uint8))
        out.append(q[b * 32:(b + 1) * 32].view(np.uint8))
    return np.concatenate(out)


def _ref_round_trip(quantize, matmul):
    # quantize_round_trip_within_tolerance (q8_0.rs:323-343)
    x = ((np.arange(64, dtype=np.float32) - np.float32(32.0)) * np.float32(0.1)).astype(np.float32)
    rc, q, s = quantize(x, 1, 64)
    assert rc == 0
    rec = q.astype(np.float32).reshape(2, 32) * s[:, None]
    assert np.all(np.abs(rec - x.reshape(2, 32)) < 0.05)


def _ref_zero(quantize, matmul):
    # quantize_zero_input_is_zero (:345-353)
    rc, q, s = quantize(np.zeros(32, np.float32), 1, 32)
    assert rc == 0 and s[0] == 0.0 and np.all(q == 0)


def _ref_pad(quantize, matmul):
    # quantize_pads_partial_block_to_zero (:355-365): 20 ones; the tail is 0
    # and (closed form) the ones quantize to 127 with scale 1/127
    rc, q, s = quantize(np.ones(20, np.float32), 1, 20)
    assert rc == 0 and np.all(q[20:] == 0) and np.all(q[:20] == 127)
    assert s[0] == np.float32(1.0) / np.float32(127.0)


def _ref_dot_full_precision(quantize, matmul):
    # dot_q8_0_row_matches_full_precision (:367-389)
    i = np.arange(96, dtype=np.float32)
    w = np.sin(i * np.float32(0.07) - np.float32(3.0)).astype(np.float32)
    x = np.cos(i * np.float32(0.11) + np.float32(1.0)).astype(np.float32)
    row = pack_q8_0_row_with(quantize, w)
    rc, xq, xs = quantize(x, 1, 96)
    assert rc == 0
    rc, got = matmul(row, xq, xs, 1, 96, 1)
    assert rc == 0
    want = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    assert abs(got[0] - want) < 0.01 * max(abs(want), 1.0)


def _ref_matmul_naive(quantize, matmul):
    # matmul_q8_0_batch_matches_naive (:391-452): in 64, out 4, 2 tokens
    in_dim, out_dim, n_tok = 64, 4, 2
    wf = np.sin(np.arange(out_dim * in_dim, dtype=np.float32) * np.float32(0.013)
                + np.float32(0.1)).astype(np.float32)
    x = np.cos(np.arange(n_tok * in_dim, dtype=np.float32) * np.float32(0.027)
               - np.float32(0.2)).astype(np.float32)
    w = np.concatenate([pack_q8_0_row_with(quantize, wf[o * in_dim:(o + 1) * in_dim])
                        for o in range(out_dim)])
    rc, xq, xs = quantize(x, n_tok, in_dim)
    assert rc == 0
    rc, out = matmul(w, xq, xs, n_tok, in_dim, out_dim)
    assert rc == 0
    want = x.reshape(n_tok, in_dim).astype(np.float64) @ wf.reshape(out_dim, in_dim).T.astype(np.float64)
    assert np.all(np.abs(out.reshape(n_tok, out_dim) - want) < 0.01 * np.maximum(np.abs(want), 1.0))


def _ref_matmul_shape(quantize, matmul):
    # matmul_rejects_shape_mismatch (:454-459): empty weights, in 32, out 4
    rc, _ = matmul(np.zeros(0, np.uint8), np.zeros(0, np.int8), np.zeros(0, np.float32), 1, 32, 4)
    assert rc == SHAPE_MISMATCH


def _ref_nan_inf(quantize, matmul):
    # quantize_rejects_nan_input / _inf_input (:461-477)
    for x in ([1.0, 2.0, np.nan, 3.0], [1.0, np.inf, 2.0]):
        x = np.array(x, np.float32)
        rc, _, _ = quantize(x, 1, x.size)
        assert rc == NON_FINITE_INPUT


def _ref_nonfinite_scale(quantize, matmul):
    # dot_q8_0_row_ignores_nonfinite_scale (:529-545): scale bits 0x7E00, quants
    # 127, xq 1, xscale 1 -> exactly 0.0; also for +-inf scales (:143-146)
    for bits in (0x7E00, 0x7C00, 0xFC00):
        row = np.concatenate([np.array([bits & 0xFF, bits >> 8], np.uint8),
                              np.full(32, 127, np.uint8)])
        rc, out = matmul(row, np.ones(32, np.int8), np.ones(1, np.float32), 1, 32, 1)
        assert rc == 0 and out[0] == 0.0 and not np.signbit(out[0])


def _closed_ties_even(quantize, matmul):
    """Closed form: amax 127 gives d = 1 and id = 1 exactly, so q = x rounded
    half to even (round_ties_even, :79): 2.5 -> 2, 3.5 -> 4, -2.5 -> -2,
    0.5 -> 0, -1.5 -> -2; a half-away-from-zero rounding fails it."""
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -1.5]
    rc, q, s = quantize(x, 1, 32)
    assert rc == 0 and s[0] == 1.0
    assert q[:8].tolist() == [127, 2, 4, -2, 0, 0, 2, -2]


def _closed_overflowing_inverse(quantize, matmul):
    """amax = 1e-40 gives a subnormal d whose inverse overflows to inf: then
    x * id is +-inf (saturating `as i32`, clamped: 127 / -128) and 0 * inf is
    NaN (`as i32` -> 0). Pins the saturating cast, the clamp bounds and
    subnormal arithmetic (no flush to zero)."""
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = np.float32(-1e-40), np.float32(1e-41), np.float32(-1e-45)
    rc, q, s = quantize(x, 1, 32)
    assert rc == 0
    assert s[0] == np.float32(1e-40) / np.float32(127.0) and s[0] != 0.0
    assert q[:4].tolist() == [-128, 127, -128, 0]


def _closed_exact_sum(quantize, matmul):
    """Power-of-two scales and small dots make every product and partial sum
    exact, so the result is the integer dot computed in Python: pins block
    order, the f16 scale byte order, signed quants, per-token scales and the
    partial last block (weight tail bytes are garbage, xq tail nonzero; only
    the first in_dim - 32 b lanes count, :183-187)."""
    for wide_w in (True, False):
        _exact_sum_case(matmul, wide_w)


def _exact_sum_case(matmul, wide_w):
    # one operand spans the full int8 range, the other |q| <= 4, and scale
    # exponents span 6 octaves: every partial sum needs at most 22 bits
    rng = np.random.default_rng(7 + wide_w)
    n_tok, in_dim, out_dim = 3, 100, 5
    blocks = 4
    wide, narrow = (-128, 128), (-4, 5)
    wq = rng.integers(*(wide if wide_w else narrow), size=(out_dim, blocks, 32)).astype(np.int8)
    xq = rng.integers(*(narrow if wide_w else wide), size=(n_tok, blocks, 32)).astype(np.int8)
    wexp = rng.integers(-2, 2, size=(out_dim, blocks))
    xexp = rng.integers(-2, 2, size=(n_tok, blocks))
    w = np.concatenate([pack_q8_0(2.0 ** int(wexp[o, b]), wq[o, b])
                        for o in range(out_dim) for b in range(blocks)])
    xs = (2.0 ** xexp).astype(np.float32).reshape(-1)
    rc, out = matmul(w, xq.reshape(-1), xs, n_tok, in_dim, out_dim)
    assert rc == 0
    want = np.zeros((n_tok, out_dim))
    for t in range(n_tok):
        for o in range(out_dim):
            acc = 0
            for b in range(blocks):
                bn = min(32, in_dim - 32 * b)
                dot = int(np.dot(wq[o, b, :bn].astype(np.int64), xq[t, b, :bn].astype(np.int64)))
                acc += dot * 2.0 ** (int(wexp[o, b]) + int(xexp[t, b]))
            want[t, o] = acc
    assert np.array_equal(out.reshape(n_tok, out_dim).astype(np.float64), want)


def _closed_sequential_order(quantize, matmul):
    """Block products 2^24, 1, 1, -2^24 summed left to right in f32 give
    (2^24 + 1 -> 2^24, ties to even) ... -> 0.0; exact summation gives 2 and
    right-to-left 2. Pins `acc += ...` in block order from 0.0 (:175-190)."""
    qs = np.zeros((4, 32), np.int8)
    qs[0, :4] = 64
    qs[1, 0] = 1
    qs[2, 0] = 1
    qs[3, :4] = -64
    w = np.concatenate([pack_q8_0(1.0, qs[b]) for b in range(4)])
    xq = np.zeros((4, 32), np.int8)
    xq[0, :4] = 64
    xq[1, 0] = 1
    xq[2, 0] = 1
    xq[3, :4] = 64
    xs = np.array([1024.0, 1.0, 1.0, 1024.0], np.float32)
    rc, out = matmul(w, xq.reshape(-1), xs, 1, 128, 1)
    assert rc == 0 and out[0] == 0.0


def _closed_scale_association(quantize, matmul):
    """The product is (wscale * xscale) * dot, each step rounded to f32
    (Rust's left-associative `wscale * xscale[b] * dot as f32`). With
    wscale = 1 + 2^-10 (f16-exact), xscale = 1 + 2^-14 + 2^-23 and
    dot = 32385 the two associations round differently."""
    ws = np.float32(np.float16(1.0 + 2.0 ** -10))
    xs = np.float32(1.0 + 2.0 ** -14 + 2.0 ** -23)
    qs = np.zeros(32, np.int8)
    xq = np.zeros(32, np.int8)
    # dot = 127 * 127 * 2 + 127 = 32385
    qs[:3] = [127, 127, 1]
    xq[:3] = [127, 127, 127]
    dot = np.float32(32385.0)
    left = np.float32(np.float32(ws * xs) * dot)
    right = np.float32(ws * np.float32(xs * dot))
    assert left != right, "choose constants whose associations differ"
    w = pack_q8_0(float(ws), qs)
    rc, out = matmul(w, xq, np.array([xs], np.float32), 1, 32, 1)
    assert rc == 0 and out[0] == left


def _closed_no_contraction(quantize, matmul):
    """`acc += p` rounds p first (Rust never contracts to an FMA): block 0
    contributes -p exactly (scale 1, xscale -p, dot 1) and block 1 the
    inexact p = (ws * xs) * dot, so the sum is exactly 0.0; a fused
    multiply-add would leave p's rounding error."""
    ws = np.float32(np.float16(1.0 + 2.0 ** -10))
    xs = np.float32(1.0 + 2.0 ** -14 + 2.0 ** -23)
    p = np.float32(np.float32(ws * xs) * np.float32(32385.0))
    from fractions import Fraction
    assert Fraction(float(np.float32(ws * xs))) * 32385 != Fraction(float(p))
    q0 = np.zeros(32, np.int8)
    q0[0] = 1
    q1 = np.zeros(32, np.int8)
    q1[:3] = [127, 127, 1]
    w = np.concatenate([pack_q8_0(1.0, q0), pack_q8_0(float(ws), q1)])
    xq = np.zeros(64, np.int8)
    xq[0] = 1
    xq[32:35] = [127, 127, 127]
    rc, out = matmul(w, xq, np.array([-p, xs], np.float32), 1, 64, 1)
    assert rc == 0 and out[0] == 0.0


def q8_kats():
    return [("ref_round_trip", _ref_round_trip), ("ref_zero", _ref_zero), ("ref_pad", _ref_pad),
            ("ref_dot_full_precision", _ref_dot_full_precision),
            ("ref_matmul_naive", _ref_matmul_naive), ("ref_matmul_shape", _ref_matmul_shape),
            ("ref_nan_inf", _ref_nan_inf), ("ref_nonfinite_scale", _ref_nonfinite_scale),
            ("closed_ties_even", _closed_ties_even),
            ("closed_overflowing_inverse", _closed_overflowing_inverse),
            ("closed_exact_sum", _closed_exact_sum),
            ("closed_sequential_order", _closed_sequential_order),
            ("closed_scale_association", _closed_scale_association),
            ("closed_no_contraction", _closed_no_contraction)]
