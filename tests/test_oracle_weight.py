"""The oracle's matmul_weight_f32 and matmul_grouped_lora_down
(rsllm-models/src/dsv4/weight.rs:113-323) pinned by the reference's own
tests of them (weight.rs:329-463) and by checks that do not reuse the C
restatement's arithmetic:

* the F32 arm is the sequential f32 sum (weight.rs:152-155), recomputed
  with numpy's strictly sequential ``add.accumulate``;
* the quantized arm is matmul_quant_f32 (already pinned by its own tests);
* the grouped form equals per-group calls on the reference's slice offsets,
  which are checked against the independent numpy Q8_0 dequantizer.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G


def seq_matmul(w, x, n_tok, in_dim, out_dim):
    """out[t, o] = ((w[o,0]*x[t,0] + w[o,1]*x[t,1]) + ...) in f32."""
    w = w.reshape(out_dim, in_dim).astype(np.float32)
    x = x.reshape(n_tok, in_dim).astype(np.float32)
    out = np.zeros((n_tok, out_dim), np.float32)
    if in_dim == 0:
        return out.reshape(-1)
    for t in range(n_tok):
        prod = (w * x[t][None, :]).astype(np.float32)
        out[t] = np.add.accumulate(prod, axis=1, dtype=np.float32)[:, -1]
    return out.reshape(-1)


def test_f32_matmul_matches_hand_dot():
    # weight.rs:329-354
    w = np.array([1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 1], np.float32)
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    rc, out = O.matmul_weight_f32(w, x, 2, 4, 3, O.F32)
    assert rc == O.OK
    assert out.tolist() == [1.0, 2.0, 7.0, 5.0, 6.0, 15.0]


def test_grouped_matmul_isolates_groups():
    # weight.rs:356-405
    w = np.array([1, 0, 1, 0, 1, 1, 2, 0, 0, 0, 2, 0], np.float32)
    x = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 40, 50, 60], np.float32)
    rc, out = O.matmul_grouped_lora_down(w, x, 2, 2, 3, 2, O.F32)
    assert rc == O.OK
    assert out.tolist() == [4.0, 5.0, 8.0, 10.0, 40.0, 50.0, 80.0, 100.0]


def test_rejects_wrong_out_shape():
    # weight.rs:447-462: out of 10 where 6 is expected
    rc, _ = O.matmul_weight_f32(np.zeros(12, np.float32), np.zeros(8, np.float32), 2, 4, 3, O.F32,
                                out_len=10)
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 10


def test_quant_slice_alignment_rejected():
    # weight.rs:407-421: 31 elements per Q8_0 group (block of 32) must fail
    rc, _ = O.matmul_grouped_lora_down(np.zeros(1024, np.uint8), np.zeros(31, np.float32), 1, 1,
                                       31, 1, O.Q8_0)
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 23


def test_quant_slice_offsets():
    # weight.rs:423-445: 4 groups of one Q8_0 block (34 bytes) in bytes 0..135;
    # group g reads bytes [34 g, 34 g + 34). Each group's single output is the
    # dot of that block (numpy dequantizer) with the group's x.
    data = np.arange(136, dtype=np.uint8)
    x = synth.activations(1, 4 * 32, 7).reshape(-1)
    rc, out = O.matmul_grouped_lora_down(data, x, 1, 4, 32, 1, O.Q8_0)
    assert rc == O.OK
    for g in range(4):
        deq = O.np_dequant_q8_0(data[34 * g: 34 * g + 34]).astype(np.float64)
        want = float(deq @ x[32 * g: 32 * g + 32].astype(np.float64))
        assert abs(out[g] - want) <= 1e-5 * np.abs(deq).max() * np.abs(x).sum()
    # block 2's scale is f16 0x4544 (bytes 68, 69) and its quants are 70..101
    assert O.np_dequant_q8_0(data[68:102])[0] == np.float16(np.frombuffer(
        bytes([68, 69]), np.float16)[0]).astype(np.float32) * 70


@pytest.mark.parametrize("n_tok,in_dim,out_dim", [(1, 1, 1), (3, 37, 5), (2, 256, 9), (4, 0, 3),
                                                  (0, 8, 8)])
def test_f32_arm_is_the_sequential_sum(n_tok, in_dim, out_dim):
    rng = np.random.default_rng(in_dim * 7 + out_dim)
    w = rng.standard_normal(out_dim * in_dim).astype(np.float32)
    x = rng.standard_normal(n_tok * in_dim).astype(np.float32)
    rc, out = O.matmul_weight_f32(w, x, n_tok, in_dim, out_dim, O.F32)
    assert rc == O.OK
    np.testing.assert_array_equal(out, seq_matmul(w, x, n_tok, in_dim, out_dim))


def test_f32_arm_errors_in_order():
    w, x = np.zeros(12, np.float32), np.zeros(8, np.float32)
    assert O.matmul_weight_f32(w, x[:7], 2, 4, 3, O.F32)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 11
    assert O.matmul_weight_f32(w[:11], x, 2, 4, 3, O.F32)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 12
    # out is checked first even when x is also wrong
    assert O.matmul_weight_f32(w, x[:7], 2, 4, 3, O.F32, out_len=5)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 10


@pytest.mark.parametrize("dt", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K])
def test_quant_arm_is_matmul_quant_f32(dt):
    w = synth.weight(dt, 6, 512, 3)
    x = synth.activations(2, 512, 4).reshape(-1)
    rc, out = O.matmul_weight_f32(w, x, 2, 512, 6, int(dt))
    rc2, want = O.matmul_quant_f32(w, x, 2, 512, 6, int(dt), n_threads=1)
    assert rc == rc2 == O.OK
    np.testing.assert_array_equal(out, want)


def test_quant_arm_maps_errors_to_shape_mismatch():
    w = synth.weight(G.Q4_K, 6, 512, 3)
    x = synth.activations(2, 512, 4).reshape(-1)
    # in_dim not a block multiple: NotBlockAligned in matmul_quant_f32
    rc, _ = O.matmul_weight_f32(w, x[:2 * 500], 2, 500, 6, int(G.Q4_K))
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 13
    rc, _ = O.matmul_weight_f32(w[:-1], x, 2, 512, 6, int(G.Q4_K))
    assert rc == O.SHAPE_MISMATCH and O.last_detail()[0] == 13
    # out_dim == 0 panics in the reference (rayon chunk size 0) and stays a panic
    rc, _ = O.matmul_weight_f32(w[:0], x, 2, 512, 0, int(G.Q4_K))
    assert rc == O.PANIC


@pytest.mark.parametrize("dt", [G.Q4_K, G.Q6_K, G.Q8_0, G.IQ2_XXS])
def test_grouped_equals_per_group_calls(dt):
    n_tok, n_groups, group_dim, rank = 3, 4, 512, 8
    w = synth.weight(dt, n_groups * rank, group_dim, 11)
    x = synth.activations(n_tok, n_groups * group_dim, 12)
    rc, out = O.matmul_grouped_lora_down(w, x, n_tok, n_groups, group_dim, rank, int(dt))
    assert rc == O.OK
    out = out.reshape(n_tok, n_groups * rank)
    stride = w.size // n_groups
    for g in range(n_groups):
        xg = np.ascontiguousarray(x[:, g * group_dim:(g + 1) * group_dim])
        rc, want = O.matmul_quant_f32(w[g * stride:(g + 1) * stride], xg, n_tok, group_dim, rank,
                                      int(dt), n_threads=1)
        assert rc == O.OK
        np.testing.assert_array_equal(out[:, g * rank:(g + 1) * rank], want.reshape(n_tok, rank))


def test_grouped_f32_is_the_sequential_sum():
    rng = np.random.default_rng(5)
    n_tok, n_groups, group_dim, rank = 2, 3, 40, 6
    w = rng.standard_normal(n_groups * rank * group_dim).astype(np.float32)
    x = rng.standard_normal((n_tok, n_groups * group_dim)).astype(np.float32)
    rc, out = O.matmul_grouped_lora_down(w, x, n_tok, n_groups, group_dim, rank, O.F32)
    assert rc == O.OK
    out = out.reshape(n_tok, -1)
    for g in range(n_groups):
        wg = w[g * rank * group_dim:(g + 1) * rank * group_dim]
        xg = np.ascontiguousarray(x[:, g * group_dim:(g + 1) * group_dim])
        np.testing.assert_array_equal(out[:, g * rank:(g + 1) * rank],
                                      seq_matmul(wg, xg, n_tok, group_dim, rank).reshape(n_tok, rank))


def test_grouped_errors_and_partial_write():
    n_tok, n_groups, group_dim, rank = 1, 3, 32, 2
    w = synth.weight(G.Q8_0, n_groups * rank, group_dim, 1)
    x = synth.activations(n_tok, n_groups * group_dim, 2).reshape(-1)
    assert O.matmul_grouped_lora_down(w, x[:-1], n_tok, n_groups, group_dim, rank,
                                      O.Q8_0)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 20
    assert O.matmul_grouped_lora_down(w, x, n_tok, n_groups, group_dim, rank, O.Q8_0,
                                      out_len=5)[0] == O.SHAPE_MISMATCH
    assert O.last_detail()[0] == 21
    assert O.matmul_grouped_lora_down(np.zeros(11, np.float32), np.zeros(6, np.float32), 1, 2, 3,
                                      2, O.F32)[0] == O.SHAPE_MISMATCH
    assert O.last_detail() == (22, 1)
    # the last group's slice ends past the blob: groups 0 and 1 are written
    # before the error, as the reference's loop does (weight.rs:241-263)
    rc, out = O.matmul_grouped_lora_down(w[:-1], x, n_tok, n_groups, group_dim, rank, O.Q8_0)
    assert rc == O.SHAPE_MISMATCH and O.last_detail() == (24, 2)
    assert np.isfinite(out[:4]).all() and np.isnan(out[4:]).all()
    # no groups: Ok, nothing written
    rc, out = O.matmul_grouped_lora_down(np.zeros(0, np.uint8), np.zeros(0, np.float32), 4, 0, 32,
                                         2, O.Q8_0)
    assert rc == O.OK and out.size == 0
