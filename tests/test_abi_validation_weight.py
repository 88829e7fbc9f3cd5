"""Argument validation of the caller-chain entry points in the reference's
order and with its error classes: matmul_weight_f32 (weight.rs:121-167) and
matmul_grouped_lora_down with grouped_weight_slice (weight.rs:219-323),
including the reference's own rejection tests (rejects_wrong_out_shape
:447-462, grouped_weight_slice_quant_path_bounds_check :407-421). Validation
runs before any device work, so these run without a GPU."""
import numpy as np
import pytest

from rsllm_amd.ggml import GgmlType as G


def mw(hip, out_len, w, x_len, n_tok, in_dim, out_dim, dtype):
    hip.matmul_weight_f32(np.zeros(out_len, np.float32), w, np.zeros(x_len, np.float32), n_tok,
                          in_dim, out_dim, dtype)


def lora(hip, out_len, w, x_len, n_tok, n_groups, group_dim, rank, dtype):
    hip.matmul_grouped_lora_down(np.zeros(out_len, np.float32), w, np.zeros(x_len, np.float32),
                                 n_tok, n_groups, group_dim, rank, dtype)


def test_rejects_wrong_out_shape(hip):
    with pytest.raises(hip.ShapeMismatch, match="matmul_weight_f32.out"):
        mw(hip, 10, np.zeros(12, np.float32), 8, 2, 4, 3, G.F32)


@pytest.mark.parametrize("args,msg", [
    ((5, np.zeros(12, np.float32), 7, 2, 4, 3, G.F32), "matmul_weight_f32.out"),  # out first
    ((6, np.zeros(12, np.float32), 7, 2, 4, 3, G.F32), "matmul_weight_f32.x"),
    ((6, np.zeros(11, np.float32), 8, 2, 4, 3, G.F32), "weight_f32"),
    ((6, np.zeros(47, np.uint8), 8, 2, 4, 3, G.F32), "weight_f32"),      # not whole f32 values
    ((4, np.zeros(2 * 144, np.uint8), 2 * 250, 2, 250, 2, G.Q4_K), "matmul_weight_f32.quant"),
    ((4, np.zeros(2 * 144 - 1, np.uint8), 2 * 256, 2, 256, 2, G.Q4_K), "matmul_weight_f32.quant"),
    ((4, np.zeros(2 * 144, np.uint8), 2 * 256, 2, 256, 2, 7), "matmul_weight_f32.quant"),  # Q5_1
])
def test_weight_f32_errors_in_order(hip, args, msg):
    with pytest.raises(hip.ShapeMismatch, match=msg):
        mw(hip, *args)


def test_weight_f32_quant_zero_out_dim_panics_in_reference(hip):
    with pytest.raises(hip.InvalidArgument):
        mw(hip, 0, np.zeros(0, np.uint8), 256, 1, 256, 0, G.Q4_K)


def test_weight_f32_empty_shapes_are_ok(hip):
    # nothing to compute: returns before touching the device
    mw(hip, 0, np.zeros(12, np.float32), 0, 0, 4, 3, G.F32)
    mw(hip, 0, np.zeros(0, np.float32), 4, 1, 4, 0, G.F32)


def test_slice_alignment_rejected(hip):
    # 31 elements per Q8_0 group
    with pytest.raises(hip.ShapeMismatch, match="alignment"):
        lora(hip, 1, np.zeros(1024, np.uint8), 31, 1, 1, 31, 1, G.Q8_0)


@pytest.mark.parametrize("args,msg", [
    ((4, np.zeros(6 * 34, np.uint8), 3 * 32 - 1, 1, 3, 32, 2, G.Q8_0), "lora_down.x"),
    ((5, np.zeros(6 * 34, np.uint8), 3 * 32, 1, 3, 32, 2, G.Q8_0), "lora_down.out"),
    ((6, np.zeros(6 * 34 - 1, np.uint8), 3 * 32, 1, 3, 32, 2, G.Q8_0), "slice.quant"),
    ((6, np.zeros(2 * 34 - 1, np.uint8), 3 * 32, 1, 3, 32, 2, G.Q8_0), "slice.quant"),
    ((4, np.zeros(11, np.float32), 6, 1, 2, 3, 2, G.F32), "slice.f32"),
    ((2 * 2 * 2, np.zeros(2 * 2 * 250 // 256 * 144, np.uint8), 2 * 2 * 250, 2, 2, 250, 2, G.Q4_K),
     "alignment"),
    ((2 * 2 * 256, np.zeros(2 * 65536 // 32 * 22, np.uint8), 2 * 2 * 256, 2, 2, 256, 256, 6),
     "matmul_weight_f32.quant"),   # Q5_0 blocks align, the matmul rejects the dtype
])
def test_lora_down_errors_in_order(hip, args, msg):
    with pytest.raises(hip.ShapeMismatch, match=msg):
        lora(hip, *args)


def test_lora_down_no_groups_is_ok(hip):
    lora(hip, 0, np.zeros(0, np.uint8), 0, 4, 0, 32, 2, G.Q8_0)


def test_lora_down_longer_blob_is_accepted_by_validation(hip):
    # the slices only need to end inside the blob (weight.rs:313-319); this
    # does not reach the device because n_tok is 0
    lora(hip, 0, np.zeros(6 * 34 + 100, np.uint8), 0, 0, 3, 32, 2, G.Q8_0)


# ---- apply_shared_expert (moe.rs:422-455: check_moe_shapes :557-573, then the
# gate, up and down matmul_weight_f32 checks) ----

def shared(hip, out_len, x_len, gate, dg, up, du, down, dd, n_tok, n_embd, n_ff):
    hip.apply_shared_expert(np.zeros(out_len, np.float32), np.zeros(x_len, np.float32), gate, dg,
                            up, du, down, dd, n_tok, n_embd, n_ff, 10.0)


_E, _F = 64, 32
_G = np.zeros(_F * _E, np.float32)
_D = np.zeros(_E * _F, np.float32)
_Q = np.zeros(_F * 2 * 34, np.uint8)   # Q8_0 [32 x 64]


@pytest.mark.parametrize("args,msg", [
    ((2 * _E, 2 * _E - 1, _G, G.F32, _G, G.F32, _D, G.F32, 2, _E, _F), "moe.x"),
    ((2 * _E - 1, 2 * _E - 1, _G, G.F32, _G, G.F32, _D, G.F32, 2, _E, _F), "moe.x"),  # x first
    ((3, 2 * _E, _G, G.F32, _G, G.F32, _D, G.F32, 2, _E, _F), "moe.out"),
    ((2 * _E, 2 * _E, _G[:-1], G.F32, _G, G.F32, _D, G.F32, 2, _E, _F), "weight_f32"),
    ((2 * _E, 2 * _E, _G, G.F32, _Q[:-1], G.Q8_0, _D, G.F32, 2, _E, _F), "matmul_weight_f32.quant"),
    ((2 * _E, 2 * _E, _G, G.F32, _Q, G.Q8_0, _D[:-1], G.F32, 2, _E, _F), "weight_f32"),
    ((2 * 96, 2 * 96, np.zeros(_F * 96, np.float32), G.F32, np.zeros(_F * 96, np.float32), G.F32,
      np.zeros(96 * 34, np.uint8), G.Q4_K, 2, 96, _F), "matmul_weight_f32.quant"),  # n_ff 32 % 256
])
def test_shared_expert_errors_in_order(hip, args, msg):
    with pytest.raises(hip.ShapeMismatch, match=msg):
        shared(hip, *args)


def test_shared_expert_no_tokens_skips_the_matmul_checks(hip):
    shared(hip, 0, 0, _G[:-1], G.F32, _G, G.F32, _D, G.F32, 0, _E, _F)


def test_shared_expert_quant_zero_n_ff_panics_in_reference(hip):
    with pytest.raises(hip.InvalidArgument):
        shared(hip, _E, _E, np.zeros(0, np.uint8), G.Q8_0, np.zeros(0, np.uint8), G.Q8_0,
               np.zeros(0, np.uint8), G.Q8_0, 1, _E, 0)
