"""Argument checks of rsllm_hip_model_upload and the model lookups. They run
before any device work, so these run without a GPU."""
import ctypes

import numpy as np
import pytest

from rsllm_amd.ggml import GgmlType as G

FP = bytes(range(32))


def test_duplicate_names_rejected(hip):
    w = np.zeros(34, np.uint8)
    with pytest.raises(hip.InvalidArgument, match="duplicate"):
        hip.model_upload(FP, [("a", w, G.Q8_0, 32), ("a", w, G.Q8_0, 32)])


@pytest.mark.parametrize("dtype,n,in_dim", [
    (G.Q8_0, 34 * 3, 48),        # in_dim not a multiple of the block
    (G.Q8_0, 34 * 3 - 1, 32),    # not whole rows
    (G.Q4_K, 144 * 3, 512),      # 3 blocks, rows of 2
    (G.F32, 4 * 10, 4),          # 10 f32 values, rows of 4
])
def test_matmul_tensor_shape_rejected(hip, dtype, n, in_dim):
    with pytest.raises(hip.ShapeMismatch, match="whole number of rows"):
        hip.model_upload(FP, [("t", np.zeros(n, np.uint8), dtype, in_dim)])


def test_null_arguments_rejected(hip):
    L = hip.LIB
    d = (hip.TensorDesc * 1)()
    d[0] = hip.TensorDesc(None, None, 0, 0, 0)
    mid = ctypes.c_uint64()
    fp = ctypes.create_string_buffer(FP, 32)
    assert L.rsllm_hip_model_upload(fp, d, 1, ctypes.byref(mid)) == hip.InvalidArgument.status
    d[0] = hip.TensorDesc(b"x", None, 16, int(G.F16), 0)
    assert L.rsllm_hip_model_upload(fp, d, 1, ctypes.byref(mid)) == hip.InvalidArgument.status
    assert L.rsllm_hip_model_upload(None, d, 0, ctypes.byref(mid)) == hip.InvalidArgument.status
    assert L.rsllm_hip_model_upload(fp, d, 0, None) == hip.InvalidArgument.status


def test_unknown_model(hip):
    with pytest.raises(hip.InvalidArgument):
        hip.model_info(987654321)
    with pytest.raises(hip.InvalidArgument):
        hip.model_tensor(987654321, "x")
    with pytest.raises(hip.InvalidArgument):
        hip.model_release(987654321)
