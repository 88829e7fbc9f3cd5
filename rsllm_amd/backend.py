"""Host-side mirror of rsllm-backend-cpu's quantized-matmul interface, backed
by librsllm_hip.so through its C ABI (include/rsllm_hip.h).

Names, argument order and error classes follow the reference:

* ``matmul_quant_f32(out, weights, x, n_tok, in_dim, out_dim, dtype, tier)``
  — backend-cpu/src/ops/quant_matmul.rs:45-54
* ``dequant_to_f32(dtype, src, dst)`` — rsllm-gguf/src/dequant/mod.rs:69
* ``Error`` subclasses — backend-cpu/src/error.rs:7-43 and
  rsllm-gguf/src/error.rs:69-80
* ``HipBackend`` — the ``CpuBackend`` handle (backend-cpu/src/lib.rs:43-107)
  with ``kind()`` / ``capability()`` (rsllm-cal/src/lib.rs:84-90)

There is no CPU fallback: if the shared library is missing, importing this
module raises.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass

import numpy as np

from .ggml import GgmlType

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librsllm_hip.so")

# ---------------------------------------------------------------------------
# Status codes (include/rsllm_hip.h)
# ---------------------------------------------------------------------------
OK = 0
ERR_SHAPE_MISMATCH = 1
ERR_NOT_BLOCK_ALIGNED = 2
ERR_NON_FINITE_INPUT = 3
ERR_UNSUPPORTED_TIER = 4
ERR_DEQUANT_SIZE_MISMATCH = 5
ERR_UNSUPPORTED_DEQUANT = 6
ERR_DEVICE = 7
ERR_INVALID_ARGUMENT = 8
ERR_UNIMPLEMENTED = 10


class SimdTier(enum.IntEnum):
    """backend-cpu/src/capability.rs:20-35. Accepted and ignored by the
    matmul, as the reference ignores it (quant_matmul.rs:55)."""

    Neon = 0
    Avx512 = 1
    Avx2 = 2
    Scalar = 3


class Error(Exception):
    status = -1

    def __init__(self, message: str = "", **fields):
        super().__init__(message)
        self.message = message
        for k, v in fields.items():
            setattr(self, k, v)


class ShapeMismatch(Error):
    status = ERR_SHAPE_MISMATCH


class NotBlockAligned(Error):
    status = ERR_NOT_BLOCK_ALIGNED


class NonFiniteInput(Error):
    status = ERR_NON_FINITE_INPUT


class UnsupportedTier(Error):
    status = ERR_UNSUPPORTED_TIER


class DequantSizeMismatch(Error):
    status = ERR_DEQUANT_SIZE_MISMATCH


class UnsupportedDequant(Error):
    status = ERR_UNSUPPORTED_DEQUANT


class DeviceError(Error):
    status = ERR_DEVICE


class InvalidArgument(Error):
    status = ERR_INVALID_ARGUMENT


class Unimplemented(Error):
    status = ERR_UNIMPLEMENTED


_ERRORS = {c.status: c for c in (ShapeMismatch, NotBlockAligned, NonFiniteInput, UnsupportedTier,
                                 DequantSizeMismatch, UnsupportedDequant, DeviceError,
                                 InvalidArgument, Unimplemented)}


class _ErrorDetail(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int32), ("message", ctypes.c_char_p), ("what", ctypes.c_char_p),
                ("actual", ctypes.c_size_t), ("block", ctypes.c_size_t),
                ("src_bytes", ctypes.c_size_t), ("expected_bytes", ctypes.c_size_t)]


class _Capability(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_char_p), ("arch", ctypes.c_char_p),
                ("q4k_matmul", ctypes.c_int), ("q6k_matmul", ctypes.c_int),
                ("q8_0_matmul", ctypes.c_int), ("q2k_matmul", ctypes.c_int),
                ("iq2xxs_matmul", ctypes.c_int), ("fp8_kv_cache", ctypes.c_int)]


class TensorDesc(ctypes.Structure):
    """rsllm_hip_tensor_desc: one GGUF tensor for rsllm_hip_model_upload."""
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("len", ctypes.c_size_t),
                ("dtype", ctypes.c_uint32), ("in_dim", ctypes.c_size_t)]


class ModelInfo(ctypes.Structure):
    _fields_ = [("device_bytes", ctypes.c_uint64), ("uploaded_bytes", ctypes.c_uint64),
                ("upload_seconds", ctypes.c_double), ("refs", ctypes.c_uint32),
                ("n_tensors", ctypes.c_uint32)]


# Every symbol include/rsllm_hip.h declares, with its ctypes signature.
_P, _S, _U32, _I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int
SIGNATURES = {
    "rsllm_hip_last_error": ([ctypes.POINTER(_ErrorDetail)], None),
    "rsllm_hip_init": ([_I], _I),
    "rsllm_hip_capability_get": ([ctypes.POINTER(_Capability)], None),
    "rsllm_hip_matmul_quant_f32": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _U32], _I),
    "rsllm_hip_matmul_quant_f32_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _P], _I),
    "rsllm_hip_matmul_quant_f32_dev_noalloc": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _P], _I),
    "rsllm_hip_register_weights": ([_P, _S, _U32, _S], _I),
    "rsllm_hip_release_weights": ([], _I),
    "rsllm_hip_device_allocations": ([], ctypes.c_uint64),
    "rsllm_hip_stream_release": ([_P], _I),
    "rsllm_hip_model_upload": ([_P, ctypes.POINTER(TensorDesc), _S,
                                ctypes.POINTER(ctypes.c_uint64)], _I),
    "rsllm_hip_model_tensor": ([ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(_P),
                                ctypes.POINTER(_S)], _I),
    "rsllm_hip_model_info_get": ([ctypes.c_uint64, ctypes.POINTER(ModelInfo)], _I),
    "rsllm_hip_model_release": ([ctypes.c_uint64], _I),
    "rsllm_hip_prepare_weights_dev": ([_P, _P, _S, _U32, _S, _P], _I),
    "rsllm_hip_dequant_to_f32": ([_U32, _P, _S, _P, _S], _I),
    "rsllm_hip_dequant_to_f32_dev": ([_U32, _P, _S, _P, _S, _P], _I),
    "rsllm_hip_xq_bytes": ([_U32, _S, _S], _S),
    "rsllm_hip_quantize_x_dev": ([_U32, _P, _S, _S, _S, _P, _S, _P], _I),
    "rsllm_hip_matmul_prequant_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _P], _I),
    "rsllm_hip_matmul_q4k_bf16_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _P], _I),
    "rsllm_hip_moe_routed_dev": ([_P, _S, _P, _S, _P, _P, _S, _P, _S, _P, _P, _S, _S, _S, _S, _S,
                                  _S, _U32, _U32, ctypes.c_float, _P], _I),
    "rsllm_hip_moe_routed": ([_P, _S, _P, _S, _P, _P, _S, _P, _S, _P, _P, _S, _S, _S, _S, _S, _S,
                              _U32, _U32, ctypes.c_float], _I),
    "rsllm_hip_quantize_q8_0_batch": ([_P, _S, _P, _S, _P, _S, _S, _S], _I),
    "rsllm_hip_quantize_q8_0_batch_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _P, _P], _I),
    "rsllm_hip_matmul_q8_0_batch": ([_P, _S, _P, _S, _P, _S, _P, _S, _S, _S, _S, _U32], _I),
    "rsllm_hip_matmul_q8_0_batch_dev": ([_P, _S, _P, _S, _P, _S, _P, _S, _S, _S, _S, _P], _I),
    "rsllm_hip_matmul_weight_f32": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32], _I),
    "rsllm_hip_matmul_weight_f32_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _U32, _P], _I),
    "rsllm_hip_matmul_grouped_lora_down": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _S, _U32], _I),
    "rsllm_hip_matmul_grouped_lora_down_dev": ([_P, _S, _P, _S, _P, _S, _S, _S, _S, _S, _U32, _P],
                                               _I),
    "rsllm_hip_apply_shared_expert": ([_P, _S, _P, _S, _P, _S, _U32, _P, _S, _U32, _P, _S, _U32,
                                       _S, _S, _S, ctypes.c_float], _I),
    "rsllm_hip_apply_shared_expert_dev": ([_P, _S, _P, _S, _P, _S, _U32, _P, _S, _U32, _P, _S,
                                           _U32, _S, _S, _S, ctypes.c_float, _P], _I),
    "rsllm_hip_stream_read_dev": ([_P, _S, _P, _S, _I, _I, _I, _I, _P], _I),
    "rsllm_hip_mfma_issue_dev": ([_P, _S, _I, _I, _I, _I, _P], _I),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m rsllm_amd.build` "
            "(there is no CPU fallback)")
    # PyTorch-ROCm ships its own libamdhip64.so.7 (same SONAME as
    # /opt/rocm's). Loading torch first makes the dynamic linker bind this
    # library to torch's copy, so the process has ONE HIP runtime and torch
    # tensors, streams and events interoperate with these entry points. Two
    # runtimes in one process do not share devices.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


def _check(rc: int) -> None:
    if rc == OK:
        return
    d = _ErrorDetail()
    LIB.rsllm_hip_last_error(ctypes.byref(d))
    cls = _ERRORS.get(rc, Error)
    msg = (d.message or b"").decode(errors="replace")
    raise cls(msg, what=(d.what or b"").decode() or None, actual=d.actual, block=d.block,
              src_bytes=d.src_bytes, expected_bytes=d.expected_bytes)


def _host_ptr(a):
    if a is None:
        return None, 0
    if isinstance(a, (bytes, bytearray, memoryview)):
        a = np.frombuffer(a, dtype=np.uint8)
    if not isinstance(a, np.ndarray):
        raise TypeError("expected a numpy array or bytes")
    if not a.flags.c_contiguous:
        raise ValueError("array must be C-contiguous")
    return (a.ctypes.data_as(ctypes.c_void_p) if a.size else None), a.size


def _host_bytes(a):
    """Pointer and byte length of any C-contiguous array (or bytes)."""
    if isinstance(a, np.ndarray) and a.dtype != np.uint8:
        if not a.flags.c_contiguous:
            raise ValueError("array must be C-contiguous")
        a = a.reshape(-1).view(np.uint8)
    return _host_ptr(a)


def _host_f32(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32):
        raise TypeError(f"{name} must be a float32 numpy array")
    return _host_ptr(a)


# ---------------------------------------------------------------------------
# Host-pointer entry points (synchronous drop-ins)
# ---------------------------------------------------------------------------

def matmul_quant_f32(out: np.ndarray, weights, x: np.ndarray, n_tok: int, in_dim: int,
                     out_dim: int, dtype, tier: SimdTier = SimdTier.Scalar) -> None:
    """out[t*out_dim + o] = sum_i deq(W)[o, i] * x[t*in_dim + i] (overwrites ``out``)."""
    po, no = _host_f32(out, "out")
    pw, nw = _host_ptr(weights)
    px, nx = _host_f32(x, "x")
    _check(LIB.rsllm_hip_matmul_quant_f32(po, no, pw, nw, px, nx, n_tok, in_dim, out_dim,
                                          int(dtype), int(tier)))


def matmul_weight_f32(out: np.ndarray, weights, x: np.ndarray, n_tok: int, in_dim: int,
                      out_dim: int, dtype) -> None:
    """matmul_weight_f32 (rsllm-models/src/dsv4/weight.rs:113-169): dtype
    GgmlType.F32 takes ``weights`` as out_dim * in_dim f32 values (an f32
    array, or its bytes); any other dtype is matmul_quant_f32 on the blob, its
    errors reported as ShapeMismatch."""
    po, no = _host_f32(out, "out")
    pw, nw = _host_bytes(weights)
    px, nx = _host_f32(x, "x")
    _check(LIB.rsllm_hip_matmul_weight_f32(po, no, pw, nw, px, nx, n_tok, in_dim, out_dim,
                                           int(dtype)))


def matmul_weight_f32_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, x_ptr: int,
                          x_len: int, n_tok: int, in_dim: int, out_dim: int, dtype,
                          stream: int = 0) -> None:
    _check(LIB.rsllm_hip_matmul_weight_f32_dev(out_ptr or None, out_len, w_ptr or None, w_len,
                                               x_ptr or None, x_len, n_tok, in_dim, out_dim,
                                               int(dtype), stream or None))


def matmul_grouped_lora_down(out: np.ndarray, weights, x: np.ndarray, n_tok: int, n_groups: int,
                             group_dim: int, rank: int, dtype) -> None:
    """matmul_grouped_lora_down (weight.rs:209-266): x [n_tok x n_groups *
    group_dim] through n_groups stacked [rank x group_dim] weights into out
    [n_tok x n_groups * rank]."""
    po, no = _host_f32(out, "out")
    pw, nw = _host_bytes(weights)
    px, nx = _host_f32(x, "x")
    _check(LIB.rsllm_hip_matmul_grouped_lora_down(po, no, pw, nw, px, nx, n_tok, n_groups,
                                                  group_dim, rank, int(dtype)))


def matmul_grouped_lora_down_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, x_ptr: int,
                                 x_len: int, n_tok: int, n_groups: int, group_dim: int, rank: int,
                                 dtype, stream: int = 0) -> None:
    _check(LIB.rsllm_hip_matmul_grouped_lora_down_dev(out_ptr or None, out_len, w_ptr or None,
                                                      w_len, x_ptr or None, x_len, n_tok, n_groups,
                                                      group_dim, rank, int(dtype), stream or None))


def dequant_to_f32(dtype, src, dst: np.ndarray) -> None:
    ps, ns = _host_ptr(src)
    pd, nd = _host_f32(dst, "dst")
    _check(LIB.rsllm_hip_dequant_to_f32(int(dtype), ps, ns, pd, nd))


def register_weights(weights: np.ndarray, dtype, in_dim: int) -> None:
    pw, nw = _host_ptr(weights)
    _check(LIB.rsllm_hip_register_weights(pw, nw, int(dtype), in_dim))


def release_weights() -> None:
    _check(LIB.rsllm_hip_release_weights())


def device_allocations() -> int:
    """Device allocations the library has made in this process so far."""
    return int(LIB.rsllm_hip_device_allocations())


def stream_release(stream: int = 0) -> None:
    """Free the device workspace the library keeps for `stream` (before the
    caller destroys it)."""
    _check(LIB.rsllm_hip_stream_release(stream or None))


def model_upload(fingerprint: bytes, tensors) -> int:
    """Upload a whole checkpoint once (rsllm_hip_model_upload). ``tensors`` is
    a sequence of (name, array, dtype, in_dim); each array is the tensor's
    payload (C-contiguous, any dtype: its bytes are taken, e.g. a slice of an
    np.memmap of the GGUF file) and must outlive its use by host-pointer
    calls. Returns the model id."""
    if len(fingerprint) != 32:
        raise ValueError("fingerprint must be 32 bytes")
    descs = (TensorDesc * max(len(tensors), 1))()
    keep = []
    for i, (name, arr, dtype, in_dim) in enumerate(tensors):
        ptr, n = _host_bytes(arr)
        nm = name.encode()
        keep.append(nm)
        descs[i] = TensorDesc(nm, ptr.value if ptr is not None else None, n, int(dtype), in_dim)
    fp = ctypes.create_string_buffer(bytes(fingerprint), 32)
    mid = ctypes.c_uint64()
    _check(LIB.rsllm_hip_model_upload(fp, descs, len(tensors), ctypes.byref(mid)))
    return mid.value


def model_tensor(model: int, name: str):
    """(device address, byte length) of one tensor of an uploaded model."""
    dev, n = _P(), _S()
    _check(LIB.rsllm_hip_model_tensor(model, name.encode(), ctypes.byref(dev), ctypes.byref(n)))
    return dev.value or 0, n.value


def model_info(model: int) -> dict:
    info = ModelInfo()
    _check(LIB.rsllm_hip_model_info_get(model, ctypes.byref(info)))
    return {f: getattr(info, f) for f, _ in ModelInfo._fields_}


def model_release(model: int) -> None:
    _check(LIB.rsllm_hip_model_release(model))


def init(device: int = 0) -> None:
    _check(LIB.rsllm_hip_init(device))


# ---------------------------------------------------------------------------
# Device-pointer entry points: arguments are raw device addresses (ints, e.g.
# torch.Tensor.data_ptr()) with element counts, and a hipStream_t (int).
# ---------------------------------------------------------------------------

def matmul_quant_f32_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, x_ptr: int,
                         x_len: int, n_tok: int, in_dim: int, out_dim: int, dtype,
                         stream: int = 0) -> None:
    _check(LIB.rsllm_hip_matmul_quant_f32_dev(out_ptr or None, out_len, w_ptr or None, w_len,
                                              x_ptr or None, x_len, n_tok, in_dim, out_dim,
                                              int(dtype), stream or None))


NOALLOC_SCRATCH_BYTES = 48 << 20


def matmul_quant_f32_dev_noalloc(out_ptr: int, out_len: int, w_ptr: int, w_len: int, x_ptr: int,
                                 x_len: int, n_tok: int, in_dim: int, out_dim: int, dtype,
                                 stream: int = 0) -> None:
    """matmul_quant_f32_dev whose workspace is the library's static per-GPU
    array (NOALLOC_SCRATCH_BYTES): no allocation in the call. Calls that
    overlap on one GPU race on that array."""
    _check(LIB.rsllm_hip_matmul_quant_f32_dev_noalloc(out_ptr or None, out_len, w_ptr or None,
                                                      w_len, x_ptr or None, x_len, n_tok, in_dim,
                                                      out_dim, int(dtype), stream or None))


def xq_bytes(dtype, n_tok: int, in_dim: int) -> int:
    return LIB.rsllm_hip_xq_bytes(int(dtype), n_tok, in_dim)


def quantize_x_dev(dtype, x_ptr: int, x_len: int, n_tok: int, in_dim: int, xq_ptr: int,
                   xq_len: int, stream: int = 0) -> None:
    _check(LIB.rsllm_hip_quantize_x_dev(int(dtype), x_ptr or None, x_len, n_tok, in_dim,
                                        xq_ptr or None, xq_len, stream or None))


def matmul_prequant_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, xq_ptr: int,
                        xq_len: int, n_tok: int, in_dim: int, out_dim: int, dtype,
                        stream: int = 0) -> None:
    _check(LIB.rsllm_hip_matmul_prequant_dev(out_ptr or None, out_len, w_ptr or None, w_len,
                                             xq_ptr or None, xq_len, n_tok, in_dim, out_dim,
                                             int(dtype), stream or None))


def matmul_q4k_bf16_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, x_ptr: int,
                        x_len: int, n_tok: int, in_dim: int, out_dim: int, dtype,
                        stream: int = 0) -> None:
    """Prefill GEMM: Q4_K weights (GGUF bytes on the device) times bf16
    activations (``x_len`` 16-bit values), fp32 output on the MFMA path."""
    _check(LIB.rsllm_hip_matmul_q4k_bf16_dev(out_ptr or None, out_len, w_ptr or None, w_len,
                                             x_ptr or None, x_len, n_tok, in_dim, out_dim,
                                             int(dtype), stream or None))


def moe_routed(out: np.ndarray, x: np.ndarray, gate, up, down, ids: np.ndarray,
               weights: np.ndarray, n_tok: int, n_embd: int, n_ff: int, n_expert: int, k: int,
               dtype_gate_up, dtype_down, clamp: float = 10.0) -> None:
    """Routed experts (accumulate_moe_outputs): ``out`` [n_tok x n_embd] is
    accumulated into. gate/up/down are the stacked expert blobs (bytes)."""
    po, no = _host_f32(out, "out")
    px, nx = _host_f32(x, "x")
    pg, ng = _host_ptr(gate)
    pu, nu = _host_ptr(up)
    pd, nd = _host_ptr(down)
    if nu != ng:
        raise ShapeMismatch("moe_routed: gate and up blobs differ in size")
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    if ids.size != weights.size:
        raise ShapeMismatch("moe_routed: ids and weights differ in length")
    pi, ni = _host_ptr(ids)
    pw, _ = _host_ptr(weights)
    _check(LIB.rsllm_hip_moe_routed(po, no, px, nx, pg, pu, ng, pd, nd, pi, pw, ni, n_tok, n_embd,
                                    n_ff, n_expert, k, int(dtype_gate_up), int(dtype_down),
                                    clamp))


def moe_routed_dev(out_ptr: int, out_len: int, x_ptr: int, x_len: int, gate_ptr: int,
                   up_ptr: int, gate_up_len: int, down_ptr: int, down_len: int, ids_ptr: int,
                   weights_ptr: int, ids_len: int, n_tok: int, n_embd: int, n_ff: int,
                   n_expert: int, k: int, dtype_gate_up, dtype_down, clamp: float = 10.0,
                   stream: int = 0) -> None:
    _check(LIB.rsllm_hip_moe_routed_dev(out_ptr or None, out_len, x_ptr or None, x_len,
                                        gate_ptr or None, up_ptr or None, gate_up_len,
                                        down_ptr or None, down_len, ids_ptr or None,
                                        weights_ptr or None, ids_len, n_tok, n_embd, n_ff,
                                        n_expert, k, int(dtype_gate_up), int(dtype_down), clamp,
                                        stream or None))


def apply_shared_expert(out: np.ndarray, x: np.ndarray, gate, dtype_gate, up, dtype_up, down,
                        dtype_down, n_tok: int, n_embd: int, n_ff: int,
                        clamp: float = 10.0) -> None:
    """apply_shared_expert (rsllm-models/src/dsv4/moe.rs:422-455): every
    token of x [n_tok x n_embd] through one SwiGLU expert (apply_expert_swiglu
    :479-502) into ``out`` (overwritten). Each blob is F32 values (dtype
    GgmlType.F32) or quantized bytes of its own dtype."""
    po, no = _host_f32(out, "out")
    px, nx = _host_f32(x, "x")
    pg, ng = _host_bytes(gate)
    pu, nu = _host_bytes(up)
    pd, nd = _host_bytes(down)
    _check(LIB.rsllm_hip_apply_shared_expert(po, no, px, nx, pg, ng, int(dtype_gate), pu, nu,
                                             int(dtype_up), pd, nd, int(dtype_down), n_tok,
                                             n_embd, n_ff, clamp))


def apply_shared_expert_dev(out_ptr: int, out_len: int, x_ptr: int, x_len: int, gate_ptr: int,
                            gate_len: int, dtype_gate, up_ptr: int, up_len: int, dtype_up,
                            down_ptr: int, down_len: int, dtype_down, n_tok: int, n_embd: int,
                            n_ff: int, clamp: float = 10.0, stream: int = 0) -> None:
    _check(LIB.rsllm_hip_apply_shared_expert_dev(out_ptr or None, out_len, x_ptr or None, x_len,
                                                 gate_ptr or None, gate_len, int(dtype_gate),
                                                 up_ptr or None, up_len, int(dtype_up),
                                                 down_ptr or None, down_len, int(dtype_down),
                                                 n_tok, n_embd, n_ff, clamp, stream or None))


def quantize_q8_0_batch(x: np.ndarray, xq: np.ndarray, scale: np.ndarray, n_tok: int,
                        in_dim: int) -> None:
    """quantize_q8_0_batch (backend-cpu/src/ops/q8_0.rs:95-129): fills ``xq``
    (int8, n_tok * ceil(in_dim/32) * 32) and ``scale`` (float32)."""
    px, nx = _host_f32(x, "x")
    if not (isinstance(xq, np.ndarray) and xq.dtype == np.int8):
        raise TypeError("xq must be an int8 numpy array")
    pq, nq = _host_ptr(xq)
    ps, ns = _host_f32(scale, "scale")
    _check(LIB.rsllm_hip_quantize_q8_0_batch(px, nx, pq, nq, ps, ns, n_tok, in_dim))


def matmul_q8_0_batch(out: np.ndarray, weights, xq: np.ndarray, xscale: np.ndarray, n_tok: int,
                      in_dim: int, out_dim: int, tier: SimdTier = SimdTier.Scalar) -> None:
    """matmul_q8_0_batch (backend-cpu/src/ops/q8_0.rs:217-263): raw GGUF Q8_0
    weight rows times pre-quantised activations; ``out`` is overwritten."""
    po, no = _host_f32(out, "out")
    pw, nw = _host_ptr(weights)
    if not (isinstance(xq, np.ndarray) and xq.dtype == np.int8):
        raise TypeError("xq must be an int8 numpy array")
    pq, nq = _host_ptr(xq)
    ps, ns = _host_f32(xscale, "xscale")
    _check(LIB.rsllm_hip_matmul_q8_0_batch(po, no, pw, nw, pq, nq, ps, ns, n_tok, in_dim, out_dim,
                                           int(tier)))


def quantize_q8_0_batch_dev(x_ptr: int, x_len: int, xq_ptr: int, xq_len: int, scale_ptr: int,
                            scale_len: int, n_tok: int, in_dim: int, status_ptr: int = 0,
                            stream: int = 0) -> None:
    _check(LIB.rsllm_hip_quantize_q8_0_batch_dev(x_ptr or None, x_len, xq_ptr or None, xq_len,
                                                 scale_ptr or None, scale_len, n_tok, in_dim,
                                                 status_ptr or None, stream or None))


def matmul_q8_0_batch_dev(out_ptr: int, out_len: int, w_ptr: int, w_len: int, xq_ptr: int,
                          xq_len: int, xscale_ptr: int, xscale_len: int, n_tok: int, in_dim: int,
                          out_dim: int, stream: int = 0) -> None:
    _check(LIB.rsllm_hip_matmul_q8_0_batch_dev(out_ptr or None, out_len, w_ptr or None, w_len,
                                               xq_ptr or None, xq_len, xscale_ptr or None,
                                               xscale_len, n_tok, in_dim, out_dim,
                                               stream or None))


def prepare_weights_dev(dst_ptr: int, src_ptr: int, nbytes: int, dtype, in_dim: int,
                        stream: int = 0) -> None:
    _check(LIB.rsllm_hip_prepare_weights_dev(dst_ptr or None, src_ptr or None, nbytes, int(dtype),
                                             in_dim, stream or None))


def dequant_to_f32_dev(dtype, src_ptr: int, src_len: int, dst_ptr: int, dst_len: int,
                       stream: int = 0) -> None:
    _check(LIB.rsllm_hip_dequant_to_f32_dev(int(dtype), src_ptr or None, src_len, dst_ptr or None,
                                            dst_len, stream or None))


def stream_read_dev(p: int, nbytes: int, sink_ptr: int, sink_len: int, n_wg: int, threads: int,
                    unroll: int, contiguous: bool, stream: int = 0) -> None:
    """Measurement aid (no reference counterpart): a pure streaming read of
    nbytes at device pointer p."""
    _check(LIB.rsllm_hip_stream_read_dev(p or None, nbytes, sink_ptr or None, sink_len, n_wg,
                                         threads, unroll, int(bool(contiguous)), stream or None))


def mfma_issue_dev(sink_ptr: int, sink_len: int, n_wg: int, iters: int, valu_per_group: int,
                   two_per_cu: bool = False, stream: int = 0) -> None:
    """Measurement aid (no reference counterpart): the matrix-core issue
    ceiling, 128 * iters v_mfma_f32_16x16x32_f16 per wavefront with
    valu_per_group packed-f16 FMAs after every four."""
    _check(LIB.rsllm_hip_mfma_issue_dev(sink_ptr or None, sink_len, n_wg, iters, valu_per_group,
                                        int(bool(two_per_cu)), stream or None))


# ---------------------------------------------------------------------------
# Backend handle
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class BackendCapability:
    backend: str
    arch: str
    q4k_matmul: bool
    q6k_matmul: bool
    q8_0_matmul: bool
    q2k_matmul: bool
    iq2xxs_matmul: bool
    fp8_kv_cache: bool


class HipBackend:
    """Analogue of ``CpuBackend``: cheap, stateless, shareable."""

    def kind(self) -> str:
        return "Rocm"

    def capability(self) -> BackendCapability:
        c = _Capability()
        LIB.rsllm_hip_capability_get(ctypes.byref(c))
        return BackendCapability(c.backend.decode(), c.arch.decode(), bool(c.q4k_matmul),
                                 bool(c.q6k_matmul), bool(c.q8_0_matmul), bool(c.q2k_matmul),
                                 bool(c.iq2xxs_matmul), bool(c.fp8_kv_cache))


__all__ = [
    "GgmlType", "SimdTier", "Error", "ShapeMismatch", "NotBlockAligned", "NonFiniteInput",
    "UnsupportedTier", "DequantSizeMismatch", "UnsupportedDequant", "DeviceError",
    "InvalidArgument", "Unimplemented", "matmul_quant_f32", "dequant_to_f32", "register_weights",
    "release_weights", "init", "matmul_quant_f32_dev", "prepare_weights_dev",
    "dequant_to_f32_dev", "xq_bytes", "quantize_x_dev", "matmul_prequant_dev",
    "matmul_q4k_bf16_dev", "moe_routed", "moe_routed_dev", "quantize_q8_0_batch",
    "matmul_q8_0_batch", "quantize_q8_0_batch_dev", "matmul_q8_0_batch_dev", "HipBackend",
    "BackendCapability", "LIB", "LIB_PATH", "SIGNATURES",
]
