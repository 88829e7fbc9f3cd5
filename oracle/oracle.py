"""Python access to the CPU oracle (test infrastructure only).

Two independent restatements of the reference's dequantizers live here:

* ``lib()``: ctypes binding of ``oracle/librsllm_oracle.so``, the C
  restatement that follows the reference operation by operation (see the
  citations in ``rsllm_oracle.c``). It is the parity oracle and the CPU
  baseline.
* ``np_dequant_*``: vectorised numpy restatements written from the block
  layouts alone (q4_k.rs:8-26, q6_k.rs:8-25, q8_0.rs:6-13, q2_k.rs:9-31,
  iq2_xxs.rs:12-33, q4_0.rs:19-28, q5_k.rs:6-24, q8_k.rs:12-23). They share no
  code with the C file and are used to cross-check it over every block of
  seeded data.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "librsllm_oracle.so")

OK, SHAPE_MISMATCH, NOT_BLOCK_ALIGNED, NON_FINITE_INPUT = 0, 1, 2, 3
DEQUANT_SIZE_MISMATCH, UNSUPPORTED_DEQUANT, PANIC = 5, 6, 9

F32, F16, Q4_0, Q8_0, Q2_K, Q4_K, Q6_K, IQ2_XXS, BF16 = 0, 1, 2, 8, 10, 12, 14, 16, 30
Q4_1, Q5_K, Q8_K = 3, 13, 15
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210), Q2_K: (256, 84), IQ2_XXS: (256, 66),
         Q4_1: (32, 20), Q5_K: (256, 176), Q8_K: (256, 292)}

_lib = None


def build() -> None:
    subprocess.run(["bash", os.path.join(HERE, "build.sh")], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(SO):
            build()
        L = ctypes.CDLL(SO)
        P, S, U32, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_q4k_scale_min.argtypes = [I, P, P, P]
        L.orc_dequant_to_f32.argtypes = [U32, P, S, P, S]
        L.orc_matmul_quant_f32.argtypes = [P, S, P, S, P, S, S, S, S, U32, I, I]
        L.orc_matmul_quant_f32_rows.argtypes = [P, P, P, S, S, S, U32, S, S, I]
        L.orc_quantize_q8_0_activation.argtypes = [P, S, P, S, P, S]
        L.orc_quantize_q8_0_batch.argtypes = [P, S, P, S, P, S, S, S]
        L.orc_dot_q8_0_row_scalar.argtypes = [P, P, P, S]
        L.orc_dot_q8_0_row_scalar.restype = ctypes.c_float
        L.orc_matmul_q8_0_batch.argtypes = [P, S, P, S, P, S, P, S, S, S, S, I]
        L.orc_silu.argtypes = [ctypes.c_float]
        L.orc_silu.restype = ctypes.c_float
        L.orc_sigmoid.argtypes = [ctypes.c_float]
        L.orc_sigmoid.restype = ctypes.c_float
        L.orc_swiglu_clamp.argtypes = [P, P, S, ctypes.c_float]
        L.orc_swiglu_clamp.restype = None
        L.orc_moe_routed.argtypes = [P, P, S, S, S, P, P, P, U32, U32, S, P, P, S, ctypes.c_float]
        L.orc_matmul_weight_f32.argtypes = [P, S, P, S, P, S, S, S, S, U32, I]
        L.orc_matmul_grouped_lora_down.argtypes = [P, S, P, S, P, S, S, S, S, S, U32, I]
        L.orc_apply_shared_expert.argtypes = [P, S, P, S, P, S, U32, P, S, U32, P, S, U32, S, S, S,
                                              ctypes.c_float]
        L.orc_last_detail.argtypes = [P, P]
        L.orc_iq2xxs_grid.argtypes = [I]
        L.orc_iq2xxs_grid.restype = ctypes.c_uint64
        L.orc_num_cores.restype = I
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None and a.size else None


def last_detail():
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    lib().orc_last_detail(ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def q4k_scale_min(j: int, q12: np.ndarray):
    sc, m = ctypes.c_uint8(), ctypes.c_uint8()
    q = np.ascontiguousarray(q12, dtype=np.uint8)
    lib().orc_q4k_scale_min(j, _p(q), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequant(dtype: int, src: np.ndarray, n: int):
    """Returns (status, float32[n])."""
    src = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1)
    dst = np.zeros(n, dtype=np.float32)
    rc = lib().orc_dequant_to_f32(dtype, _p(src), src.size, _p(dst), n)
    return rc, dst


def matmul_quant_f32(w, x, n_tok, in_dim, out_dim, dtype, allow_q6k=True, n_threads=0, out_len=None):
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n_out = n_tok * out_dim if out_len is None else out_len
    out = np.full(max(n_out, 0), np.nan, dtype=np.float32)
    rc = lib().orc_matmul_quant_f32(_p(out), out.size, _p(w), w.size, _p(x), x.size, n_tok, in_dim,
                                    out_dim, dtype, int(allow_q6k), n_threads)
    return rc, out


def _weight_bytes(w):
    """Byte view of a weight blob: f32 arrays keep their bytes."""
    w = np.ascontiguousarray(w)
    return w.reshape(-1).view(np.uint8)


def matmul_weight_f32(w, x, n_tok, in_dim, out_dim, dtype, allow_q6k=True, out_len=None):
    """Returns (status, out); ``w`` is float32 for dtype F32, else bytes."""
    wb = _weight_bytes(w)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n_out = n_tok * out_dim if out_len is None else out_len
    out = np.full(max(n_out, 0), np.nan, dtype=np.float32)
    rc = lib().orc_matmul_weight_f32(_p(out), out.size, _p(wb), wb.size, _p(x), x.size, n_tok,
                                     in_dim, out_dim, dtype, int(allow_q6k))
    return rc, out


def matmul_grouped_lora_down(w, x, n_tok, n_groups, group_dim, rank, dtype, allow_q6k=True,
                             out_len=None):
    """Returns (status, out); out starts as NaN so unwritten groups show."""
    wb = _weight_bytes(w)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n_out = n_tok * n_groups * rank if out_len is None else out_len
    out = np.full(max(n_out, 0), np.nan, dtype=np.float32)
    rc = lib().orc_matmul_grouped_lora_down(_p(out), out.size, _p(wb), wb.size, _p(x), x.size,
                                            n_tok, n_groups, group_dim, rank, dtype,
                                            int(allow_q6k))
    return rc, out


def matmul_quant_f32_rows(w, x, n_tok, in_dim, out_dim, dtype, row0, row1, n_threads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(n_tok * out_dim, dtype=np.float32)
    rc = lib().orc_matmul_quant_f32_rows(_p(out), _p(w), _p(x), n_tok, in_dim, out_dim, dtype,
                                         row0, row1, n_threads)
    assert rc == OK
    return out


def quantize_q8_0_activation(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    blocks = (x.size + 31) // 32
    xq = np.full(blocks * 32, 99, dtype=np.int8)
    sc = np.zeros(blocks, dtype=np.float32)
    rc = lib().orc_quantize_q8_0_activation(_p(x), x.size, _p(xq), xq.size, _p(sc), sc.size)
    return rc, xq, sc


def quantize_q8_0_batch(x: np.ndarray, n_tok: int, in_dim: int):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    blocks = (in_dim + 31) // 32
    xq = np.zeros(n_tok * blocks * 32, dtype=np.int8)
    sc = np.zeros(n_tok * blocks, dtype=np.float32)
    rc = lib().orc_quantize_q8_0_batch(_p(x), x.size, _p(xq), xq.size, _p(sc), sc.size, n_tok, in_dim)
    return rc, xq, sc


def dot_q8_0_row_scalar(row, xq, xscale, in_dim) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xscale = np.ascontiguousarray(xscale, dtype=np.float32)
    return lib().orc_dot_q8_0_row_scalar(_p(row), _p(xq), _p(xscale), in_dim)


def matmul_q8_0_batch(w, xq, xscale, n_tok, in_dim, out_dim, n_threads=0):
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1)
    xscale = np.ascontiguousarray(xscale, dtype=np.float32).reshape(-1)
    out = np.full(n_tok * out_dim, np.nan, dtype=np.float32)
    rc = lib().orc_matmul_q8_0_batch(_p(out), out.size, _p(w), w.size, _p(xq), xq.size, _p(xscale),
                                     xscale.size, n_tok, in_dim, out_dim, n_threads)
    return rc, out


def silu(x: float) -> float:
    return lib().orc_silu(x)


def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def swiglu_clamp(gate: np.ndarray, up: np.ndarray, c: float):
    """apply_swiglu_clamp on copies; returns (gate, up)."""
    g = np.ascontiguousarray(gate, dtype=np.float32).copy()
    u = np.ascontiguousarray(up, dtype=np.float32).copy()
    assert g.size == u.size
    lib().orc_swiglu_clamp(_p(g), _p(u), g.size, ctypes.c_float(c))
    return g, u


def moe_routed(out, x, n_tok, n_embd, n_ff, gate, up, down, dtype_gu, dtype_down, n_expert, ids,
               weights, k, clamp):
    """Accumulates into ``out`` (float32 [n_tok*n_embd]) in place; returns status."""
    assert out.dtype == np.float32 and out.flags.c_contiguous
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    return lib().orc_moe_routed(_p(out), _p(x), n_tok, n_embd, n_ff, _p(gate), _p(up), _p(down),
                                dtype_gu, dtype_down, n_expert, _p(ids), _p(weights), k,
                                ctypes.c_float(clamp))


def apply_shared_expert(x, gate, dt_gate, up, dt_up, down, dt_down, n_tok, n_embd, n_ff, clamp,
                        out_len=None):
    """Returns (status, out); weights are float32 arrays for F32, else bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    g, u, d = _weight_bytes(gate), _weight_bytes(up), _weight_bytes(down)
    n_out = n_tok * n_embd if out_len is None else out_len
    out = np.full(max(n_out, 0), np.nan, dtype=np.float32)
    rc = lib().orc_apply_shared_expert(_p(out), out.size, _p(x), x.size, _p(g), g.size, dt_gate,
                                       _p(u), u.size, dt_up, _p(d), d.size, dt_down, n_tok, n_embd,
                                       n_ff, ctypes.c_float(clamp))
    return rc, out


def num_cores() -> int:
    return lib().orc_num_cores()


# --------------------------------------------------------------------------
# Independent numpy restatement (written from the block layouts).
# --------------------------------------------------------------------------

def _f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32).reshape(-1)


def np_scale_min(q12: np.ndarray):
    """[n, 12] -> (sc[n, 8], m[n, 8]) by bit fields: sub-blocks 0-3 use the
    low 6 bits of bytes 0-3 (scales) and 4-7 (mins); sub-blocks 4-7 take the
    low/high nibble of bytes 8-11 as bits 0-3 and bits 6-7 of bytes 0-3
    (scales) / 4-7 (mins) as bits 4-5."""
    q = q12.astype(np.uint32)
    sc = np.empty((q.shape[0], 8), np.uint32)
    m = np.empty((q.shape[0], 8), np.uint32)
    sc[:, :4] = q[:, 0:4] & 63
    m[:, :4] = q[:, 4:8] & 63
    sc[:, 4:] = (q[:, 8:12] & 15) | ((q[:, 0:4] >> 6) << 4)
    m[:, 4:] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    return sc, m


def np_dequant_q4k(src: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1, 144)
    d = _f16(b[:, 0:2])[:, None]
    dmin = _f16(b[:, 2:4])[:, None]
    sc, m = np_scale_min(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32)                    # [n, pair, l]
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)  # [n, j, l]
    ds = (d * sc.astype(np.float32)).astype(np.float32)  # exact products
    mm = (dmin * m.astype(np.float32)).astype(np.float32)
    prod = (ds[:, :, None] * q).astype(np.float32)
    return (prod - mm[:, :, None]).astype(np.float32).reshape(-1)


def np_q6k_values(src: np.ndarray):
    """[n, 256] integer q-32 and [n, 256] int8 scale for every element."""
    b = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1, 210)
    n = b.shape[0]
    e = np.arange(256)
    h, k, l = e // 128, (e % 128) // 32, e % 32
    ql_idx = 64 * h + l + 32 * (k % 2)
    nib = b[:, ql_idx].astype(np.int32)
    nib = np.where(k >= 2, nib >> 4, nib & 15)
    hi = (b[:, 128 + 32 * h + l].astype(np.int32) >> (2 * k)) & 3
    q = (nib | (hi << 4)) - 32
    sc = b[:, 192:208].view(np.int8)[:, e // 16].astype(np.int32)
    return q.reshape(n, 256), sc.reshape(n, 256)


def np_dequant_q6k(src: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1, 210)
    d = _f16(b[:, 208:210])[:, None]
    q, sc = np_q6k_values(b)
    return ((d * sc.astype(np.float32)).astype(np.float32) * q.astype(np.float32)).astype(np.float32).reshape(-1)


def np_dequant_q8_0(src: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1, 34)
    d = _f16(b[:, 0:2])[:, None]
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d).astype(np.float32).reshape(-1)


def np_dequant_q2k(src: np.ndarray) -> np.ndarray:
    """Q2_K from the block layout (q2_k.rs:9-31), vectorised: element e of a
    block: sub-block e // 16, code at shift 2 ((e % 128) // 32) of qs byte
    32 (e // 128) + e % 32; (d * sc) * q - dmin * m in float32."""
    b = np.asarray(src, np.uint8).reshape(-1, 84)
    d = b[:, 80:82].copy().view(np.float16).astype(np.float32)
    dmin = b[:, 82:84].copy().view(np.float16).astype(np.float32)
    e = np.arange(256)
    sc = b[:, e // 16]
    byte = b[:, 16 + 32 * (e // 128) + e % 32]
    q = ((byte >> (2 * ((e % 128) // 32))) & 3).astype(np.float32)
    dl = (d * (sc & 15).astype(np.float32)).astype(np.float32)
    ml = (dmin * (sc >> 4).astype(np.float32)).astype(np.float32)
    return ((dl * q).astype(np.float32) - ml).astype(np.float32).reshape(-1)


def np_dequant_q4_1(src: np.ndarray) -> np.ndarray:
    """Q4_1 from the block layout (q4_0.rs:19-28): [d f16 | m f16 | 16 code
    bytes], element j < 16 the low nibble of byte j, j >= 16 the high nibble
    of byte j - 16; code * d + m in float32."""
    b = np.asarray(src, np.uint8).reshape(-1, 20)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    m = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    qs = b[:, 4:20]
    code = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)
    return ((code * d).astype(np.float32) + m).astype(np.float32).reshape(-1)


def np_dequant_q5k(src: np.ndarray) -> np.ndarray:
    """Q5_K from the block layout (q5_k.rs:6-24): [d | dmin | scales 12 |
    qh 32 | qs 128]; element 32 j + l (sub-block j) has low bits from the
    low (even j) or high (odd j) nibble of qs[32 (j // 2) + l] and bit 4
    from bit j of qh[l]; (d * sc_j) * q - dmin * m_j in float32."""
    b = np.asarray(src, np.uint8).reshape(-1, 176)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    sc, m = np_scale_min(b[:, 4:16])
    qh = b[:, 16:48].astype(np.uint32)
    qs = b[:, 48:176].reshape(-1, 4, 32).astype(np.uint32)
    j = np.arange(8)
    nib = np.where((j % 2 == 0)[None, :, None], qs[:, j // 2, :] & 15, qs[:, j // 2, :] >> 4)
    hb = (qh[:, None, :] >> j[None, :, None]) & 1
    q = (nib | (hb << 4)).astype(np.float32)                     # [n, j, l]
    ds = (d * sc.astype(np.float32)).astype(np.float32)
    mm = (dmin * m.astype(np.float32)).astype(np.float32)
    return ((ds[:, :, None] * q).astype(np.float32) - mm[:, :, None]).astype(np.float32).reshape(-1)


def np_dequant_q8k(src: np.ndarray) -> np.ndarray:
    """Q8_K from the block layout (q8_k.rs:12-23): [d f32 | qs 256 int8 |
    bsums]; d * q in float32."""
    b = np.asarray(src, np.uint8).reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32)
    q = b[:, 4:260].view(np.int8).astype(np.float32)
    return (d * q).astype(np.float32).reshape(-1)


def iq2xxs_grid() -> np.ndarray:
    """The IQ2_XXS codebook as [256, 8] int8 (from the C restatement)."""
    g = np.array([lib().orc_iq2xxs_grid(i) for i in range(256)], np.uint64)
    return g.view(np.uint8).reshape(256, 8).view(np.int8)


def np_dequant_iq2xxs(src: np.ndarray) -> np.ndarray:
    """IQ2_XXS from the block layout (iq2_xxs.rs:12-33), vectorised; the sign
    byte of index i is i with bit 7 = parity(i)."""
    b = np.asarray(src, np.uint8).reshape(-1, 66)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    aux = b[:, 2:66].copy().view(np.uint32).reshape(-1, 8, 2)
    grid = iq2xxs_grid().astype(np.float32)
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    db = (d[:, None] * (np.float32(0.5) + (aux[:, :, 1] >> 28).astype(np.float32)) *
          np.float32(0.25)).astype(np.float32)
    for l in range(4):
        gi = (aux[:, :, 0] >> (8 * l)) & 0xFF
        si = (aux[:, :, 1] >> (7 * l)) & 0x7F
        par = np.zeros_like(si)
        for bit in range(7):
            par ^= (si >> bit) & 1
        signs = si | (par << 7)
        neg = ((signs[:, :, None] >> np.arange(8)) & 1).astype(bool)
        v = (db[:, :, None] * grid[gi]).astype(np.float32)
        out[:, :, l, :] = np.where(neg, -v, v)
    return out.reshape(-1)


NP_DEQUANT = {Q4_K: np_dequant_q4k, Q6_K: np_dequant_q6k, Q8_0: np_dequant_q8_0,
              Q2_K: np_dequant_q2k, IQ2_XXS: np_dequant_iq2xxs, Q4_1: np_dequant_q4_1,
              Q5_K: np_dequant_q5k, Q8_K: np_dequant_q8k}
