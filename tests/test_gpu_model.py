"""Whole-model residency (rsllm_hip_model_upload) on the GPU: a synthetic
GGUF-like checkpoint written to a file and memory-mapped, as GgufFile::open
maps the real one (rsllm-gguf/src/file.rs:81-97), with tensor payloads
borrowed from the mapping (tensor_bytes :181-187).

* Every resident tensor is byte-identical to what the per-tensor path holds:
  the GGUF bytes for Q4_K / F32 / F16, rsllm_hip_prepare_weights_dev of the
  whole tensor for the converted formats, including tensors larger than one
  staging chunk and block counts that are not multiples of 8.
* Host-pointer matmuls on the mapped ranges use the resident copies and agree
  with the oracle (1e-3) and, bit for bit, with the same calls after release
  (weights uploaded per call).
* Reuse by fingerprint + tensor table + full payload hash (a byte changed
  outside the sampled windows gives a new model), and release."""
import ctypes
import os

import numpy as np
import pytest

from conftest import REL_TOL, rel_err
from rsllm_amd import synth
from rsllm_amd.ggml import GgmlType as G

pytestmark = pytest.mark.gpu

FP = bytes(range(100, 132))


def _hip_runtime():
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            L = ctypes.CDLL(name)
            L.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            return L
        except OSError:
            continue
    raise RuntimeError("libamdhip64.so not found")


def device_bytes(ptr, n):
    out = np.empty(n, np.uint8)
    assert _hip_runtime().hipMemcpy(out.ctypes.data, ptr, n, 2) == 0  # device -> host
    return out


def checkpoint_spec():
    """(name, payload, dtype, in_dim): a layer's worth of DS-V4-like tensors."""
    f32 = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    f16 = np.random.default_rng(2).standard_normal(1000).astype(np.float16)
    return [
        ("token_embd.weight", f16.view(np.uint8), G.F16, 0),
        ("output_norm.weight", f32.view(np.uint8), G.F32, 4096),
        ("blk.0.attn_q_a.weight", synth.weight(G.Q8_0, 300, 512, 3), G.Q8_0, 512),
        ("blk.0.attn_output_a.weight", synth.weight(G.Q8_0, 8 * 64, 1024, 4), G.Q8_0, 1024),
        ("blk.0.ffn_gate_exps.weight", synth.weight(G.IQ2_XXS, 4 * 256, 512, 5), G.IQ2_XXS, 512),
        ("blk.0.ffn_up_exps.weight", synth.weight(G.IQ2_XXS, 4 * 256, 512, 6), G.IQ2_XXS, 512),
        ("blk.0.ffn_down_exps.weight", synth.weight(G.Q2_K, 4 * 512, 256, 7), G.Q2_K, 256),
        ("blk.0.ffn_up_shexp.weight", synth.weight(G.Q6_K, 257, 1024, 8), G.Q6_K, 1024),
        ("blk.0.attn_output.weight", synth.weight(G.Q4_K, 96, 2048, 9), G.Q4_K, 2048),
        ("blk.0.attn_kv.weight", synth.weight(G.Q4_0, 64, 256, 10), G.Q4_0, 256),
        # larger than one 64 MiB staging chunk: 2 chunks each
        ("blk.1.ffn_big.weight", synth.weight(G.Q6_K, 20000, 4096, 11), G.Q6_K, 4096),
        ("blk.1.ffn_big_q4k.weight", synth.weight(G.Q4_K, 30000, 4096, 12), G.Q4_K, 4096),
    ]


def write_and_map(path, spec):
    """Write the payloads at 32-byte aligned offsets (GGUF's default
    alignment, file.rs:29) and map the file read-only."""
    offs, pos = [], 0
    with open(path, "wb") as f:
        for _, arr, _, _ in spec:
            pad = (-pos) % 32
            f.write(b"\0" * pad)
            pos += pad
            offs.append(pos)
            b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
            f.write(b.tobytes())
            pos += b.size
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    views = []
    for (name, arr, dt, in_dim), o in zip(spec, offs):
        n = np.ascontiguousarray(arr).view(np.uint8).size
        views.append((name, mm[o:o + n], dt, in_dim))
    return mm, views


@pytest.fixture(scope="module")
def mapped(tmp_path_factory):
    spec = checkpoint_spec()
    path = os.path.join(tmp_path_factory.mktemp("gguf"), "model.bin")
    mm, views = write_and_map(path, spec)
    yield spec, views
    del mm


def prepared_reference(hip, arr, dtype, in_dim):
    import torch
    raw = torch.from_numpy(np.array(arr, copy=True)).cuda()  # a writable copy (arr may be a read-only view)
    out = torch.empty_like(raw)
    hip.prepare_weights_dev(out.data_ptr(), raw.data_ptr(), raw.numel(), dtype, in_dim,
                            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_resident_bytes_match_the_per_tensor_layout(hip, mapped):
    spec, views = mapped
    mid = hip.model_upload(FP, views)
    try:
        info = hip.model_info(mid)
        total = sum(v[1].size for v in views)
        assert info["uploaded_bytes"] == total and info["n_tensors"] == len(views)
        assert info["device_bytes"] >= total and info["refs"] == 1
        print(f"upload {total / 1e6:.1f} MB in {info['upload_seconds'] * 1e3:.1f} ms")
        for name, view, dt, in_dim in views:
            ptr, n = hip.model_tensor(mid, name)
            assert n == view.size and ptr % 256 == 0
            got = device_bytes(ptr, n)
            if dt in (G.Q6_K, G.Q8_0, G.Q4_0, G.Q2_K, G.IQ2_XXS) and in_dim:
                want = prepared_reference(hip, view, dt, in_dim)
            else:
                want = np.asarray(view)
            assert np.array_equal(got, want), name
    finally:
        hip.model_release(mid)


def test_host_calls_use_resident_copies(oracle, hip, mapped):
    spec, views = mapped
    by = {v[0]: v for v in views}
    mid = hip.model_upload(FP, views)
    results = {}
    try:
        # plain matmuls on the mapped ranges
        for name in ("blk.0.attn_q_a.weight", "blk.0.ffn_up_shexp.weight",
                     "blk.0.attn_output.weight", "blk.0.attn_kv.weight", "blk.1.ffn_big.weight"):
            _, w, dt, in_dim = by[name]
            out_dim = w.size // (in_dim // dt.block_elements() * dt.block_bytes())
            x = synth.activations(3, in_dim, 5).reshape(-1)
            got = np.full(3 * out_dim, np.nan, np.float32)
            hip.matmul_quant_f32(got, w, x, 3, in_dim, out_dim, dt)
            rc, want = oracle.matmul_quant_f32(np.asarray(w), x, 3, in_dim, out_dim, int(dt))
            assert rc == 0 and rel_err(got, want) <= REL_TOL, name
            results[name] = (got, w, x, in_dim, out_dim, dt)
        # the F32 norm through matmul_weight_f32 (one row of 4096)
        _, wn, _, _ = by["output_norm.weight"]
        xn = synth.activations(2, 4096, 6).reshape(-1)
        got_n = np.full(2, np.nan, np.float32)
        hip.matmul_weight_f32(got_n, wn, xn, 2, 4096, 1, G.F32)
        rc, want_n = oracle.matmul_weight_f32(np.asarray(wn), xn, 2, 4096, 1, oracle.F32)
        assert rc == 0 and rel_err(got_n, want_n) <= REL_TOL
        # grouped LoRA-down over the stacked [8 x 64 x 1024] Q8_0 tensor
        _, wl, _, _ = by["blk.0.attn_output_a.weight"]
        xl = synth.activations(2, 8 * 1024, 7)
        got_l = np.full(2 * 8 * 64, np.nan, np.float32)
        hip.matmul_grouped_lora_down(got_l, wl, xl.reshape(-1), 2, 8, 1024, 64, G.Q8_0)
        rc, want_l = oracle.matmul_grouped_lora_down(np.asarray(wl), xl, 2, 8, 1024, 64,
                                                     int(G.Q8_0))
        assert rc == 0 and rel_err(got_l, want_l) <= REL_TOL
        # routed experts on the stacked IQ2_XXS / Q2_K tensors (4 experts)
        g, u, d = (by[f"blk.0.ffn_{m}_exps.weight"][1] for m in ("gate", "up", "down"))
        xm = synth.activations(2, 512, 8)
        ids, wts = synth.moe_routing(2, 4, 2, 9)
        got_m = np.zeros(2 * 512, np.float32)
        hip.moe_routed(got_m, xm.reshape(-1), g, u, d, ids, wts, 2, 512, 256, 4, 2, G.IQ2_XXS,
                       G.Q2_K, 10.0)
        want_m = np.zeros(2 * 512, np.float32)
        assert oracle.moe_routed(want_m, xm, 2, 512, 256, np.asarray(g), np.asarray(u),
                                 np.asarray(d), int(G.IQ2_XXS), int(G.Q2_K), 4, ids, wts, 2,
                                 10.0) == 0
        assert rel_err(got_m, want_m) <= REL_TOL
    finally:
        hip.model_release(mid)
    # after release the same calls upload per call: bit-identical results
    for name, (got, w, x, in_dim, out_dim, dt) in results.items():
        again = np.full(got.size, np.nan, np.float32)
        hip.matmul_quant_f32(again, w, x, 3, in_dim, out_dim, dt)
        assert np.array_equal(again.view(np.uint32), got.view(np.uint32)), name


def test_reuse_by_fingerprint_and_release(hip, mapped, tmp_path):
    spec, views = mapped
    a = hip.model_upload(FP, views)
    try:
        b = hip.model_upload(FP, views)             # same file, same table: reused
        assert b == a and hip.model_info(a)["refs"] == 2
        other_fp = bytes(32)
        c = hip.model_upload(other_fp, views[:4])   # another fingerprint: a new model
        assert c != a and hip.model_info(c)["refs"] == 1
        # same fingerprint, table and content at other host addresses: reused
        copies = [(n, np.array(v), dt, k) for n, v, dt, k in views[:4]]
        assert hip.model_upload(other_fp, copies) == c
        assert hip.model_info(c)["refs"] == 2
        # one byte changed outside the 16 sampled windows (byte 300 of a
        # 557 KB tensor: the windows start at 0, 37 KB, 74 KB, ...): the full
        # payload hash tells it apart, a new model
        assert copies[3][1].size > 16 * 4096
        copies[3][1][300] ^= 0x01
        e = hip.model_upload(other_fp, copies)
        assert e not in (a, c)
        assert hip.model_info(e)["uploaded_bytes"] == sum(v[1].size for v in copies)
        ptr, n = hip.model_tensor(e, copies[3][0])
        assert np.array_equal(device_bytes(ptr, n), prepared_reference(hip, copies[3][1], copies[3][2],
                                                                       copies[3][3]))
        # the same changed bytes again: that model is reused
        assert hip.model_upload(other_fp, copies) == e
        # one sampled byte changed: a new model
        copies[2][1][0] ^= 0xFF
        d = hip.model_upload(other_fp, copies)
        assert d not in (a, c, e)
        assert hip.model_info(d)["uploaded_bytes"] == sum(v[1].size for v in copies)
        for m in (d, e, e, c, c):
            hip.model_release(m)
        with pytest.raises(hip.InvalidArgument):
            hip.model_info(c)
        hip.model_release(b)
        assert hip.model_info(a)["refs"] == 1
        name = views[2][0]
        ptr, n = hip.model_tensor(a, name)
        assert n == views[2][1].size
    finally:
        hip.model_release(a)
    with pytest.raises(hip.InvalidArgument):
        hip.model_info(a)


def test_release_weights_leaves_models_alone(oracle, hip, mapped):
    spec, views = mapped
    mid = hip.model_upload(FP, views[:3])
    try:
        hip.release_weights()
        assert hip.model_info(mid)["refs"] == 1
        _, w, dt, in_dim = views[2]
        x = synth.activations(1, in_dim, 3).reshape(-1)
        out_dim = w.size // (in_dim // 32 * 34)
        got = np.full(out_dim, np.nan, np.float32)
        hip.matmul_quant_f32(got, w, x, 1, in_dim, out_dim, dt)
        rc, want = oracle.matmul_quant_f32(np.asarray(w), x, 1, in_dim, out_dim, int(dt))
        assert rel_err(got, want) <= REL_TOL
    finally:
        hip.model_release(mid)
