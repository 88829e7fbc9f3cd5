"""The C-ABI library loads (no GPU needed) and exports every entry point that
include/rsllm_hip.h (the drop-in boundary) and include/rsllm_hip_probe.h
(the benchmark's measurement aids) declare; the Python mirror declares a
signature for each of them. No compute calls are made."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rsllm_hip.h")
PROBE_HEADER = os.path.join(ROOT, "include", "rsllm_hip_probe.h")


def declared_functions(headers=(HEADER, PROBE_HEADER)):
    text = "".join(open(h).read() for h in headers)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)  # drop comments
    names = re.findall(r"^\s*(?:int|size_t|void|uint64_t)\s+(rsllm_hip_\w+)\s*\(", text, flags=re.M)
    assert names, "no declarations parsed from the header"
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions((HEADER,))
    assert not any(n.endswith(("_stream_read_dev", "_mfma_issue_dev")) for n in names)
    for required in ("rsllm_hip_matmul_quant_f32", "rsllm_hip_matmul_quant_f32_dev",
                     "rsllm_hip_dequant_to_f32", "rsllm_hip_release_weights",
                     "rsllm_hip_matmul_q4k_bf16_dev"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from rsllm_amd import backend as B
    lib = ctypes.CDLL(B.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_mirror_covers_every_symbol():
    from rsllm_amd import backend as B
    assert sorted(B.SIGNATURES) == declared_functions()


def test_product_does_not_link_the_oracle():
    from rsllm_amd import backend as B
    blob = open(B.LIB_PATH, "rb").read()
    assert b"orc_" not in blob and b"rsllm_oracle" not in blob
