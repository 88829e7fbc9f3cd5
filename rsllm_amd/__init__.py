"""rsllm_amd — MI355X (gfx950) quantized mat-vec / mat-mul backend for rsLLM.

``rsllm_amd.backend`` binds the C ABI of librsllm_hip.so (include/rsllm_hip.h)
and mirrors rsllm-backend-cpu's operator interface. ``rsllm_amd.synth`` makes
the seeded synthetic GGUF tensors the benchmark and tests use.
"""
from .ggml import GgmlType  # noqa: F401
