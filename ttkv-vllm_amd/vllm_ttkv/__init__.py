"""vllm_ttkv for MI355X: the compressed-KV (pre-RoPE tensor-train) attention backend, with its
hot path in hand-written gfx950 HIP kernels behind the C ABI in include/ttkv_hip.h.

Importing this package does not import vLLM. `register()` does, and only when called by vLLM's
plugin loader (reference: vllm_ttkv/__init__.py:36-76).
"""
from __future__ import annotations

__all__ = ["register"]


def register() -> None:
    """vLLM general-plugin entry point: register the backend as AttentionBackendEnum.CUSTOM."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, "vllm_ttkv.backend.TTKVAttentionBackend")
