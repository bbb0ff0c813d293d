"""vLLM general-plugin entry point (flashdec/vllm_plugin.py:6-21).

Entry point: ``vllm.general_plugins: flashdec_amd = flashdec_amd.vllm_plugin:register``.
vLLM is imported inside ``register`` only, so the kernels and runtime work
without vLLM installed.
"""

from __future__ import annotations

BACKEND_CLASS_PATH = "flashdec_amd.vllm_backend.FlashDecAttentionBackend"


def register() -> None:
    """Register the HIP decode backend as vLLM's ``CUSTOM`` attention backend."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, BACKEND_CLASS_PATH)
