"""Minimal stand-ins for the vLLM modules the backend imports (vLLM is not installed).

They provide only the names ``flashdec_amd.vllm_backend`` and ``vllm_plugin``
touch: ``AttentionType``, the Triton backend/impl/metadata classes, and the
backend registry.  The fake Triton ``forward`` records its calls so tests can
see when the backend falls back.
"""

import importlib
import sys
import types


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"


class TritonAttentionMetadata:
    pass


class TritonAttentionBackend:
    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
        return (num_blocks, 2, block_size, num_kv_heads, head_size)


class TritonAttentionImpl:
    fallback_calls = []

    def __init__(self, num_heads, head_size, scale, num_kv_heads, *args, **kwargs):
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.attn_type = AttentionType.DECODER
        self.need_to_return_lse_for_decode = False
        self.kv_cache_dtype = kwargs.get("kv_cache_dtype", "auto")
        self.alibi_slopes = None
        self.sinks = None
        self.sliding_window = (-1, -1)
        self.logits_soft_cap = 0

    def forward(self, *args):
        TritonAttentionImpl.fallback_calls.append(args)
        return "vllm-triton-fallback"


def install(monkeypatch):
    """Put the fake modules in ``sys.modules`` and return a fresh ``flashdec_amd.vllm_backend``."""
    names = ["vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends"]
    for name in names:
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    backend = types.ModuleType("vllm.v1.attention.backend")
    backend.AttentionType = AttentionType
    triton_attn = types.ModuleType("vllm.v1.attention.backends.triton_attn")
    triton_attn.TritonAttentionBackend = TritonAttentionBackend
    triton_attn.TritonAttentionImpl = TritonAttentionImpl
    triton_attn.TritonAttentionMetadata = TritonAttentionMetadata
    registry = types.ModuleType("vllm.v1.attention.backends.registry")
    registry.AttentionBackendEnum = types.SimpleNamespace(CUSTOM="custom")
    registry.calls = []
    registry.register_backend = lambda enum, path: registry.calls.append((enum, path))
    for mod in (backend, triton_attn, registry):
        monkeypatch.setitem(sys.modules, mod.__name__, mod)
    monkeypatch.delitem(sys.modules, "flashdec_amd.vllm_backend", raising=False)
    TritonAttentionImpl.fallback_calls = []
    module = importlib.import_module("flashdec_amd.vllm_backend")
    return module, registry
