"""flashdec_amd: MI355X-native paged single-token decode path.

A drop-in for cysong2025/flashdec's decode data path (``import flashdec_amd as
flashdec``): the same public names for paged decode attention, fused RoPE +
paged KV append, the paged KV cache with multi-layer token transactions, the
decode engine and the vLLM ``CUSTOM`` backend hook.  The compute runs in
hand-written gfx950 HIP kernels behind the C ABI in ``include/flashdec_hip.h``
(``libflashdec_hip.so``); attributes are imported lazily like the
reference's package (flashdec/__init__.py:58-247).
"""

__all__ = [
    "PagedKVCache",
    "KVTokenTransactionView",
    "AdmissionResult",
    "DecodeLayerResult",
    "DecodeEngine",
    "DecodeStepTransaction",
    "DecodeStepResult",
    "DecodeStepGraph",
    "RopeAppendResult",
    "__version__",
    "apply_rope",
    "cuda_kv_append",
    "decode",
    "dense_decode_attention_ref",
    "fused_rope_kv_append",
    "load_cuda_kv_append_extension",
    "load_fused_rope_kv_append_extension",
    "paged_decode_attention",
    "paged_decode_attention_into",
    "paged_decode_attention_ref",
    "rope_paged_kv_append",
    "rope_paged_kv_append_ref",
]

__version__ = "0.1.0"

_LAZY = {
    "PagedKVCache": ("cache", "PagedKVCache"),
    "KVTokenTransactionView": ("cache", "KVTokenTransactionView"),
    "AdmissionResult": ("engine", "AdmissionResult"),
    "DecodeLayerResult": ("engine", "DecodeLayerResult"),
    "DecodeEngine": ("engine", "DecodeEngine"),
    "DecodeStepTransaction": ("engine", "DecodeStepTransaction"),
    "DecodeStepResult": ("engine", "DecodeStepResult"),
    "DecodeStepGraph": ("engine", "DecodeStepGraph"),
    "RopeAppendResult": ("rope", "RopeAppendResult"),
    "apply_rope": ("rope", "apply_rope"),
    "rope_paged_kv_append": ("rope", "rope_paged_kv_append"),
    "rope_paged_kv_append_ref": ("rope", "rope_paged_kv_append_ref"),
    "cuda_kv_append": ("_kv_append", "cuda_kv_append"),
    "load_cuda_kv_append_extension": ("_kv_append", "load_cuda_kv_append_extension"),
    "fused_rope_kv_append": ("_fused_rope_kv_append", "fused_rope_kv_append"),
    "load_fused_rope_kv_append_extension": ("_fused_rope_kv_append", "load_fused_rope_kv_append_extension"),
    "decode": ("paged_decode", "paged_decode_attention"),
    "paged_decode_attention": ("paged_decode", "paged_decode_attention"),
    "paged_decode_attention_into": ("paged_decode", "paged_decode_attention_into"),
    "paged_decode_attention_ref": ("paged_reference", "paged_decode_attention_ref"),
    "dense_decode_attention_ref": ("reference", "dense_decode_attention_ref"),
}


def __getattr__(name):
    target = _LAZY.get(name)
    if target is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    import importlib

    module = importlib.import_module(f".{target[0]}", __name__)
    value = getattr(module, target[1])
    globals()[name] = value
    return value


def __dir__():
    return sorted(set(globals()) | set(__all__))
