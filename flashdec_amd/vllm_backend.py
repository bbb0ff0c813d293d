"""vLLM attention backend that runs eligible decode batches on the HIP kernels.

Follows flashdec/vllm_backend.py:155-389.
- The backend inherits vLLM's Triton attention backend.
- vLLM keeps ownership of KV-cache allocation and of the separate KV update (``forward_includes_kv_cache_update = False``). It also keeps metadata, prefill, mixed batches and every feature outside the narrow path.
- This backend replaces uniform single-token decoder attention over an fp16/bf16 paged cache with head_size 128 and 4/8/16 query heads per KV head.

An eligible batch:
- is one ``_vllm_paged_decode_attention_into`` call over vLLM's own 5-D cache ``[blocks, 2, block_size, kv_heads, head_size]``, through its strides;
- uses vLLM's split workspace (``softmax_segm_*``);
- takes the newest token's K/V from ``key``/``value``;
- carries ``slot_mapping == -1`` graph-padding rows, which stay inert inside the kernel, with no host read.

``FLASHDEC_VLLM_NUM_SPLITS`` picks the split count:
- 0 = auto; otherwise 1, 2, 4, 8 or 16.
- A split count of 1 falls back to vLLM's own kernel, as in the reference.
- Auto uses the reference's policy (power of two nearest the program target, capped by the context). The target is the device's compute-unit count (256 on MI355X) rather than the reference's fixed 128, so one decode layer fills the chip, and every automatic split keeps at least 128 tokens (one 32-token unit per wave).

The reference's split-attestation files (benchmark provenance) are not part of this path.
"""

from __future__ import annotations

import os

import torch
from vllm.v1.attention.backend import AttentionType
from vllm.v1.attention.backends.triton_attn import (
    TritonAttentionBackend,
    TritonAttentionImpl,
    TritonAttentionMetadata,
)

from .paged_decode import _vllm_paged_decode_attention_into
from .vllm_splits import (  # noqa: F401  (re-exported: the hook's policy lives beside it)
    _AUTO_MIN_SPLIT_TOKENS,
    _REFERENCE_TARGET_PROGRAMS,
    _VALID_NUM_SPLITS,
    _VALID_REQUESTED_SPLITS,
    _parse_requested_splits,
    _select_num_splits,
)

_MIN_CONTEXT = 512  # below this the split kernel does not pay (vllm_backend.py:254)


def _parse_kv_reuse(value: str) -> bool:
    """``FLASHDEC_VLLM_KV_REUSE`` -> plain (cached) K/V loads; no counterpart in the reference."""
    if value not in ("0", "1"):
        raise ValueError("FLASHDEC_VLLM_KV_REUSE must be 0 or 1")
    return value == "1"


_TARGETS: dict = {}


def _target_programs(device) -> int:
    """Compute units of ``device`` (one workgroup per CU fills the chip)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    target = _TARGETS.get(index)
    if target is None:
        target = int(torch.cuda.get_device_properties(index).multi_processor_count)
        _TARGETS[index] = target
    return target


class FlashDecAttentionBackend(TritonAttentionBackend):
    """vLLM backend that substitutes the HIP decode kernels for eligible decode batches."""

    # vLLM's separate KV update stays on every path (and its graph ordering);
    # the fused kernel stores the same token again, which is harmless.
    forward_includes_kv_cache_update = False

    @staticmethod
    def get_name() -> str:
        # vLLM maps the selected class back through its registry by this name
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type["FlashDecAttentionImpl"]:
        return FlashDecAttentionImpl


class FlashDecAttentionImpl(TritonAttentionImpl):
    """HIP kernels for the narrow decode path; vLLM's Triton implementation for the rest."""

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        self._requested_splits = _parse_requested_splits(os.environ.get("FLASHDEC_VLLM_NUM_SPLITS", "0"))
        # "1" when requests share cache blocks (prefix caching with common
        # prompts): K/V re-reads then come from the caches instead of HBM
        self._kv_reuse = _parse_kv_reuse(os.environ.get("FLASHDEC_VLLM_KV_REUSE", "0"))

    def _supports_flashdec_decode(self, query, key, value, kv_cache, attn_metadata, output, output_scale,
                                  output_block_scale) -> bool:
        """Eligibility of one forward call (vllm_backend.py:225-280)."""
        if attn_metadata is None or self.attn_type != AttentionType.DECODER:
            return False
        if attn_metadata.max_seq_len < _MIN_CONTEXT:
            return False
        if attn_metadata.max_query_len != 1 or attn_metadata.use_cascade or attn_metadata.causal is not True:
            return False
        if self.need_to_return_lse_for_decode or output_scale is not None or output_block_scale is not None:
            return False
        if self.kv_cache_dtype not in ("auto", "float16", "bfloat16"):
            return False
        if query.dtype not in (torch.float16, torch.bfloat16) or kv_cache.dtype != query.dtype:
            return False
        if query.ndim != 3 or key.ndim != 3 or value.ndim != 3 or output.ndim != 3 or kv_cache.ndim != 5:
            return False
        if self.head_size != 128:
            return False
        if (kv_cache.shape[1] != 2 or kv_cache.shape[2] not in (16, 32) or kv_cache.shape[3] != self.num_kv_heads
                or kv_cache.shape[4] != self.head_size):
            return False
        if self.alibi_slopes is not None or self.sinks is not None:
            return False
        if self.sliding_window != (-1, -1) or self.logits_soft_cap != 0:
            return False
        return self.num_heads % self.num_kv_heads == 0 and self.num_heads // self.num_kv_heads in (4, 8, 16)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata: TritonAttentionMetadata, output,
                output_scale=None, output_block_scale=None):
        owns_kv = getattr(layer, "kv_sharing_target_layer_name", None) is None and key is not None \
            and value is not None
        if not owns_kv or not self._supports_flashdec_decode(query, key, value, kv_cache, attn_metadata, output,
                                                             output_scale, output_block_scale):
            return super().forward(layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                                   output_block_scale)
        # one query token per metadata row; under graph replay the row count
        # includes padding rows, which slot_mapping == -1 keeps inert
        num_reqs = attn_metadata.query_start_loc.shape[0] - 1
        block_size = kv_cache.shape[2]
        logical_blocks = (attn_metadata.max_seq_len + block_size - 1) // block_size
        num_splits = _select_num_splits(self._requested_splits, num_reqs=num_reqs, num_kv_heads=self.num_kv_heads,
                                        logical_blocks=logical_blocks,
                                        target_programs=_target_programs(query.device),
                                        auto_min_tokens=_AUTO_MIN_SPLIT_TOKENS, block_size=block_size)
        if num_reqs > attn_metadata.softmax_segm_output.shape[0]:
            num_splits = 1
        if num_splits == 1:
            return super().forward(layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                                   output_block_scale)
        _vllm_paged_decode_attention_into(
            query,
            key,
            value,
            kv_cache,
            attn_metadata.block_table,
            attn_metadata.seq_lens,
            output,
            attn_metadata.slot_mapping,
            attn_metadata.softmax_segm_output,
            attn_metadata.softmax_segm_max,
            attn_metadata.softmax_segm_expsum,
            num_reqs=num_reqs,
            num_q_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_size,
            block_size=block_size,
            sm_scale=self.scale,
            num_splits=num_splits,
            max_seq_len=attn_metadata.max_seq_len,
            kv_reuse=self._kv_reuse,
        )
        return output
