"""Split-count policy of the vLLM hook (flashdec/vllm_backend.py:155-188), free of vLLM imports.

``FLASHDEC_VLLM_NUM_SPLITS`` = 0 selects the power of two whose program count
(rows x KV heads x splits) is nearest a target, capped by the context's
logical blocks; 1, 2, 4, 8 or 16 request that count (still capped).  The hook
passes the device's compute-unit count as the target (the reference's fixed
target is 128) and keeps automatic splits at >= 128 tokens.
"""

from __future__ import annotations

_VALID_REQUESTED_SPLITS = (0, 1, 2, 4, 8, 16)
_VALID_NUM_SPLITS = _VALID_REQUESTED_SPLITS[1:]
_REFERENCE_TARGET_PROGRAMS = 128
# the hook's automatic splits keep one 32-token unit per wave of the HIP
# kernel (B8 ctx1024 bs16: 8 instead of 16 splits)
_AUTO_MIN_SPLIT_TOKENS = 128


def _parse_requested_splits(value: str) -> int:
    """``FLASHDEC_VLLM_NUM_SPLITS`` -> requested split count (0 = auto)."""
    try:
        requested = int(value)
    except ValueError:
        requested = -1
    if requested not in _VALID_REQUESTED_SPLITS:
        raise ValueError("FLASHDEC_VLLM_NUM_SPLITS must be one of 0, 1, 2, 4, 8, or 16 (0 selects auto)")
    return requested


def _select_num_splits(requested_splits: int, *, num_reqs: int, num_kv_heads: int, logical_blocks: int,
                       target_programs: int = _REFERENCE_TARGET_PROGRAMS, auto_min_tokens: int = 0,
                       block_size: int = 1) -> int:
    """Split count: the power of two whose program count is nearest the target, capped by the context.

    ``auto_min_tokens`` > 0 (no counterpart in the reference) also keeps every
    automatically chosen split at least that many tokens long (the HIP
    kernel's four waves take one 32-token unit each: 128).  Explicit requests
    keep the reference's cap only.
    """
    cap = max(s for s in _VALID_NUM_SPLITS if s <= max(1, logical_blocks))
    if requested_splits == 0:
        per_split = max(1, num_reqs * num_kv_heads)
        requested_splits = min(_VALID_NUM_SPLITS, key=lambda s: (abs(per_split * s - target_programs), s))
        if auto_min_tokens > 0:
            units = max(1, logical_blocks * block_size // auto_min_tokens)
            cap = min(cap, max(s for s in _VALID_NUM_SPLITS if s <= units))
    return min(requested_splits, cap)
