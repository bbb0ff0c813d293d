"""vLLM backend split-count policy (pure Python).  Test infrastructure only.

Restates cysong2025/flashdec ``flashdec/vllm_backend.py:155-188``
(``_parse_requested_splits`` and ``_select_num_splits``): requested splits in
{0 (auto), 1, 2, 4, 8, 16}; auto picks the power of two whose program count
``num_reqs * num_kv_heads * s`` is nearest to 128 (ties to the smaller s),
then the choice is capped by the largest power of two <= logical blocks.
"""

VALID_REQUESTED = (0, 1, 2, 4, 8, 16)
VALID_SPLITS = VALID_REQUESTED[1:]


def parse_requested_splits(value):
    try:
        requested = int(value)
    except ValueError:
        requested = -1
    if requested not in VALID_REQUESTED:
        raise ValueError("FLASHDEC_VLLM_NUM_SPLITS must be one of 0, 1, 2, 4, 8, or 16 (0 selects auto)")
    return requested


def select_num_splits(requested, *, num_reqs, num_kv_heads, logical_blocks, target_programs=128):
    cap = max(s for s in VALID_SPLITS if s <= max(1, logical_blocks))
    if requested == 0:
        per = max(1, num_reqs * num_kv_heads)
        requested = min(VALID_SPLITS, key=lambda s: (abs(per * s - target_programs), s))
    return min(requested, cap)
