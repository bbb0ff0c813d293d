"""vLLM CUSTOM backend and plugin on the CPU, against fake vLLM modules.

Scenarios follow the reference's tests/test_vllm_backend.py and
tests/test_vllm_plugin.py: identity and cache contract, which calls reach the
HIP launcher (and with which arguments), and every fallback to vLLM's own
Triton path.
"""

import importlib
from types import SimpleNamespace

import pytest
import torch

from tests import vllm_fakes


@pytest.fixture
def vb(monkeypatch):
    module, registry = vllm_fakes.install(monkeypatch)
    monkeypatch.setattr(module, "_target_programs", lambda device: 256)
    module._registry = registry
    return module


def make_impl(vb, **overrides):
    impl = vb.FlashDecAttentionImpl(16, 128, 128 ** -0.5, 2)
    for key, value in overrides.items():
        setattr(impl, key, value)
    return impl


def metadata(num_reqs=3, max_seq_len=1024, workspace_capacity=64, **overrides):
    md = SimpleNamespace(
        query_start_loc=torch.empty(num_reqs + 1, dtype=torch.int32),
        max_seq_len=max_seq_len,
        max_query_len=1,
        use_cascade=False,
        causal=True,
        block_table=torch.empty((num_reqs, 64), dtype=torch.int32),
        seq_lens=torch.empty(num_reqs, dtype=torch.int32),
        slot_mapping=torch.empty(num_reqs, dtype=torch.int64),
        softmax_segm_output=torch.empty((workspace_capacity, 16, 16, 128)),
        softmax_segm_max=torch.empty((workspace_capacity, 16, 16)),
        softmax_segm_expsum=torch.empty((workspace_capacity, 16, 16)),
    )
    for key, value in overrides.items():
        setattr(md, key, value)
    return md


def tensors(num_tokens=4, dtype=torch.float16, blocks=65, block_size=16):
    q = torch.empty((num_tokens, 16, 128), dtype=dtype)
    k = torch.empty((num_tokens, 2, 128), dtype=dtype)
    return q, k, torch.empty_like(k), torch.empty((blocks, 2, block_size, 2, 128), dtype=dtype), torch.empty_like(q)


def owning_layer():
    return SimpleNamespace(kv_sharing_target_layer_name=None)


def record_launches(vb, monkeypatch):
    calls = []

    def launcher(*args, **kwargs):
        calls.append((args, kwargs))
        return args[6]

    monkeypatch.setattr(vb, "_vllm_paged_decode_attention_into", launcher)
    return calls


def test_backend_identity_and_cache_contract(vb):
    assert vb.FlashDecAttentionBackend.get_name() == "CUSTOM"
    assert vb.FlashDecAttentionBackend.get_impl_cls() is vb.FlashDecAttentionImpl
    assert vb.FlashDecAttentionBackend.forward_includes_kv_cache_update is False
    assert vb.FlashDecAttentionBackend.get_kv_cache_shape(7, 16, 2, 128) == (7, 2, 16, 2, 128)


@pytest.mark.parametrize(("max_seq_len", "splits"), [(512, 4), (1024, 8), (2048, 16)])
def test_eligible_decode_passes_vllm_tensors_to_the_hip_launcher(vb, monkeypatch, max_seq_len, splits):
    calls = record_launches(vb, monkeypatch)
    impl = make_impl(vb)
    q, k, v, cache, out = tensors()
    md = metadata(max_seq_len=max_seq_len)
    assert impl.forward(owning_layer(), q, k, v, cache, md, out) is out
    (args, kwargs), = calls
    expected_args = (q, k, v, cache, md.block_table, md.seq_lens, out, md.slot_mapping, md.softmax_segm_output,
                     md.softmax_segm_max, md.softmax_segm_expsum)
    assert len(args) == len(expected_args) and all(a is b for a, b in zip(args, expected_args))
    assert kwargs == {"num_reqs": 3, "num_q_heads": 16, "num_kv_heads": 2, "head_dim": 128, "block_size": 16,
                      "sm_scale": 128 ** -0.5, "num_splits": splits, "max_seq_len": max_seq_len, "kv_reuse": False}
    assert vllm_fakes.TritonAttentionImpl.fallback_calls == []


@pytest.mark.parametrize("num_reqs,max_seq_len,expected", [(8, 8192, 16), (32, 8192, 4), (64, 8192, 2),
                                                           (16, 8192, 8)])
def test_auto_split_targets_the_device_compute_units(vb, monkeypatch, num_reqs, max_seq_len, expected):
    calls = record_launches(vb, monkeypatch)
    q, k, v, cache, out = tensors(num_tokens=num_reqs, blocks=600)
    make_impl(vb).forward(owning_layer(), q, k, v, cache, metadata(num_reqs=num_reqs, max_seq_len=max_seq_len),
                          out)
    assert calls[0][1]["num_splits"] == expected


@pytest.mark.parametrize("requested,num_reqs,capacity", [(1, 3, 64), (0, 128, 128), (0, 3, 2)],
                         ids=("explicit-one", "auto-one-high-batch", "workspace-forces-one"))
def test_single_split_falls_back_to_vllm(vb, monkeypatch, requested, num_reqs, capacity):
    calls = record_launches(vb, monkeypatch)
    impl = make_impl(vb, _requested_splits=requested)
    q, k, v, cache, out = tensors(num_tokens=num_reqs)
    md = metadata(num_reqs=num_reqs, workspace_capacity=capacity)
    layer = owning_layer()
    assert impl.forward(layer, q, k, v, cache, md, out) == "vllm-triton-fallback"
    assert calls == []
    assert vllm_fakes.TritonAttentionImpl.fallback_calls == [(layer, q, k, v, cache, md, out, None, None)]


@pytest.mark.parametrize("change", [
    dict(impl=dict(head_size=64)), dict(impl=dict(num_heads=4)), dict(impl=dict(sliding_window=(128, 0))),
    dict(impl=dict(alibi_slopes=torch.ones(16))), dict(impl=dict(logits_soft_cap=30.0)),
    dict(impl=dict(kv_cache_dtype="fp8")), dict(impl=dict(need_to_return_lse_for_decode=True)),
    dict(impl=dict(attn_type="encoder")), dict(md=dict(max_seq_len=511)), dict(md=dict(max_query_len=2)),
    dict(md=dict(use_cascade=True)), dict(md=dict(causal=False)), dict(dtype=torch.float32),
    dict(block_size=8), dict(output_scale=True)])
def test_ineligible_calls_fall_back(vb, monkeypatch, change):
    calls = record_launches(vb, monkeypatch)
    impl = make_impl(vb, **change.get("impl", {}))
    q, k, v, cache, out = tensors(dtype=change.get("dtype", torch.float16), block_size=change.get("block_size", 16))
    md = metadata(**change.get("md", {}))
    extra = (torch.ones(1),) if change.get("output_scale") else ()
    assert impl.forward(owning_layer(), q, k, v, cache, md, out, *extra) == "vllm-triton-fallback"
    assert calls == []


@pytest.mark.parametrize("layer,md", [(SimpleNamespace(kv_sharing_target_layer_name="shared.0"), "metadata"),
                                      (SimpleNamespace(kv_sharing_target_layer_name=None), None)])
def test_non_owning_or_profiling_calls_fall_back(vb, monkeypatch, layer, md):
    calls = record_launches(vb, monkeypatch)
    md = metadata() if md == "metadata" else None
    assert make_impl(vb).forward(layer, object(), object(), object(), object(), md, object()) == "vllm-triton-fallback"
    assert calls == []


def test_launcher_failure_propagates(vb, monkeypatch):
    def failing(*args, **kwargs):
        raise RuntimeError("launch failed")

    monkeypatch.setattr(vb, "_vllm_paged_decode_attention_into", failing)
    q, k, v, cache, out = tensors()
    with pytest.raises(RuntimeError, match="launch failed"):
        make_impl(vb).forward(owning_layer(), q, k, v, cache, metadata(), out)


@pytest.mark.parametrize("value", ["auto", "-1", "3", "6", "11", "12", "17"])
def test_invalid_split_environment_rejected_at_construction(vb, monkeypatch, value):
    monkeypatch.setenv("FLASHDEC_VLLM_NUM_SPLITS", value)
    with pytest.raises(ValueError, match=r"0, 1, 2, 4, 8, or 16 \(0 selects auto\)"):
        make_impl(vb)


@pytest.mark.parametrize("value", ["0", "1", "2", "4", "8", "16"])
def test_valid_split_environment(vb, monkeypatch, value):
    monkeypatch.setenv("FLASHDEC_VLLM_NUM_SPLITS", value)
    assert make_impl(vb)._requested_splits == int(value)


@pytest.mark.parametrize("value,expected", [("0", False), ("1", True)])
def test_kv_reuse_environment_reaches_the_launcher(vb, monkeypatch, value, expected):
    monkeypatch.setenv("FLASHDEC_VLLM_KV_REUSE", value)
    calls = record_launches(vb, monkeypatch)
    q, k, v, cache, out = tensors()
    make_impl(vb).forward(owning_layer(), q, k, v, cache, metadata(), out)
    (_, kwargs), = calls
    assert kwargs["kv_reuse"] is expected


@pytest.mark.parametrize("value", ["", "yes", "2", "true"])
def test_invalid_kv_reuse_environment_rejected_at_construction(vb, monkeypatch, value):
    monkeypatch.setenv("FLASHDEC_VLLM_KV_REUSE", value)
    with pytest.raises(ValueError, match="FLASHDEC_VLLM_KV_REUSE must be 0 or 1"):
        make_impl(vb)


def test_automatic_splits_keep_128_tokens_and_requests_keep_the_reference_cap(vb):
    # auto: 3 rows x 2 heads at 256 programs -> 16, capped to ctx / 128
    for ctx, expected in [(512, 4), (1024, 8), (1100, 8), (2048, 16), (8192, 16)]:
        assert vb._select_num_splits(0, num_reqs=3, num_kv_heads=2, logical_blocks=-(-ctx // 16),
                                     target_programs=256, auto_min_tokens=128, block_size=16) == expected
    # an explicit request is capped by the logical blocks only, as in the reference
    assert vb._select_num_splits(16, num_reqs=3, num_kv_heads=2, logical_blocks=32, target_programs=256,
                                 auto_min_tokens=128, block_size=16) == 16


def test_reference_split_policy_is_the_default_target(vb):
    # the reference's own table (tests/test_vllm_backend.py:96-121) at its 128-program target
    for num_reqs, expected in [(4, 16), (5, 16), (6, 8), (10, 8), (11, 4), (12, 4)]:
        assert vb._select_num_splits(0, num_reqs=num_reqs, num_kv_heads=2, logical_blocks=64) == expected


def test_plugin_is_import_safe_and_registers(monkeypatch):
    plugin = importlib.import_module("flashdec_amd.vllm_plugin")
    assert callable(plugin.register)
    _, registry = vllm_fakes.install(monkeypatch)
    plugin.register()
    assert registry.calls == [("custom", "flashdec_amd.vllm_backend.FlashDecAttentionBackend")]
