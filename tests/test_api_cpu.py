"""Public API on the CPU: argument checks that run before any launch, the torch
baselines of the reference API, and the single-layer RoPE + append path on a
CPU cache, all against the oracle."""

import numpy as np
import pytest
import torch

import flashdec_amd
from flashdec_amd import paged_reference, reference
from flashdec_amd.cache import PagedKVCache
from flashdec_amd.rope import RopeAppendResult, apply_rope, rope_paged_kv_append, rope_paged_kv_append_ref
from oracle import attention as oa
from oracle import rope as orope


def test_hip_entry_points_reject_cpu_tensors_before_launch():
    q = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 1, 32, 128, dtype=torch.bfloat16)
    table = torch.zeros(1, 1, dtype=torch.int32)
    lens = torch.ones(1, dtype=torch.int32)
    with pytest.raises(ValueError, match="must be CUDA tensors"):
        flashdec_amd.decode(q, cache, cache, table, lens)
    with pytest.raises(ValueError, match="must be CUDA tensors"):
        flashdec_amd.paged_decode_attention_into(q, cache, cache, table, lens, torch.empty_like(q))
    k = torch.zeros(1, 1, 4)
    c4 = torch.zeros(1, 1, 2, 4)
    idx = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(ValueError, match="q must be a CUDA tensor"):
        flashdec_amd.fused_rope_kv_append(torch.zeros(1, 2, 4), k, k, c4, c4, idx, idx, idx)
    with pytest.raises(ValueError, match="k_cache must be a CUDA tensor"):
        flashdec_amd.cuda_kv_append(c4, c4, idx, idx, k, k)


def test_public_names():
    assert flashdec_amd.decode is flashdec_amd.paged_decode_attention
    for name in ("decode", "paged_decode_attention", "paged_decode_attention_into", "fused_rope_kv_append",
                 "cuda_kv_append", "PagedKVCache", "KVTokenTransactionView", "DecodeEngine", "apply_rope",
                 "rope_paged_kv_append", "RopeAppendResult", "paged_decode_attention_ref",
                 "dense_decode_attention_ref"):
        assert name in flashdec_amd.__all__, name
        assert getattr(flashdec_amd, name) is not None


def test_apply_rope_validation():
    x = torch.zeros(2, 3, 8)
    pos = torch.zeros(2, dtype=torch.long)
    with pytest.raises(ValueError, match="positive, even"):
        apply_rope(x, pos, rotary_dim=3)
    with pytest.raises(ValueError, match="non-negative"):
        apply_rope(x, -torch.ones(2, dtype=torch.long))
    with pytest.raises(ValueError, match="positive finite"):
        apply_rope(x, pos, base=0.0)
    with pytest.raises(ValueError, match="shape \\[batch\\]"):
        apply_rope(x, torch.zeros(3, dtype=torch.long))
    with pytest.raises(ValueError, match="int32 or int64"):
        apply_rope(x, pos.float())


def test_rope_paged_kv_append_torch_path_against_oracle():
    cache = PagedKVCache(1, 2, 8, 4, 8, dtype=torch.float32, device="cpu")
    g = torch.Generator().manual_seed(2)
    for step in range(6):
        q = torch.randn(2, 4, 8, generator=g)
        k = torch.randn(2, 2, 8, generator=g)
        v = torch.randn(2, 2, 8, generator=g)
        res = (rope_paged_kv_append_ref if step % 2 else rope_paged_kv_append)(cache, 0, ["a", "b"], q, k, v,
                                                                               rotary_dim=4)
        assert isinstance(res, RopeAppendResult)
        assert res.positions.tolist() == [step, step] and res.seq_lens.tolist() == [step + 1, step + 1]
        np.testing.assert_allclose(res.q.numpy(), orope.apply_rope(q.numpy(), res.positions.numpy(), 4), atol=1e-6)
        blk = res.block_tables[:, step // 4].tolist()
        for row in range(2):
            np.testing.assert_allclose(cache.k_cache[0, blk[row], :, step % 4].numpy(),
                                       orope.apply_rope(k.numpy(), res.positions.numpy(), 4)[row], atol=1e-6)
            assert torch.equal(cache.v_cache[0, blk[row], :, step % 4], v[row])
    assert res.block_tables.tolist() == [[0, 2], [1, 3]]
    with pytest.raises(ValueError, match="append_backend"):
        rope_paged_kv_append(cache, 0, ["a"], q[:1], k[:1], v[:1], append_backend="nope")


def test_torch_baselines_match_oracle():
    rng = np.random.default_rng(8)
    lens = [0, 5, 17, 40]
    pool = 20
    table = np.full((4, 10), -1, dtype=np.int32)
    perm = rng.permutation(pool)
    c = 0
    for b, n in enumerate(lens):
        nb = (n + 7) // 8
        table[b, :nb] = perm[c:c + nb]
        c += nb
    q = rng.standard_normal((4, 8, 16)).astype(np.float32)
    k = rng.standard_normal((pool, 2, 8, 16)).astype(np.float32)
    v = rng.standard_normal((pool, 2, 8, 16)).astype(np.float32)
    expected = oa.paged_decode_attention(q, k, v, table, lens)
    got = paged_reference.paged_decode_attention_ref(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                                     torch.from_numpy(table), torch.tensor(lens))
    np.testing.assert_allclose(got.numpy(), expected, atol=1e-5, rtol=1e-5)
    kd, vd = oa.paged_to_dense(k, v, table, lens)
    dense = reference.dense_decode_attention_ref(torch.from_numpy(q), torch.from_numpy(kd), torch.from_numpy(vd),
                                                 torch.tensor(lens))
    np.testing.assert_allclose(dense.numpy(), expected, atol=1e-5, rtol=1e-5)
    # dim-major layout through the reference API
    km = np.ascontiguousarray(k.transpose(0, 1, 3, 2))
    vm = np.ascontiguousarray(v.transpose(0, 1, 3, 2))
    got_dm = paged_reference.paged_decode_attention_ref(torch.from_numpy(q), torch.from_numpy(km),
                                                        torch.from_numpy(vm), torch.from_numpy(table),
                                                        torch.tensor(lens), kv_layout="dim_major")
    np.testing.assert_allclose(got_dm.numpy(), expected, atol=1e-5, rtol=1e-5)
