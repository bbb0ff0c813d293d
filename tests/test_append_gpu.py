"""Fused RoPE + K/V append and plain K/V append on the GPU, bit-exact against the oracle.

The oracle evaluates inv_freq and cos/sin in float64 and rounds once to fp32,
then rotates with unfused fp32 products and sums (oracle/rope.py); the HIP
kernel computes the same numbers, so q_out and every cache byte must match
exactly.  Cases follow the reference's tests/test_fused_rope_kv_append.py and
tests/test_cuda_kv_append.py, plus the C3 shape (B64 Hq16 Hkv2 D128, base 1e6).
"""

import numpy as np
import pytest
import torch

import flashdec_amd
from flashdec_amd import _fused_rope_kv_append as fused_module
from flashdec_amd._fused_rope_kv_append import _fused_rope_kv_append_trusted, fused_rope_kv_append
from flashdec_amd._kv_append import cuda_kv_append
from flashdec_amd.cache import PagedKVCache
from flashdec_amd.rope import apply_rope, rope_paged_kv_append
from oracle import rope as orope

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def bits(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy()
    return t.view(torch.int16).numpy()


def oracle_bits(values, dtype):
    return bits(torch.from_numpy(np.ascontiguousarray(values)).to(dtype))


def c3_case(dtype, batch=64, hq=16, hkv=2, d=128, bs=32, seed=251, rotary_dim=None, idx_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    num_blocks = batch * 8 + 3
    pos = torch.randint(1, 8192, (batch,), generator=g)
    perm = torch.randperm(num_blocks, generator=g)[:batch]
    q = torch.randn(batch, hq, d, generator=g).to(dtype)
    k = torch.randn(batch, hkv, d, generator=g).to(dtype)
    v = torch.randn(batch, hkv, d, generator=g).to(dtype)
    kc = torch.randn(num_blocks, hkv, bs, d, generator=g).to(dtype)
    vc = torch.randn(num_blocks, hkv, bs, d, generator=g).to(dtype)
    blk = perm.to(idx_dtype)
    off = (pos % bs).to(idx_dtype)
    return q, k, v, kc, vc, blk, off, pos.to(idx_dtype)


def expected(q, k, v, kc, vc, blk, off, pos, rotary_dim, base, dtype):
    f = lambda t: t.float().numpy()
    return orope.rope_kv_append(f(q), f(k), f(v), f(kc), f(vc), blk.numpy(), off.numpy(), pos.numpy(),
                                rotary_dim=rotary_dim, base=base, dtype=NAME[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [
    dict(batch=64, hq=16, hkv=2, d=128, bs=32, rotary_dim=None, base=1e6),   # C3
    dict(batch=5, hq=8, hkv=8, d=64, bs=16, rotary_dim=32, base=1e4),        # partial rotary, MHA
    dict(batch=3, hq=4, hkv=1, d=256, bs=8, rotary_dim=256, base=5e5),
])
def test_fused_rope_append_is_bit_exact(dtype, shape):
    shape = dict(shape)
    rotary_dim, base = shape.pop("rotary_dim"), shape.pop("base")
    print(f"fused rope append {dtype} {shape} R={rotary_dim} base={base}", flush=True)
    q, k, v, kc, vc, blk, off, pos = c3_case(dtype, **shape)
    exp_q, exp_k, exp_v = expected(q, k, v, kc, vc, blk, off, pos, rotary_dim, base, dtype)
    dev = [t.cuda() for t in (q, k, v, kc, vc, blk, off, pos)]
    q_out = fused_rope_kv_append(*dev, rotary_dim=rotary_dim, base=base)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_out), oracle_bits(exp_q, dtype))
    assert np.array_equal(bits(dev[3]), oracle_bits(exp_k, dtype))  # untouched slots keep their bytes too
    assert np.array_equal(bits(dev[4]), oracle_bits(exp_v, dtype))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_matches_reference_small_case(dtype):
    """The reference's own fixture: rows (block 3, offset 2, pos 0) and (block 1, offset 0, pos 7), R=4."""
    torch.manual_seed(241)
    q = torch.randn((2, 4, 8), device="cuda", dtype=dtype)
    k = torch.randn((2, 2, 8), device="cuda", dtype=dtype)
    v = torch.randn_like(k)
    kc = torch.zeros((4, 2, 3, 8), device="cuda", dtype=dtype)
    vc = torch.zeros_like(kc)
    blk = torch.tensor([3, 1], device="cuda", dtype=torch.int32)
    off = torch.tensor([2, 0], device="cuda", dtype=torch.int64)
    pos = torch.tensor([0, 7], device="cuda", dtype=torch.int64)
    q_out = fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, rotary_dim=4)
    exp_k = apply_rope(k, pos, rotary_dim=4)
    torch.testing.assert_close(q_out, apply_rope(q, pos, rotary_dim=4), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(kc[3, :, 2], exp_k[0], atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(kc[1, :, 0], exp_k[1], atol=1e-2, rtol=1e-2)
    assert torch.equal(vc[3, :, 2], v[0]) and torch.equal(vc[1, :, 0], v[1])
    assert torch.count_nonzero(kc[0]).item() == 0 and torch.count_nonzero(vc[2]).item() == 0
    zeros = np.zeros((4, 2, 3, 8), np.float32)
    exp_q, exp_k, exp_v = orope.rope_kv_append(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                               v.float().cpu().numpy(), zeros, zeros, [3, 1], [2, 0], [0, 7],
                                               rotary_dim=4, dtype=NAME[dtype])
    assert np.array_equal(bits(q_out), oracle_bits(exp_q, dtype))
    assert np.array_equal(bits(kc), oracle_bits(exp_k, dtype))
    assert np.array_equal(bits(vc), oracle_bits(exp_v, dtype))


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_trusted_equals_checked(idx_dtype):
    q, k, v, kc, vc, blk, off, pos = [t.cuda() for t in c3_case(torch.bfloat16, batch=16, idx_dtype=idx_dtype)]
    kc2, vc2 = kc.clone(), vc.clone()
    a = fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, base=1e6)
    b = _fused_rope_kv_append_trusted(q, k, v, kc2, vc2, blk.long(), off.long(), pos.long(), base=1e6)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(kc, kc2) and torch.equal(vc, vc2)
    with pytest.raises(ValueError, match="trusted transaction metadata must use int64"):
        _fused_rope_kv_append_trusted(q, k, v, kc, vc, blk.int(), off.int(), pos.int())


@pytest.mark.parametrize("blk,off,pos,message", [
    ([-1], [0], [0], "block_ids"), ([2], [0], [0], "block_ids"), ([0], [-1], [0], "block_offsets"),
    ([0], [2], [0], "block_offsets"), ([0], [0], [-1], "positions")])
def test_public_primitive_checks_index_values_before_launch(blk, off, pos, message, monkeypatch):
    q = torch.zeros((1, 2, 4), device="cuda")
    k = torch.zeros((1, 1, 4), device="cuda")
    cache = torch.zeros((2, 1, 2, 4), device="cuda")

    def no_launch(*_a, **_k):
        raise AssertionError("invalid indices must not reach the launch")

    monkeypatch.setattr(fused_module, "_launch", no_launch)
    t = lambda x: torch.tensor(x, device="cuda", dtype=torch.int64)
    with pytest.raises(ValueError, match=message):
        fused_rope_kv_append(q, k, k, cache, cache, t(blk), t(off), t(pos))


def test_kernel_range_checks_block_and_offset():
    """Out-of-range rows given through the trusted path write no K/V; q_out is still produced."""
    q, k, v, kc, vc, blk, off, pos = [t.cuda() for t in c3_case(torch.bfloat16, batch=4)]
    blk[1] = kc.shape[0]  # one past the pool
    off[2] = kc.shape[2]  # one past the block
    before_k, before_v = kc.clone(), vc.clone()
    q_out = _fused_rope_kv_append_trusted(q, k, v, kc, vc, blk, off, pos, base=1e6)
    torch.cuda.synchronize()
    exp_q = orope.apply_rope(q.float().cpu().numpy(), pos.cpu().numpy(), base=1e6, out_dtype="bfloat16")
    assert np.array_equal(bits(q_out), oracle_bits(exp_q, torch.bfloat16))
    written = sorted([blk[0].item(), blk[3].item()])
    assert sorted((kc != before_k).any(dim=(1, 2, 3)).nonzero().flatten().tolist()) == written
    assert sorted((vc != before_v).any(dim=(1, 2, 3)).nonzero().flatten().tolist()) == written


@pytest.mark.parametrize("dtype", DTYPES)
def test_kv_append_is_bit_exact(dtype):
    q, k, v, kc, vc, blk, off, pos = c3_case(dtype, batch=33, idx_dtype=torch.int32)
    exp_k, exp_v = orope.kv_append(k.float().numpy(), v.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                   blk.numpy(), off.numpy())
    kc, vc = kc.cuda(), vc.cuda()
    cuda_kv_append(kc, vc, blk.cuda(), off.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), oracle_bits(exp_k, dtype))
    assert np.array_equal(bits(vc), oracle_bits(exp_v, dtype))


def test_kv_append_rejects_out_of_range():
    cache = torch.zeros((2, 1, 2, 4), device="cuda")
    k = torch.zeros((1, 1, 4), device="cuda")
    t = lambda x: torch.tensor(x, device="cuda")
    with pytest.raises(ValueError, match="block_ids must be within"):
        cuda_kv_append(cache, cache, t([2]), t([0]), k, k)
    with pytest.raises(ValueError, match="block_offsets must be within"):
        cuda_kv_append(cache, cache, t([0]), t([2]), k, k)


# ------------------------------------------------------------- cache paths
def gpu_cache(dtype=torch.bfloat16, num_layers=1, hkv=2, d=128, bs=32, max_blocks=16):
    return PagedKVCache(num_layers=num_layers, num_kv_heads=hkv, head_dim=d, block_size=bs, max_blocks=max_blocks,
                        dtype=dtype, device="cuda")


@pytest.mark.parametrize("dtype", DTYPES)
def test_append_cuda_matches_torch_append(dtype):
    a, b = gpu_cache(dtype, bs=4), gpu_cache(dtype, bs=4)
    g = torch.Generator().manual_seed(3)
    for step in range(9):
        ids = [1, 2, 3] if step % 3 else [2, 3]
        k = torch.randn(len(ids), 2, 128, generator=g).to(dtype).cuda()
        v = torch.randn(len(ids), 2, 128, generator=g).to(dtype).cuda()
        ta = a.append(0, ids, k, v)
        tb = b.append_cuda(0, ids, k, v)
        assert torch.equal(ta, tb)
    torch.cuda.synchronize()
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache)
    assert a.metrics() == b.metrics()
    assert b.validate_invariants()


def test_append_cuda_failures_keep_allocator_atomic():
    cache = gpu_cache(max_blocks=1, bs=4)
    kv = torch.zeros(2, 2, 128, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        cache.append_cuda(0, [1, 2], kv, kv)
    with pytest.raises(KeyError, match="unknown request_id"):
        cache.request_state(1)
    strided = torch.zeros(1, 2, 256, device="cuda", dtype=torch.bfloat16)[..., ::2]
    with pytest.raises(ValueError, match="requires contiguous"):
        cache.append_cuda(0, [1], strided, strided)
    with pytest.raises(KeyError, match="unknown request_id"):
        cache.request_state(1)
    assert cache.validate_invariants()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rope_tables", [True, False])
def test_rope_paged_kv_append_backends_agree(dtype, rope_tables):
    """With the cache's own cos/sin tables (the default) the fused backend rotates q and K
    exactly as the torch backend (the reference's rope.py:66-82 expression) does, bit for
    bit; with them off the kernel's own evaluation equals the float64 oracle bit for bit."""
    caches = {name: gpu_cache(dtype, bs=8) for name in ("torch", "cuda", "fused_cuda")}
    caches["fused_cuda"].rope_tables = rope_tables
    g = torch.Generator().manual_seed(11)
    for step in range(12):
        ids = [5, 6, 7]
        q = torch.randn(3, 16, 128, generator=g).to(dtype).cuda()
        k = torch.randn(3, 2, 128, generator=g).to(dtype).cuda()
        v = torch.randn(3, 2, 128, generator=g).to(dtype).cuda()
        results = {n: rope_paged_kv_append(c, 0, ids, q, k, v, base=1e6, append_backend=n) for n, c in caches.items()}
        pos = results["torch"].positions
        assert all(torch.equal(r.positions, pos) for r in results.values())
        assert all(torch.equal(r.block_tables, results["torch"].block_tables) for r in results.values())
        exp_q = orope.apply_rope(q.float().cpu().numpy(), pos.cpu().numpy(), base=1e6, out_dtype=NAME[dtype])
        if rope_tables:
            assert torch.equal(results["torch"].q.view(torch.int16), results["fused_cuda"].q.view(torch.int16))
        else:
            assert np.array_equal(bits(results["fused_cuda"].q), oracle_bits(exp_q, dtype))
        # torch's fp32 pow/cos/sin may differ from the correctly rounded values by an ulp
        torch.testing.assert_close(results["torch"].q, results["fused_cuda"].q, atol=2e-2, rtol=1e-2)
    torch.cuda.synchronize()
    assert torch.equal(caches["torch"].v_cache, caches["fused_cuda"].v_cache)
    if rope_tables:
        assert torch.equal(caches["torch"].k_cache.view(torch.int16), caches["fused_cuda"].k_cache.view(torch.int16))
    torch.testing.assert_close(caches["torch"].k_cache, caches["fused_cuda"].k_cache, atol=2e-2, rtol=1e-2)
    assert caches["torch"].metrics() == caches["fused_cuda"].metrics()


def test_public_api_exports():
    assert flashdec_amd.fused_rope_kv_append is fused_rope_kv_append
    assert flashdec_amd.cuda_kv_append is cuda_kv_append
    assert callable(flashdec_amd.load_fused_rope_kv_append_extension)
    assert "_fused_rope_kv_append_trusted" not in flashdec_amd.__all__
