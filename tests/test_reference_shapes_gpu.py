"""GPU parity at the head layout of the reference's own benchmark rows.

The reference's grouped-decode, default-profile and RoPE + append benchmarks all
run Hq32 / Hkv8 / D128 (four query heads per KV head), block size 32,
token-major, in fp16 and bf16 (benchmarks/run_flashinfer_baseline.py,
benchmarks/profile_paged_decode.py:83-86, benchmarks/run_rope_kv_append_bench.py:18-22).
Here, at those heads:

- decode through the public API against the fp32 oracle: full-length rows at
  the small benchmark shapes, lengths drawn from U{L/2..L} as the default
  profile draws them, and explicit split counts beside the planned one;
- ``rope_paged_kv_append`` with the fused backend on a cache seeded with
  context, against the torch backend (bit for bit with the cache's cos/sin
  tables, the default) and the RoPE oracle, for several consecutive tokens;
  then decode of the appended cache against the attention oracle.

Tolerance: atol 2e-2 / rtol 1e-2 against the fp32 oracle.
"""

import numpy as np
import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.paged_decode import paged_decode_attention, paged_decode_attention_into
from flashdec_amd.rope import rope_paged_kv_append
from oracle.attention import paged_decode_attention as oracle_decode
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 32
DTYPES = [torch.float16, torch.bfloat16]
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _oracle(q, k, v, table, lens):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lens", [[128], [1024] * 4, [1, 31, 32, 33, 600], [0, 257, 0]])
def test_grouped_rows_match_oracle(lens, dtype):
    q, k, v, table, sl = make_paged_inputs(lens, HQ, HKV, D, BS, dtype, seed=len(lens) + sum(lens) % 97)
    out = paged_decode_attention(q, k, v, table, sl)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("batch", "max_len"), [(16, 1024), (3, 4096)])
def test_default_profile_lengths_match_oracle(batch, max_len, dtype):
    rng = np.random.default_rng(batch + max_len)
    lens = [int(x) for x in rng.integers(max_len // 2, max_len + 1, size=batch)]
    q, k, v, table, sl = make_paged_inputs(lens, HQ, HKV, D, BS, dtype, seed=batch)
    out = torch.empty_like(q)
    paged_decode_attention_into(q, k, v, table, sl, out)  # library-planned splits
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("num_splits", [2, 5, 16, 32])
def test_explicit_splits_match_oracle(num_splits, dtype):
    q, k, v, table, sl = make_paged_inputs([1500, 65, 1024], HQ, HKV, D, BS, dtype, seed=num_splits)
    ws = (torch.empty((3, HQ, num_splits, D), device="cuda"), torch.empty((3, HQ, num_splits), device="cuda"),
          torch.empty((3, HQ, num_splits), device="cuda"))
    out = torch.empty_like(q)
    paged_decode_attention_into(q, k, v, table, sl, out, split_kv_workspace=ws, num_splits=num_splits)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_append_on_seeded_context_then_decode(dtype):
    """The RoPE + append benchmark's call (rope_paged_kv_append, fused backend, base 10000) on a
    cache seeded with context, as the reference benchmark builds it, for five consecutive tokens."""
    batch, ctx = 4, 100
    caches = {}
    for name in ("torch", "fused_cuda"):
        cache = PagedKVCache(1, HKV, D, BS, 64, dtype=dtype, device="cuda")
        for r in range(batch):
            cache.add_request(r)
        gen = torch.Generator().manual_seed(5)
        seed_k = torch.randn((1, batch, ctx, HKV, D), generator=gen).to(dtype).cuda()
        seed_v = torch.randn((1, batch, ctx, HKV, D), generator=gen).to(dtype).cuda()
        cache.seed_context(list(range(batch)), ctx, k=seed_k, v=seed_v)
        caches[name] = cache
    g = torch.Generator().manual_seed(17)
    ids = list(range(batch))
    for _ in range(5):
        q = torch.randn((batch, HQ, D), generator=g).to(dtype).cuda()
        k = torch.randn((batch, HKV, D), generator=g).to(dtype).cuda()
        v = torch.randn((batch, HKV, D), generator=g).to(dtype).cuda()
        res = {n: rope_paged_kv_append(c, 0, ids, q, k, v, append_backend=n) for n, c in caches.items()}
        pos = res["torch"].positions
        assert pos.tolist() == res["fused_cuda"].positions.tolist()
        assert torch.equal(res["torch"].q.view(torch.int16), res["fused_cuda"].q.view(torch.int16))
        exp_q = orope.apply_rope(q.float().cpu().numpy(), pos.cpu().numpy(), out_dtype=NAME[dtype])
        np.testing.assert_allclose(res["fused_cuda"].q.float().cpu().numpy(), exp_q, atol=2e-2, rtol=1e-2)
        fused = caches["fused_cuda"]
        table = fused.block_tables(ids).cuda()
        lens = fused.seq_lens_tensor(ids).cuda()
        out = paged_decode_attention(res["fused_cuda"].q, fused.k_cache[0], fused.v_cache[0], table, lens)
        assert_close_to_oracle(out, _oracle(res["fused_cuda"].q, fused.k_cache[0], fused.v_cache[0], table, lens))
    torch.cuda.synchronize()
    assert torch.equal(caches["torch"].k_cache.view(torch.int16), caches["fused_cuda"].k_cache.view(torch.int16))
    assert torch.equal(caches["torch"].v_cache, caches["fused_cuda"].v_cache)
    assert caches["torch"].metrics() == caches["fused_cuda"].metrics()
