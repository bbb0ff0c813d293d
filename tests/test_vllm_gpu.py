"""vLLM CUSTOM backend on the GPU: forward() through the real HIP kernels.

vLLM is not installed, so its modules are the fakes of tests/vllm_fakes.py.
The backend code, launcher and kernels are the product's.  The cache is
vLLM's ``[blocks, 2, block_size, kv_heads, head_size]`` allocation.  vLLM
has already written the newest token (its separate KV update), and the
kernel stores the same bytes again.  Rows past the live requests carry
``slot_mapping = -1`` graph padding.
"""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests import vllm_fakes
from tests.helpers import assert_close_to_oracle, bits16

pytestmark = pytest.mark.gpu


def vllm_batch(lens, padded_rows, bs=16, hq=16, hkv=2, d=128, dtype=torch.bfloat16, seed=5, table_width=None):
    g = torch.Generator().manual_seed(seed)
    nblk = [(n + bs - 1) // bs for n in lens]
    width = table_width or max(nblk)
    pool = sum(width for _ in lens) + 4
    cache = torch.randn((pool, 2, bs, hkv, d), generator=g).to(dtype).cuda()
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros((padded_rows, width), dtype=torch.int32)
    for b in range(len(lens)):
        table[b] = perm[b * width:(b + 1) * width].to(torch.int32)
    seq_lens = torch.zeros(padded_rows, dtype=torch.int32)
    seq_lens[: len(lens)] = torch.tensor(lens, dtype=torch.int32)
    slot = torch.full((padded_rows,), -1, dtype=torch.int64)
    key = torch.zeros((padded_rows, hkv, d), dtype=dtype)
    value = torch.zeros((padded_rows, hkv, d), dtype=dtype)
    for b, n in enumerate(lens):
        blk = int(table[b, (n - 1) // bs])
        off = (n - 1) % bs
        slot[b] = blk * bs + off
        key[b] = cache[blk, 0, off].cpu()
        value[b] = cache[blk, 1, off].cpu()
    q = torch.randn((padded_rows, hq, d), generator=g).to(dtype)
    md = SimpleNamespace(
        query_start_loc=torch.arange(padded_rows + 1, dtype=torch.int32).cuda(),
        max_seq_len=max(lens),
        max_query_len=1,
        use_cascade=False,
        causal=True,
        block_table=table.cuda(),
        seq_lens=seq_lens.cuda(),
        slot_mapping=slot.cuda(),
        softmax_segm_output=torch.empty((padded_rows, hq, 16, d), device="cuda"),
        softmax_segm_max=torch.empty((padded_rows, hq, 16), device="cuda"),
        softmax_segm_expsum=torch.empty((padded_rows, hq, 16), device="cuda"),
    )
    return q.cuda(), key.cuda(), value.cuda(), cache, md


def expected_rows(q, cache, md, live):
    k = cache[:, 0].permute(0, 2, 1, 3).float().cpu().numpy()  # [NB, Hkv, bs, D]
    v = cache[:, 1].permute(0, 2, 1, 3).float().cpu().numpy()
    return oracle_decode(q[:live].float().cpu().numpy(), k, v, md.block_table[:live].cpu().numpy(),
                         md.seq_lens[:live].cpu().numpy())


@pytest.fixture
def vb(monkeypatch):
    module, _ = vllm_fakes.install(monkeypatch)
    return module


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lens,padded", [([2048] * 8, 8), ([700, 513, 4000], 8), ([600, 1200], 2)])
def test_forward_matches_oracle_with_padding_rows(vb, dtype, lens, padded):
    impl = vb.FlashDecAttentionImpl(16, 128, 1 / math.sqrt(128), 2)
    q, key, value, cache, md = vllm_batch(lens, padded, dtype=dtype)
    before = cache.clone()
    out = torch.full_like(q, 7)
    layer = SimpleNamespace(kv_sharing_target_layer_name=None)
    assert impl.forward(layer, q, key, value, cache, md, out) is out
    torch.cuda.synchronize()
    assert vllm_fakes.TritonAttentionImpl.fallback_calls == []
    assert_close_to_oracle(out[: len(lens)], expected_rows(q, cache, md, len(lens)))
    assert torch.count_nonzero(out[len(lens):]) == 0  # padding rows are zero
    assert np.array_equal(bits16(cache), bits16(before))  # re-stored newest token has the same bytes


def test_forward_under_graph_capture_follows_growing_rows(vb):
    """Capture once at the batch's current max_seq_len, replay as rows grow (vLLM's decode graphs)."""
    impl = vb.FlashDecAttentionImpl(16, 128, 1 / math.sqrt(128), 2)
    final = [1500, 900, 2600, 520]
    q, key, value, cache, md = vllm_batch(final, 6, table_width=(2600 + 15) // 16, seed=9)
    out = torch.empty_like(q)
    layer = SimpleNamespace(kv_sharing_target_layer_name=None)

    def set_lengths(lengths):
        for b, n in enumerate(lengths):
            md.seq_lens[b] = n
            blk = int(md.block_table[b, (n - 1) // 16])
            off = (n - 1) % 16
            md.slot_mapping[b] = blk * 16 + off
            key[b] = cache[blk, 0, off]
            value[b] = cache[blk, 1, off]

    set_lengths([1000, 600, 1100, 512])
    md.max_seq_len = 1100
    impl.forward(layer, q, key, value, cache, md, out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph):
            impl.forward(layer, q, key, value, cache, md, out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for lengths in ([1001, 601, 1101, 513], final, [1300, 899, 2000, 515]):
        set_lengths(lengths)
        out.fill_(3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_close_to_oracle(out[:4], expected_rows(q, cache, md, 4))
        assert torch.count_nonzero(out[4:]) == 0
