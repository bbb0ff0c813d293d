"""GPU parity of balanced (per-row) split counts for ragged batches.

With ``balance_target`` V > 0 each row's split count follows its own length,
computed on the device from seq_lens (no counterpart in the reference, whose
split count is per launch, flashdec/kernels/paged_decode.py:408-411).  The
result must equal plain paged decode, so the oracle is the paged-decode
oracle.  Cases: block sizes 8/16/32, fp16/bf16, zero-length and one-token
rows, targets from 1 to beyond the row count, split caps below the rows'
counts, the ``ragged=True`` Python path, a graph replayed after the lengths
change, and an engine step graph captured on a ragged batch.  Tolerance:
atol 2e-2 / rtol 1e-2.
"""

import math

import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

RAGGED = [700, 3, 0, 129, 2000, 64, 31, 1]


def _oracle(q, k, v, table, lens):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy())


def _launch(q, k, v, table, lens, out, block_size, splits, target):
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out,
                    k.shape[1], block_size, 1.0 / math.sqrt(q.shape[2]))
    args.num_blocks = k.shape[0]
    args.max_seq_len = table.shape[1] * block_size
    stream = _lib.current_stream_handle(q.device)
    acc, mx, sm, _ = pd._auto_workspace(q, k.shape[1], splits, stream)
    pd._fill_workspace(args, acc, mx, sm, splits)
    args.balance_target = target
    _lib.paged_decode(args, stream)
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize(("target", "splits"), [(1, 2), (3, 5), (17, 9), (100, 64), (6, 3)])
def test_balanced_splits_match_oracle(target, splits, block_size, dtype):
    q, k, v, table, lens = make_paged_inputs(RAGGED, 16, 2, 128, block_size, dtype, seed=block_size + target)
    out = _launch(q, k, v, table, lens, torch.empty_like(q), block_size, splits, target)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))
    assert torch.count_nonzero(out[2]) == 0  # the zero-length row


@pytest.mark.parametrize(("hq", "hkv"), [(16, 2), (8, 1), (32, 2), (4, 4)])
def test_ragged_flag_matches_oracle(hq, hkv):
    import flashdec_amd as fd

    q, k, v, table, lens = make_paged_inputs([4000, 10, 250, 0, 1500, 33, 7, 900, 60], hq, hkv, 128, 32,
                                             torch.bfloat16, seed=hq)
    out = fd.decode(q, k, v, table, lens, ragged=True)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_balanced_graph_follows_new_lengths():
    # the split counts are recomputed from seq_lens at every replay (every
    # row owns 3000 tokens of blocks; the lengths vary below that)
    q, k, v, table, lens = make_paged_inputs([3000] * 4, 16, 2, 128, 16, torch.bfloat16, seed=5)
    lens.copy_(torch.tensor([3000, 40, 500, 2], dtype=lens.dtype))
    out = torch.empty_like(q)
    _launch(q, k, v, table, lens, out, 16, 24, 24)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph):
            _launch(q, k, v, table, lens, out, 16, 24, 24)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for lengths in ([3000, 40, 500, 2], [10, 3000, 3000, 0], [1, 2, 3, 2999], [0, 0, 0, 0]):
        lens.copy_(torch.tensor(lengths, dtype=lens.dtype))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_engine_step_graph_on_a_ragged_batch():
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine
    from oracle import attention as oa
    from oracle import rope as orope

    layers, hq, hkv, d, bs = 2, 16, 2, 128, 16
    cache = PagedKVCache(layers, hkv, d, bs, max_blocks=320, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(3)
    cache.k_cache.copy_(torch.randn(cache.k_cache.shape, device="cuda", generator=g))
    cache.v_cache.copy_(torch.randn(cache.v_cache.shape, device="cuda", generator=g))
    cache.enable_graph_metadata(4, 160)
    engine = DecodeEngine(cache)
    contexts = {"a": 2000, "b": 30, "c": 70, "d": 5}
    for rid, n in contexts.items():
        engine.add_request(rid)
    engine.admit(list(contexts))
    for rid, n in contexts.items():
        cache.seed_context([rid], n)
    sg = engine.capture_step_graph(4, hq, base=1e6)
    assert sg.balance_target > 0  # the batch is ragged: per-row split counts
    for step in range(3):
        q = torch.randn((layers, 4, hq, d), device="cuda", generator=g).to(torch.bfloat16)
        sg.q.copy_(q)
        sg.k.copy_(torch.randn((layers, 4, hkv, d), device="cuda", generator=g).to(torch.bfloat16))
        sg.v.copy_(torch.randn((layers, 4, hkv, d), device="cuda", generator=g).to(torch.bfloat16))
        tx = engine.begin_step()
        out = engine.step_graph(tx, sg)
        torch.cuda.synchronize()
        for layer in range(layers):
            q_rot = orope.apply_rope(q[layer].float().cpu().numpy(), tx.positions.cpu().numpy(), base=1e6,
                                     out_dtype="bfloat16")
            expected = oa.paged_decode_attention(q_rot, cache.k_cache[layer].float().cpu().numpy(),
                                                 cache.v_cache[layer].float().cpu().numpy(),
                                                 tx.block_tables.cpu().numpy(), tx.effective_seq_lens.cpu().numpy())
            assert_close_to_oracle(out[layer], expected)
        engine.commit_step(tx)
    assert engine.validate_invariants()


def test_full_c4_ragged_shape_rows_match_oracle():
    """The ragged long-context shape at full size: B32, L ~ logU[128, 32768] (seed 1701),
    Hq16/Hkv2, D128, bf16, bs32.  Both split policies are checked against the
    oracle on the longest row, the shortest and three others."""
    import numpy as np

    import flashdec_amd as fd

    rng = np.random.default_rng(1701)
    lens_list = [int(round(math.exp(x))) for x in rng.uniform(math.log(128), math.log(32768), size=32)]
    bs, hkv, hq, d = 32, 2, 16, 128
    nblk = [-(-n // bs) for n in lens_list]
    pool = int(sum(nblk) * 1.25) + 1
    g = torch.Generator(device="cuda").manual_seed(1701)
    perm = torch.randperm(pool, device="cuda", generator=g).to(torch.int32)
    table = torch.full((32, max(nblk)), -1, device="cuda", dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n
    k = torch.randn((pool, hkv, bs, d), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((pool, hkv, bs, d), device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((32, hq, d), device="cuda", generator=g).to(torch.bfloat16)
    lens = torch.tensor(lens_list, device="cuda", dtype=torch.int32)
    rows = sorted({int(np.argmax(lens_list)), int(np.argmin(lens_list)), 3, 17, 30})
    k_np, v_np = np32(k), np32(v)
    for ragged in (False, True):
        out = fd.decode(q, k, v, table, lens, ragged=ragged)
        torch.cuda.synchronize()
        sel = torch.tensor(rows, device="cuda")
        expected = oracle_decode(np32(q[sel]), k_np, v_np, table[sel].cpu().numpy(), lens[sel].cpu().numpy())
        assert_close_to_oracle(out[sel], expected)
