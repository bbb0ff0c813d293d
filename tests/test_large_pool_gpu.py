"""KV pools past 2^32 elements (8.6 GB per cache): every kernel family addresses far blocks.

A vLLM or engine cache for one layer easily holds more than 2^31 elements
(vLLM sizes it to the free HBM; 288 GB on this part), so a block id times a
block stride must not wrap in 32 bits anywhere: neither in an element offset
nor in a byte offset.  The reference's kernels take such caches as plain
tensors (flashdec/kernels/paged_decode.py:28-543 index with
``block_id * stride``); its tests use small pools only.

One pair of [524544, 2, 32, 128] bf16 caches (2^32 + 2^21 elements each) is
shared by the module and reinterpreted per case (token-major or dim-major,
head_dim 128 or 64).  Rows draw their blocks from around element 2^31 (byte
2^32) and from the last blocks past element 2^32, mixed with low blocks, so
that one row's units straddle both boundaries.  Each launch is checked
against the float64 oracle on a compact copy of the blocks it uses, appended
K/V bytes bit for bit, and the launch record names the kernel each case is
meant to reach.
"""

import math

import numpy as np
import pytest
import torch

from oracle import rope as orope
from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, bits16, np32

pytestmark = pytest.mark.gpu

HKV, BS, D = 2, 32, 128
ELEMS_PER_BLOCK = HKV * BS * D          # 8192
NB = (1 << 32) // ELEMS_PER_BLOCK + 256  # 524544 blocks: the last ones start past element 2^32


@pytest.fixture(scope="module")
def pool():
    k = torch.empty((NB, HKV, BS, D), device="cuda", dtype=torch.bfloat16)
    v = torch.empty_like(k)
    assert k.numel() > (1 << 32) and k.numel() * k.element_size() > (1 << 33)
    yield k, v
    del k, v
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _views(k, v, layout, head_dim):
    """The pool's memory as [nb, 2, 32, head_dim] (token-major) or [nb, 2, head_dim, 32] (dim-major)."""
    nb = k.numel() // (HKV * BS * head_dim)
    shape = (nb, HKV, BS, head_dim) if layout == "token_major" else (nb, HKV, head_dim, BS)
    return k.view(shape), v.view(shape), nb


def _far_ids(nb, count, seed, exclude=()):
    """``count`` distinct block ids of an ``nb``-block view: low blocks, blocks around element 2^31 and
    the last blocks (past element 2^32)."""
    # every view holds about 2^32 + 2^21 elements: block nb/2 starts 2^20 elements past element 2^31,
    # and the 600 blocks below it reach across that boundary
    mid = nb // 2
    cands = np.concatenate([np.arange(0, 400), np.arange(mid - 600, mid + 600), np.arange(nb - 1200, nb)])
    cands = np.setdiff1d(cands, np.asarray(exclude, dtype=np.int64))
    ids = np.random.default_rng(seed).choice(cands, size=count, replace=False)
    assert ids.max() < nb
    return ids


def _fill(k, v, lens, hq, head_dim, seed, width=None, exclude=()):
    """Random q and blocks for rows of ``lens``; returns q, table, seq_lens and the compact oracle inputs."""
    nb = k.shape[0]
    nblk = [(n + BS - 1) // BS for n in lens]
    ids = _far_ids(nb, sum(nblk), seed, exclude)
    width = max(nblk) if width is None else width
    table = np.full((len(lens), width), -1, dtype=np.int32)
    compact = np.full((len(lens), width), -1, dtype=np.int32)
    cursor = 0
    for b, n in enumerate(nblk):
        table[b, :n] = ids[cursor:cursor + n]
        compact[b, :n] = np.arange(cursor, cursor + n)
        cursor += n
    gen = torch.Generator().manual_seed(seed)
    blocks = torch.randn((len(ids),) + tuple(k.shape[1:]), generator=gen).to(torch.bfloat16)
    vblocks = torch.randn((len(ids),) + tuple(k.shape[1:]), generator=gen).to(torch.bfloat16)
    idx = torch.from_numpy(ids).cuda()
    k[idx] = blocks.cuda()
    v[idx] = vblocks.cuda()
    q = torch.randn((len(lens), hq, head_dim), generator=gen).to(torch.bfloat16).cuda()
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    return q, torch.from_numpy(table).cuda(), sl, (np32(blocks), np32(vblocks), compact)


def _expected(q, lens, compact_inputs, layout="token_major"):
    kc, vc, table = compact_inputs
    return oracle_decode(np32(q), kc, vc, table, np.asarray(lens), kv_layout=layout)


@pytest.fixture
def record():
    from flashdec_amd import _lib

    _lib.record_launches(True)
    yield _lib
    _lib.record_launches(False)


@pytest.mark.parametrize(("layout", "head_dim", "hq", "lens", "kernel"), [
    ("token_major", 128, 16, [2048, 777, 33, 1500], "fd::decode_mfma_kernel<__bf16, 32, 0, false, 32, true, 128, 1>"),
    ("token_major", 128, 16, [8192, 6000, 100, 7000], "fd::decode_mfma_kernel<__bf16, 32, 0, false, 16, true, 128, 1>"),
    ("token_major", 128, 64, [3000, 900], "fd::decode_mfma_kernel<__bf16, 32, 0, false, "),
    ("token_major", 64, 16, [2500, 40, 1300], "fd::decode_mfma_kernel<__bf16, 32, 0, false, "),
    ("dim_major", 128, 16, [2048, 700, 1], "fd::decode_dm_kernel<__bf16, 32, true, 128, 0>"),
    ("dim_major", 64, 16, [3000, 65], "fd::decode_dm_kernel<__bf16, 32, true, 64, 0>"),
])
def test_decode_reads_blocks_past_2_pow_32_elements(pool, record, layout, head_dim, hq, lens, kernel):
    import flashdec_amd as fd

    k, v, _ = _views(*pool, layout, head_dim)
    q, table, sl, compact = _fill(k, v, lens, hq, head_dim, seed=sum(lens) + hq + head_dim)
    out = fd.decode(q, k, v, table, sl, kv_layout=layout)
    names = record.last_launch()
    assert names[0].startswith(kernel), names
    assert_close_to_oracle(out, _expected(q, lens, compact, layout))


def test_per_row_splits_read_far_blocks(pool, record):
    import flashdec_amd as fd

    k, v, _ = _views(*pool, "token_major", D)
    lens = [6000, 10, 250, 0, 1500, 33, 7, 900]
    q, table, sl, compact = _fill(k, v, lens, 16, D, seed=5)
    out = fd.decode(q, k, v, table, sl, ragged=True)
    assert record.last_launch()[0] == "fd::decode_balanced_kernel<__bf16, 32, true>"
    assert_close_to_oracle(out, _expected(q, lens, compact))


def test_generic_kernel_reads_far_blocks(pool, record):
    import flashdec_amd as fd

    # the pool one element in: a 2-byte aligned base leaves both MFMA kernels, so the VALU kernel
    # addresses the far blocks
    k, v = pool
    n = (NB - 1) * ELEMS_PER_BLOCK
    kk = k.view(-1)[1:1 + n].view(NB - 1, HKV, BS, D)
    vv = v.view(-1)[1:1 + n].view(NB - 1, HKV, BS, D)
    lens = [1200, 77]
    q, table, sl, compact = _fill(kk, vv, lens, 16, D, seed=17)
    out = fd.decode(q, kk, vv, table, sl)
    assert record.last_launch()[0].startswith("fd::decode_generic_kernel<__bf16, "), record.last_launch()
    assert_close_to_oracle(out, _expected(q, lens, compact))


@pytest.mark.parametrize("num_splits", [1, 8])
def test_fused_append_writes_far_slots(pool, num_splits):
    import flashdec_amd as fd

    k, v, nb = _views(*pool, "token_major", D)
    lens = [1025, 64, 3000]
    # the appended token's slot: each row's last block is moved to one of the last three blocks
    last = [nb - 1, nb - 2, nb - 3]
    q, table, sl, (kc, vc, compact) = _fill(k, v, lens, 16, D, seed=23 + num_splits, exclude=last)
    for b, n in enumerate(lens):
        j = (n - 1) // BS
        table[b, j] = last[b]
    gen = torch.Generator().manual_seed(99)
    append_k = torch.randn((3, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    append_v = torch.randn((3, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    slots = []
    kc, vc = kc.copy(), vc.copy()
    for b, n in enumerate(lens):
        j, off = (n - 1) // BS, (n - 1) % BS
        # the moved block holds the same tokens as the compact copy, the new token from append_k/v
        ci = compact[b, j]
        k[last[b]] = torch.from_numpy(kc[ci]).to(torch.bfloat16).cuda()
        v[last[b]] = torch.from_numpy(vc[ci]).to(torch.bfloat16).cuda()
        k[last[b], :, off] = float("nan")
        v[last[b], :, off] = float("nan")
        kc[ci, :, off] = np32(append_k[b])
        vc[ci, :, off] = np32(append_v[b])
        slots.append(last[b] * BS + off)
    ws = (torch.empty((3, 16, 8, D), device="cuda"), torch.empty((3, 16, 8), device="cuda"),
          torch.empty((3, 16, 8), device="cuda"))
    out = torch.empty_like(q)
    fd.paged_decode_attention_into(q, k, v, table, sl, out, split_kv_workspace=ws if num_splits > 1 else None,
                                   num_splits=num_splits,
                                   append_k=append_k, append_v=append_v,
                                   slot_mapping=torch.tensor(slots, device="cuda", dtype=torch.int64))
    assert_close_to_oracle(out, oracle_decode(np32(q), kc, vc, compact, np.asarray(lens)))
    for b, n in enumerate(lens):
        off = (n - 1) % BS
        assert np.array_equal(bits16(k[last[b], :, off]), bits16(append_k[b])), b
        assert np.array_equal(bits16(v[last[b], :, off]), bits16(append_v[b])), b


def test_vllm_5d_cache_past_2_pow_32_elements():
    from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into

    bs = 16
    nb = (1 << 32) // (2 * bs * HKV * D) + 64  # [nb, 2, 16, 2, 128]: 2^32 + 2^20 elements
    cache = torch.empty((nb, 2, bs, HKV, D), device="cuda", dtype=torch.bfloat16)
    try:
        lens = [900, 31, 1600]
        nblk = [(n + bs - 1) // bs for n in lens]
        mid = (1 << 31) // (2 * bs * HKV * D)
        rng = np.random.default_rng(7)
        cands = np.concatenate([np.arange(0, 100), np.arange(mid - 100, mid + 100), np.arange(nb - 200, nb)])
        ids = rng.choice(cands, size=sum(nblk), replace=False)
        table = np.full((3, max(nblk)), -1, dtype=np.int32)
        compact = np.full_like(table, -1)
        cursor = 0
        for b, n in enumerate(nblk):
            table[b, :n] = ids[cursor:cursor + n]
            compact[b, :n] = np.arange(cursor, cursor + n)
            cursor += n
        gen = torch.Generator().manual_seed(8)
        blocks = torch.randn((len(ids), 2, bs, HKV, D), generator=gen).to(torch.bfloat16)
        cache[torch.from_numpy(ids).cuda()] = blocks.cuda()
        q = torch.randn((3, 16, D), generator=gen).to(torch.bfloat16).cuda()
        append_k = torch.empty((3, HKV, D), device="cuda", dtype=torch.bfloat16)
        append_v = torch.empty_like(append_k)
        slots = []
        for b, n in enumerate(lens):
            blk, off = int(table[b, (n - 1) // bs]), (n - 1) % bs
            append_k[b] = cache[blk, 0, off]
            append_v[b] = cache[blk, 1, off]
            cache[blk, :, off] = float("nan")  # the launch writes the token back from append_k/v
            slots.append(blk * bs + off)
        splits = 8
        ws = (torch.empty((3, 16, splits, D), device="cuda"), torch.empty((3, 16, splits), device="cuda"),
              torch.empty((3, 16, splits), device="cuda"))
        out = torch.empty_like(q)
        _vllm_paged_decode_attention_into(q, append_k, append_v, cache, torch.from_numpy(table).cuda(),
                                          torch.tensor(lens, device="cuda", dtype=torch.int32), out,
                                          torch.tensor(slots, device="cuda", dtype=torch.int64), *ws, num_reqs=3,
                                          num_q_heads=16, num_kv_heads=HKV, head_dim=D, block_size=bs,
                                          sm_scale=1.0 / math.sqrt(D), num_splits=splits)
        kc = np32(blocks[:, 0].permute(0, 2, 1, 3))  # [n, Hkv, bs, D]
        vc = np32(blocks[:, 1].permute(0, 2, 1, 3))
        assert_close_to_oracle(out, oracle_decode(np32(q), kc, vc, compact, np.asarray(lens)))
        for b, s in enumerate(slots):
            blk, off = divmod(s, bs)
            assert np.array_equal(bits16(cache[blk, 0, off]), bits16(blocks[np.where(ids == blk)[0][0], 0, off]))
            assert np.array_equal(bits16(cache[blk, 1, off]), bits16(blocks[np.where(ids == blk)[0][0], 1, off]))
    finally:
        del cache
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def test_cascade_shared_prefix_in_far_blocks(pool, record):
    from flashdec_amd.cascade import paged_decode_attention_cascade

    k, v, nb = _views(*pool, "token_major", D)
    prefix = np.arange(nb - 40, nb)  # 40 shared blocks at the very end of the pool
    tails = [[300, 301, 302], [262100, 262101], [5, 6, 7, 8], [262200]]
    tail_lens = [70, 40, 100, 9]
    rows = [40 * BS + n for n in tail_lens]
    width = max(40 + len(t) for t in tails)
    table = np.full((4, width), -1, dtype=np.int32)
    for b, t in enumerate(tails):
        table[b, :40] = prefix
        table[b, 40:40 + len(t)] = t
    used = np.unique(table[table >= 0])
    gen = torch.Generator().manual_seed(31)
    kb = torch.randn((len(used), HKV, BS, D), generator=gen).to(torch.bfloat16)
    vb = torch.randn((len(used), HKV, BS, D), generator=gen).to(torch.bfloat16)
    idx = torch.from_numpy(used).cuda()
    k[idx] = kb.cuda()
    v[idx] = vb.cuda()
    q = torch.randn((4, 16, D), generator=gen).to(torch.bfloat16).cuda()
    sl = torch.tensor(rows, dtype=torch.int32, device="cuda")
    out = paged_decode_attention_cascade(q, k, v, torch.from_numpy(table).cuda(), sl)
    assert any(n.startswith("fd::cascade_decode_kernel<") for n in record.last_launch()), record.last_launch()
    compact = np.where(table >= 0, np.searchsorted(used, np.maximum(table, 0)), -1).astype(np.int32)
    assert_close_to_oracle(out, oracle_decode(np32(q), np32(kb), np32(vb), compact, np.asarray(rows)))


def test_rope_append_and_kv_append_write_far_slots(pool):
    import flashdec_amd as fd

    k, v, nb = _views(*pool, "token_major", D)
    B = 6
    gen = torch.Generator().manual_seed(41)
    q = torch.randn((B, 16, D), generator=gen).to(torch.bfloat16).cuda()
    kin = torch.randn((B, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    vin = torch.randn((B, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    mid = (1 << 31) // ELEMS_PER_BLOCK
    blocks = torch.tensor([nb - 1, nb - 2, mid, mid - 1, nb - 100, 3], dtype=torch.int64, device="cuda")
    offs = torch.tensor([31, 0, 17, 31, 5, 9], dtype=torch.int64, device="cuda")
    pos = torch.tensor([8191, 1, 4000, 77, 12345, 0], dtype=torch.int64, device="cuda")
    q_out = fd.fused_rope_kv_append(q, kin, vin, k, v, blocks, offs, pos, base=1e6)
    p = pos.cpu().numpy()
    assert np.array_equal(bits16(q_out), bits16(torch.from_numpy(
        orope.apply_rope(np32(q), p, base=1e6, out_dtype="bfloat16")).to(torch.bfloat16)))
    k_rot = torch.from_numpy(orope.apply_rope(np32(kin), p, base=1e6, out_dtype="bfloat16")).to(torch.bfloat16)
    for b in range(B):
        blk, off = int(blocks[b]), int(offs[b])
        assert np.array_equal(bits16(k[blk, :, off]), bits16(k_rot[b])), b
        assert np.array_equal(bits16(v[blk, :, off]), bits16(vin[b])), b
    # the plain K/V scatter into the same far slots
    k2 = torch.randn((B, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    v2 = torch.randn((B, HKV, D), generator=gen).to(torch.bfloat16).cuda()
    fd.cuda_kv_append(k, v, blocks, offs, k2, v2)
    for b in range(B):
        blk, off = int(blocks[b]), int(offs[b])
        assert np.array_equal(bits16(k[blk, :, off]), bits16(k2[b])), b
        assert np.array_equal(bits16(v[blk, :, off]), bits16(v2[b])), b
