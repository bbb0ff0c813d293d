"""Shared builders for parity tests: seeded paged inputs and tolerance checks."""

from __future__ import annotations

import numpy as np
import torch

# Parity bar for attention against an fp32 reference: atol 2e-2 / rtol 1e-2
ATOL = 2e-2
RTOL = 1e-2


def make_paged_inputs(
    seq_lens,
    num_q_heads,
    num_kv_heads,
    head_dim,
    block_size,
    dtype=torch.bfloat16,
    seed=61,
    device="cuda",
    pool_factor=1.25,
    kv_layout="token_major",
    table_width=None,
    pad_value=-1,
):
    """Random N(0,1) q and paged K/V with block tables drawn from a shuffled pool.

    Each request's blocks are a slice of ``randperm(pool)`` so logical
    neighbours are physically scattered (the reference's fixtures assert the
    same property, tests/test_paged_decode.py:113).  Unused table slots hold
    ``pad_value``.
    """
    gen = torch.Generator().manual_seed(seed)
    nblk = [(int(n) + block_size - 1) // block_size for n in seq_lens]
    total = max(1, sum(nblk))
    pool = max(total + 1, int(total * pool_factor))
    width = max(1, max(nblk)) if table_width is None else table_width
    perm = torch.randperm(pool, generator=gen)
    table = torch.full((len(seq_lens), width), pad_value, dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[cursor:cursor + n].to(torch.int32)
        cursor += n
    shape = (pool, num_kv_heads, block_size, head_dim)
    k = torch.randn(shape, generator=gen).to(dtype)
    v = torch.randn(shape, generator=gen).to(dtype)
    q = torch.randn((len(seq_lens), num_q_heads, head_dim), generator=gen).to(dtype)
    if kv_layout == "dim_major":
        k = k.permute(0, 1, 3, 2).contiguous()
        v = v.permute(0, 1, 3, 2).contiguous()
    sl = torch.tensor([int(x) for x in seq_lens], dtype=torch.int32)
    return q.to(device), k.to(device), v.to(device), table.to(device), sl.to(device)


def np32(t):
    return t.detach().float().cpu().numpy()


def assert_close_to_oracle(actual, expected, atol=ATOL, rtol=RTOL):
    a = np32(actual)
    e = np.asarray(expected, dtype=np.float32)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.all(np.isfinite(a)), "non-finite output"
    err = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    worst = float((err - bound).max())
    assert worst <= 0, f"max |err| {float(err.max()):.3e} exceeds atol {atol} + rtol {rtol}*|ref| (by {worst:.3e})"


def bits16(t):
    """Bit patterns of a 16-bit float tensor (for bit-exact comparisons)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


def rope_pair_bound(x, pos, rotary_dim, base):
    """Per-element bound on how far two fp32 evaluations of split-half RoPE may differ when each
    one's inv_freq is within an ulp of the correctly rounded value (cos/sin within an ulp too).

    Frequency i's angle error is at most (pos + 1) * ulp(inv_i) <= (pos + 1) * inv_i * 2^-23 per
    evaluation; each rotated element moves by at most (|x_lo| + |x_hi|) times the angle error plus
    the products' and sum's rounding (2^-21 relative).  Low frequencies (inv_i << 1) therefore get
    a bound far below the position-independent 2^-23 * pos * max|x|.
    """
    half = rotary_dim // 2
    inv = np.array([base ** (-2.0 * i / rotary_dim) for i in range(half)])
    pair = np.abs(x[..., :half]) + np.abs(x[..., half:rotary_dim])
    per = pair * (2.0 * (np.asarray(pos, dtype=np.float64)[:, None, None] + 1) * inv * 2.0**-23 + 2.0**-21)
    return np.concatenate([per, per], axis=-1)


def device_rope(x, positions, rotary_dim=None, base=10_000.0):
    """float32 numpy of the reference's torch RoPE (flashdec/rope.py:26-85, restated as
    ``flashdec_amd.rope.apply_rope``) evaluated on x's device, in x's dtype: the HIP RoPE
    launches that read the cache's cos/sin tables (the engine's and the cache's default)
    reproduce it bit for bit."""
    from flashdec_amd.rope import apply_rope

    pos = torch.as_tensor(np.asarray(positions), dtype=torch.int64).to(x.device)
    return apply_rope(x, pos, rotary_dim=rotary_dim, base=base).float().cpu().numpy()
