"""CPU checks of the score profiles the score-range GPU tests rely on.

``steps`` must move a column's running maximum past the kernels' slack of 8
(base 2) many times within a split, and ``falling`` never after the first
unit (the profiles are built in tests/test_score_range_gpu.py).  On
``steps``, a float64 restatement of the kernels' lazy update equals the
softmax, and the same update with its rescale dropped (a planted mistake)
misses the GPU tests' tolerance.
"""

import numpy as np
import torch

from tests.helpers import make_paged_inputs
from tests.test_score_range_gpu import _shape_scores


def test_profiles_move_the_maximum_past_the_slack():
    # one row's head 0, unit by unit (16 tokens), as the kernels track it
    for profile, expect_moves in (("steps", True), ("falling", False)):
        q, k, v, table, sl = make_paged_inputs([4096], 16, 2, 128, 16, torch.bfloat16, seed=93, device="cpu")
        _shape_scores(profile, q, k, v, table, sl, 16, 93)
        rows = k[table[0].long()].permute(1, 0, 2, 3).reshape(2, -1, 128)[0, :4096].float()
        s = (rows @ q[0, 0].float()) / 128**0.5 / np.log(2.0)  # base-2 scores of head 0
        ref = -np.inf
        moves = 0
        for u in range(0, 4096, 16):
            mx = float(s[u : u + 16].max())
            if mx > ref + 8:
                moves += ref != -np.inf
                ref = mx
        assert (moves >= 20) == expect_moves, (profile, moves)


def _lazy_softmax_v(s, vrows, unit=16, slack=8.0, drop_rescale=False):
    """The kernels' per-column online softmax (base 2, reference maximum that
    moves only past ``slack``), restated in float64 for one column."""
    ref = -np.inf
    acc = np.zeros(vrows.shape[1])
    den = 0.0
    for u in range(0, len(s), unit):
        su = s[u : u + unit]
        mx = su.max()
        if mx > ref + slack:
            if ref != -np.inf and not drop_rescale:
                alpha = 2.0 ** (ref - mx)
                acc *= alpha
                den *= alpha
            ref = mx
        p = 2.0 ** (su - ref)
        acc += p @ vrows[u : u + unit]
        den += p.sum()
    return acc / den


def test_rescale_on_moves_is_what_the_profiles_check():
    # on the "steps" profile the lazy update with its rescales equals the
    # softmax, and the same update with the rescale dropped misses the
    # GPU tests' tolerance by far
    q, k, v, table, sl = make_paged_inputs([4096], 16, 2, 128, 16, torch.bfloat16, seed=93, device="cpu")
    _shape_scores("steps", q, k, v, table, sl, 16, 93)
    krows = k[table[0].long()].permute(1, 0, 2, 3).reshape(2, -1, 128)[0, :4096].double().numpy()
    vrows = v[table[0].long()].permute(1, 0, 2, 3).reshape(2, -1, 128)[0, :4096].double().numpy()
    s = krows @ q[0, 0].double().numpy() / 128**0.5 / np.log(2.0)
    w = 2.0 ** (s - s.max())
    exact = (w / w.sum()) @ vrows
    bound = 2e-2 + 1e-2 * np.abs(exact)
    assert np.all(np.abs(_lazy_softmax_v(s, vrows) - exact) <= 1e-9 + 1e-9 * np.abs(exact))
    assert np.any(np.abs(_lazy_softmax_v(s, vrows, drop_rescale=True) - exact) > bound)
