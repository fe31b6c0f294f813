"""The MoE parts of the oracle (CPU): the token floor against the reference's own blend
(tests/golden/moe_blend.npz, written from hi2.moe.blend with the experts' sum of
hi2/layerwise.py:241-257), and the routed batch order of hi2/moe.py:83-100."""

import os

import numpy as np
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_top_up_equals_the_reference_blend():
    g = np.load(os.path.join(GOLDEN, "moe_blend.npz"))
    out, out_n = oracle.moe_top_up(g["sums"], g["counts"], int(g["need"]))
    assert out_n == g["out_n"].tolist()
    assert np.array_equal(out, g["out"])
    # experts at or above the floor are untouched; the floor is the reference's own test
    # identity (tests/test_moe.py:201-213) to rounding
    counts = g["counts"]
    need = int(g["need"])
    tot = g["sums"].astype(np.float64).sum(0)
    for e, n in enumerate(counts):
        if n >= need:
            assert np.array_equal(out[e], g["sums"][e])
        else:
            want = g["sums"][e] + (need - n) * tot / counts.sum()
            assert np.allclose(out[e], want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_top_up_without_tokens_changes_nothing():
    s = np.random.default_rng(0).standard_normal((3, 8, 8)).astype(np.float32)
    out, n = oracle.moe_top_up(s, [0, 0, 0], 4096)
    assert n == [0, 0, 0] and np.array_equal(out, s)


def test_route_order_is_the_reference_expert_loop():
    """hi2_amd.moe.route_order (a stable sort of the flat expert indices, the counts'
    prefix sums) against the reference's loop written out: expert by expert, the routed
    slots in token order."""
    from hi2_amd.moe import route_order

    g = torch.Generator().manual_seed(5)
    e, t, k = 9, 50, 3
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
    rows, offs = route_order(idx, e)
    want_rows, want_offs = [], [0]
    for ex in range(e):
        for tok in range(t):
            for pos in range(k):
                if int(idx[tok, pos]) == ex:
                    want_rows.append(tok)
        want_offs.append(len(want_rows))
    assert rows.tolist() == want_rows and offs.tolist() == want_offs
