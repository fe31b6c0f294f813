"""The oracle's local code refinement (``or_refine``) pinned against the reference's
``refine_groups`` golden vectors, the reference's own invariants
(``tests/test_refine.py``) and an independent unblocked float64 column loop — CPU only."""

import numpy as np
import pytest

import oracle
from golden_data import refine_cases

CASES = list(refine_cases())


def _cat(groups):
    """Rows of every group in one sweep: per-row block and top, ladders padded."""
    ldp = max(g["lo"].shape[1] for g in groups)
    pad = lambda a: np.pad(a, ((0, 0), (0, ldp - a.shape[1])))  # noqa: E731
    w = np.concatenate([g["w"] for g in groups])
    codes = np.concatenate([g["codes_in"] for g in groups])
    lo = np.concatenate([pad(g["lo"]) for g in groups])
    st = np.concatenate([pad(g["step"]) for g in groups])
    block = np.concatenate([np.full(len(g["w"]), g["block"]) for g in groups])
    top = np.concatenate([np.full(len(g["w"]), 2 ** g["nbits"] - 1.0) for g in groups])
    return w, codes, lo, st, block, top


def _objective(w, codes, lo, st, block, hs):
    """sum_r e_r Hs e_r^T in float64 (hi2/refine.py:23-36), e = fp16(lo + c st) - w."""
    idx = np.arange(w.shape[1]) // block
    rec = (lo[:, idx] + codes.astype(np.float32) * st[:, idx]).astype(np.float16)
    e = rec.astype(np.float64) - w.astype(np.float64)
    return float(np.einsum("ij,jk,ik->", e, hs.astype(np.float64), e))


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_refine_equals_reference_golden(case):
    tag, hs, passes, groups = case
    w, codes, lo, st, block, top = _cat(groups)
    got, moved, sweeps = oracle.refine(w, codes, lo, st, block, top, hs, passes)
    want = np.concatenate([g["codes"] for g in groups])
    assert np.array_equal(got, want)
    assert sweeps <= passes
    if passes:
        assert moved.sum() >= (got != codes).sum()


@pytest.mark.parametrize("tag", ["a", "b", "c", "e"])
def test_a_sweep_never_raises_the_objective_and_keeps_codes_in_range(tag):
    # the reference's tests/test_refine.py:37-55 invariants, on the golden inputs
    _, hs, _, groups = next(c for c in CASES if c[0] == tag)
    (g,) = groups
    w, c0, lo, st, block, top = _cat(groups)
    before = _objective(w, c0, lo, st, g["block"], hs)
    two, _, _ = oracle.refine(w, c0, lo, st, block, top, hs, 2)
    one, _, _ = oracle.refine(w, c0, lo, st, block, top, hs, 1)
    assert two.max() <= 2 ** g["nbits"] - 1
    after = _objective(w, two, lo, st, g["block"], hs)
    assert after <= before and after < 0.99 * before
    assert _objective(w, one, lo, st, g["block"], hs) >= after - 1e-6
    assert np.abs(one.astype(int) - c0.astype(int)).max() <= 1  # single steps per sweep


def test_zero_passes_return_the_input_and_a_converged_sweep_is_a_fixed_point():
    _, hs, _, groups = next(c for c in CASES if c[0] == "conv")
    w, c0, lo, st, block, top = _cat(groups)
    zero, moved, sweeps = oracle.refine(w, c0, lo, st, block, top, hs, 0)
    assert np.array_equal(zero, c0) and sweeps == 0 and moved.sum() == 0
    conv, _, sweeps = oracle.refine(w, c0, lo, st, block, top, hs, 40)
    assert sweeps < 40  # stopped after a sweep that moved nothing
    again, moved, sweeps = oracle.refine(w, conv, lo, st, block, top, hs, 1)
    assert np.array_equal(again, conv) and moved.sum() == 0 and sweeps == 1


def _plain_loop(w, codes, lo, st, block, top, hs, passes):
    """An independent statement of the refinement: unblocked, g updated over every
    column after every move, in float64 (the reference's tests/test_refine.py:58-87
    cross-check)."""
    w = w.astype(np.float64)
    hs = hs.astype(np.float64)
    c = codes.astype(np.float64).copy()
    n, k = w.shape
    idx = np.arange(k) // block
    lo_x = lo[:, idx].astype(np.float32)
    st_x = st[:, idx].astype(np.float32)

    def dec(cc):
        return (lo_x + cc.astype(np.float32) * st_x).astype(np.float16).astype(np.float64)

    g = (dec(c) - w) @ hs
    for _ in range(passes):
        for j in range(k):
            cur = dec(c)[:, j]
            best = np.zeros(n)
            best_d = np.zeros(n)
            best_dw = np.zeros(n)
            for d in (1.0, -1.0):
                cn = c[:, j] + d
                cc = c.copy()
                cc[:, j] = cn
                dw = dec(cc)[:, j] - cur
                ok = (cn >= 0) & (cn <= top) & (st_x[:, j] > 0)
                gain = np.where(ok, -(2 * dw * g[:, j] + dw * dw * hs[j, j]), -np.inf)
                better = gain > best
                best = np.where(better, gain, best)
                best_d = np.where(better, d, best_d)
                best_dw = np.where(better, dw, best_dw)
            c[:, j] += best_d
            g += best_dw[:, None] * hs[j][None, :]
    return c.astype(np.uint8)


def test_block_lazy_sweep_makes_the_decisions_of_a_plain_column_loop():
    _, hs, _, groups = next(c for c in CASES if c[0] == "a")
    (g,) = groups
    w, c0, lo, st, block, top = _cat(groups)
    w, c0, lo, st = w[:8], c0[:8], lo[:8], st[:8]
    blocked, _, _ = oracle.refine(w, c0, lo, st, block[:8], top[:8], hs, 2)
    plain = _plain_loop(w, c0, lo, st, g["block"], top[:8], hs, 2)
    ref = _objective(w, plain, lo, st, g["block"], hs)
    got = _objective(w, blocked, lo, st, g["block"], hs)
    assert got == pytest.approx(ref, rel=1e-4)
    assert (blocked != plain).mean() < 0.01


def test_mixed_candidates_share_a_sweep_with_the_result_of_each_alone():
    _, hs, passes, groups = next(c for c in CASES if c[0] == "mixed")
    w, c0, lo, st, block, top = _cat(groups)
    both, _, _ = oracle.refine(w, c0, lo, st, block, top, hs, passes)
    o = 0
    for g in groups:
        n = len(g["w"])
        alone, _, _ = oracle.refine(g["w"], g["codes_in"], g["lo"], g["step"], g["block"],
                                    2 ** g["nbits"] - 1, hs, passes)
        assert np.array_equal(both[o:o + n], alone)
        o += n
