"""The oracle's composition of ``encode_many`` (``hi2/calibrate.py:297-424``) pinned to
the reference's own ``encode_many`` output (``tests/golden/encode_many.npz``: factor
sharing over q/k, act-order, refinement, nearest rows, ``comp``), given the factors the
reference computed there — CPU only."""

import numpy as np
import pytest

import oracle
from golden_data import encode_many_case

CANDS, TENSORS, CONFIGS = encode_many_case()
FIELDS = ("codes", "code_off", "blk_params", "param_off", "row_consts", "row_nbits",
          "row_block", "had")


@pytest.mark.parametrize("tag", list(CONFIGS))
def test_oracle_encode_many_equals_reference_golden(tag):
    cfg = CONFIGS[tag]
    got = oracle.encode_many(TENSORS, CANDS, cfg, cfg["factors"])
    for t, (packed, comp) in zip(TENSORS, got):
        want = cfg["out"][t["name"]]
        for f in FIELDS:
            assert np.array_equal(np.asarray(packed[f]).reshape(-1),
                                  np.asarray(want[f]).reshape(-1)), (t["name"], f)
        if t["comp"]:
            assert np.array_equal(comp, want["comp"]), t["name"]
        else:
            assert want["comp"] is None


def test_fixture_covers_factor_sharing_refinement_and_comp():
    # q and k read one input with one transform: three factors for four GPTQ tensors
    assert [len(CONFIGS[t]["factors"]) for t in ("g", "ga", "gr", "nr")] == [3, 3, 3, 0]
    g, r = CONFIGS["g"]["out"], CONFIGS["gr"]["out"]
    for t in TENSORS:
        moved = int((g[t["name"]]["codes"] != r[t["name"]]["codes"]).sum())
        # refinement moves codes, except for the QAD start (comp) and nearest rows
        assert (moved > 0) == (not t["comp"] and t["sigma"] is not None), t["name"]
    assert np.array_equal(g["k"]["comp"], r["k"]["comp"])


def test_oracle_own_factors_stay_close_to_the_reference():
    """With the oracle's own Cholesky chain (not bit-identical to LAPACK) the packed
    layout is the same and almost every code agrees."""
    cfg = CONFIGS["g"]
    got = oracle.encode_many(TENSORS, CANDS, cfg)
    for t, (packed, _) in zip(TENSORS, got):
        want = cfg["out"][t["name"]]
        for f in ("code_off", "param_off", "row_nbits", "row_block", "had"):
            assert np.array_equal(np.asarray(packed[f]).reshape(-1), want[f].reshape(-1))
        assert (packed["codes"] != want["codes"]).mean() < 0.05


def test_per_tensor_calls_equal_one_batched_call():
    cfg = CONFIGS["gr"]
    both = oracle.encode_many(TENSORS, CANDS, cfg, cfg["factors"])
    # factors per tensor alone: q, k (shared), o, n (none), v
    fac = {"q": 0, "k": 0, "o": 1, "v": 2}
    for t, (packed, comp) in zip(TENSORS, both):
        f = [cfg["factors"][fac[t["name"]]]] if t["name"] in fac else []
        (alone, comp1), = oracle.encode_many([t], CANDS, cfg, f)
        assert np.array_equal(alone["codes"], packed["codes"]), t["name"]
        assert (comp is None and comp1 is None) or np.array_equal(comp, comp1)
