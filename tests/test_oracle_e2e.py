"""The oracle against the reference's whole encode pipeline on BASELINE configurations
(tests/golden/e2e_*.npz, written by make_golden.py e2e from hi2's own HessianStats,
transform_sigma, inverse_factor, fwht_groups, GPTQ and encode_many; inputs from
tests/e2e_recipes.py).  CPU tests.

Pinned here, per case:
- the recipes reproduce the fixture's inputs (SHA-256 of X, W and the allocation);
- the oracle's transform of the reference's Sigma is the reference's Hs bit for bit;
- given the reference's Hs, factor U and rotated rows, the oracle's GPTQ gives the
  reference's codes, params, consts, sse and comp bit for bit (the trailing update's
  sequential FMA chain is the reference BLAS call's rounding at these shapes), and its
  packing gives the reference's packed buffers;
- the oracle's Hessian of the bf16 tokens is within 1e-5 of the reference's Sigma (the
  reference's fp32 GEMM sums in another order) and its float64-accumulated factor within
  the LAPACK fp32 factor's rounding of the reference's U.
"""

import numpy as np
import pytest
import torch

import oracle
from e2e_recipes import CANDIDATES, CASES, FULL_CASES, input_digests, inputs, sha
from golden_data import e2e_case

FULL = list(FULL_CASES)


@pytest.mark.parametrize("case", list(CASES))
def test_recipes_reproduce_the_fixture_inputs(case):
    g = e2e_case(case)
    dg = input_digests(case)
    assert dg["x"] == g["digest_x"] and dg["w"] == g["digest_w"]
    assert dg["picks"] == g["digest_picks"]


@pytest.mark.parametrize("case", FULL)
def test_oracle_given_the_reference_factor_equals_the_reference(case):
    g = e2e_case(case)
    _, w, picks, had = inputs(case)
    hs = oracle.transform_sigma(g["sigma"], None, had)
    assert sha(hs) == g["hs_sha"]
    d = np.diag(hs).copy()
    assert np.array_equal(d, g["d"])
    wt = oracle.fwht16(w, had)
    pieces = []
    for ci, rows, params, consts in g["groups"]:
        nb, b = CANDIDATES[ci]
        e = oracle.encode_rows_gptq(wt[rows], d, g["u"], nb, b, "normal")
        assert np.array_equal(e["codes"], g["codes"][rows]), (case, ci)
        assert np.array_equal(e["params"], params)
        assert np.array_equal(e["consts"].view(np.uint16), consts)
        assert np.array_equal(e["sse"], g["sse"][rows])
        assert np.array_equal(e["comp"], g["comp"][rows])
        pieces.append((rows, e["codes"], e["params"], e["consts"]))
    nbits = np.array([CANDIDATES[c][0] for c in picks], np.int64)
    block = np.array([CANDIDATES[c][1] for c in picks], np.int64)
    p = oracle.assemble(pieces, nbits, block, w.shape[1])
    assert np.array_equal(np.asarray(p["codes"]).reshape(-1).view(np.int32),
                          g["packed_codes"].reshape(-1))
    assert np.array_equal(np.asarray(p["blk_params"]).reshape(-1),
                          g["packed_blk_params"].reshape(-1))
    assert np.array_equal(np.asarray(p["row_consts"]).reshape(-1).view(np.uint16),
                          g["packed_row_consts"].reshape(-1))


@pytest.mark.parametrize("case", FULL)
def test_oracle_hessian_and_factor_within_the_reference_rounding(case):
    g = e2e_case(case)
    xb, _, _, had = inputs(case)
    k = xb.shape[1]
    s = np.zeros((k, k), np.float32)
    oracle.hessian_update(s, xb.view(torch.int16).numpy().view(np.uint16))
    sigma = s / np.float32(xb.shape[0])
    rel = np.abs(sigma - g["sigma"]).max() / np.abs(g["sigma"]).max()
    assert rel < 1e-5, rel
    u, att = oracle.inverse_factor(oracle.transform_sigma(g["sigma"], None, had), 0.01)
    assert att == 0
    urel = np.abs(u - g["u"]).max() / np.abs(g["u"]).max()
    print(f"{case}: sigma rel {rel:.3g}  factor rel {urel:.3g}")
    assert urel < 1e-3, urel


def _oracle_pipeline(case):
    xb, w, picks, had = inputs(case)
    k = w.shape[1]
    s = np.zeros((k, k), np.float32)
    oracle.hessian_update(s, xb.view(torch.int16).numpy().view(np.uint16))
    hs = oracle.transform_sigma(s / np.float32(xb.shape[0]), None, had)
    d = np.diag(hs).copy()
    u, _ = oracle.inverse_factor(hs, 0.01)
    return oracle.fwht16(w, had), d, u


@pytest.mark.parametrize("case", FULL)
def test_oracle_pipeline_departs_from_the_reference_only_at_ties(case):
    """The oracle's own fp32 Hessian and float64-accumulated factor against the
    reference's: an independent pipeline whose every diverging row must start at a
    ladder tie (fit errors equal to 1e-5) or a rounding tie; >= 99.9 % of codes equal.
    This pins the tie classification the GPU end-to-end tests apply."""
    from e2e_check import first_divergences, summarise

    g = e2e_case(case)
    wt, d, u = _oracle_pipeline(case)
    divs, equal, total = [], 0, 0
    for ci, rows, params, consts in g["groups"]:
        nb, b = CANDIDATES[ci]
        e = oracle.encode_rows_gptq(wt[rows], d, u, nb, b, "normal")
        equal += int((e["codes"] == g["codes"][rows]).sum())
        total += e["codes"].size
        divs += first_divergences(wt[rows], e["codes"], g["codes"][rows], e["params"], params,
                                  e["consts"].view(np.uint16), consts, e["comp"],
                                  g["comp"][rows], d, g["d"], nb, b)
    print(f"{case}: codes equal {equal / total:.6f}; " + summarise(divs, len(wt)))
    assert equal / total >= 0.999
    for x in divs:
        assert x["tie"] < (1e-5 if x["kind"] == "ladder" else 0.02), x
