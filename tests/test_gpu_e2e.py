"""The whole encode path on the MI355X against the reference's own pipeline on BASELINE
configurations (tests/golden/e2e_*.npz from hi2's HessianStats, transform_sigma,
inverse_factor, fwht_groups, GPTQ and encode_many; inputs tests/e2e_recipes.py):

- cfg1 down-scaled to 512 x 512 with 512 tokens (rank-deficient) and 2048 tokens (full
  rank), a cfg2-style case (heavy-tailed rows, 30 % INT2/B32 + 70 % INT4/B64, 2048
  tokens), and cfg1 at its full 2048 x 2048 with 512 tokens (digests, every row's sse
  and a 64-row slice);
- (a) given the reference's Sigma and factor: Hs, codes, params, consts, sse, comp and
  the packed buffers bit for bit;
- (b) free running (the GPU's own bf16-MFMA Hessian, factor, rotation, GPTQ and
  packing): Sigma within 1e-5, U within 1e-3 of the reference's (LAPACK) factor, every
  row that departs from the reference doing so at a ladder tie (the two fits' weighted
  errors equal to 1e-5) or a rounding tie (the two runs' pre-rounding quotients within
  1e-3 steps), codes equal on >= 99.9 % of entries where the Hessian has full rank, and
  the total reconstruction error (sum of the rows' sse) within the stated bound of the
  reference's.

A row that departs at a tie follows another, equally good path for the rest of its
columns (error feedback), so where the Hessian is rank-deficient (512 tokens for 512 or
2048 channels: only the damping makes it definite, and the factor's rounding differences
are amplified) the share of equal codes is bounded below by the tie rate, not by this
build: there the classification of every departure is the bar, and the share of equal
codes is reported and held to the measured level.
"""

import numpy as np
import pytest
import torch

from e2e_check import classify_departures, first_divergences, summarise
from e2e_recipes import (CANDIDATES, CASES, FULL_CASES, WIDE_CASES, input_digests, inputs,
                         row_digests, segment_digests, sha)
from golden_data import e2e_case

pytestmark = pytest.mark.gpu

FULL = list(FULL_CASES)
WIDE = list(WIDE_CASES)
# every departure at a tie: a ladder tie's two weighted fit errors equal to this relative
# gap, a rounding tie's two pre-rounding quotients within this many ladder steps
# (measured on the MI355X: fit gaps <= 6.7e-6, quotient distances <= 3.3e-4 steps)
LADDER_TIE = 1e-5
ROUNDING_TIE = 1e-3
# a ladder departure where only the digests are at hand: the two runs' d (the fit's
# weights) within this relative difference in the blocks whose fits differ
D_TIE = 1e-5
# the wide cases, against the reference's own variation: the fixtures hold the reference
# against itself with its Hessian summed in 2048-token chunks instead of 4096 (rows
# departing 67 / 846, codes equal 99.956 % / 98.2 %, total sse 9.9e-5 / 1.2e-3 at K = 4096
# / 14336).  The GPU sums its Hessian in an entirely different order, so it may depart on
# a small multiple of that: rows departing <= 2.5 x the reference's own, 512-column
# segments unequal <= 3 x its own, total sse <= 1.5 x its own (at least 1e-4).  Measured
# on the MI355X: 126 and 1574 rows, segments 98.3 % and 77.5 %, total sse 6.7e-5 and
# 1.1e-3, U 1.5e-5 and 7.6e-4 of the largest entry (rank 4096 at K = 14336: only the
# damping makes it definite)
WIDE_ROWS, WIDE_SEGMENTS, WIDE_SSE = 2.5, 3.0, 1.5
WIDE_U = {"cfg3_q_proj": 3e-5, "cfg2_down_proj": 2e-3}
# share of equal codes: the north-star 99.9 % on full-rank Hessians; the measured level
# with margin on the rank-deficient ones (measured on the MI355X: 99.897 % at 512 x 512
# with 512 tokens, 98.71 % on cfg1's first 64 rows, 7 of them departing at ties; the
# full-rank cases 99.981 % and 99.996 %)
CODES_EQUAL = {"cfg1_k512_t512": 0.998, "cfg1_k512_t2048": 0.999, "cfg2_k512_t2048": 0.999,
               "cfg1_full": 0.98}
# total reconstruction error of the free-running pipeline against the reference's: the
# rows that follow another path at a tie change their own sse by a few per cent either
# way (measured on the MI355X: 4.6e-4, 7.1e-4, 1.8e-5 on the 512 x 512 cases, 2.1e-5 on
# cfg1's 2048 rows; the oracle pipeline 0.7e-4 .. 4.2e-4 on the 512 x 512 cases)
SSE_REL = {"cfg1_k512_t512": 2e-3, "cfg1_k512_t2048": 2e-3, "cfg2_k512_t2048": 2e-3,
           "cfg1_full": 5e-3}


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N(t):
    return t.detach().cpu().numpy()


def _encode_groups(wt, d, u, picks, dev):
    """GPTQ of every candidate group through the drop-in (encode_jobs_gptq), then packing
    (assemble).  Returns codes, comp, sse, per-group (params, consts) and the packed
    tensor."""
    from hi2_amd.format import assemble
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq

    n, k = wt.shape
    groups, jobs = [], []
    for ci, (nb, b) in enumerate(CANDIDATES):
        rows = np.nonzero(picks == ci)[0]
        if rows.size:
            groups.append((ci, rows))
            jobs.append(GptqJob(wt.index_select(0, T(rows, dev)), d, u, nb, b))
    encs = encode_jobs_gptq(jobs, "normal", comp=True)
    codes = np.zeros((n, k), np.uint8)
    comp = np.zeros((n, k), np.float32)
    sse = np.zeros(n, np.float32)
    per, pieces = {}, []
    for (ci, rows), e in zip(groups, encs):
        codes[rows] = N(e.codes)
        comp[rows] = N(e.comp)
        sse[rows] = N(e.sse)
        per[ci] = (N(e.params), N(e.consts.view(torch.int16)).view(np.uint16))
        pieces.append((torch.from_numpy(rows), e.codes, e.params, e.consts))
    nbits = torch.tensor([CANDIDATES[c][0] for c in picks])
    block = torch.tensor([CANDIDATES[c][1] for c in picks])
    had = torch.ones(k // 16, dtype=torch.uint8)
    packed = assemble(pieces, nbits, block, had, k)
    return dict(codes=codes, comp=comp, sse=sse, per=per, packed=packed)


def _pipeline(case, dev):
    """The free-running GPU pipeline on the case's inputs."""
    from hi2_amd.format import fwht_groups
    from hi2_amd.hessian import HessianStats, inverse_factor

    xb, w, picks, had = inputs(case)
    k = w.shape[1]
    st = HessianStats(k, dev)
    st.update(xb.to(dev))
    hs = st.transformed(None, T(had, dev))
    sigma = st.mean()
    u = inverse_factor(hs, 0.01)
    wt = fwht_groups(T(w, dev), T(had, dev))
    d = hs.diagonal().clone()
    out = _encode_groups(wt, d, u, picks, dev)
    out.update(sigma=sigma, hs=hs, u=u, d=N(d), wt=N(wt), picks=picks)
    return out


@pytest.mark.parametrize("case", FULL)
def test_given_the_reference_factor_the_encoding_is_bit_exact(case, dev):
    """(a): the GPU's transform of the reference's Sigma, then rotation, GPTQ and packing
    with the reference's factor: every output bit for bit."""
    from hi2_amd.format import fwht_groups
    from hi2_amd.hessian import transform_sigma

    print(f"e2e (a) {case}", flush=True)
    g = e2e_case(case)
    _, w, picks, had = inputs(case)
    assert input_digests(case)["w"] == g["digest_w"]
    hs = transform_sigma(T(g["sigma"], dev), None, T(had, dev))
    assert sha(N(hs)) == g["hs_sha"]
    d = hs.diagonal().clone()
    assert np.array_equal(N(d), g["d"])
    wt = fwht_groups(T(w, dev), T(had, dev))
    o = _encode_groups(wt, d, T(g["u"], dev), picks, dev)
    assert np.array_equal(o["codes"], g["codes"])
    assert np.array_equal(o["sse"], g["sse"])
    assert np.array_equal(o["comp"], g["comp"])
    for ci, rows, params, consts in g["groups"]:
        assert np.array_equal(o["per"][ci][0], params), ci
        assert np.array_equal(o["per"][ci][1], consts), ci
    p = o["packed"]
    for f in ("codes", "code_off", "blk_params", "param_off", "row_nbits", "row_block"):
        assert np.array_equal(getattr(p, f).numpy().reshape(-1),
                              g[f"packed_{f}"].reshape(-1)), f
    assert np.array_equal(p.row_consts.view(torch.int16).numpy().view(np.uint16).reshape(-1),
                          g["packed_row_consts"].reshape(-1))


def _agreement(case, o, g, rows_of_slice=None):
    """Codes agreement, tie classification and the reconstruction error of a free run:
    the share of equal codes, the departures, the total sse's relative difference and the
    largest relative sse difference over the rows that do not depart (all rows of a full
    case, the slice of a sliced one)."""
    codes_r, comp_r = (g["codes"], g["comp"]) if rows_of_slice is None else \
        (g["codes_slice"], g["comp_slice"])
    keep = np.arange(len(codes_r))
    divs, equal, total, departed = [], 0, 0, []
    for ci, rows, params, consts in g["groups"]:
        nb, b = CANDIDATES[ci]
        sel = np.isin(np.nonzero(o["picks"] == ci)[0], rows)
        po, co = o["per"][ci][0][sel], o["per"][ci][1][sel]
        rr = rows[np.isin(rows, keep)]
        equal += int((o["codes"][rr] == codes_r[rr]).sum())
        total += o["codes"][rr].size
        dv = first_divergences(o["wt"][rr], o["codes"][rr], codes_r[rr], po, params, co,
                               consts, o["comp"][rr], comp_r[rr], o["d"], g["d"], nb, b)
        departed += [int(rr[x["row"]]) for x in dv]
        divs += dv
    so, sr = o["sse"].astype(np.float64), g["sse"].astype(np.float64)
    sse_rel = abs(so.sum() / sr.sum() - 1)
    stay = np.setdiff1d(keep, departed)
    sse_keep = float(np.max(np.abs(so[stay] - sr[stay]) / np.maximum(sr[stay], 1e-30)))
    msg = (f"{case}: codes equal {equal / total:.6f} of {total}; " + summarise(divs, len(keep))
           + f"; total sse rel {sse_rel:.3g}; sse of the rows that stay {sse_keep:.3g}")
    return equal / total, divs, sse_rel, sse_keep, msg, sorted(departed)


@pytest.mark.parametrize("case", FULL)
def test_free_running_pipeline_departs_from_the_reference_only_at_ties(case, dev):
    """(b) at 512 x 512: the whole GPU pipeline against the reference's pipeline."""
    print(f"e2e (b) {case}", flush=True)
    g = e2e_case(case)
    o = _pipeline(case, dev)
    sig = N(o["sigma"])
    srel = np.abs(sig - g["sigma"]).max() / np.abs(g["sigma"]).max()
    urel = np.abs(N(o["u"]) - g["u"]).max() / np.abs(g["u"]).max()
    frac, divs, sse_rel, sse_keep, msg, _ = _agreement(case, o, g)
    print(f"sigma rel {srel:.3g}  factor rel {urel:.3g}  " + msg, flush=True)
    assert srel < 1e-5 and urel < 1e-3
    assert frac >= CODES_EQUAL[case], msg
    for x in divs:
        assert x["tie"] < (LADDER_TIE if x["kind"] == "ladder" else ROUNDING_TIE), (x, msg)
    assert sse_keep < 1e-4, msg
    assert sse_rel < SSE_REL[case], msg


def test_free_running_pipeline_at_cfg1_full_size(dev):
    """(b) at cfg1's own size, 2048 x 2048 with 512 tokens (rank 512: the damping alone
    makes the Hessian definite, and error feedback amplifies the factor's rounding
    differences): Sigma and U on the stored rows, the first 64 rows' codes and ties,
    and every row's sse."""
    case = "cfg1_full"
    print(f"e2e (b) {case}", flush=True)
    g = e2e_case(case)
    o = _pipeline(case, dev)
    sig = N(o["sigma"])
    srel = max(np.abs(sig[:16] - g["sigma_rows"]).max() / np.abs(g["sigma_rows"]).max(),
               np.abs(np.diag(sig) - g["sigma_diag"]).max() / np.abs(g["sigma_diag"]).max())
    u = N(o["u"])
    urel = np.abs(u[:16] - g["u_rows"]).max() / np.abs(g["u_rows"]).max()
    frac, divs, sse_rel, sse_keep, msg, _ = _agreement(case, o, g, rows_of_slice=True)
    print(f"sigma rel {srel:.3g}  factor rel {urel:.3g}  " + msg, flush=True)
    assert srel < 1e-5 and urel < 3e-3
    assert frac >= CODES_EQUAL[case], msg
    for x in divs:
        assert x["tie"] < (LADDER_TIE if x["kind"] == "ladder" else ROUNDING_TIE), (x, msg)
    assert sse_keep < 1e-4, msg
    assert sse_rel < SSE_REL[case], msg


def _params_digests(o, n):
    """8-byte digests of every row's ladder bytes (rows of each candidate group)."""
    out = np.zeros(n, np.uint64)
    for ci in o["per"]:
        rows = np.nonzero(o["picks"] == ci)[0]
        out[rows] = row_digests(o["per"][ci][0])
    return out


@pytest.mark.parametrize("case", WIDE)
def test_free_running_pipeline_at_the_benchmark_widths(case, dev):
    """(b) at the bench's own widths, where the factor's large products run on the fp16
    split planes: cfg3's q_proj input (K = 4096, 8192 tokens, full rank) and cfg2's
    down_proj (K = 14336, 4096 tokens, rank 4096).  Against the reference's pipeline:
    Sigma and U on the stored rows and diagonals; over every row, which rows depart (their
    codes, ladder bytes or consts differ from the reference's: per-row digests) and the
    share of equal codes (bounded below by the 512-column segments whose digests agree);
    on the slice rows the tie of every departure; the sse of every row that stays within
    1e-4 of the reference's, and the total sse."""
    print(f"e2e (b) {case}", flush=True)
    g = e2e_case(case)
    assert input_digests(case)["w"] == g["digest_w"]
    o = _pipeline(case, dev)
    n, k = o["codes"].shape
    rs = g["factor_rows"]
    sig, u = N(o["sigma"]), N(o["u"])
    srel = max(np.abs(sig[rs] - g["sigma_rows"]).max() / np.abs(g["sigma_rows"]).max(),
               np.abs(np.diag(sig) - g["sigma_diag"]).max() / np.abs(g["sigma_diag"]).max())
    urel = max(np.abs(u[rs] - g["u_rows"]).max() / np.abs(g["u_rows"]).max(),
               np.abs(np.diag(u) - g["u_diag"]).max() / np.abs(g["u_diag"]).max())
    consts = np.zeros((n, 3), np.uint16)
    for ci in o["per"]:
        consts[np.nonzero(o["picks"] == ci)[0]] = o["per"][ci][1]
    depart = ((row_digests(o["codes"]) != g["codes_digest"])
              | (_params_digests(o, n) != g["params_digest"])
              | (consts != g["consts_all"]).any(axis=1))
    seg_equal = float((segment_digests(o["codes"]) == g["codes_segments"]).mean())
    # every departing row: a ladder departure (the oracle's fit from the reference's d
    # reproduces the reference's ladder bytes and differs from this build's at a tie) or
    # a departure in the codes alone
    cls = []
    for ci, (nb, b) in enumerate(CANDIDATES):
        rows = np.nonzero(o["picks"] == ci)[0]
        if rows.size == 0:
            continue
        dep = np.nonzero(depart[rows])[0]
        cls += classify_departures(o["wt"][rows], dep, o["d"], g["d"], nb, b,
                                   g["params_digest"][rows], g["consts_all"][rows],
                                   o["per"][ci][0], o["per"][ci][1])
    lad = [x["tie"] for x in cls if x["kind"] == "ladder"]
    n_rnd = sum(x["kind"] == "rounding" for x in cls)
    g["codes"], g["comp"] = g["codes_slice"], g["comp_slice"]
    r = len(g["codes_slice"])
    frac_s, divs, _, _, msg, departed = _agreement(case, o, g, rows_of_slice=True)
    so, sr = o["sse"].astype(np.float64), g["sse"].astype(np.float64)
    sse_rel = abs(so.sum() / sr.sum() - 1)
    stay = ~depart
    sse_keep = float(np.max(np.abs(so[stay] - sr[stay]) / np.maximum(sr[stay], 1e-30)))
    self_dep = ((g["self_codes_digest"] != g["codes_digest"])
                | (g["self_params_digest"] != g["params_digest"]))
    self_seg = float((g["self_codes_segments"] == g["codes_segments"]).mean())
    print(f"{case}: the reference against itself (2048-token chunks): rows departing "
          f"{int(self_dep.sum())}/{n}, codes equal {float(g['self_codes_equal']):.6f} "
          f"(>= {self_seg:.6f} by segments), total sse rel "
          f"{abs(g['self_sse'].astype(np.float64).sum() / g['sse'].astype(np.float64).sum() - 1):.3g}",
          flush=True)
    print(f"{case}: sigma rel {srel:.3g}  factor rel {urel:.3g}  rows departing "
          f"{int(depart.sum())}/{n}  codes equal >= {seg_equal:.6f} (512-column segments)  "
          f"(ladder {len(lad)}, their d within {max(lad, default=0):.2g} rel., fit gaps "
          f"<= {max((x['fit_gap'] for x in cls if x['kind'] == 'ladder'), default=0):.2g}; "
          f"codes alone {n_rnd}; "
          f"unexplained {sum(not x['explained'] for x in cls)})  "
          f"total sse rel {sse_rel:.3g}  sse of the rows that stay {sse_keep:.3g}; "
          f"slice of {r} rows: {msg}", flush=True)
    assert srel < 1e-5 and urel < WIDE_U[case]
    assert list(np.nonzero(depart[:r])[0]) == departed  # the digests see what the slice shows
    for x in divs:
        assert x["tie"] < (LADDER_TIE if x["kind"] == "ladder" else ROUNDING_TIE), (x, msg)
    assert all(x["explained"] for x in cls)
    assert max(lad, default=0) < D_TIE
    self_sse = abs(g["self_sse"].astype(np.float64).sum() / sr.sum() - 1)
    assert 1 - seg_equal <= WIDE_SEGMENTS * (1 - self_seg)
    assert depart.sum() <= WIDE_ROWS * self_dep.sum()
    assert sse_keep < 1e-4
    assert sse_rel < max(1e-4, WIDE_SSE * self_sse)


def test_encode_many_from_the_device_hessian_equals_the_direct_path(dev):
    """The drop-in orchestration (hi2_amd.calibrate.encode_many) fed the device's own
    Sigma gives the same packed buffers and comp as the direct path of the free run
    (same kernels, same factor)."""
    from hi2_amd.calibrate import Config, EncodeRequest, Executor, TensorTable, encode_many

    case = "cfg2_k512_t2048"
    o = _pipeline(case, dev)
    _, w, picks, had = inputs(case)
    n, k = w.shape
    table = TensorTable(case, (n, k), torch.from_numpy(had), torch.zeros(1), list(CANDIDATES),
                        0.0, CASES[case][3], None)
    req = EncodeRequest(torch.from_numpy(w), None, table, torch.from_numpy(picks), o["sigma"],
                        "x", {})
    got = encode_many([req], Config(candidates=list(CANDIDATES)), Executor([str(dev)]))[0]
    for f in ("codes", "code_off", "blk_params", "param_off", "row_consts", "row_nbits",
              "row_block"):
        assert torch.equal(getattr(got, f), getattr(o["packed"], f)), f
    assert np.array_equal(req.comp_out["comp"].numpy(), o["comp"])
