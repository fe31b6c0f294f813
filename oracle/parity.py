"""Agreement of a free-running encode pipeline with the reference's, and the
classification of every row where the two differ (test infrastructure: the checker of
``tests/`` and of ``bench.py``'s parity object; the product path never imports it).

Two fp32 pipelines that sum the Hessian GEMM in different orders and factor it with
different blockings produce Sigma, Hs and U that differ in the last bits.  From there a
row of the encoding can only come apart at a discrete decision:

* a **ladder tie**: the ladder fit of some block (argmin over the grid and the LSQ
  refits on the row's uncompensated weights, weighted by diag(Hs),
  ``hi2/encode.py:53-92``) picks another (lo, step) because two candidates' weighted
  errors are equal to fp32 precision, or the 8-bit quantisation of the row's ladders
  (``hi2/encode.py:95-119``) lands on other bytes; from that block on the row follows
  another, equally good, path;
* a **rounding tie**: with the same ladder, the compensated value of a column lies so
  close to a rounding boundary (``hi2/hessian.py:248-261``) that the two runs'
  accumulated fp32 differences put it on different sides.

``first_divergences`` finds, per row, the first column where the runs differ (a code,
or the first column of a block whose decoded ladder differs) and measures the tie: for
a ladder tie the relative gap between the two fits' weighted errors (float64, the
reference's weights), for a rounding tie the distance, in ladder steps, between the two
runs' pre-rounding quotients at that column.  ``classify_departures`` does the same for
rows of which only the reference's digests are known.
"""

import hashlib

import numpy as np

from . import fit_ladder, params


def row_digests(a: np.ndarray) -> np.ndarray:
    """An 8-byte BLAKE2b digest of every row of a 2-D (or [rows, ...]) array, as uint64:
    rows whose digests are equal hold the same bytes."""
    a = np.ascontiguousarray(a).reshape(a.shape[0], -1).view(np.uint8)
    return np.array([int.from_bytes(hashlib.blake2b(r.tobytes(), digest_size=8).digest(),
                                    "little") for r in a], np.uint64)


def f16_bits_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def decode(params, consts_bits):
    """decode_params (hi2/format.py:45-60): lo = fp16(f32(f64(u) f64(lo_scale) +
    f64(lo_min))), step = fp16(f32(u) f32(step_scale)); returns f32 [rows, nb] each."""
    c = f16_bits_to_f32(consts_bits).astype(np.float64)
    lo_u = params[..., 0].astype(np.float64)
    st_u = params[..., 1].astype(np.float32)
    lo = (lo_u * c[:, 1:2] + c[:, 0:1]).astype(np.float32).astype(np.float16)
    st = (st_u * c[:, 2:3].astype(np.float32)).astype(np.float16)
    return lo.astype(np.float32), st.astype(np.float32)


def _fit_err(wb, db, lo, st, nlev):
    safe = st if st != 0 else 1.0
    q = np.clip(np.rint((wb - lo) / safe), 0, nlev - 1)
    rec = lo + q * st
    return float((db * (rec - wb) ** 2).sum())


def first_divergences(wt, codes_o, codes_r, params_o, params_r, consts_o, consts_r, comp_o,
                      comp_r, d_o, d_r, nbits, block):
    """Per diverging row of one candidate group (rows ``wt`` [n, K] in the stored basis,
    ``*_o`` this build's, ``*_r`` the reference's): dicts with ``row``, ``col``, ``kind``
    ("ladder" or "rounding") and ``tie`` (the relative fit-error gap of the blocks whose
    fits differ, or the quotient distance in steps); a ladder tie also carries ``d_rel``,
    the largest relative difference of the two runs' d over those blocks."""
    n, k = codes_o.shape
    nb = k // block
    lo_o, st_o = decode(params_o, consts_o)
    lo_r, st_r = decode(params_r, consts_r)
    lad_diff = (lo_o != lo_r) | (st_o != st_r)
    out = []
    for i in range(n):
        cd = np.nonzero(codes_o[i] != codes_r[i])[0]
        ld = np.nonzero(lad_diff[i])[0]
        if cd.size == 0 and ld.size == 0:
            continue
        first_code = int(cd[0]) if cd.size else k
        first_lad = int(ld[0]) * block if ld.size else k
        if first_lad <= first_code:
            # the raw fits of both runs: every block whose fit differs must be a tie
            wb = wt[i].reshape(1, nb, block)
            fo = fit_ladder(wb, d_o.reshape(1, nb, block), 2 ** nbits, "normal")
            fr = fit_ladder(wb, d_r.reshape(1, nb, block), 2 ** nbits, "normal")
            gap = d_rel = 0.0
            w64 = wt[i].reshape(nb, block).astype(np.float64)
            d64 = d_r.reshape(nb, block).astype(np.float64)
            for b in range(nb):
                if fo[0][0, b] == fr[0][0, b] and fo[1][0, b] == fr[1][0, b]:
                    continue
                eo = _fit_err(w64[b], d64[b], float(fo[0][0, b]), float(fo[1][0, b]), 2 ** nbits)
                er = _fit_err(w64[b], d64[b], float(fr[0][0, b]), float(fr[1][0, b]), 2 ** nbits)
                gap = max(gap, abs(eo - er) / max(eo, er, 1e-300))
                do = d_o[b * block:(b + 1) * block].astype(np.float64)
                d_rel = max(d_rel, float(np.max(np.abs(do - d64[b])
                                                / np.maximum(np.abs(d64[b]), 1e-300))))
            out.append(dict(row=i, col=first_lad, kind="ladder", tie=gap, d_rel=d_rel))
        else:
            j = first_code
            b = j // block
            qo = (float(comp_o[i, j]) - float(lo_o[i, b])) / float(st_o[i, b])
            qr = (float(comp_r[i, j]) - float(lo_r[i, b])) / float(st_r[i, b])
            out.append(dict(row=i, col=j, kind="rounding", tie=abs(qo - qr),
                            boundary=min(int(codes_o[i, j]), int(codes_r[i, j])) + 0.5,
                            q=(qo, qr)))
    return out


def summarise(divs, n_rows):
    lad = [x["tie"] for x in divs if x["kind"] == "ladder"]
    rnd = [x["tie"] for x in divs if x["kind"] == "rounding"]
    return (f"rows diverging {len(divs)}/{n_rows} (ladder ties {len(lad)}, max fit gap "
            f"{max(lad, default=0):.2g}; rounding ties {len(rnd)}, max quotient distance "
            f"{max(rnd, default=0):.3g} steps)")


def classify_departures(wt, rows, d_o, d_r, nbits, block, params_digest_r, consts_r,
                        params_o, consts_o):
    """Every departing row of one candidate group when only the reference's per-row
    digests are at hand (the wide fixtures): ``rows`` (indices into the group's rows
    ``wt`` [n, K], ``params_o`` [n, nb, 2] and ``consts_o`` [n, 3], this build's ladder)
    depart.  The
    reference's ladder of such a row is recomputed by the oracle's fit (bit-exact with the
    reference given the same inputs) from the reference's own weights d_r; a row is a
    **ladder** departure when that ladder differs from this build's (which is the oracle's
    fit from d_o), **explained** when the recomputed ladder bytes and consts have the
    reference's digests.  The two fits then differ only because d does: the rotated rows
    are bit-identical, so the fit's decision lies within that difference of its boundary,
    and the tie is the largest relative difference |d_o - d_r| / d_r over the blocks whose
    raw fits differ (``fit_gap``: the largest relative gap between the two fits' weighted
    errors there, which the fit's discrete least-squares refits can make large).  A row
    whose ladders agree departs in its codes alone: a **rounding** departure.  Returns
    dicts with ``row``, ``kind``, ``tie`` and ``fit_gap`` (ladder only), ``explained``."""
    k = wt.shape[1]
    nb = k // block
    out = []
    for i in rows:
        wb = wt[i].reshape(1, nb, block)
        fr = fit_ladder(wb, d_r.reshape(1, nb, block), 2 ** nbits, "normal")
        lo_u, st_u, cr, _, _ = params(*fr)
        pr = np.stack([lo_u[0], st_u[0]], -1)[None]
        explained = bool(row_digests(pr)[0] == params_digest_r[i]
                         and np.array_equal(cr[0], consts_r[i]))
        if np.array_equal(pr[0], params_o[i]) and np.array_equal(cr[0], consts_o[i]):
            out.append(dict(row=int(i), kind="rounding", tie=None, explained=explained))
            continue
        fo = fit_ladder(wb, d_o.reshape(1, nb, block), 2 ** nbits, "normal")
        w64 = wt[i].reshape(nb, block).astype(np.float64)
        d64 = d_r.reshape(nb, block).astype(np.float64)
        gap = tie = 0.0
        for b in range(nb):
            if fo[0][0, b] == fr[0][0, b] and fo[1][0, b] == fr[1][0, b]:
                continue
            eo = _fit_err(w64[b], d64[b], float(fo[0][0, b]), float(fo[1][0, b]), 2 ** nbits)
            er = _fit_err(w64[b], d64[b], float(fr[0][0, b]), float(fr[1][0, b]), 2 ** nbits)
            gap = max(gap, abs(eo - er) / max(eo, er, 1e-300))
            do = d_o[b * block:(b + 1) * block].astype(np.float64)
            tie = max(tie, float(np.max(np.abs(do - d64[b]) / np.maximum(np.abs(d64[b]),
                                                                          1e-300))))
        out.append(dict(row=int(i), kind="ladder", tie=tie, fit_gap=gap, explained=explained))
    return out


def compare_groups(groups):
    """Agreement of two encodings of one tensor, group by group.  ``groups`` holds, per
    candidate group, dicts ``wt`` (the rotated rows [n, K], identical for both runs),
    ``o`` and ``r`` (this build's and the reference's: ``codes`` u8 [n, K], ``params``
    u8 [n, nb, 2], ``consts`` u16 [n, 3], ``sse`` f32 [n], ``comp`` f32 [n, K]), ``d_o``,
    ``d_r`` (each run's ladder weights diag(Hs)), ``nbits`` and ``block``.  Returns the
    share of equal codes, the departing rows by kind with their largest tie (ladder: the
    fit-error gap and the d difference; rounding: the quotient distance in steps), the
    total sse's relative difference and the largest relative sse difference over the rows
    that do not depart."""
    equal = total = rows = 0
    lad, rnd = [], []
    sse_o, sse_r, stay_rel = [], [], 0.0
    for g in groups:
        o, r = g["o"], g["r"]
        n = o["codes"].shape[0]
        dep = ((o["codes"] != r["codes"]).any(1)
               | (o["params"].reshape(n, -1) != r["params"].reshape(n, -1)).any(1)
               | (o["consts"] != r["consts"]).any(1))
        idx = np.nonzero(dep)[0]
        equal += int((o["codes"] == r["codes"]).sum())
        total += o["codes"].size
        rows += n
        if idx.size:
            divs = first_divergences(g["wt"][idx], o["codes"][idx], r["codes"][idx],
                                     o["params"][idx], r["params"][idx], o["consts"][idx],
                                     r["consts"][idx], o["comp"][idx], r["comp"][idx],
                                     g["d_o"], g["d_r"], g["nbits"], g["block"])
            lad += [x for x in divs if x["kind"] == "ladder"]
            rnd += [x for x in divs if x["kind"] == "rounding"]
        so, sr = o["sse"].astype(np.float64), r["sse"].astype(np.float64)
        sse_o.append(so.sum())
        sse_r.append(sr.sum())
        keep = ~dep
        if keep.any():
            stay_rel = max(stay_rel, float(np.max(np.abs(so[keep] - sr[keep])
                                                  / np.maximum(sr[keep], 1e-30))))
    return {"codes_equal": equal / max(total, 1), "codes": total, "rows": rows,
            "rows_departing": len(lad) + len(rnd),
            "ladder": {"rows": len(lad),
                       "max_fit_gap": max((x["tie"] for x in lad), default=0.0),
                       "max_d_rel": max((x["d_rel"] for x in lad), default=0.0)},
            "rounding": {"rows": len(rnd),
                         "max_quotient_distance_steps": max((x["tie"] for x in rnd),
                                                            default=0.0)},
            "sse_rel_total": abs(sum(sse_o) / max(sum(sse_r), 1e-300) - 1),
            "sse_rel_max_rows_that_stay": stay_rel}
