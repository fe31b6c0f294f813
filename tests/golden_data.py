"""Loaders for the reference's golden vectors in tests/golden (written by
tests/golden/make_golden.py from the reference's own functions)."""

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = [(2, 16), (2, 32), (2, 64), (4, 16), (4, 32), (4, 64), (8, 32), (8, 64)]


def gptq_cases():
    """Yields (nbits, block, effort, act_order, dict of arrays)."""
    for nbits in (2, 4, 8):
        g = np.load(os.path.join(GOLDEN, f"gptq_int{nbits}.npz"))
        tags = sorted({k.rsplit("_", 1)[0] for k in g.files})
        for tag in tags:
            b, ao, effort = tag.split("_")
            arr = {f: g[f"{tag}_{f}"] for f in ("w", "d", "u", "perm", "codes", "params",
                                                "consts", "sse", "comp")}
            if arr["perm"].size == 0:
                arr["perm"] = None
            yield nbits, int(b[1:]), effort, ao == "ao1", arr


def fit_cases():
    g = np.load(os.path.join(GOLDEN, "fit_ladder.npz"))
    tags = sorted({k.rsplit("_", 1)[0] for k in g.files if not k.startswith("effort")})
    for tag in tags:
        n, b, effort = tag.split("_")
        yield int(n[1:]), int(b[1:]), effort, {f: g[f"{tag}_{f}"] for f in ("wb", "db", "lo", "step")}


def inverse_cases():
    g = np.load(os.path.join(GOLDEN, "inverse_factor.npz"))
    tags = sorted({k.rsplit("_", 1)[0] for k in g.files})
    for tag in tags:
        yield tag, g[f"{tag}_hs"], g[f"{tag}_u"]


def refine_cases():
    """Yields (tag, hs, passes, groups) for the reference's refine_groups fixtures
    (tests/golden/refine_*.npz); each group is a dict with nbits, block, w, codes_in,
    params, consts, lo, step (decoded) and codes (the reference's refined codes)."""
    for fname in ("refine_1.npz", "refine_2.npz"):
        g = np.load(os.path.join(GOLDEN, fname))
        tags = sorted({k.split("_", 1)[0] for k in g.files})
        for tag in tags:
            groups = []
            gi = 0
            while f"{tag}_g{gi}_spec" in g.files:
                p = f"{tag}_g{gi}"
                nbits, block = (int(v) for v in g[f"{p}_spec"])
                grp = {f: g[f"{p}_{f}"] for f in ("w", "codes_in", "params", "consts", "lo",
                                                   "step", "codes")}
                grp.update(nbits=nbits, block=block)
                groups.append(grp)
                gi += 1
            yield tag, g[f"{tag}_hs"], int(g[f"{tag}_passes"]), groups


def colstats_case():
    """The reference ColumnStats fixture (tests/golden/colstats.npz): input as bf16 bits
    [t, 64], the split of the two update calls, flags, inv_scale, and per input dtype
    ("bf16", "f32": the same values as float32) the reference's S, n and diag variants."""
    g = np.load(os.path.join(GOLDEN, "colstats.npz"))
    return {f: g[f] for f in g.files}


def encode_many_case():
    """The reference encode_many fixture (tests/golden/encode_many.npz).  Returns
    (candidates, tensors, configs): tensors is a list of dicts (name, w float32 [R, K],
    w_bf16 (bf16 bits) or None, had, picks, col_scale (fp16 bits) or None, sigma or None,
    sigma_id or None, stats (S, n) or None, comp); configs maps a tag to a dict
    (rounding, act_order, refine_passes, effort, factors: the reference's factors in
    call order, out: per tensor name the packed fields and comp)."""
    g = np.load(os.path.join(GOLDEN, "encode_many.npz"))
    cands = [tuple(int(v) for v in c) for c in g["candidates"]]
    cs = g["in0_col_scale"].view(np.uint16)
    tensors = []
    for name in g["names"]:
        name = str(name)
        inp, sid, smooth, comp, has_sigma, has_stats = (str(v) for v in g[f"meta_{name}"])
        w = g[f"w_{name}"]
        wb = None
        if w.dtype == np.int16:
            wb = w.view(np.uint16)
            w = (wb.astype(np.uint32) << 16).view(np.float32)
        tensors.append(dict(
            name=name, w=w, w_bf16=wb, had=g[f"had_{name}"], picks=g[f"picks_{name}"],
            col_scale=cs if smooth == "1" else None,
            sigma=g[f"{inp}_sigma"] if has_sigma == "1" else None, sigma_id=sid or None,
            stats=(g[f"{inp}_S"], int(g[f"{inp}_n"])) if has_stats == "1" else None,
            comp=comp == "1"))
    configs = {}
    for tag in g["configs"]:
        tag = str(tag)
        rounding, ao, passes, effort = (str(v) for v in g[f"{tag}_cfg"])
        out = {}
        for t in tensors:
            p = f"{tag}_{t['name']}_"
            o = {f: g[p + f] for f in ("codes", "code_off", "blk_params", "param_off",
                                       "row_nbits", "row_block", "had")}
            o["row_consts"] = g[p + "row_consts"].view(np.uint16)
            o["comp"] = g[p + "comp"] if p + "comp" in g.files else None
            out[t["name"]] = o
        configs[tag] = dict(rounding=rounding, act_order=ao == "1", refine_passes=int(passes),
                            effort=effort, out=out,
                            factors=[g[f"{tag}_u{j}"] for j in range(int(g[f"{tag}_nfactors"]))])
    return cands, tensors, configs


def qad_cases():
    """The reference QAD fixture (tests/golden/qad.npz, hi2.qad.FakeQuantLinear's torch
    graph).  Yields (tag, case): latent [R, K], unit [R, K] or None, had, col_scale (fp16
    bits), groups (rows, consts (fp16 bits), nbits, block, lo_u, st_u and the reference's
    gradients g_lo/g_st of the stored values and og_lo/og_st of the original-basis
    weights), grad / grad2 (the output gradients), stored, g_latent, original, og_latent."""
    g = np.load(os.path.join(GOLDEN, "qad.npz"))
    for tag in ("abs", "step", "clamp"):
        p = f"{tag}_"
        unit = g[p + "unit"]
        case = dict(latent=g[p + "latent"], unit=unit if unit.size else None, had=g["had"],
                    col_scale=g["col_scale"].view(np.uint16), w=g["w"], groups=[])
        for gi in range(int(g[p + "ngroups"])):
            q = f"{p}g{gi}_"
            nbits, block = (int(v) for v in g[q + "spec"])
            grp = {f: g[q + f] for f in ("rows", "lo_u", "st_u", "g_lo", "g_st", "og_lo",
                                          "og_st")}
            grp.update(consts=g[q + "consts"].view(np.uint16), nbits=nbits, block=block)
            case["groups"].append(grp)
        for f in ("grad", "grad2", "stored", "g_latent", "original", "og_latent"):
            case[f] = g[p + f]
        yield tag, case


def unpack_rows(words, code_off, row_nbits, k):
    """Codes [R, K] uint8 of rdna_hint_flex packed words (LSB first, 32 / nbits codes per
    int32 word, row r's words at code_off[r]:code_off[r + 1])."""
    words = np.asarray(words).view(np.uint32)
    out = np.zeros((len(row_nbits), k), np.uint8)
    for r, nb in enumerate(np.asarray(row_nbits, np.int64)):
        wr = words[int(code_off[r]):int(code_off[r + 1])]
        per = 32 // int(nb)
        sh = (np.arange(per, dtype=np.uint32) * np.uint32(nb))
        out[r] = ((wr[:, None] >> sh[None, :]) & np.uint32((1 << int(nb)) - 1)).reshape(-1)
    return out


def e2e_case(case):
    """The reference pipeline's fixture of an end-to-end case (tests/e2e_recipes.py, written
    by make_golden.py e2e).  Full cases: sigma [K, K], u [K, K] (upper), d, hs_sha, codes
    [N, K] (unpacked from the reference's packed words), comp, sse, packed fields, per
    candidate group (rows, params, consts).  cfg1_full: digests, sse, sigma_diag, u_diag,
    16 rows of sigma and u, and the first 64 rows' codes, comp, params and consts.  Wide
    cases: see below."""
    from e2e_recipes import CASES, FULL_CASES, WIDE_CASES, from_upper

    _, k, n, _, _ = CASES[case]
    if case in WIDE_CASES:
        # wide cases (K = 4096, 14336): digests, every row's sse, consts and digests of its
        # codes and ladder bytes, d, Sigma/U diagonals and factor_rows of each, and the
        # first rows' codes, comp, params and consts
        out = {}
        for part in ("factor", "out", "comp"):
            with np.load(os.path.join(GOLDEN, f"e2e_{case}_{part}.npz")) as f:
                out.update({name: f[name] for name in f.files})
        out["consts_all"] = out["consts_all"].view(np.uint16)
    elif case not in FULL_CASES:
        g = np.load(os.path.join(GOLDEN, f"e2e_{case}.npz"))
        out = {f: g[f] for f in g.files}
    else:
        f1 = np.load(os.path.join(GOLDEN, f"e2e_{case}_factor.npz"))
        f2 = np.load(os.path.join(GOLDEN, f"e2e_{case}_out.npz"))
        f3 = np.load(os.path.join(GOLDEN, f"e2e_{case}_comp.npz"))
        out = {f: f1[f] for f in f1.files}
        out.update({f: f2[f] for f in f2.files})
        out["comp"] = f3["comp"]
        out["sigma"] = from_upper(out.pop("sigma_tri"), k, True)
        out["u"] = from_upper(out.pop("u_tri"), k, False)
        out["packed_row_consts"] = out["packed_row_consts"].view(np.uint16)
        out["codes"] = unpack_rows(out["packed_codes"], out["packed_code_off"],
                                   out["packed_row_nbits"], k)
    groups = []
    gi = 0
    for gi in range(4):
        if f"g{gi}_rows" in out:
            groups.append((gi, out.pop(f"g{gi}_rows"), out.pop(f"g{gi}_params"),
                           out.pop(f"g{gi}_consts").view(np.uint16)))
    out["groups"] = groups
    for f in [f for f in out if isinstance(out[f], np.ndarray) and out[f].dtype.kind == "U"]:
        out[f] = str(out[f])
    return out
