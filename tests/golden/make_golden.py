"""Write the golden vectors that pin the oracle where closed forms cannot.

This script imports the reference package from ``/root/reference`` (read-only) in the
build container and records inputs and outputs of the three functions whose exact bits
depend on the reference's own torch-CPU arithmetic:

* ``hi2.hessian.inverse_factor`` (LAPACK ``cholesky`` -> ``cholesky_inverse`` ->
  ``cholesky(upper)`` with the damping retry, ``hi2/hessian.py:71-86``);
* ``hi2.encode.fit_ladder`` (grid search + weighted LSQ refits on torch reductions,
  ``hi2/encode.py:53-92``);
* ``hi2.hessian.encode_rows_gptq_reference`` (the verbatim column loop with the BLAS
  trailing update, ``hi2/hessian.py:89-175``), on the inputs of the reference's own
  ``tests/test_gptq_fast.py:19-36`` ``_layer`` recipe;
* ``hi2.refine.refine_groups`` (the local code refinement torch loop with its two BLAS
  products, ``hi2/refine.py:43-144``), on the inputs of the reference's own
  ``tests/test_refine_kernel.py:25-32`` ``_rows`` recipe;
* ``hi2.stats.ColumnStats`` (``update`` per 4096-token chunk through torch's fp32
  einsum, ``diag`` with and without rotation flags and smoothing, ``hi2/stats.py:26-55``);
* ``hi2.qad.FakeQuantLinear`` (the torch graph of the fused QAD decode,
  ``hi2/qad.py:366-422``: stored values, the original-basis weights, and the autograd
  gradients of both for the latent weights and both ladder bytes of every block);
* ``hi2.calibrate.encode_many`` (factor sharing, candidate grouping, refinement,
  ``comp`` and packing of several tensors, ``hi2/calibrate.py:297-424``), with every
  factor it computed recorded beside the packed output;
* the reference's whole encode pipeline on BASELINE configurations (``e2e_*.npz``):
  ``HessianStats`` over bf16 calibration tokens, ``mean``, ``transform_sigma``,
  ``inverse_factor``, ``fwht_groups`` and GPTQ with packing through ``encode_many``, on
  the seeded inputs of ``tests/e2e_recipes.py`` (cfg1 down-scaled to 512 x 512 with 512
  and 2048 tokens, a cfg2-style mixed INT2/INT4 case, and cfg1 at its full 2048 x 2048
  as digests and a 64-row slice), and at the benchmark's widths (cfg3's q_proj at
  K = 4096 with 8192 tokens, cfg2's down_proj at K = 14336) as digests, every row's sse
  and per-row digests, and a slice of rows;
* the MoE token floor (``hi2/layerwise.py:241-257`` with ``hi2.moe.blend``) on seven
  experts' sums (``moe_blend.npz``);
* ``hi2.encode.encode_rows`` (nearest rounding, ``hi2/encode.py:133-173``) at INT2/B32,
  INT4/B64 and INT8/B64 (``nearest.npz``).

The fixtures are plain ``.npz`` data (inputs and expected outputs); nothing of the
reference is stored.  Run from the repository root:

    python tests/golden/make_golden.py            # every fixture
    python tests/golden/make_golden.py refine     # refine_*.npz only
    python tests/golden/make_golden.py colstats   # colstats.npz only
    python tests/golden/make_golden.py encode_many  # encode_many.npz only
    python tests/golden/make_golden.py qad          # qad.npz only
    python tests/golden/make_golden.py e2e          # e2e_*.npz only (small cases)
    python tests/golden/make_golden.py e2e_wide [case ...]  # the K = 4096 / 14336 cases
    python tests/golden/make_golden.py moe          # moe_blend.npz only
    python tests/golden/make_golden.py nearest      # nearest.npz only
"""

import os
import sys

import numpy as np
import torch

REF = os.environ.get("HI2_REFERENCE", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))
# the repository root: tests/e2e_recipes.py digests rows with the oracle's helper
sys.path.insert(0, os.path.dirname(os.path.dirname(OUT)))

CASES = [(2, 16), (2, 32), (2, 64), (4, 16), (4, 32), (4, 64), (8, 32), (8, 64)]


def _layer(rows, k, seed, act_order, inverse_factor):
    # same recipe as the reference's tests/test_gptq_fast.py:19-36
    g = torch.Generator().manual_seed(seed)
    mix = torch.randn(k, k, generator=g) * 0.1 + torch.eye(k)
    x = torch.randn(4 * k, k, generator=g) @ mix
    x *= torch.exp(0.5 * torch.randn(1, k, generator=g))
    hs = x.T @ x / x.shape[0]
    w = torch.randn(rows, k, generator=g) * torch.exp(
        0.4 * torch.randn(rows, 1, generator=g)
    )
    w[:, :: max(1, k // 5)] *= 8
    d = hs.diagonal().clone()
    perm = None
    if act_order:
        perm = torch.argsort(d, descending=True)
        hs = hs[perm][:, perm]
    u = inverse_factor(hs, 0.01)
    return w, d, u, perm, hs


def _correlated(t, k, seed):
    # reference tests/test_hessian.py:18-23
    g = torch.Generator().manual_seed(seed)
    mix = torch.randn(k, k, generator=g) * 0.15 + torch.eye(k)
    x = torch.randn(t, k, generator=g) @ mix
    x *= torch.exp(0.5 * torch.randn(1, k, generator=g))
    return x


def _refine_rows(nbits, block, n, k, seed, encode_rows_gptq_reference, inverse_factor):
    # same recipe as the reference's tests/test_refine_kernel.py:25-32
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(500, k, generator=g) * torch.exp(0.5 * torch.randn(k, generator=g))
    hs = (x.T @ x) / 500
    w = torch.randn(n, k, generator=g) * 0.3
    enc = encode_rows_gptq_reference(w, hs.diagonal().clone(), inverse_factor(hs), nbits, block)
    return w, enc, hs


REFINE_CASES = {  # file: [(tag, [(nbits, block, rows)], k, seed, passes)]
    "refine_1.npz": [
        ("a", [(2, 32, 64)], 256, 64, 3),
        ("b", [(4, 64, 100)], 192, 100, 3),
        ("c", [(2, 16, 37)], 160, 37, 2),
        ("d", [(4, 16, 1)], 128, 1, 3),
        ("zero", [(2, 32, 33)], 128, 2, 0),
    ],
    "refine_2.npz": [
        ("e", [(2, 32, 40)], 384, 40, 2),
        ("mixed", [(2, 32, 70), (4, 64, 45)], 192, 1, 2),
        ("conv", [(2, 32, 33)], 128, 2, 40),
    ],
}


def make_refine():
    sys.path.insert(0, REF)
    from hi2.format import decode_params
    from hi2.hessian import encode_rows_gptq_reference, inverse_factor
    from hi2.refine import refine_groups

    torch.set_num_threads(1)
    for fname, cases in REFINE_CASES.items():
        arrs = {}
        for tag, groups, k, seed, passes in cases:
            _refine_case(arrs, tag, groups, k, seed, passes, decode_params,
                         encode_rows_gptq_reference, inverse_factor, refine_groups)
        np.savez_compressed(os.path.join(OUT, fname), **arrs)


def _refine_case(arrs, tag, groups, k, seed, passes, decode_params,
                 encode_rows_gptq_reference, inverse_factor, refine_groups):
    grp, hs = [], None
    for nbits, block, n in groups:
        w, enc, h = _refine_rows(nbits, block, n, k, seed, encode_rows_gptq_reference,
                                 inverse_factor)
        hs = h if hs is None else hs  # mixed: both groups use the first group's Hessian
        grp.append((w, enc, nbits, block))
    out = refine_groups(grp, hs, passes)
    arrs[f"{tag}_hs"] = hs.numpy()
    arrs[f"{tag}_passes"] = np.array(passes, np.int64)
    for gi, ((w, enc, nbits, block), codes) in enumerate(zip(grp, out)):
        lo, step = decode_params(enc.params[..., 0], enc.params[..., 1],
                                 enc.consts[:, 0:1], enc.consts[:, 1:2], enc.consts[:, 2:3])
        p = f"{tag}_g{gi}"
        arrs[f"{p}_spec"] = np.array([nbits, block], np.int64)
        arrs[f"{p}_w"] = w.numpy()
        arrs[f"{p}_codes_in"] = enc.codes.numpy()
        arrs[f"{p}_params"] = enc.params.numpy()
        arrs[f"{p}_consts"] = enc.consts.view(torch.int16).numpy()
        arrs[f"{p}_lo"] = lo.float().numpy()
        arrs[f"{p}_step"] = step.float().numpy()
        arrs[f"{p}_codes"] = codes.numpy()


def make_colstats():
    sys.path.insert(0, REF)
    from hi2.stats import ColumnStats

    torch.set_num_threads(1)
    g = torch.Generator().manual_seed(3)
    k, t1, t2 = 64, 4500, 700  # the first update spans two 4096-token chunks
    x = (torch.randn(t1 + t2, k, generator=g) * torch.exp(0.7 * torch.randn(k, generator=g)))
    xb = x.to(torch.bfloat16)
    arrs = {"x_bf16": xb.view(torch.int16).numpy(), "split": np.array([t1, t2], np.int64)}
    flags = torch.tensor([1, 0, 1, 1], dtype=torch.uint8)
    inv = 1.0 / (torch.rand(k, generator=g) + 0.5).half().float()
    arrs["flags"] = flags.numpy()
    arrs["inv_scale"] = inv.numpy()
    for tag, xs in (("bf16", xb), ("f32", xb.float())):
        st = ColumnStats(k)
        st.update(xs[:t1])
        st.update(xs[t1:])
        arrs[f"{tag}_S"] = st.S.numpy()
        arrs[f"{tag}_n"] = np.array(st.n, np.int64)
        arrs[f"{tag}_diag"] = st.diag().numpy()
        arrs[f"{tag}_diag_rot"] = st.diag(flags).numpy()
        arrs[f"{tag}_diag_inv"] = st.diag(None, inv).numpy()
        arrs[f"{tag}_diag_rot_inv"] = st.diag(flags, inv).numpy()
    np.savez_compressed(os.path.join(OUT, "colstats.npz"), **arrs)


# encode_many requests: name -> (rows, input, sigma_id, smoothed, flags, weight dtype, comp)
EM_TENSORS = {
    "q": (36, "in0", "in0", True, "mixed", torch.bfloat16, False),
    "k": (20, "in0", "in0", True, "mixed", torch.bfloat16, True),
    "o": (28, "in1", None, False, "ones", torch.float32, False),
    "n": (12, "in0", None, True, "mixed", torch.bfloat16, True),  # no sigma: nearest rows
    "v": (16, "in0", "in0", True, "ones", torch.float32, False),  # same input, other flags
}
EM_INPUTS = {"in0": (128, 1200), "in1": (64, 700)}  # K, tokens
# config tag -> (rounding, act_order, refine_passes, effort)
EM_CONFIGS = {
    "g": ("gptq", False, 0, "normal"),
    "ga": ("gptq", True, 0, "fast"),
    "gr": ("gptq", False, 2, "normal"),
    "nr": ("nearest", False, 0, "normal"),
}


def make_encode_many():
    sys.path.insert(0, REF)
    import hi2.hessian as H
    from hi2.calibrate import (ALL_CANDIDATES, INT8_CANDIDATES, Config, EncodeRequest,
                               TensorTable, encode_many, smoothing_scale)
    from hi2.executor import Executor
    from hi2.format import GROUP
    from hi2.stats import ColumnStats

    torch.set_num_threads(1)
    g = torch.Generator().manual_seed(29)
    cands = list(ALL_CANDIDATES) + list(INT8_CANDIDATES)
    arrs = {"candidates": np.array(cands, np.int64), "names": np.array(list(EM_TENSORS)),
            "configs": np.array(list(EM_CONFIGS))}
    for tag, (rounding, ao, passes, effort) in EM_CONFIGS.items():
        arrs[f"{tag}_cfg"] = np.array([rounding, str(int(ao)), str(passes), effort])
    stats, sigma = {}, {}
    for inp, (k, t) in EM_INPUTS.items():
        x = torch.randn(t, k, generator=g) * torch.exp(0.6 * torch.randn(k, generator=g))
        x[:, :: 7] *= 5.0
        x = x.to(torch.bfloat16)
        st = ColumnStats(k)
        st.update(x)
        stats[inp] = st
        xf = x.float()
        sigma[inp] = (xf.T @ xf) / t
        arrs[f"{inp}_S"] = st.S.numpy()
        arrs[f"{inp}_n"] = np.array(st.n, np.int64)
        arrs[f"{inp}_sigma"] = sigma[inp].numpy()
    s16 = smoothing_scale(stats["in0"], 0.5)
    arrs["in0_col_scale"] = s16.view(torch.int16).numpy()
    reqs_in = []
    for name, (rows, inp, sid, smooth, fl, dt, comp) in EM_TENSORS.items():
        k = EM_INPUTS[inp][0]
        w = torch.randn(rows, k, generator=g) * torch.exp(0.4 * torch.randn(rows, 1, generator=g))
        w[:, :: max(1, k // 5)] *= 6
        w = (w * 0.05).to(dt)
        if fl == "ones":
            had = torch.ones(k // GROUP, dtype=torch.uint8)
        else:
            had = (torch.arange(k // GROUP) % 3 != 1).to(torch.uint8)
        picks = torch.randint(0, len(cands), (rows,), generator=g)
        arrs[f"w_{name}"] = (w.view(torch.int16) if dt == torch.bfloat16 else w).numpy()
        arrs[f"had_{name}"] = had.numpy()
        arrs[f"picks_{name}"] = picks.numpy().astype(np.int64)
        arrs[f"meta_{name}"] = np.array([inp, sid or "", str(int(smooth)), str(int(comp)),
                                         str(int(name != "n")), str(int(name != "o"))])
        reqs_in.append((name, w, inp, sid, s16 if smooth else None, had, picks, comp))
    orig = H.inverse_factor
    for tag, (rounding, ao, passes, effort) in EM_CONFIGS.items():
        cfg = Config(candidates=cands, rounding=rounding, act_order=ao, refine_passes=passes,
                     effort=effort)
        reqs = []
        for name, w, inp, sid, cs, had, picks, comp in reqs_in:
            k = w.shape[1]
            table = TensorTable(name, (w.shape[0], k), had.clone(),
                                torch.zeros(len(cands), w.shape[0]), cands, 0.0,
                                stats[inp].n, None if cs is None else cs.clone())
            sig = None if name == "n" else sigma[inp]
            reqs.append(EncodeRequest(w, None if name == "o" else stats[inp], table, picks,
                                      sig, sid, {} if comp else None))
        factors = []

        def record(hs, damp=0.01):
            u = orig(hs, damp)
            factors.append(u.clone())
            return u

        H.inverse_factor = record
        try:
            out = encode_many(reqs, cfg, Executor(["cpu"]))
        finally:
            H.inverse_factor = orig
        arrs[f"{tag}_nfactors"] = np.array(len(factors), np.int64)
        for j, u in enumerate(factors):
            arrs[f"{tag}_u{j}"] = u.numpy()
        for r, o in zip(reqs, out):
            nm = r.table.name
            for f in ("codes", "code_off", "blk_params", "param_off", "row_nbits",
                      "row_block", "had"):
                arrs[f"{tag}_{nm}_{f}"] = getattr(o, f).numpy()
            arrs[f"{tag}_{nm}_row_consts"] = o.row_consts.view(torch.int16).numpy()
            if r.comp_out is not None:
                arrs[f"{tag}_{nm}_comp"] = r.comp_out["comp"].numpy()
    np.savez_compressed(os.path.join(OUT, "encode_many.npz"), **arrs)


# QAD cases: tag -> (latent units, zero-step and far-off blocks, clamped first 16 columns)
QAD_CASES = {"abs": ("abs", False, False), "step": ("step", True, False),
             "clamp": ("abs", True, True)}


def make_qad():
    sys.path.insert(0, REF)
    from hi2.calibrate import (ALL_CANDIDATES, INT8_CANDIDATES, Config, EncodeRequest,
                               TensorTable, encode_many)
    from hi2.executor import Executor
    from hi2.format import GROUP
    from hi2.qad import FakeQuantLinear

    torch.set_num_threads(1)
    g = torch.Generator().manual_seed(37)
    cands = list(ALL_CANDIDATES) + list(INT8_CANDIDATES)
    r, k = 40, 128
    w = torch.randn(r, k, generator=g) * torch.exp(0.4 * torch.randn(r, 1, generator=g)) * 0.05
    cs = (torch.rand(k, generator=g) * 1.5 + 0.5).half()
    had = (torch.arange(k // GROUP) % 3 != 1).to(torch.uint8)
    picks = torch.randint(0, len(cands), (r,), generator=g)
    table = TensorTable("t", (r, k), had, torch.zeros(len(cands), r), cands, 0.0, 0, cs)
    cfg = Config(candidates=cands, rounding="nearest")
    t0 = encode_many([EncodeRequest(w, None, table, picks)], cfg, Executor(["cpu"]))[0]
    arrs = {"w": w.numpy(), "had": had.numpy(), "col_scale": cs.view(torch.int16).numpy()}
    for tag, (units, zero_blocks, clamp) in QAD_CASES.items():
        fq = FakeQuantLinear(w, t0, None, "weights", units)
        with torch.no_grad():
            fq.latent.add_(0.3 * fq.latent.std() * torch.randn(r, k, generator=g))
            for gr in fq.groups:
                gr.lo_u.add_(0.7 * torch.randn(gr.lo_u.shape, generator=g))
                gr.step_u.add_(0.7 * torch.randn(gr.step_u.shape, generator=g))
                if zero_blocks:
                    gr.step_u[::3, ::2] = 0.0
                    gr.lo_u[1::4] += 40.0
            fq.project()
            if clamp:
                fq.latent[:, :16] += 50.0 * fq.latent.abs().max()
        params = [fq.latent] + [p for gr in fq.groups for p in (gr.lo_u, gr.step_u)]
        grad = torch.randn(r, k, generator=g)
        grad2 = torch.randn(r, k, generator=g)
        stored = fq.stored(False).detach()
        st_grads = torch.autograd.grad(fq.stored(True), params, grad)
        orig = fq()
        or_grads = torch.autograd.grad(orig, params, grad2)
        p = f"{tag}_"
        arrs[p + "latent"] = fq.latent.detach().numpy()
        arrs[p + "unit"] = fq.unit.numpy()
        arrs[p + "ngroups"] = np.array(len(fq.groups), np.int64)
        for gi, gr in enumerate(fq.groups):
            q = f"{p}g{gi}_"
            arrs[q + "rows"] = gr.rows.numpy()
            arrs[q + "consts"] = gr.consts.view(torch.int16).numpy()
            arrs[q + "spec"] = np.array([gr.nbits, gr.block], np.int64)
            arrs[q + "lo_u"] = gr.lo_u.detach().numpy()
            arrs[q + "st_u"] = gr.step_u.detach().numpy()
            arrs[q + "g_lo"] = st_grads[1 + 2 * gi].numpy()
            arrs[q + "g_st"] = st_grads[2 + 2 * gi].numpy()
            arrs[q + "og_lo"] = or_grads[1 + 2 * gi].numpy()
            arrs[q + "og_st"] = or_grads[2 + 2 * gi].numpy()
        arrs[p + "grad"] = grad.numpy()
        arrs[p + "grad2"] = grad2.numpy()
        arrs[p + "stored"] = stored.numpy()
        arrs[p + "g_latent"] = st_grads[0].numpy()
        arrs[p + "original"] = orig.detach().numpy()
        arrs[p + "og_latent"] = or_grads[0].numpy()
    np.savez_compressed(os.path.join(OUT, "qad.npz"), **arrs)


def make_e2e():
    sys.path.insert(0, REF)
    sys.path.insert(0, os.path.dirname(OUT))
    import hi2.hessian as H
    from e2e_recipes import CANDIDATES, CASES, DAMP, FULL_CASES, SLICE_ROWS, WIDE_CASES, \
        input_digests, inputs, sha, upper
    from hi2.calibrate import Config, EncodeRequest, TensorTable, encode_many
    from hi2.executor import Executor
    from hi2.format import fwht_groups
    from hi2.hessian import GptqJob, HessianStats, encode_jobs_gptq, transform_sigma

    torch.set_num_threads(1)
    orig = H.inverse_factor
    for case, (_recipe, k, n, t, _seed) in CASES.items():
        if case in WIDE_CASES:
            continue
        print(case, flush=True)
        xb, w, picks, had = inputs(case)
        had_t = torch.from_numpy(had)
        st = HessianStats(k)
        st.update(xb)
        sigma = st.mean()
        factors = []

        def record(hs, damp=0.01):
            u = orig(hs, damp)
            factors.append(u.clone())
            return u

        table = TensorTable(case, (n, k), had_t.clone(), torch.zeros(len(CANDIDATES), n),
                            list(CANDIDATES), 0.0, st.n, None)
        req = EncodeRequest(torch.from_numpy(w), None, table, torch.from_numpy(picks), sigma,
                            "x", {})
        cfg = Config(candidates=list(CANDIDATES), rounding="gptq", act_order=False,
                     refine_passes=0, effort="normal", damp=DAMP)
        H.inverse_factor = record
        try:
            packed = encode_many([req], cfg, Executor(["cpu"]))[0]
        finally:
            H.inverse_factor = orig
        assert len(factors) == 1
        u = factors[0]
        # the per-row outputs encode_many does not return (sse, the unpacked codes), from
        # the reference's GPTQ entry on the same inputs; comp must equal encode_many's
        hs = transform_sigma(sigma, None, had_t)
        d = hs.diagonal().clone()
        wt = fwht_groups(torch.from_numpy(w), had_t)
        codes = np.zeros((n, k), np.uint8)
        comp = np.zeros((n, k), np.float32)
        sse = np.zeros(n, np.float32)
        groups = []
        for ci, (nb, b) in enumerate(CANDIDATES):
            rows = np.nonzero(picks == ci)[0]
            if rows.size == 0:
                continue
            e = encode_jobs_gptq([GptqJob(wt[torch.from_numpy(rows)], d, u, nb, b)],
                                 "normal", comp=True)[0]
            codes[rows] = e.codes.numpy()
            comp[rows] = e.comp.numpy()
            sse[rows] = e.sse.numpy()
            groups.append((ci, rows, e.params.numpy(), e.consts.view(torch.int16).numpy()))
        assert np.array_equal(comp, req.comp_out["comp"].numpy())
        meta = {"case": np.array(case), "digest_x": np.array(input_digests(case)["x"]),
                "digest_w": np.array(input_digests(case)["w"]),
                "digest_picks": np.array(input_digests(case)["picks"]),
                "sigma_sha": np.array(sha(sigma.numpy())), "hs_sha": np.array(sha(hs.numpy())),
                "u_sha": np.array(sha(u.numpy())), "codes_sha": np.array(sha(codes)),
                "comp_sha": np.array(sha(comp)), "sse": sse,
                "packed_sha": np.array(sha(packed.codes.numpy())),
                "d": d.numpy(), "sigma_diag": np.diag(sigma.numpy()).copy(),
                "u_diag": np.diag(u.numpy()).copy()}
        if case in FULL_CASES:
            np.savez_compressed(os.path.join(OUT, f"e2e_{case}_factor.npz"), **meta,
                                sigma_tri=upper(sigma.numpy()), u_tri=upper(u.numpy()))
            # codes travel packed (the reference's own words); comp in a file of its own
            np.savez_compressed(os.path.join(OUT, f"e2e_{case}_comp.npz"), comp=comp)
            out = {}
            for f in ("codes", "code_off", "blk_params", "param_off", "row_nbits",
                      "row_block"):
                out[f"packed_{f}"] = getattr(packed, f).numpy()
            out["packed_row_consts"] = packed.row_consts.view(torch.int16).numpy()
            for ci, rows, params, consts in groups:
                out[f"g{ci}_rows"] = rows
                out[f"g{ci}_params"] = params
                out[f"g{ci}_consts"] = consts
            np.savez_compressed(os.path.join(OUT, f"e2e_{case}_out.npz"), **out)
        else:
            r = SLICE_ROWS
            out = dict(meta, codes_slice=codes[:r], comp_slice=comp[:r],
                       u_rows=u.numpy()[:16].copy(), sigma_rows=sigma.numpy()[:16].copy())
            for ci, rows, params, consts in groups:
                keep = rows < r
                out[f"g{ci}_rows"] = rows[keep]
                out[f"g{ci}_params"] = params[keep]
                out[f"g{ci}_consts"] = consts[keep]
            np.savez_compressed(os.path.join(OUT, f"e2e_{case}.npz"), **out)


def make_e2e_wide(cases=None):
    """The reference's pipeline at the benchmark's widths (tests/e2e_recipes.py
    WIDE_CASES: K = 4096 with 8192 tokens, K = 14336 with 4096 tokens), where this build's
    factor runs its fp16 split-plane products: HessianStats over the bf16 tokens, mean,
    transform_sigma, inverse_factor, fwht_groups, GPTQ of every candidate group through
    encode_jobs_gptq (comp on) and assemble.  Stored per case, in three files near 1 MB:
    digests of the inputs, of Sigma, Hs, U, the codes, comp, sse and every packed field;
    every row's sse, consts and 8-byte digests of its codes and ladder bytes, 4-byte
    digests of its codes per 512 columns; d; the
    diagonals and a few evenly spread rows of Sigma and U; the first rows' codes, ladder
    bytes and comp in full.  Beside it, the same digests of the reference against itself
    with its Hessian accumulated in 2048-token chunks (``HessianStats.update``'s chunk
    argument), and the share of codes the two reference runs have equal.  Torch runs on 8
    threads here (recorded as "threads"): the case is too large for one."""
    sys.path.insert(0, REF)
    sys.path.insert(0, os.path.dirname(OUT))
    from e2e_recipes import (CANDIDATES, CASES, DAMP, WIDE_CASES, WIDE_SLICE_ROWS,
                             factor_rows, input_digests, inputs, row_digests,
                             segment_digests, sha)
    from hi2.format import assemble, fwht_groups
    from hi2.hessian import (GptqJob, HessianStats, encode_jobs_gptq, inverse_factor,
                             transform_sigma)

    threads = 8
    torch.set_num_threads(threads)
    for case in cases or WIDE_CASES:
        _recipe, k, n, t, _seed = CASES[case]
        print(case, flush=True)
        xb, w, picks, had = inputs(case)
        had_t = torch.from_numpy(had)
        st = HessianStats(k)
        st.update(xb)
        sigma = st.mean()
        hs = transform_sigma(sigma, None, had_t)
        d = hs.diagonal().clone()
        u = inverse_factor(hs, DAMP)
        wt = fwht_groups(torch.from_numpy(w), had_t)
        codes = np.zeros((n, k), np.uint8)
        comp = np.zeros((n, k), np.float32)
        sse = np.zeros(n, np.float32)
        consts = np.zeros((n, 3), np.uint16)
        pdig = np.zeros(n, np.uint64)
        groups, pieces = [], []
        for ci, (nb, b) in enumerate(CANDIDATES):
            rows = np.nonzero(picks == ci)[0]
            if rows.size == 0:
                continue
            print(f"  gptq INT{nb}/B{b}: {rows.size} rows", flush=True)
            e = encode_jobs_gptq([GptqJob(wt[torch.from_numpy(rows)], d, u, nb, b)],
                                 "normal", comp=True)[0]
            codes[rows] = e.codes.numpy()
            comp[rows] = e.comp.numpy()
            sse[rows] = e.sse.numpy()
            cb = e.consts.view(torch.int16).numpy().view(np.uint16)
            consts[rows] = cb
            pdig[rows] = row_digests(e.params.numpy())
            groups.append((ci, rows, e.params.numpy(), cb))
            pieces.append((torch.from_numpy(rows), e.codes, e.params, e.consts))
        nbits = torch.tensor([CANDIDATES[c][0] for c in picks])
        block = torch.tensor([CANDIDATES[c][1] for c in picks])
        packed = assemble(pieces, nbits, block, had_t, k)
        dg = input_digests(case)
        rs = factor_rows(case)
        sg, un = sigma.numpy(), u.numpy()
        meta = {"case": np.array(case), "threads": np.array(threads),
                "digest_x": np.array(dg["x"]), "digest_w": np.array(dg["w"]),
                "digest_picks": np.array(dg["picks"]), "sigma_sha": np.array(sha(sg)),
                "hs_sha": np.array(sha(hs.numpy())), "u_sha": np.array(sha(un)),
                "codes_sha": np.array(sha(codes)), "comp_sha": np.array(sha(comp)),
                "sse_sha": np.array(sha(sse))}
        for f in ("codes", "code_off", "blk_params", "param_off", "row_consts"):
            meta[f"packed_{f}_sha"] = np.array(sha(getattr(packed, f).numpy()))
        np.savez_compressed(os.path.join(OUT, f"e2e_{case}_factor.npz"), **meta,
                            factor_rows=rs, sigma_rows=sg[rs].copy(), u_rows=un[rs].copy(),
                            sigma_diag=np.diag(sg).copy(), u_diag=np.diag(un).copy())
        r = WIDE_SLICE_ROWS[case]
        out = dict(d=d.numpy(), sse=sse, consts_all=consts, codes_digest=row_digests(codes),
                   codes_segments=segment_digests(codes), params_digest=pdig,
                   codes_slice=codes[:r])
        for ci, rows, params, cb in groups:
            keep = rows < r
            out[f"g{ci}_rows"] = rows[keep]
            out[f"g{ci}_params"] = params[keep]
            out[f"g{ci}_consts"] = cb[keep]
        # the reference against itself: the same pipeline with its Hessian accumulated in
        # 2048-token chunks (HessianStats.update's own chunk argument) instead of 4096 —
        # the departures two correct fp32 runs of the reference show between them
        st2 = HessianStats(k)
        st2.update(xb, chunk=2048)
        hs2 = transform_sigma(st2.mean(), None, had_t)
        d2 = hs2.diagonal().clone()
        u2 = inverse_factor(hs2, DAMP)
        codes2 = np.zeros((n, k), np.uint8)
        pdig2 = np.zeros(n, np.uint64)
        sse2 = np.zeros(n, np.float32)
        for ci, (nb, b) in enumerate(CANDIDATES):
            rows = np.nonzero(picks == ci)[0]
            if rows.size == 0:
                continue
            print(f"  self-check, 2048-token chunks: INT{nb}/B{b}", flush=True)
            e = encode_jobs_gptq([GptqJob(wt[torch.from_numpy(rows)], d2, u2, nb, b)],
                                 "normal")[0]
            codes2[rows] = e.codes.numpy()
            sse2[rows] = e.sse.numpy()
            pdig2[rows] = row_digests(e.params.numpy())
        out.update(self_codes_digest=row_digests(codes2), self_params_digest=pdig2,
                   self_codes_segments=segment_digests(codes2), self_sse=sse2,
                   self_codes_equal=np.array((codes2 == codes).mean()))
        np.savez_compressed(os.path.join(OUT, f"e2e_{case}_out.npz"), **out)
        np.savez_compressed(os.path.join(OUT, f"e2e_{case}_comp.npz"), comp_slice=comp[:r])
        del st, sigma, hs, u, wt, codes, comp, st2, hs2, u2, codes2


def make_moe():
    """The MoE token floor: hi2/layerwise.py:241-257 (the experts' sum, need, which experts
    are short) with the reference's own blend (hi2/moe.py:152-156) on every short expert."""
    sys.path.insert(0, REF)
    from hi2.moe import blend

    torch.set_num_threads(1)
    g = torch.Generator().manual_seed(53)
    k = 64
    counts = [5000, 300, 0, 4096, 1200, 70, 9000]
    sums = []
    for n in counts:
        x = torch.randn(max(n, 1), k, generator=g) * torch.exp(0.5 * torch.randn(k, generator=g))
        s_ = x.T @ x if n else torch.zeros(k, k)
        sums.append(s_.float())
    need = int(2.0 * 2048)  # min_tokens x the expert's widest input (cfg5: 2 x 2048)
    tot_n = sum(counts)
    tot_s = sum(sums)  # the reference's Python sum over the experts, as layerwise._merge
    out, out_n = [], []
    for s_, n in zip(sums, counts):
        if n >= need or tot_n == 0:
            out.append(s_)
            out_n.append(n)
            continue
        b, nn_ = blend(s_, n, tot_s, tot_n, need)
        out.append(b)
        out_n.append(nn_)
    np.savez_compressed(os.path.join(OUT, "moe_blend.npz"), counts=np.array(counts, np.int64),
                        need=np.array(need, np.int64), sums=np.stack([t.numpy() for t in sums]),
                        out=np.stack([t.numpy() for t in out]),
                        out_n=np.array(out_n, np.int64))


def make_nearest():
    """hi2.encode.encode_rows (nearest rounding, hi2/encode.py:133-173) on the rotated
    cfg1_k512_t2048 rows with the reference's own diag(Hs) as the weights: INT2/B32 on
    the first 96 rows, INT4/B64 on the next 96, INT8/B64 on 32."""
    sys.path.insert(0, REF)
    sys.path.insert(0, os.path.dirname(OUT))
    from e2e_recipes import inputs
    from hi2.encode import encode_rows
    from hi2.format import fwht_groups
    from hi2.hessian import HessianStats, transform_sigma

    torch.set_num_threads(1)
    xb, w, picks, had = inputs("cfg1_k512_t2048")
    st = HessianStats(w.shape[1])
    st.update(xb)
    d = transform_sigma(st.mean(), None, torch.from_numpy(had)).diagonal().clone()
    wt = fwht_groups(torch.from_numpy(w), torch.from_numpy(had))
    arrs = {"d": d.numpy(), "wt": wt[:224].numpy()}
    for tag, (nb, b, a, z) in {"int2": (2, 32, 0, 96), "int4": (4, 64, 96, 192),
                                "int8": (8, 64, 192, 224)}.items():
        e = encode_rows(wt[a:z], d, nb, b, "normal")
        arrs[f"{tag}_codes"] = e.codes.numpy()
        arrs[f"{tag}_params"] = e.params.numpy()
        arrs[f"{tag}_consts"] = e.consts.view(torch.int16).numpy()
        arrs[f"{tag}_sse"] = e.sse.numpy()
    np.savez_compressed(os.path.join(OUT, "nearest.npz"), **arrs)


def main():
    if sys.argv[1:] == ["nearest"]:
        make_nearest()
        return
    if sys.argv[1:] == ["moe"]:
        make_moe()
        return
    if sys.argv[1:2] == ["e2e_wide"]:
        make_e2e_wide(sys.argv[2:] or None)
        return
    if sys.argv[1:] == ["e2e"]:
        make_e2e()
        return
    if sys.argv[1:] == ["qad"]:
        make_qad()
        return
    if sys.argv[1:] == ["encode_many"]:
        make_encode_many()
        return
    if sys.argv[1:] == ["refine"]:
        make_refine()
        return
    if sys.argv[1:] == ["colstats"]:
        make_colstats()
        return
    sys.path.insert(0, REF)
    from hi2.encode import EFFORT, fit_ladder
    from hi2.hessian import encode_rows_gptq_reference, inverse_factor

    torch.set_num_threads(1)
    meta = dict(torch=torch.__version__, threads=1)

    # ---- GPTQ end to end (codes/params/consts/sse/comp) ------------------------
    for nbits in (2, 4, 8):
        arrs = {}
        for (nb, b) in CASES:
            if nb != nbits:
                continue
            for ao in (False, True):
                for effort in ("fast", "normal"):
                    if effort == "normal" and ao:
                        continue
                    seed = nb * 100 + b + (7 if effort == "normal" else 0)
                    w, d, u, perm, _ = _layer(24, 192, seed, ao, inverse_factor)
                    enc = encode_rows_gptq_reference(w, d, u, nb, b, effort, perm)
                    tag = f"b{b}_ao{int(ao)}_{effort}"
                    arrs[f"{tag}_w"] = w.numpy()
                    arrs[f"{tag}_d"] = d.numpy()
                    arrs[f"{tag}_u"] = u.numpy()
                    arrs[f"{tag}_perm"] = (
                        perm.numpy().astype(np.int64)
                        if perm is not None
                        else np.zeros(0, np.int64)
                    )
                    arrs[f"{tag}_codes"] = enc.codes.numpy()
                    arrs[f"{tag}_params"] = enc.params.numpy()
                    arrs[f"{tag}_consts"] = enc.consts.view(torch.int16).numpy()
                    arrs[f"{tag}_sse"] = enc.sse.numpy()
                    arrs[f"{tag}_comp"] = enc.comp.numpy()
        np.savez_compressed(os.path.join(OUT, f"gptq_int{nbits}.npz"), **arrs)

    # ---- inverse_factor ---------------------------------------------------------
    arrs = {}
    for k, t, seed in ((32, 500, 0), (64, 1000, 1), (200, 4000, 2)):
        x = _correlated(t, k, seed)
        hs = x.T @ x / t
        arrs[f"k{k}_hs"] = hs.numpy()
        arrs[f"k{k}_u"] = inverse_factor(hs, 0.01).numpy()
    sing = torch.zeros(16, 16)
    sing[0, 0] = 1.0
    arrs["singular_hs"] = sing.numpy()
    arrs["singular_u"] = inverse_factor(sing, 0.01).numpy()
    # indefinite: the first attempts fail, a later damping succeeds
    ind = torch.eye(16)
    ind[15, 15] = -0.2
    arrs["indef_hs"] = ind.numpy()
    arrs["indef_u"] = inverse_factor(ind, 0.01).numpy()
    np.savez_compressed(os.path.join(OUT, "inverse_factor.npz"), **arrs)

    # ---- fit_ladder -----------------------------------------------------------------
    arrs = {}
    g = torch.Generator().manual_seed(11)
    for n, b, effort in ((4, 16, "normal"), (16, 64, "normal"), (4, 32, "fast"),
                         (16, 32, "max"), (256, 64, "normal")):
        wb = torch.randn(48, 6, b, generator=g) * torch.exp(
            0.5 * torch.randn(48, 6, 1, generator=g)
        )
        wb[:, :, :: max(1, b // 5)] *= 4
        db = torch.rand(1, 6, b, generator=g) + 0.25
        lo, step = fit_ladder(wb, db, n, effort)
        tag = f"n{n}_b{b}_{effort}"
        arrs[f"{tag}_wb"] = wb.numpy()
        arrs[f"{tag}_db"] = db.numpy()
        arrs[f"{tag}_lo"] = lo.numpy()
        arrs[f"{tag}_step"] = step.numpy()
    arrs["effort_normal_grid"] = np.array(EFFORT["normal"]["grid"], np.float64)
    np.savez_compressed(os.path.join(OUT, "fit_ladder.npz"), **arrs)

    make_refine()
    make_colstats()
    make_encode_many()
    make_qad()
    make_e2e()
    make_moe()
    make_nearest()

    with open(os.path.join(OUT, "golden_meta.txt"), "w") as f:
        for k, v in meta.items():
            f.write(f"{k}={v}\n")


if __name__ == "__main__":
    main()
