"""The HIP path against the oracle and the reference's golden vectors (MI355X).

Bit-exact wherever the reference's arithmetic is a fixed sequence of IEEE operations
(ladder fit, params, column loop and its MFMA cross-block update, finish, Hadamard,
transform_sigma, packing); tolerance for the Hessian GEMM and the Cholesky chain,
whose reference rounding comes from BLAS/LAPACK blocking (rtol stated per test)."""

import numpy as np
import pytest
import torch

import oracle
from golden_data import CASES, fit_cases, gptq_cases, inverse_cases

pytestmark = pytest.mark.gpu


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.detach().cpu().numpy()


def _same(got, want: dict):
    assert np.array_equal(N(got.codes), want["codes"]), "codes"
    assert np.array_equal(N(got.params), want["params"]), "params"
    assert np.array_equal(N(got.consts).view(np.int16), want["consts"].view(np.int16)), "consts"
    assert np.array_equal(N(got.sse), want["sse"]), "sse"
    if want.get("comp") is not None:
        assert got.comp is not None
        assert np.array_equal(N(got.comp), want["comp"]), "comp"


def _layer(rows, k, seed, act_order=False):
    """Seeded layer like the reference's tests/test_gptq_fast.py:19-36 (numpy RNG),
    with the factor from the oracle (the same U goes to both sides)."""
    rng = np.random.default_rng(seed)
    mix = rng.standard_normal((k, k)) * 0.1 + np.eye(k)
    x = rng.standard_normal((4 * k, k)) @ mix
    x *= np.exp(0.5 * rng.standard_normal((1, k)))
    hs = (x.T @ x / x.shape[0]).astype(np.float32)
    w = (rng.standard_normal((rows, k)) * np.exp(0.4 * rng.standard_normal((rows, 1)))).astype(np.float32)
    w[:, :: max(1, k // 5)] *= 8
    d = np.diag(hs).copy()
    perm = None
    if act_order:
        perm = np.argsort(-d, kind="stable")
        hs = hs[perm][:, perm]
    u, _ = oracle.inverse_factor(hs, 0.01)
    return w, d, u, perm, hs


# ---- the reference's golden vectors ---------------------------------------------------
@pytest.mark.parametrize(
    "case", list(gptq_cases()), ids=lambda c: f"int{c[0]}_b{c[1]}_{c[2]}_ao{int(c[3])}"
)
@pytest.mark.parametrize("schedule", ["batched", "per_block"])
def test_gptq_equals_reference_golden(dev, case, schedule):
    from hi2_amd.hessian import encode_rows_gptq, encode_rows_gptq_reference

    nbits, block, effort, _, a = case
    perm = None if a["perm"] is None else T(a["perm"], dev)
    fn = encode_rows_gptq if schedule == "batched" else encode_rows_gptq_reference
    got = fn(T(a["w"], dev), T(a["d"], dev), T(a["u"], dev), nbits, block, effort, perm)
    _same(got, a)


@pytest.mark.parametrize("case", list(fit_cases()), ids=lambda c: f"n{c[0]}_b{c[1]}_{c[2]}")
def test_fit_ladder_equals_reference_golden(dev, case):
    from hi2_amd.encode import fit_ladder

    n, b, effort, a = case
    lo, st = fit_ladder(T(a["wb"], dev), T(a["db"], dev), n, effort)
    assert np.array_equal(N(lo), a["lo"]) and np.array_equal(N(st), a["step"])


@pytest.mark.parametrize("case", list(inverse_cases()), ids=lambda c: c[0])
def test_inverse_factor_matches_reference_golden(dev, case):
    from hi2_amd.hessian import inverse_factor

    _, hs, u_ref = case
    u = N(inverse_factor(T(hs, dev), 0.01))
    assert np.array_equal(np.tril(u, -1), np.zeros_like(u))
    scale = np.abs(u_ref).max()
    # fp32 factorisations in different orders: agreement to the conditioning allows
    assert np.allclose(u, u_ref, rtol=1e-3, atol=1e-4 * scale), np.abs(u - u_ref).max() / scale


# ---- the column loop ------------------------------------------------------------------
@pytest.mark.parametrize("nbits,block", CASES)
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("k", [192, 448])  # last block shorter than 128
def test_gptq_equals_oracle(dev, nbits, block, act_order, k):
    from hi2_amd.hessian import encode_rows_gptq

    w, d, u, perm, _ = _layer(200, k, nbits * 7 + block + k, act_order)
    want = oracle.encode_rows_gptq(w, d, u, nbits, block, "fast", perm)
    got = encode_rows_gptq(T(w, dev), T(d, dev), T(u, dev), nbits, block, "fast",
                           None if perm is None else T(perm, dev))
    _same(got, want)


def test_gptq_block_one_launch_equals_oracle(dev):
    """hi2x_gptq_block alone (the gptq_kernel.gptq_block contract), three row groups
    with different factors, column maps and code counts, a 96-column last block."""
    from hi2_amd import gptq_kernel

    rng = np.random.default_rng(7)
    k, i1, length = 224, 128, 96
    sizes = [37, 64, 70]
    n = sum(sizes)
    us, blks, nmax = [], [], []
    for g, nb in enumerate((4, 16, 256)):
        _, _, u, perm, _ = _layer(4, k, 100 + g, act_order=g == 1)
        us.append(u)
        blks.append((np.arange(k) if perm is None else perm) // 32)
        nmax.append(nb - 1)
    wc = (rng.standard_normal((n, k)) * 0.3).astype(np.float32)
    ldp = k // 16
    lo = (rng.standard_normal((n, ldp)) * 0.2 - 0.5).astype(np.float32)
    st = (rng.random((n, ldp)) * 0.1).astype(np.float32)
    st[5, 4] = 0.0
    row_grp = np.repeat(np.arange(3), sizes).astype(np.int32)
    blk = np.stack(blks).astype(np.int32)
    nm = np.array(nmax, np.float32)
    err_w, codes_w, comp_w = oracle.gptq_block(wc, i1, length, lo, st, row_grp, us, blk, nm)
    ut = [T(u, dev) for u in us]
    u_ptrs = torch.tensor([u.data_ptr() for u in ut], dtype=torch.int64, device=dev)
    err1 = torch.empty(n, length, dtype=torch.float32, device=dev)
    codes = torch.zeros(n, k, dtype=torch.uint8, device=dev)
    comp = torch.zeros(n, k, dtype=torch.float32, device=dev)
    gptq_kernel.gptq_block(T(wc, dev), i1, length, err1, codes, T(lo, dev), T(st, dev),
                           T(row_grp, dev), u_ptrs, T(blk, dev), T(nm, dev), comp)
    assert np.array_equal(N(err1), err_w)
    assert np.array_equal(N(codes), codes_w)
    assert np.array_equal(N(comp), comp_w)


@pytest.mark.parametrize("sb", [1, 2, 3, 8])
def test_super_block_schedule_is_bit_identical(dev, sb):
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq

    w, d, u, perm, _ = _layer(150, 1024, 5, act_order=True)
    job = GptqJob(T(w, dev), T(d, dev), T(u, dev), 4, 64, T(perm, dev))
    ref = encode_jobs_gptq([job], "normal", comp=True, super_blocks=1)[0]
    got = encode_jobs_gptq([job], "normal", comp=True, super_blocks=sb)[0]
    for f in ("codes", "params", "consts", "sse", "comp"):
        assert torch.equal(getattr(got, f), getattr(ref, f)), f


def test_background_stream_leaves_results_unchanged(dev):
    """hi2x_stream_background only changes how many of the cross-block update's
    workgroups share a CU: the same job on a background stream gives the same bits.
    4096 rows x 4096 columns, so the far updates take the 128-tile path and the near
    ones the 64-tile path."""
    from hi2_amd import _lib
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq, inverse_factor

    k, n = 4096, 4096
    g = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(2 * k, k, device=dev, generator=g)
    hs = (x.T @ x / x.shape[0]).contiguous()
    del x
    u = inverse_factor(hs, 0.01)
    w = torch.randn(n, k, device=dev, generator=g) * 0.02
    job = GptqJob(w, torch.diagonal(hs).clone(), u, 4, 64)
    st = torch.cuda.Stream(device=dev)
    st.wait_stream(torch.cuda.current_stream(dev))
    try:
        with torch.cuda.stream(st):
            ref = encode_jobs_gptq([job], "normal", comp=True)[0]
            _lib.stream_background(st)
            got = encode_jobs_gptq([job], "normal", comp=True)[0]
    finally:
        _lib.stream_background(st, False)
    torch.cuda.current_stream(dev).wait_stream(st)
    for f in ("codes", "params", "consts", "sse", "comp"):
        assert torch.equal(getattr(got, f), getattr(ref, f)), f


def _shared_factor_batch(k, seed):
    """Five row groups over two factors in the order A A B A A (A in storage order, B in
    act order), 71 rows unpadded (sizes 5, 20, 9, 30, 7): workgroups of 16 rows and
    64-row tiles straddle groups of one factor and of two."""
    rng = np.random.default_rng(seed)
    sizes = [5, 20, 9, 30, 7]
    _, _, ua, _, _ = _layer(4, k, seed + 1)
    _, _, ub, perm_b, _ = _layer(4, k, seed + 2, act_order=True)
    which = [0, 0, 1, 0, 0]
    us = [(ua, ub)[w] for w in which]
    blks = [np.arange(k) // 32, np.arange(k) // 64, perm_b // 32, np.arange(k) // 16,
            np.arange(k) // 64]
    nmax = np.array([3, 15, 255, 15, 3], np.float32)
    n = sum(sizes)
    wc = (rng.standard_normal((n, k)) * 0.3).astype(np.float32)
    ldp = k // 16
    lo = (rng.standard_normal((n, ldp)) * 0.2 - 0.5).astype(np.float32)
    st = (rng.random((n, ldp)) * 0.1 + 0.01).astype(np.float32)
    row_grp = np.repeat(np.arange(5), sizes).astype(np.int32)
    return sizes, which, (ua, ub), us, np.stack(blks).astype(np.int32), nmax, wc, lo, st, row_grp


def test_groups_sharing_a_factor_share_passes(dev):
    """Consecutive row groups whose factor is one matrix (one address in u_ptrs: the row
    classes of one input) run as one pass of the column loop and of the cross-block tile
    update, each row with its own group's block map and highest code; a group of another
    factor in between splits the run.  hi2x_gptq_block against the oracle, and
    hi2x_gptq_run over the whole unpadded batch (K = 448: a short last block, two-block
    super-blocks) against one call per group, bit for bit."""
    from hi2_amd import _lib, gptq_kernel

    k, i1, length = 224, 128, 96
    sizes, which, (ua, ub), us, blk, nm, wc, lo, st, row_grp = _shared_factor_batch(k, 30)
    n = sum(sizes)
    err_w, codes_w, comp_w = oracle.gptq_block(wc, i1, length, lo, st, row_grp, us, blk, nm)
    uf = [T(ua, dev), T(ub, dev)]
    u_ptrs = torch.tensor([uf[w].data_ptr() for w in which], dtype=torch.int64, device=dev)
    err1 = torch.empty(n, length, dtype=torch.float32, device=dev)
    codes = torch.zeros(n, k, dtype=torch.uint8, device=dev)
    comp = torch.zeros(n, k, dtype=torch.float32, device=dev)
    gptq_kernel.gptq_block(T(wc, dev), i1, length, err1, codes, T(lo, dev), T(st, dev),
                           T(row_grp, dev), u_ptrs, T(blk, dev), T(nm, dev), comp)
    assert np.array_equal(N(err1), err_w)
    assert np.array_equal(N(codes), codes_w)
    assert np.array_equal(N(comp), comp_w)

    k, sb = 448, 2
    sizes, which, (ua, ub), us, blk, nm, wc, lo, st, row_grp = _shared_factor_batch(k, 40)
    n = sum(sizes)
    uf = [T(ua, dev), T(ub, dev)]

    def run(rows, grp, ptrs, blk_t, nm_t):
        m = rows.shape[0]
        # every device buffer is bound to a name until the launches have run (a temporary
        # would be freed once its address is taken, and its block handed to the next one)
        w, lo_t, st_t = T(wc[rows], dev), T(lo[rows], dev), T(st[rows], dev)
        grp_t, blk_d, nm_d = T(grp, dev), T(blk_t, dev), T(nm_t, dev)
        assert grp_t.shape == (m,) and int(grp_t.max()) < ptrs.numel() == blk_d.shape[0]
        out = torch.zeros(m, k, dtype=torch.uint8, device=dev)
        cmp = torch.zeros(m, k, dtype=torch.float32, device=dev)
        ws = torch.empty(m, 128 * sb, dtype=torch.float32, device=dev)
        _lib.call("hi2x_gptq_run", dev, _lib.ptr(w), m, k, _lib.ptr(out), _lib.ptr(lo_t),
                  _lib.ptr(st_t), k // 16, _lib.ptr(grp_t), _lib.ptr(ptrs), _lib.ptr(blk_d),
                  _lib.ptr(nm_d), _lib.ptr(cmp), _lib.ptr(ws), sb)
        torch.cuda.synchronize()
        return N(w), N(out), N(cmp)

    ptrs = torch.tensor([uf[w].data_ptr() for w in which], dtype=torch.int64, device=dev)
    whole = run(np.arange(n), row_grp, ptrs, blk, nm)
    off = 0
    for g, m in enumerate(sizes):
        rows = np.arange(off, off + m)
        one = run(rows, np.zeros(m, np.int32),
                  torch.tensor([uf[which[g]].data_ptr()], dtype=torch.int64, device=dev),
                  blk[g:g + 1], nm[g:g + 1])
        for a, b in zip(whole, one):
            assert np.array_equal(a[off:off + m], b), g
        off += m


def test_batched_jobs_match_one_call_each(dev, monkeypatch):
    # reference tests/test_gptq_fast.py:58-72: several row chunks and batches, two widths
    import hi2_amd.hessian as hm

    monkeypatch.setattr(hm, "ROW_ELEMS", 256 * 5)
    monkeypatch.setattr(hm, "BATCH_ELEMS", 256 * 23)
    jobs, refs = [], []
    for i, (nb, b) in enumerate(CASES):
        k = 256 if i % 3 else 128
        w, d, u, perm, _ = _layer(13 + i, k, i, act_order=i % 2 == 1)
        jobs.append(hm.GptqJob(T(w, dev), T(d, dev), T(u, dev), nb, b,
                               None if perm is None else T(perm, dev)))
        refs.append(oracle.encode_rows_gptq(w, d, u, nb, b, "fast", perm))
    for got, ref in zip(hm.encode_jobs_gptq(jobs, "fast", comp=True), refs):
        _same(got, ref)


def test_lone_chunk_at_an_offset_leaves_the_job_rows_alone(dev, monkeypatch):
    """An fp32 job cut into row chunks where a chunk at s > 0 runs alone in its batch
    (K = 256, 40 rows, 16 rows per chunk, one chunk per batch): the chunk's working copy
    must be a copy (hi2/hessian.py:211 clones), not a view of the job's rows that the
    column loop would overwrite with compensated values.  Codes, sse and comp equal the
    oracle bit for bit, and the job's w is unchanged."""
    import hi2_amd.hessian as hm

    monkeypatch.setattr(hm, "ROW_ELEMS", 256 * 16)
    monkeypatch.setattr(hm, "BATCH_ELEMS", 256 * 16)
    w, d, u, _, _ = _layer(40, 256, 9)
    wt = T(w, dev)
    before = wt.clone()
    got = hm.encode_rows_gptq(wt, T(d, dev), T(u, dev), 4, 32, "normal", comp=True)
    assert torch.equal(wt, before), "the caller's rows were modified"
    _same(got, oracle.encode_rows_gptq(w, d, u, 4, 32, "normal"))


@pytest.mark.parametrize("scale", [3e-31, 1e-39])
def test_tiny_rows_take_the_exact_division_path(dev, scale):
    """Rows whose error quotients fall outside the reciprocal iteration's exact range
    (numerators below 2^-100: tiny weights, 3e-31 normal and 1e-39 subnormal) next to
    ordinary rows in the same waves: the column loop's flagged waves run the block again
    with IEEE division, and codes, sse and comp equal the oracle (IEEE) bit for bit."""
    w, d, u, _, _ = _layer(48, 256, 31)
    w[::3] *= np.float32(scale)
    got = _encode(dev, w, d, u)
    _same(got, oracle.encode_rows_gptq(w, d, u, 4, 64, "normal"))


@pytest.mark.parametrize("kind", ["huge", "tiny_step", "huge_step", "zero_rows"])
def test_rows_outside_the_column_loops_bounds_take_the_rerun(dev, kind):
    """The column loop keeps a wave on the reciprocal iteration only while its per-block
    bounds hold (|1 / step| <= 2^40, |lo| <= 2^40, |step| <= 2^32, 1 / U[c][c] in
    [2^-50, 2^50]) and its per-step ones (|num| in [2^-50, 2^50] or num = +0).  Rows that
    break them, next to ordinary rows in the same waves, and rows of exact zeros (num = +0
    at every step, which must not need the rerun): codes, params, sse and comp equal the
    oracle (IEEE division) bit for bit.  Rows beyond fp16's range overflow the rounded
    value wq to infinity, in the oracle as here: their sse and comp are NaN in the same
    places (compared with NaN equal to NaN)."""
    w, d, u, _, _ = _layer(48, 256, 37)
    rng = np.random.default_rng(41)
    if kind == "huge":  # ladder origins and steps beyond 2^40
        w[::3] *= np.float32(2.0 ** 45)
    elif kind == "tiny_step":  # near-constant blocks: steps below 2^-40 (1 / step above)
        w[1::3] = np.float32(0.75) + rng.standard_normal(w[1::3].shape).astype(np.float32) * np.float32(2.0 ** -46)
    elif kind == "huge_step":  # steps beyond 2^32 with origins below 2^40
        w[2::3] = (rng.standard_normal(w[2::3].shape) * 2.0 ** 36).astype(np.float32)
    else:
        w[::4] = 0.0
    got = _encode(dev, w, d, u)
    want = oracle.encode_rows_gptq(w, d, u, 4, 64, "normal")
    if kind in ("huge", "huge_step"):
        assert np.array_equal(N(got.codes), want["codes"])
        assert np.array_equal(N(got.params), want["params"])
        assert np.array_equal(N(got.consts).view(np.int16), want["consts"].view(np.int16))
        assert np.array_equal(N(got.sse), want["sse"], equal_nan=True)
        assert np.array_equal(N(got.comp), want["comp"], equal_nan=True)
        assert np.isnan(want["sse"]).any()  # the overflow does happen
    else:
        _same(got, want)


def _encode(dev, w, d, u):
    from hi2_amd.hessian import encode_rows_gptq

    return encode_rows_gptq(T(w, dev), T(d, dev), T(u, dev), 4, 64, "normal", comp=True)


def test_nearest_encode_rows_equals_oracle(dev):
    """encode_rows (ladder fit, params, hi2x_nearest_codes, the finish's sse) against the
    oracle's nearest rounding, with zero-step blocks (constant rows) among them."""
    from hi2_amd.encode import encode_rows

    rng = np.random.default_rng(3)
    w = (rng.standard_normal((40, 256)) * np.exp(rng.standard_normal((1, 256)))).astype(np.float32)
    w[5] = 0.25
    w[7, :64] = -1.5
    d = (rng.random(256) + 0.1).astype(np.float32)
    want = oracle.encode_rows(w, d, 2, 32, "fast")
    got = encode_rows(T(w, dev), T(d, dev), 2, 32, "fast")
    _same(got, {**want, "comp": None})


@pytest.mark.parametrize("tag,spec", [("int2", (2, 32, 0, 96)), ("int4", (4, 64, 96, 192)),
                                      ("int8", (8, 64, 192, 224))])
def test_nearest_encode_rows_equals_reference_golden(dev, tag, spec):
    """encode_rows against hi2.encode.encode_rows itself (tests/golden/nearest.npz)."""
    import os

    from hi2_amd.encode import encode_rows

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "nearest.npz"))
    nb, b, a, z = spec
    got = encode_rows(T(g["wt"][a:z], dev), T(g["d"], dev), nb, b, "normal")
    assert np.array_equal(N(got.codes), g[f"{tag}_codes"])
    assert np.array_equal(N(got.params), g[f"{tag}_params"])
    assert np.array_equal(N(got.consts).view(np.int16), g[f"{tag}_consts"])
    assert np.array_equal(N(got.sse), g[f"{tag}_sse"])


# ---- ladder, params, finish -------------------------------------------------------------
@pytest.mark.parametrize("n,b,effort", [(4, 16, "normal"), (16, 32, "max"), (256, 64, "fast"),
                                        (4, 64, "normal")])
def test_fit_ladder_equals_oracle(dev, n, b, effort):
    from hi2_amd.encode import fit_ladder

    rng = np.random.default_rng(n + b)
    wb = (rng.standard_normal((101, 640 // b * 4, b)) * np.exp(rng.standard_normal((101, 1, 1)))).astype(np.float32)
    db = (rng.random((1, wb.shape[1], b)) + 0.5).astype(np.float32)
    lo_w, st_w = oracle.fit_ladder(wb, db, n, effort)
    lo, st = fit_ladder(T(wb, dev), T(db, dev), n, effort)
    assert np.array_equal(N(lo), lo_w) and np.array_equal(N(st), st_w)


@pytest.mark.parametrize("n,b", [(4, 64), (16, 32), (256, 64)])
def test_fit_ladder_ties_equal_oracle(dev, n, b):
    """Weights on the midpoints between ladder levels: (w - lo) / step lands on (or next to)
    half-integers for the first grid candidates, where rounding the quotient to a code
    must follow the IEEE division exactly (the kernel's reciprocal shortcut falls back to
    the division there)."""
    from hi2_amd.encode import fit_ladder

    rng = np.random.default_rng(n * b)
    rows, nb = 64, 640 // b
    h = np.float32(2.0) ** rng.integers(-8, 3, (rows, nb, 1)).astype(np.float32)
    k = rng.integers(0, n - 1, (rows, nb, b)).astype(np.float32)
    wb = ((k + np.float32(0.5)) * h).astype(np.float32)
    wb[:, :, 0] = 0.0                        # lo = 0 on the first candidate
    wb[:, :, 1] = np.float32(n - 1) * h[:, :, 0]  # span = (n - 1) h: step = h
    wb[::3] += rng.standard_normal(wb[::3].shape).astype(np.float32) * np.float32(1e-6)
    db = (rng.random((1, nb, b)) + 0.5).astype(np.float32)
    for effort in ("fast", "normal"):
        lo_w, st_w = oracle.fit_ladder(wb, db, n, effort)
        lo, st = fit_ladder(T(wb, dev), T(db, dev), n, effort)
        assert np.array_equal(N(lo), lo_w) and np.array_equal(N(st), st_w), effort


@pytest.mark.parametrize("b", [16, 32, 64])
def test_fit_ladder_extremes_equal_oracle(dev, b):
    """Blocks whose min / max are repeated, signed zeros or at the block's first element:
    the fit's span comes from a sequential scan with strict comparisons (the first
    element equal to the extreme), which the two-lane kernel rebuilds from each lane's
    scan and the element positions.  Also all-zero, constant and two-valued blocks, where
    every candidate's step is zero or the refit's determinant vanishes."""
    from hi2_amd.encode import fit_ladder

    rng = np.random.default_rng(b)
    rows, nb = 48, 640 // b
    wb = (rng.standard_normal((rows, nb, b)) * 0.02).astype(np.float32)
    for r in range(rows):
        for j in range(nb):
            kind = (r * nb + j) % 8
            blk = wb[r, j]
            if kind == 0:    # +0 and -0 as the minimum at several positions
                blk[:] = np.abs(blk)
                blk[rng.choice(b, 3, replace=False)] = np.float32(-0.0)
                blk[rng.choice(b, 2, replace=False)] = np.float32(0.0)
            elif kind == 1:  # -0 and +0 as the maximum
                blk[:] = -np.abs(blk)
                blk[rng.choice(b, 2, replace=False)] = np.float32(0.0)
                blk[rng.choice(b, 2, replace=False)] = np.float32(-0.0)
            elif kind == 2:  # the extremes at element 0 and repeated later
                blk[0] = blk.min() - np.float32(0.01)
                blk[rng.choice(np.arange(1, b), 3, replace=False)] = blk[0]
            elif kind == 3:  # all zeros, mixed signs
                blk[:] = np.where(rng.random(b) < 0.5, np.float32(0.0), np.float32(-0.0))
            elif kind == 4:  # constant
                blk[:] = np.float32(0.013)
            elif kind == 5:  # two values
                blk[:] = np.where(rng.random(b) < 0.5, np.float32(-0.01), np.float32(0.02))
            elif kind == 6:  # the extremes in the last positions of each lane's half
                blk[b - 1] = np.float32(0.5)
                blk[3] = np.float32(-0.5)
                blk[7] = np.float32(-0.5)
    db = (rng.random((1, nb, b)) + 0.5).astype(np.float32)
    for n in (4, 16, 256):
        for effort in ("fast", "normal"):
            lo_w, st_w = oracle.fit_ladder(wb, db, n, effort)
            lo, st = fit_ladder(T(wb, dev), T(db, dev), n, effort)
            lo, st = N(lo), N(st)
            assert np.array_equal(lo.view(np.uint32), lo_w.view(np.uint32)), (n, effort)
            assert np.array_equal(st.view(np.uint32), st_w.view(np.uint32)), (n, effort)


@pytest.mark.parametrize("b", [16, 32, 64])
def test_fit_ladder_subnormal_steps_equal_oracle(dev, b):
    """Blocks whose spans are so small that the candidate steps span / nm are subnormal
    (their reciprocals overflow): the kernels take the IEEE division for those codes.  The
    fit's outputs equal the oracle's bit for bit (its errors underflow to zero there, so
    the first candidate wins; the host check of divrcp.h covers the codes themselves)."""
    from hi2_amd.encode import fit_ladder

    rng = np.random.default_rng(1000 + b)
    rows, nb = 32, 640 // b
    tiny = np.float32(2.0) ** -140  # subnormal unit
    base = np.where(rng.random((rows, nb, 1)) < 0.5, np.float32(0.0),
                    np.float32(2.0) ** rng.integers(-135, -117, (rows, nb, 1)).astype(np.float32))
    wb = (base + rng.integers(0, 1 << 12, (rows, nb, b)).astype(np.float32) * tiny)
    wb = (wb * np.where(rng.random((rows, nb, 1)) < 0.5, 1, -1)).astype(np.float32)
    db = (rng.random((1, nb, b)) + 0.5).astype(np.float32)
    for n in (4, 16, 256):
        for effort in ("fast", "normal"):
            lo_w, st_w = oracle.fit_ladder(wb, db, n, effort)
            lo, st = fit_ladder(T(wb, dev), T(db, dev), n, effort)
            lo, st = N(lo), N(st)
            assert np.array_equal(lo.view(np.uint32), lo_w.view(np.uint32)), (n, effort)
            assert np.array_equal(st.view(np.uint32), st_w.view(np.uint32)), (n, effort)
            assert np.isfinite(lo).all() and np.isfinite(st).all()


def test_params_equal_oracle(dev):
    from hi2_amd.encode import params_decoded, quantize_params
    from hi2_amd.format import decode_params

    rng = np.random.default_rng(4)
    lo = (rng.standard_normal((300, 70)) * 0.4).astype(np.float32)
    st = (rng.random((300, 70)) * 0.05).astype(np.float32)
    st[10] = 0
    st[11, ::2] = -0.01
    lo[12] = -0.125
    want = oracle.params(lo, st)
    got = params_decoded(T(lo, dev), T(st, dev))
    for g, w in zip(got, want):
        g = N(g)
        assert np.array_equal(g.view(w.dtype) if g.dtype == np.float16 else g, w)
    lo_u8, st_u8, consts = quantize_params(T(lo, dev), T(st, dev))
    dl, ds = decode_params(lo_u8, st_u8, consts[:, 0:1], consts[:, 1:2], consts[:, 2:3])
    assert np.array_equal(N(dl).astype(np.float32), want[3])
    assert np.array_equal(N(ds).astype(np.float32), want[4])


# ---- format ------------------------------------------------------------------------------
def test_fwht_equals_oracle_and_is_an_involution(dev):
    from hi2_amd.format import fwht_groups

    rng = np.random.default_rng(1)
    x = (rng.standard_normal((333, 512)) * np.exp(rng.standard_normal((333, 512)))).astype(np.float32)
    fl = rng.integers(0, 2, 32).astype(np.uint8)
    y = fwht_groups(T(x, dev), T(fl, dev))
    assert np.array_equal(N(y), oracle.fwht16(x, fl))
    back = fwht_groups(y.double(), T(fl, dev))  # y carries fp32 rounding
    xd = T(x, dev).double()
    assert torch.allclose(back, xd, rtol=1e-5, atol=1e-6 * float(xd.abs().max()))
    xb = T(x, dev).to(torch.bfloat16)  # non-fp32 input: float64 work, cast back
    yb = fwht_groups(xb, T(fl, dev))
    assert yb.dtype == torch.bfloat16
    with pytest.raises(ValueError):
        fwht_groups(T(x[:, :24], dev), T(fl[:1], dev))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotate_rows_equals_cast_scale_fwht_select(dev, dtype):
    """rotate_rows(w, flags, rows, s) == fwht_groups(w.float() * s, flags)[rows] bit for
    bit (the product one fp32 rounding), against the oracle's fwht16; rows repeated and
    out of order, a strided row view, no rows (every row), no flags (no transform)."""
    from hi2_amd.format import rotate_rows

    rng = np.random.default_rng(5)
    n, k = 300, 768
    x = (rng.standard_normal((n, k)) * np.exp(rng.standard_normal((n, 1)))).astype(np.float32)
    w = T(x, dev).to(dtype)
    wf = N(w.float())
    fl = rng.integers(0, 2, k // 16).astype(np.uint8)
    cs = (rng.random(k) + 0.5).astype(np.float32)
    rows = rng.integers(0, n, 257).astype(np.int64)
    rows[:5] = [3, 3, n - 1, 0, 7]
    got = rotate_rows(w, T(fl, dev), T(rows, dev), T(cs, dev))
    assert np.array_equal(N(got), oracle.fwht16((wf * cs)[rows], fl))
    got = rotate_rows(w, T(fl, dev))
    assert np.array_equal(N(got), oracle.fwht16(wf, fl))
    got = rotate_rows(w, None, torch.from_numpy(rows))  # host rows: range-checked
    assert np.array_equal(N(got), wf[rows])
    wide = torch.zeros(n, k + 64, dtype=dtype, device=dev)
    wide[:, :k] = w
    got = rotate_rows(wide[:, :k], T(fl, dev), T(rows, dev))
    assert np.array_equal(N(got), oracle.fwht16(wf[rows], fl))
    with pytest.raises(IndexError):
        rotate_rows(w, T(fl, dev), torch.tensor([0, n]))
    bad = rotate_rows(w, T(fl, dev), T(np.array([1, n, -1], np.int64), dev))
    assert np.isnan(N(bad[1:])).all() and np.array_equal(N(bad[:1]), oracle.fwht16(wf[1:2], fl))


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_pack_and_assemble_equal_oracle(dev, nbits):
    from hi2_amd.format import assemble, pack_codes

    rng = np.random.default_rng(nbits)
    codes = rng.integers(0, 2**nbits, (37, 256)).astype(np.uint8)
    assert np.array_equal(N(pack_codes(T(codes, dev), nbits)), oracle.pack_codes(codes, nbits))
    if nbits < 8:
        bad = codes.copy()
        bad[3, 7] = 2**nbits
        with pytest.raises(ValueError):
            pack_codes(T(bad, dev), nbits)
    k, r = 128, 9
    row_nbits = rng.choice([2, 4, 8], r)
    row_block = rng.choice([16, 32, 64], r)
    pieces_np, pieces = [], []
    for nb in (2, 4, 8):
        for b in (16, 32, 64):
            rows = np.nonzero((row_nbits == nb) & (row_block == b))[0]
            if not rows.size:
                continue
            c = rng.integers(0, 2**nb, (rows.size, k)).astype(np.uint8)
            p = rng.integers(0, 256, (rows.size, k // b, 2)).astype(np.uint8)
            rc = rng.standard_normal((rows.size, 3)).astype(np.float16)
            pieces_np.append((rows, c, p, rc.view(np.uint16)))
            pieces.append((T(rows, dev), T(c, dev), T(p, dev), T(rc, dev)))
    want = oracle.assemble(pieces_np, row_nbits, row_block, k)
    got = assemble(pieces, torch.from_numpy(row_nbits), torch.from_numpy(row_block),
                   torch.zeros(k // 16, dtype=torch.uint8), k)
    assert np.array_equal(got.codes.numpy(), want["codes"])
    assert np.array_equal(got.blk_params.numpy(), want["blk_params"])
    assert np.array_equal(got.row_consts.numpy().view(np.uint16), want["row_consts"])
    assert np.array_equal(got.code_off.numpy(), want["code_off"])
    assert np.array_equal(got.param_off.numpy(), want["param_off"])


def test_assemble_many_equals_assemble_per_tensor(dev):
    """The batched packing of several tensors (hi2x_assemble_batch: one call for every
    piece of every tensor) equals assemble on each tensor, field by field."""
    from hi2_amd.format import assemble, assemble_many

    rng = np.random.default_rng(2)
    tensors = []
    for ti, (r, k) in enumerate(((37, 256), (64, 128), (20, 512))):
        perm = rng.permutation(r)
        cuts = [(2, 32, perm[: r // 3]), (4, 64, perm[r // 3: 2 * r // 3]), (8, 64, perm[2 * r // 3:])]
        nbits = np.zeros(r, np.int64)
        block = np.zeros(r, np.int64)
        pieces = []
        for nb, b, rows in cuts:
            rows = np.sort(rows)
            nbits[rows] = nb
            block[rows] = b
            codes = rng.integers(0, 2 ** nb, (rows.size, k)).astype(np.uint8)
            params = rng.integers(0, 256, (rows.size, k // b, 2)).astype(np.uint8)
            consts = rng.standard_normal((rows.size, 3)).astype(np.float16)
            pieces.append((torch.from_numpy(rows), T(codes, dev), T(params, dev),
                           T(consts, dev)))
        tensors.append(dict(pieces=pieces, row_nbits=torch.from_numpy(nbits),
                            row_block=torch.from_numpy(block),
                            had=torch.ones(k // 16, dtype=torch.uint8), k=k))
    many = assemble_many(tensors)
    for t, got in zip(tensors, many):
        want = assemble(t["pieces"], t["row_nbits"], t["row_block"], t["had"], t["k"])
        for f in ("codes", "code_off", "blk_params", "param_off", "row_nbits", "row_block",
                  "had"):
            assert torch.equal(getattr(got, f), getattr(want, f)), f
        assert torch.equal(got.row_consts.view(torch.int16), want.row_consts.view(torch.int16))
        assert got.shape == want.shape


def _offset_copy(a: np.ndarray, dev, shift: int):
    """A device copy of a that starts `shift` bytes into its allocation (misaligned for
    shift % 16 != 0)."""
    flat = torch.zeros(a.nbytes + shift, dtype=torch.uint8, device=dev)
    flat[shift:] = T(np.ascontiguousarray(a).view(np.uint8).reshape(-1), dev)
    return flat[shift:].view(getattr(torch, a.dtype.name)).view(a.shape)


def test_assemble_batch_over_many_launches_and_misaligned_pieces(dev):
    """hi2x_assemble_batch with more pieces than one launch carries (40 pieces of three
    tensors, K up to 14336: several workgroups per row), some pieces' codes and ladder
    bytes starting off their vector boundaries (the byte-load path), against the oracle's
    assemble of each tensor."""
    from hi2_amd.format import assemble_many

    rng = np.random.default_rng(7)
    tensors, want = [], []
    for ti, (r, k) in enumerate(((48, 4096), (40, 960), (32, 14336))):
        nbits = np.zeros(r, np.int64)
        block = np.zeros(r, np.int64)
        pieces, pieces_np = [], []
        order = rng.permutation(r)
        for pi, rows in enumerate(np.array_split(order, 14 if ti == 0 else 13)):
            rows = np.sort(rows)
            nb = int(rng.choice([2, 4, 8]))
            b = int(rng.choice([16, 32, 64]))
            nbits[rows] = nb
            block[rows] = b
            c = rng.integers(0, 2 ** nb, (rows.size, k)).astype(np.uint8)
            p = rng.integers(0, 256, (rows.size, k // b, 2)).astype(np.uint8)
            rc = rng.standard_normal((rows.size, 3)).astype(np.float16)
            pieces_np.append((rows, c, p, rc.view(np.uint16)))
            shift = (pi % 3) * 5  # 0: aligned; 5, 10: off the 16-byte and 2-byte grids
            pieces.append((torch.from_numpy(rows), _offset_copy(c, dev, shift),
                           _offset_copy(p, dev, shift), T(rc, dev)))
        tensors.append(dict(pieces=pieces, row_nbits=torch.from_numpy(nbits),
                            row_block=torch.from_numpy(block),
                            had=torch.ones(k // 16, dtype=torch.uint8), k=k))
        want.append(oracle.assemble(pieces_np, nbits, block, k))
    assert sum(len(t["pieces"]) for t in tensors) == 40
    for got, w in zip(assemble_many(tensors), want):
        assert np.array_equal(got.codes.numpy(), w["codes"])
        assert np.array_equal(got.blk_params.numpy(), w["blk_params"])
        assert np.array_equal(got.row_consts.numpy().view(np.uint16), w["row_consts"])
        assert np.array_equal(got.code_off.numpy(), w["code_off"])
        assert np.array_equal(got.param_off.numpy(), w["param_off"])


# ---- Hessian, transform, factor --------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("t,k", [(700, 320), (4096, 256)])
def test_hessian_stats_equal_xtx(dev, dtype, t, k):
    from hi2_amd.hessian import HessianStats

    rng = np.random.default_rng(t + k)
    x = (rng.standard_normal((t, k)) * np.exp(rng.standard_normal((1, k)))).astype(np.float32)
    x[:, 3] *= 20  # outlier channel
    xt = T(x, dev).to(dtype)
    st = HessianStats(k, dev)
    st.update(xt[: t // 3])
    other = HessianStats(k, dev)
    other.update(xt[t // 3:])
    st.merge(other)
    assert st.n == t
    xd = xt.double().cpu().numpy()
    want = xd.T @ xd
    got = N(st.S).astype(np.float64)
    assert np.array_equal(N(st.S), N(st.S).T)  # exactly symmetric
    # f32 accumulation of exact products over t terms
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
    assert torch.allclose(st.mean(), st.S / t)


@pytest.mark.parametrize("k,t0,t", [(8448, 256, 640), (8448, 1024, 2560), (4096, 1536, 3584)])
def test_hessian_stats_large_k_super_schedule(dev, k, t0, t):
    """K = 8448 (33 tiles of 256, 561 upper tiles): the bf16 SYRK runs its super-tile
    schedule and accumulates into a nonzero S (two updates); with 1024 and 1536 tokens per
    update the 49 tiles past the last whole round of 256 run token-split in a launch of
    their own, their partials summed into S afterwards.  K = 4096 (136 tiles): the token
    range split three ways.  Checked against X^T X in float64 on the device (bf16
    products are exact, the sums are f32)."""
    from hi2_amd.hessian import HessianStats

    print(f"hessian k={k} tokens {t0} + {t - t0}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    x = (torch.randn(t, k, device=dev, generator=g)
         * torch.exp(torch.randn(1, k, device=dev, generator=g))).to(torch.bfloat16)
    st = HessianStats(k, dev)
    st.update(x[:t0])
    st.update(x[t0:])
    xd = x.double()
    want = xd.T @ xd
    got = st.S.double()
    assert torch.equal(st.S, st.S.T)
    # the tolerance of the other Hessian tests (f32 sums of exact products over t terms)
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-4 * want.abs().max().item())
    # the diagonal sums positive terms only: relative agreement entry by entry
    dg = torch.diagonal(got), torch.diagonal(want)
    assert ((dg[0] - dg[1]).abs() / dg[1]).max().item() < 1e-5


@pytest.mark.parametrize("smooth", [False, True])
def test_transform_sigma_equals_oracle(dev, smooth):
    from hi2_amd.hessian import transform_sigma

    rng = np.random.default_rng(2)
    k = 320
    a = rng.standard_normal((k, k)).astype(np.float32)
    sigma = (a @ a.T / k).astype(np.float32)
    sigma = (sigma + sigma.T) / 2
    had = rng.integers(0, 2, k // 16).astype(np.uint8)
    cs = (rng.random(k) * 2 + 0.3).astype(np.float16) if smooth else None
    want = oracle.transform_sigma(sigma, None if cs is None else cs.view(np.uint16), had)
    got = transform_sigma(T(sigma, dev), None if cs is None else T(cs, dev), T(had, dev))
    assert np.array_equal(N(got), want)


@pytest.mark.parametrize("k", [48, 320, 1040])
@pytest.mark.parametrize("smooth", [False, True])
def test_transformed_equals_transform_of_mean(dev, k, smooth):
    """HessianStats.transformed (one pass over the upper triangle of S, no mirror) equals
    the oracle's transform of S / n and transform_sigma(mean()) bit for bit: K not a
    multiple of the 64-wide tiles, n not a power of two, mixed Hadamard flags."""
    from hi2_amd.hessian import HessianStats, transform_sigma

    rng = np.random.default_rng(k + smooth)
    t = 777
    x = (rng.standard_normal((t, k)) * np.exp(rng.standard_normal((1, k)))).astype(np.float32)
    xb = T(x, dev).to(torch.bfloat16)
    had = rng.integers(0, 2, k // 16).astype(np.uint8)
    cs = (rng.random(k) * 2 + 0.3).astype(np.float16) if smooth else None
    cs_d = None if cs is None else T(cs, dev)
    st = HessianStats(k, dev)
    st.update(xb[:300])
    st.update(xb[300:])
    got = st.transformed(cs_d, T(had, dev))
    assert st._upper_only  # S has not been mirrored for it
    s_full = N(st.S)
    assert np.array_equal(s_full, s_full.T)
    mean = s_full / np.float32(t)
    assert np.array_equal(N(st.mean()), mean)  # IEEE division, as the reference's CPU mean
    want = oracle.transform_sigma(mean, None if cs is None else cs.view(np.uint16), had)
    assert np.array_equal(N(got), want)
    assert torch.equal(got, transform_sigma(st.mean(), cs_d, T(had, dev)))


def test_upper_update_then_mirror_equals_full_update(dev):
    """hi2x_hessian_syrk_upper + the mirror on first read of S == hi2x_hessian_syrk."""
    from hi2_amd import _lib
    from hi2_amd.hessian import HessianStats

    k, t = 1040, 500
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(t, k, device=dev, generator=g).to(torch.bfloat16)
    st = HessianStats(k, dev)
    st.update(x)
    full = torch.zeros(k, k, device=dev)
    ws = _lib.workspace(dev, "hi2x_hessian_workspace_bytes", 2, t, k)
    _lib.call("hi2x_hessian_syrk", dev, _lib.ptr(x), 2, t, k, _lib.ptr(full), _lib.ptr(ws),
              ws.numel())
    assert torch.equal(st.S, full)


@pytest.mark.parametrize("k", [16, 100, 1000, 4108, 8448])
def test_damping_lambda_equals_oracle(dev, k):
    """The damping term (hi2/hessian.py:75-79) bit for bit: torch's CPU reduction order
    of the strided diagonal, reproduced by the parallel step sums of diag_mean_kernel."""
    from hi2_amd import _lib

    rng = np.random.default_rng(k)
    d = ((rng.standard_normal(k) * np.exp(rng.standard_normal(k))) ** 2).astype(np.float32)
    hs = torch.diag(T(d, dev))
    lam = torch.zeros(1, dtype=torch.float32, device=dev)
    for a in (0, 2, 5):
        _lib.call("hi2x_chol_lambda", dev, _lib.ptr(hs), k, 0.01, a, _lib.ptr(lam))
        want = oracle.damp_lambda(np.diag(d), 0.01, a)
        assert N(lam)[0] == want, (a, N(lam)[0], want)


@pytest.mark.parametrize("k", [96, 320, 1000 - 1000 % 16])
def test_inverse_factor_inverts(dev, k):
    from hi2_amd.hessian import inverse_factor

    rng = np.random.default_rng(k)
    mix = rng.standard_normal((k, k)) * 0.15 + np.eye(k)
    x = rng.standard_normal((3 * k, k)) @ mix
    x *= np.exp(0.5 * rng.standard_normal((1, k)))
    hs = (x.T @ x / x.shape[0]).astype(np.float32)
    u = N(inverse_factor(T(hs, dev), 0.01)).astype(np.float64)
    assert np.array_equal(np.tril(u, -1), np.zeros_like(u))
    assert (np.diag(u) > 0).all()
    damped = hs.astype(np.float64) + 0.01 * np.diag(hs).mean() * np.eye(k)
    assert np.allclose(u.T @ u @ damped, np.eye(k), atol=2e-3)
    u_o, _ = oracle.inverse_factor(hs, 0.01)
    scale = np.abs(u_o).max()
    assert np.allclose(u, u_o, rtol=1e-3, atol=2e-4 * scale)


def test_inverse_factor_inverts_large(dev):
    """K = 8448: every product of the top recursion levels runs the super-tile schedule
    of the large-grid path (4356 tiles); checked by U^T U (Hs + lam I) = I in float64 on
    the device (the CPU oracle would take minutes at this size)."""
    from hi2_amd.hessian import inverse_factor

    k = 8448
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(2 * k, k, device=dev, generator=g)
    x = x * torch.exp(0.5 * torch.randn(1, k, device=dev, generator=g))
    hs = (x.T.double() @ x.double() / x.shape[0]).float().contiguous()
    u = inverse_factor(hs, 0.01).double()
    assert torch.equal(torch.tril(u, -1), torch.zeros_like(u))
    assert bool((torch.diagonal(u) > 0).all())
    h = hs.double()
    damped = h + 0.01 * torch.diagonal(h).mean() * torch.eye(k, device=dev, dtype=torch.float64)
    r = u.T @ (u @ damped)
    err = (r - torch.eye(k, device=dev, dtype=torch.float64)).abs().max().item()
    assert err < 5e-3, err


@pytest.mark.parametrize("lo, hi", [(-40, 40), (40, 52)])
def test_inverse_factor_wide_channel_scales(dev, lo, hi):
    """K = 4096 with channel scales 2^u, u uniform in [lo, hi]: Hessian entries over a
    range of 2^160, or all large (up to ~2^107, operand rows whose largest element is above
    2^100, while the damping's diagonal sum stays finite in fp32).  The big products' operand rows are split into fp16
    planes after a power-of-two row scale, so every row of U keeps fp32-level accuracy
    relative to its own largest element.  Reference: the float64 inverse Cholesky factor
    of the same damped matrix (torch.linalg on the device)."""
    from hi2_amd.hessian import inverse_factor

    k = 4096
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(2 * k, k, device=dev, generator=g, dtype=torch.float64)
    x = x * torch.exp(0.5 * torch.randn(1, k, device=dev, generator=g, dtype=torch.float64))
    h0 = x.T @ x / x.shape[0]
    del x
    dsc = torch.exp2(torch.randint(lo, hi + 1, (k,), device=dev, generator=g).double())
    h = (dsc[:, None] * h0 * dsc[None, :]).float().contiguous()
    u = inverse_factor(h, 0.01).double()
    hd = h.double()
    hd = hd + 0.01 * torch.diagonal(hd).mean() * torch.eye(k, device=dev, dtype=torch.float64)
    rev = torch.arange(k - 1, -1, -1, device=dev)
    lo = torch.linalg.cholesky(hd[rev][:, rev])
    eye = torch.eye(k, device=dev, dtype=torch.float64)
    u64 = torch.linalg.solve_triangular(lo, eye, upper=False)[rev][:, rev]
    rel = ((u - u64).abs() / u64.abs().amax(dim=1, keepdim=True)).max().item()
    assert rel < 1e-5, rel


_FP32_FACTOR = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from hi2_amd.hessian import inverse_factor
h = torch.from_numpy(np.load(sys.argv[2])).cuda()
np.save(sys.argv[3], inverse_factor(h, 0.01).cpu().numpy())
"""


def test_inverse_factor_elementwise_on_decaying_rows(dev, tmp_path):
    """K = 4096 with channel scales rising smoothly over 2^16 across the columns, so each
    row of U = U_A D^-1 decays by up to 2^16 from its largest element.  The big products'
    fp16 split bounds their error by the operand rows' largest elements, not element by
    element: the entries of U above 2^-20 of their row's largest are compared one by one
    with the float64 factor, for the default (split) factor and for the fp32 MFMA one
    (HI2X_CHOL_FP32=1, read once per process, so in a child process).  Measured: both
    0.0032 at most and 4.6e-5 / 5.1e-5 at the 99.9th percentile over entries down to 2^-20
    of their row's largest: the split factor is as accurate element by element."""
    import os
    import subprocess
    import sys

    from hi2_amd.hessian import inverse_factor

    k = 4096
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(2 * k, k, device=dev, generator=g, dtype=torch.float64)
    h0 = x.T @ x / x.shape[0]
    del x
    dsc = torch.exp2(torch.linspace(0.0, 16.0, k, device=dev, dtype=torch.float64))
    h = (dsc[:, None] * h0 * dsc[None, :]).float().contiguous()
    del h0
    u = inverse_factor(h, 0.01).double()
    hd = h.double()
    hd = hd + 0.01 * torch.diagonal(hd).mean() * torch.eye(k, device=dev, dtype=torch.float64)
    rev = torch.arange(k - 1, -1, -1, device=dev)
    lo = torch.linalg.cholesky(hd[rev][:, rev])
    eye = torch.eye(k, device=dev, dtype=torch.float64)
    u64 = torch.linalg.solve_triangular(lo, eye, upper=False)[rev][:, rev]
    del lo, eye, hd
    hp, up = tmp_path / "h.npy", tmp_path / "u32.npy"
    np.save(hp, h.cpu().numpy())
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, HI2X_CHOL_FP32="1")
    r = subprocess.run([sys.executable, "-c", _FP32_FACTOR, root, str(hp), str(up)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    u32 = torch.from_numpy(np.load(up)).to(dev).double()
    rowmax = u64.abs().amax(dim=1, keepdim=True)
    live = u64.abs() >= rowmax * 2.0 ** -20
    decay = (rowmax / u64.abs().clamp_min(1e-300))[live].max().item()

    def elementwise(v):
        rel = ((v - u64).abs() / u64.abs().clamp_min(1e-300))[live]
        return rel.max().item(), torch.quantile(rel[:1 << 24].float(), 0.999).item()

    e_split, q_split = elementwise(u)
    e_fp32, q_fp32 = elementwise(u32)
    print(f"decay {decay:.3g}; elementwise rel. error max / 99.9 %: split {e_split:.3g} / "
          f"{q_split:.3g}, fp32 {e_fp32:.3g} / {q_fp32:.3g}")
    assert decay > 2.0 ** 12  # the rows do decay
    assert e_split < 2 * e_fp32 + 1e-6, (e_split, e_fp32)
    assert q_split < 2 * q_fp32 + 1e-7, (q_split, q_fp32)


def test_inverse_factor_256_tiles_equal_128_tiles(dev, monkeypatch):
    """K = 8448: the top level's three rectangular products (17 x 17 tiles of 256, the
    last row and column of tiles partial) run on the 256-tile kernel; with
    HI2X_CHOL_TILE256=0 every product runs on the 128-tiles.  Same terms in the same order
    per element: the factors are equal bit for bit."""
    from hi2_amd.hessian import inverse_factor

    k = 8448
    g = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn(2 * k, k, device=dev, generator=g)
    x = x * torch.exp(0.5 * torch.randn(1, k, device=dev, generator=g))
    hs = (x.T @ x / x.shape[0]).contiguous()
    del x
    u256 = inverse_factor(hs, 0.01)
    monkeypatch.setenv("HI2X_CHOL_TILE256", "0")
    u128 = inverse_factor(hs, 0.01)
    assert torch.equal(u256, u128)


_SPLIT_CASES = r"""
import hashlib
import sys
import torch
sys.path.insert(0, sys.argv[1])
from hi2_amd.hessian import inverse_factor, inverse_factors_batched


def hessian(k, seed, batch=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(max(batch, 1), 2 * k, k, device="cuda", generator=g)
    x = x * torch.exp(0.5 * torch.randn(max(batch, 1), 1, k, device="cuda", generator=g))
    hs = (torch.matmul(x.transpose(1, 2).contiguous(), x) / x.shape[1]).contiguous()
    return hs if batch else hs[0]


for k, seed, batch in ((8448, 21, 0), (6148, 22, 0), (4096, 23, 2)):
    hs = hessian(k, seed, batch)
    u = inverse_factors_batched(hs, 0.01) if batch else inverse_factor(hs, 0.01)
    torch.cuda.synchronize()
    print(k, batch, hashlib.sha256(u.cpu().numpy().tobytes()).hexdigest(), flush=True)
"""


def test_inverse_factor_one_pass_splits_equal_the_pair(tmp_path):
    """The split-plane products' row-major operands go through split_rows_kernel (rb rows
    per workgroup staged in LDS, maxima and planes in one pass), the transposed ones
    through rowmax_kernel + split2_kernel; HI2X_CHOL_SPLIT_ROWS=0 (read once per process,
    so in a child process each) sends every operand through the pair.  Same elements,
    maxima and conversions: the factors are equal bit for bit.  K = 8448 (the top level's
    operands 4 rows per workgroup, the next level's 8), K = 6148 (the top level's 2948-row
    operands at 8 rows per workgroup: the last row block partial) and a batch of two
    K = 4096 factors (8 rows per workgroup, two batch entries per launch)."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = {}
    for flag in ("1", "0"):
        env = dict(os.environ, HI2X_CHOL_SPLIT_ROWS=flag)
        print(f"factor digests, HI2X_CHOL_SPLIT_ROWS={flag}", flush=True)
        r = subprocess.run([sys.executable, "-c", _SPLIT_CASES, root], env=env,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        out[flag] = [line for line in r.stdout.splitlines() if line.strip()]
        print("\n".join(out[flag]), flush=True)
    assert len(out["1"]) == 3
    assert out["1"] == out["0"]


def test_inverse_factor_rejects_width_not_multiple_of_4(dev):
    """The factor's leaves move 16-byte vectors: a width that is not a multiple of 4 (no
    Hessian of the reference has one) is refused before any launch."""
    from hi2_amd.hessian import inverse_factor

    with pytest.raises(Exception, match="multiple of 4"):
        inverse_factor(torch.eye(30, device=dev), 0.01)


def test_inverse_factor_retries_and_survives_singular(dev):
    from hi2_amd.hessian import inverse_factor

    sing = torch.zeros(16, 16, device=dev)
    sing[0, 0] = 1.0
    assert torch.isfinite(inverse_factor(sing, 0.01)).all()
    ind = torch.eye(16, device=dev)
    ind[15, 15] = -0.2
    u = N(inverse_factor(ind, 0.01))
    u_o, att = oracle.inverse_factor(N(ind), 0.01)
    assert att == 2
    assert np.allclose(u, u_o, rtol=1e-5, atol=1e-6)


# ---- end to end: Hessian -> transform -> factor -> GPTQ -> pack ---------------------------
def test_small_config_end_to_end_against_oracle(dev):
    """cfg1 scaled down (512 x 512, 256 tokens): the GPU pipeline against the oracle
    pipeline.  The factor differs in rounding (LAPACK-free fp32 vs float64), so codes are
    compared at the north-star tolerance: >= 99.9 % equal."""
    from hi2_amd.format import assemble, fwht_groups
    from hi2_amd.hessian import HessianStats, encode_rows_gptq, inverse_factor, transform_sigma

    rng = np.random.default_rng(0)
    k, n, t = 512, 512, 256
    x = rng.standard_normal((t, k)).astype(np.float32)
    x[:, rng.permutation(k)[: k // 100 + 1]] *= 20
    xb = T(x, dev).to(torch.bfloat16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    had = np.ones(k // 16, np.uint8)
    st = HessianStats(k, dev)
    st.update(xb)
    hs = transform_sigma(st.mean(), None, T(had, dev))
    d = hs.diagonal().clone()
    u = inverse_factor(hs, 0.01)
    wt = fwht_groups(T(w, dev), T(had, dev))
    enc = encode_rows_gptq(wt, d, u, 4, 64, "normal")
    # oracle pipeline
    s = np.zeros((k, k), np.float32)
    oracle.hessian_update(s, N(xb.view(torch.int16)).view(np.uint16))
    hs_o = oracle.transform_sigma(s / np.float32(t), None, had)
    u_o, _ = oracle.inverse_factor(hs_o, 0.01)
    wt_o = oracle.fwht16(w, had)
    assert np.array_equal(N(wt), wt_o)
    want = oracle.encode_rows_gptq(wt_o, np.diag(hs_o).copy(), u_o, 4, 64, "normal")
    match = (N(enc.codes) == want["codes"]).mean()
    assert match >= 0.999, match
    sse_rel = np.abs(N(enc.sse) / want["sse"] - 1).max()
    assert sse_rel < 1e-2, sse_rel
    t_ = assemble([(torch.arange(n), enc.codes, enc.params, enc.consts)],
                  torch.full((n,), 4), torch.full((n,), 64), torch.from_numpy(had), k)
    assert t_.codes.numel() == n * k * 4 // 32
