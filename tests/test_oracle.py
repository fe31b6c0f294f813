"""The CPU oracle (oracle/) pinned against the reference's golden vectors, closed
forms, invariants and brute force — CPU only."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from golden_data import fit_cases, gptq_cases, inverse_cases


@pytest.fixture(scope="module", autouse=True)
def _one_thread():
    n = torch.get_num_threads()
    torch.set_num_threads(1)  # torch's reductions split across threads otherwise
    yield
    torch.set_num_threads(n)


def _tsum(x):
    L = oracle.lib()
    L.or_torch_sum.restype = ctypes.c_float
    L.or_torch_sum.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    x = np.ascontiguousarray(x, np.float32)
    return L.or_torch_sum(oracle._p(x), x.size)


# ---- number formats and reduction order -------------------------------------------------
def test_f16_conversion_is_ieee_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(4000) * np.exp2(rng.integers(-30, 17, 4000))).astype(np.float32),
        np.array([65504, 65519.99, 65520, 6.1e-5, 6.0e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0,
                  -0.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11], np.float32),
    ])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [16, 24, 32, 64, 192, 1024, 2048, 4096, 14336, 65536])
def test_sum_order_is_torch_cpu_order(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * np.exp(2 * rng.standard_normal(n))).astype(np.float32)
    assert _tsum(x) == torch.from_numpy(x).sum().item()


@pytest.mark.parametrize("n,stride", [(16, 17), (48, 49), (100, 101), (1000, 1001),
                                      (4108, 4109), (14336, 2), (65540, 3)])
def test_strided_sum_is_torch_cpu_order(n, stride):
    """The diagonal reduction of inverse_factor's damping (hi2/hessian.py:75) is torch's
    CPU sum of a strided vector: pinned against torch itself."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((n - 1) * stride + 1) * np.exp(2 * rng.standard_normal(1))).astype(np.float32)
    want = torch.as_strided(torch.from_numpy(x), (n,), (stride,)).sum().item()
    assert oracle.torch_sum_strided(x, n, stride) == np.float32(want)


@pytest.mark.parametrize("k", [16, 100, 1000, 4108])
def test_damp_lambda_is_the_reference_expression(k):
    # hi2/hessian.py:75-79: mean = hs.diagonal().mean().clamp_min(1e-12); damp*mean*10**a
    rng = np.random.default_rng(k)
    hs = (rng.standard_normal((k, k)) * 0.01).astype(np.float32)
    hs[np.diag_indices(k)] = (rng.standard_normal(k) * np.exp(rng.standard_normal(k))) ** 2
    mean = torch.from_numpy(hs).diagonal().mean().clamp_min(1e-12)
    for a in (0, 1, 3, 5):
        want = (0.01 * mean * 10**a).item()
        assert oracle.damp_lambda(hs, 0.01, a) == np.float32(want), a


# ---- fit_ladder / params ---------------------------------------------------------------
@pytest.mark.parametrize("case", list(fit_cases()), ids=lambda c: f"n{c[0]}_b{c[1]}_{c[2]}")
def test_fit_ladder_equals_reference_golden(case):
    n, b, effort, a = case
    lo, st = oracle.fit_ladder(a["wb"], a["db"], n, effort)
    assert np.array_equal(lo, a["lo"]) and np.array_equal(st, a["step"])


def _params_numpy(lo, step):
    """hi2/encode.py:95-119 and hi2/format.py:45-60 with numpy's IEEE ops."""
    f16 = lambda v: np.asarray(v, np.float32).astype(np.float16)  # noqa: E731
    step = np.maximum(step, np.float32(0))
    ss = f16(step.max(-1, keepdims=True) / np.float32(255)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        su = np.where(ss > 0, np.rint(step / np.maximum(ss, np.float32(1e-30))), 0)
    su = np.clip(su, 0, 255).astype(np.uint8)
    lm = f16(lo.min(-1, keepdims=True)).astype(np.float32)
    ls = f16(np.maximum(lo.max(-1, keepdims=True) - lm, 0) / np.float32(255)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        lu = np.where(ls > 0, np.rint((lo - lm) / np.maximum(ls, np.float32(1e-30))), 0)
    lu = np.clip(lu, 0, 255).astype(np.uint8)
    lo_d = f16((lu.astype(np.float64) * ls.astype(np.float64) + lm.astype(np.float64)).astype(np.float32))
    st_d = f16(su.astype(np.float32) * ss)
    consts = np.concatenate([f16(lm), f16(ls), f16(ss)], -1).view(np.uint16)
    return lu, su, consts, lo_d.astype(np.float32), st_d.astype(np.float32)


def test_params_equal_closed_form():
    rng = np.random.default_rng(3)
    lo = (rng.standard_normal((50, 37)) * 0.3).astype(np.float32)
    st = (rng.random((50, 37)) * 0.1).astype(np.float32)
    st[3] = 0.0
    st[5, ::3] = -1e-3
    lo[7] = 0.25
    got = oracle.params(lo, st)
    want = _params_numpy(lo, st)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_params_keep_constant_and_zero_blocks_exact():
    # reference tests/test_format.py:90-98
    lo = np.array([[0.5, -0.2, 0.1]], np.float32)
    step = np.array([[0.0, 0.03, 0.0]], np.float32)
    _, _, _, lo_d, st_d = oracle.params(lo, step)
    assert st_d[0, 0] == 0 and st_d[0, 2] == 0
    assert np.allclose(lo_d, lo, atol=2e-3)


# ---- GPTQ -----------------------------------------------------------------------------
@pytest.mark.parametrize(
    "case", list(gptq_cases()), ids=lambda c: f"int{c[0]}_b{c[1]}_{c[2]}_ao{int(c[3])}"
)
def test_gptq_equals_reference_golden(case):
    nbits, block, effort, _, a = case
    out = oracle.encode_rows_gptq(a["w"], a["d"], a["u"], nbits, block, effort, a["perm"])
    assert np.array_equal(out["codes"], a["codes"])
    assert np.array_equal(out["params"], a["params"])
    assert np.array_equal(out["consts"].view(np.int16), a["consts"])
    assert np.array_equal(out["sse"], a["sse"])
    assert np.array_equal(out["comp"], a["comp"])


def _correlated(t, k, seed):
    rng = np.random.default_rng(seed)
    mix = rng.standard_normal((k, k)) * 0.15 + np.eye(k)
    x = rng.standard_normal((t, k)) @ mix
    return (x * np.exp(0.5 * rng.standard_normal((1, k)))).astype(np.float32)


def _recon(out, block, k):
    n = out["codes"].shape[0]
    rec = (out["lo_d"].repeat(block, 1) + out["codes"].astype(np.float32)
           * out["step_d"].repeat(block, 1))
    return rec.astype(np.float16).astype(np.float64).reshape(n, k)


def test_diagonal_hessian_gives_nearest_rounding():
    # reference tests/test_hessian.py:107-115: with a diagonal H no error propagates
    rng = np.random.default_rng(2)
    k = 64
    w = rng.standard_normal((24, k)).astype(np.float32)
    d = (rng.random(k) + 0.5).astype(np.float32)
    u, _ = oracle.inverse_factor(np.diag(d), 0.0)
    got = oracle.encode_rows_gptq(w, d, u, 2, 32, "fast")
    lo, st = oracle.fit_ladder(w.reshape(24, 2, 32), d.reshape(1, 2, 32), 4, "fast")
    _, _, _, lo_d, st_d = oracle.params(lo, st)
    safe = np.where(st_d == 0, 1, st_d).repeat(32, 1)
    near = np.clip(np.rint((w - lo_d.repeat(32, 1)) / safe), 0, 3)
    near = np.where(st_d.repeat(32, 1) == 0, 0, near)
    assert np.array_equal(got["codes"], near.astype(np.uint8))


@pytest.mark.parametrize("nbits,block", [(2, 32), (2, 16), (4, 64)])
def test_compensation_lowers_the_hessian_error(nbits, block):
    # reference tests/test_hessian.py:83-104
    k, rows = 128, 48
    x = _correlated(6000, k, 1)
    hs = (x.T.astype(np.float64) @ x / x.shape[0]).astype(np.float32)
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((rows, k)) * np.exp(0.3 * rng.standard_normal((1, k)))).astype(np.float32)
    d = np.diag(hs).copy()
    u, _ = oracle.inverse_factor(hs, 0.01)
    comp = oracle.encode_rows_gptq(w, d, u, nbits, block, "fast")
    # a diagonal factor propagates no error: nearest rounding on the same ladders
    near = oracle.encode_rows_gptq(w, d, np.diag(1 / np.sqrt(d)).astype(np.float32), nbits,
                                   block, "fast")
    assert np.array_equal(comp["params"], near["params"])

    def herr(o):
        e = _recon(o, block, k) - w
        return float(((e @ hs) * e).sum())

    assert herr(comp) < herr(near) * 0.97


# ---- Hadamard ---------------------------------------------------------------------------
def _h16():
    i = np.arange(16)
    par = np.vectorize(lambda v: bin(v).count("1") & 1)(i[:, None] & i[None, :])
    return np.where(par, -0.25, 0.25)


def test_fwht_is_the_normalised_hadamard_and_an_involution():
    h = _h16()
    assert np.allclose(h @ h, np.eye(16))
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    fl = np.array([1, 0, 1, 1], np.uint8)
    y = oracle.fwht16(x, fl)
    assert np.array_equal(y[:, 16:32], x[:, 16:32])
    ref = (x.astype(np.float64).reshape(5, 4, 16) @ h).reshape(5, 64)
    assert np.allclose(y[:, :16], ref[:, :16], rtol=1e-6, atol=1e-6)
    assert np.allclose(oracle.fwht16(y, fl), x, atol=1e-5)
    ints = rng.integers(-50, 50, (3, 32)).astype(np.float32)  # every sum exact
    assert np.array_equal(oracle.fwht16(ints, np.ones(2, np.uint8)),
                          (ints.astype(np.float64).reshape(3, 2, 16) @ h).reshape(3, 32).astype(np.float32))
    with pytest.raises(ValueError):
        oracle.fwht16(x, fl[:3])


def test_fwht_order_is_the_reference_matmul_order():
    # the reference evaluates x @ H16 with torch's fp32 matmul (hi2/format.py:39)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((40, 64)) * np.exp(2 * rng.standard_normal((40, 64)))).astype(np.float32)
    fl = np.ones(4, np.uint8)
    want = (torch.from_numpy(x).reshape(40, 4, 16) @ torch.from_numpy(_h16()).float()).reshape(40, 64)
    assert np.array_equal(oracle.fwht16(x, fl), want.numpy())


# ---- Hessian accumulation and transform -----------------------------------------------------
@pytest.mark.parametrize("bf16", [False, True])
def test_hessian_update_is_xtx(bf16):
    x = _correlated(300, 48, 4)
    if bf16:
        xb = torch.from_numpy(x).to(torch.bfloat16)
        xin = xb.view(torch.int16).numpy().view(np.uint16)
        xd = xb.double().numpy()
    else:
        xin, xd = x, x.astype(np.float64)
    s = np.zeros((48, 48), np.float32)
    oracle.hessian_update(s, xin[:100])
    oracle.hessian_update(s, xin[100:])
    assert np.allclose(s, xd.T @ xd, rtol=1e-6, atol=1e-4)
    assert np.array_equal(s, s.T)


@pytest.mark.parametrize("smooth", [False, True])
@pytest.mark.parametrize("flags", [[0, 0, 0, 0], [1, 0, 1, 1]])
def test_transform_sigma_is_the_covariance_of_the_transformed_activation(smooth, flags):
    # reference tests/test_hessian.py:57-67
    x = _correlated(2000, 64, 0)
    fl = np.array(flags, np.uint8)
    rng = np.random.default_rng(9)
    s = (rng.random(64) * 2 + 0.5).astype(np.float16) if smooth else None
    xt = x / s.astype(np.float32) if smooth else x
    xt = xt.astype(np.float64).reshape(-1, 4, 16)
    xt = np.where(fl.astype(bool)[None, :, None], xt @ _h16(), xt).reshape(-1, 64)
    want = xt.T @ xt / x.shape[0]
    sigma = (x.T.astype(np.float64) @ x / x.shape[0]).astype(np.float32)
    got = oracle.transform_sigma(sigma, None if s is None else s.view(np.uint16), fl)
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3 * np.abs(want).max())
    assert np.array_equal(got, got.T)


def test_transform_sigma_order_is_the_reference_einsum_order():
    # hi2/hessian.py:57-68 evaluated by torch's fp32 einsum (the reference's own ops)
    rng = np.random.default_rng(11)
    k = 96
    a = rng.standard_normal((k, k)).astype(np.float32)
    sigma = (a @ a.T).astype(np.float32)
    cs = (rng.random(k) * 2 + 0.5).astype(np.float16)
    had = np.array([1, 0, 1, 1, 0, 1], np.uint8)
    s = torch.from_numpy(sigma)
    inv = 1.0 / torch.from_numpy(cs).float()
    s = s * inv[:, None] * inv[None, :]
    h = torch.from_numpy(_h16()).float()
    m = torch.where(torch.from_numpy(had).bool().reshape(-1, 1, 1), h, torch.eye(16))
    s4 = s.reshape(6, 16, 6, 16)
    s4 = torch.einsum("gij,gjhk->gihk", m, s4)
    s4 = torch.einsum("gihk,hlk->gihl", s4, m)
    s = s4.reshape(k, k)
    want = (0.5 * (s + s.T)).numpy()
    got = oracle.transform_sigma(sigma, cs.view(np.uint16), had)
    assert np.array_equal(got, want)


# ---- inverse_factor ------------------------------------------------------------------------
@pytest.mark.parametrize("case", list(inverse_cases()), ids=lambda c: c[0])
def test_inverse_factor_matches_reference_golden(case):
    tag, hs, u_ref = case
    u, att = oracle.inverse_factor(hs, 0.01)
    assert np.allclose(np.tril(u, -1), 0)
    scale = np.abs(u_ref).max()
    assert np.allclose(u, u_ref, rtol=1e-3, atol=1e-4 * scale), np.abs(u - u_ref).max() / scale


def test_inverse_factor_inverts_and_retries():
    # reference tests/test_hessian.py:70-80
    x = _correlated(500, 32, 0)
    hs = (x.T.astype(np.float64) @ x / 500).astype(np.float32)
    u, att = oracle.inverse_factor(hs, 0.01)
    assert att == 0
    damped = hs + 0.01 * np.diag(hs).mean() * np.eye(32)
    assert np.allclose(u.T.astype(np.float64) @ u @ damped, np.eye(32), atol=1e-3)
    sing = np.zeros((16, 16), np.float32)
    sing[0, 0] = 1
    u2, _ = oracle.inverse_factor(sing, 0.01)
    assert np.isfinite(u2).all()
    ind = np.eye(16, dtype=np.float32)
    ind[15, 15] = -0.2
    _, att3 = oracle.inverse_factor(ind, 0.01)
    assert att3 == 2  # lam = 0.00925 * 10^a first exceeds 0.2 at a = 2


# ---- packing ---------------------------------------------------------------------------------
@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_pack_is_lsb_first(nbits):
    # reference tests/test_format.py:41-49
    rng = np.random.default_rng(nbits)
    codes = rng.integers(0, 2**nbits, (5, 64)).astype(np.uint8)
    words = oracle.pack_codes(codes, nbits)
    per = 32 // nbits
    u = words.view(np.uint32)
    back = np.stack([(u >> (nbits * i)) & (2**nbits - 1) for i in range(per)], -1).reshape(5, 64)
    assert np.array_equal(back, codes)
    one = np.zeros((1, 32), np.uint8)
    one[0, 1] = 3 if nbits == 2 else 9
    assert int(oracle.pack_codes(one, nbits)[0, 0]) == int(one[0, 1]) << nbits
    if nbits < 8:  # reference tests/test_format.py:52-54
        with pytest.raises(ValueError):
            oracle.pack_codes(np.full((1, 16), 2**nbits, np.uint8), nbits)


def test_assemble_mixed_rows_offsets():
    # reference tests/test_format.py:113-133 (offset KAT)
    k = 128
    nbits = np.array([2, 4, 2, 4])
    block = np.array([32, 64, 64, 32])
    pieces = []
    rng = np.random.default_rng(0)
    for nb in (2, 4):
        for b in (32, 64):
            rows = np.nonzero((nbits == nb) & (block == b))[0]
            if rows.size:
                c = rng.integers(0, 2**nb, (rows.size, k)).astype(np.uint8)
                p = rng.integers(0, 256, (rows.size, k // b, 2)).astype(np.uint8)
                rc = rng.integers(0, 2**15, (rows.size, 3)).astype(np.uint16)
                pieces.append((rows, c, p, rc))
    t = oracle.assemble(pieces, nbits, block, k)
    assert t["code_off"].tolist() == [0, 8, 24, 32, 48]
    assert t["param_off"].tolist() == [0, 4, 6, 8, 12]
    assert t["codes"].size == 48 and t["blk_params"].size == 24
    for rows, c, p, rc in pieces:
        for i, r in enumerate(rows):
            nb = int(nbits[r])
            w0 = t["code_off"][r]
            assert np.array_equal(t["codes"][w0:w0 + k * nb // 32], oracle.pack_codes(c[i:i + 1], nb)[0])
            p0 = t["param_off"][r] * 2
            assert np.array_equal(t["blk_params"][p0:p0 + p[i].size], p[i].reshape(-1))
            assert np.array_equal(t["row_consts"][r], rc[i])


NEAREST_SPECS = {"int2": (2, 32, 0, 96), "int4": (4, 64, 96, 192), "int8": (8, 64, 192, 224)}


@pytest.mark.parametrize("tag", list(NEAREST_SPECS))
def test_encode_rows_equals_the_reference_nearest_golden(tag):
    """oracle.encode_rows against hi2.encode.encode_rows (tests/golden/nearest.npz):
    codes, params, consts and sse bit for bit; and it equals the GPTQ flow with an
    identity factor (no error is propagated), the identity the old nearest path used."""
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "nearest.npz"))
    nb, b, a, z = NEAREST_SPECS[tag]
    e = oracle.encode_rows(g["wt"][a:z], g["d"], nb, b, "normal")
    assert np.array_equal(e["codes"], g[f"{tag}_codes"])
    assert np.array_equal(e["params"], g[f"{tag}_params"])
    assert np.array_equal(e["consts"].view(np.int16), g[f"{tag}_consts"])
    assert np.array_equal(e["sse"], g[f"{tag}_sse"])
    k = g["wt"].shape[1]
    via = oracle.encode_rows_gptq(g["wt"][a:z], g["d"], np.eye(k, dtype=np.float32), nb, b,
                                  "normal")
    assert np.array_equal(via["codes"], e["codes"]) and np.array_equal(via["sse"], e["sse"])
