"""The oracle's QAD decode (``or_qad_*``) pinned to the reference's torch graph of the
fake-quantised Linear (``tests/golden/qad.npz`` from ``hi2.qad.FakeQuantLinear``): stored
values and latent gradients bit-exact, the per-block byte gradients and the original-basis
transform within float32 summation rounding; exact sums on integer-valued inputs (where the
order cannot matter); the butterfly against the H16 product in float64 — CPU only."""

import numpy as np
import pytest

import oracle
from golden_data import qad_cases

CASES = list(qad_cases())


def _stored(c):
    out = np.zeros_like(c["latent"])
    for g in c["groups"]:
        oracle.qad_decode_fwd(c["latent"], c["unit"], g["lo_u"], g["st_u"], g["consts"],
                              g["rows"], g["block"], g["nbits"], out)
    return out


def _bwd(c, grad):
    g_lat = np.zeros_like(c["latent"])
    out = []
    for g in c["groups"]:
        _, g_lo, g_st = oracle.qad_decode_bwd(grad, c["latent"], c["unit"], g["lo_u"], g["st_u"],
                                              g["consts"], g["rows"], g["block"], g["nbits"],
                                              g_lat)
        out.append((g_lo, g_st))
    return g_lat, out


def _close(a, b, rel):
    scale = float(np.abs(a).max()) + 1e-12
    return float(np.abs(a - b).max()) <= rel * scale


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_stored_values_and_gradients_equal_the_reference_torch_graph(case):
    tag, c = case
    assert np.array_equal(_stored(c), c["stored"])
    g_lat, per = _bwd(c, c["grad"])
    assert np.array_equal(g_lat, c["g_latent"])
    for g, (g_lo, g_st) in zip(c["groups"], per):
        # autograd sums the block in its own order: agreement to fp32 summation rounding
        assert _close(g["g_lo"], g_lo, 1e-5) and _close(g["g_st"], g_st, 1e-5)
    if tag == "clamp":  # clamped latents get no gradient, their blocks' bytes do
        assert not g_lat[:, :16].any()


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_original_basis_and_its_gradients_match_the_reference(case):
    _, c = case
    stored = _stored(c)
    orig = oracle.qad_wht_scale(stored, c["had"], c["col_scale"], False)
    assert _close(c["original"], orig, 1e-6)  # the torch path rotates with a matmul
    g = oracle.qad_wht_scale(c["grad2"], c["had"], c["col_scale"], True)
    g_lat, per = _bwd(c, g)
    assert _close(c["og_latent"], g_lat, 1e-5)
    for gr, (g_lo, g_st) in zip(c["groups"], per):
        assert _close(gr["og_lo"], g_lo, 1e-4) and _close(gr["og_st"], g_st, 1e-4)


def test_block_sums_are_exact_on_integer_inputs():
    """lo_scale = step_scale = 1 and lo_min = 0 make lo and step the bytes; integer latents
    and gradients make every term and partial sum an exact integer, so any order gives the
    float64 sum: a wrong block or lane index cannot hide."""
    rng = np.random.default_rng(3)
    for block in (16, 32, 64):
        n, k, nbits = 6, 256, 4
        nb = k // block
        latent = rng.integers(-4, 24, (n + 2, k)).astype(np.float32)
        rows = np.array([5, 0, 7, 2, 3, 1], np.int64)
        lo_u = rng.integers(0, 4, (n, nb)).astype(np.float32)
        st_u = np.ones((n, nb), np.float32)
        st_u[1, ::2] = 0.0  # zero-step blocks
        consts = np.tile(np.array([0, 0x3C00, 0x3C00], np.uint16), (n, 1))  # 0, 1.0, 1.0
        grad = rng.integers(-8, 9, (n + 2, k)).astype(np.float32)
        g_lat, g_lo, g_st = oracle.qad_decode_bwd(grad, latent, None, lo_u, st_u, consts, rows,
                                                  block, nbits)
        top = 2 ** nbits - 1
        for i, r in enumerate(rows):
            for b in range(nb):
                sl = slice(b * block, (b + 1) * block)
                lo, st = lo_u[i, b], st_u[i, b]
                safe = st if st else 1.0
                z = (latent[r, sl] - lo) / safe
                q = np.where(st == 0, 0.0, np.clip(np.rint(z), 0, top))
                inside = (z >= 0) & (z <= top)
                gz = np.where(inside, grad[r, sl] * st, 0.0)
                assert np.array_equal(g_lat[r, sl], gz / safe)
                want_lo = np.sum(grad[r, sl].astype(np.float64) - gz / safe)
                want_st = np.sum(grad[r, sl] * q - (gz * (z / safe) if st else 0.0))
                assert g_lo[i, b] == want_lo and g_st[i, b] == want_st


def test_butterfly_is_the_normalised_hadamard_transform():
    rng = np.random.default_rng(4)
    k = 64
    i = np.arange(16)
    h = np.where(np.vectorize(lambda a: bin(a).count("1") % 2)(i[:, None] & i[None, :]),
                 -0.25, 0.25)
    flags = np.array([1, 0, 1, 1], np.uint8)
    x = rng.integers(-50, 50, (5, k)).astype(np.float32)  # exact in any order
    y = oracle.qad_wht_scale(x, flags, None, False)
    for g in range(4):
        sl = slice(16 * g, 16 * g + 16)
        want = x[:, sl].astype(np.float64) @ h if flags[g] else x[:, sl]
        assert np.array_equal(y[:, sl], want)
    xr = rng.standard_normal((5, k)).astype(np.float32)
    yr = oracle.qad_wht_scale(xr, flags, None, False)
    back = oracle.qad_wht_scale(yr, flags, None, False)  # an involution up to rounding
    assert np.abs(back - xr).max() <= 1e-6 * np.abs(xr).max()
    s = (rng.random(k) + 0.5).astype(np.float16)
    post = oracle.qad_wht_scale(xr, flags, s.view(np.uint16), False)
    assert np.array_equal(post, (yr / s.astype(np.float32)).astype(np.float32))
    pre = oracle.qad_wht_scale(xr, flags, s.view(np.uint16), True)
    assert np.array_equal(pre, oracle.qad_wht_scale(xr / s.astype(np.float32), flags, None,
                                                    False))
