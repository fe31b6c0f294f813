"""The QAD decode kernels on the MI355X (hi2x_qad_*) against the oracle (bit for bit,
including the per-block gradient sums) and the reference's torch graph of the
fake-quantised Linear (tests/golden/qad.npz): the stored values and latent gradients
bit-exact, the rest within float32 summation rounding; the autograd wrappers of the
``qad_kernel`` mirror end to end."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from golden_data import qad_cases

pytestmark = pytest.mark.gpu

CASES = list(qad_cases())


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.detach().cpu().numpy()


def _h(bits, dev):
    return T(bits.view(np.int16), dev).view(torch.float16)


def _oracle_stored(c):
    out = np.zeros_like(c["latent"])
    for g in c["groups"]:
        oracle.qad_decode_fwd(c["latent"], c["unit"], g["lo_u"], g["st_u"], g["consts"],
                              g["rows"], g["block"], g["nbits"], out)
    return out


def _oracle_bwd(c, grad):
    g_lat = np.zeros_like(c["latent"])
    per = []
    for g in c["groups"]:
        _, g_lo, g_st = oracle.qad_decode_bwd(grad, c["latent"], c["unit"], g["lo_u"], g["st_u"],
                                              g["consts"], g["rows"], g["block"], g["nbits"],
                                              g_lat)
        per.append((g_lo, g_st))
    return g_lat, per


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_kernels_equal_the_oracle_and_the_reference_graph(case, dev):
    from hi2_amd.qad_kernel import load

    tag, c = case
    print(f"qad kernels {tag}", flush=True)
    mod = load()
    lat = T(c["latent"], dev)
    unit = T(c["unit"], dev) if c["unit"] is not None else torch.ones(0, device=dev)
    out = torch.zeros_like(lat)
    grad = T(c["grad"], dev)
    g_lat = torch.zeros_like(lat)
    want_lat, want = _oracle_bwd(c, c["grad"])
    for g, (o_lo, o_st) in zip(c["groups"], want):
        args = (T(g["lo_u"], dev), T(g["st_u"], dev), _h(g["consts"], dev), T(g["rows"], dev))
        mod.decode_fwd(lat, unit, *args, g["block"], float(2 ** g["nbits"] - 1), out)
        g_lo, g_st = torch.empty_like(args[0]), torch.empty_like(args[0])
        mod.decode_bwd(grad, lat, unit, *args, g["block"], float(2 ** g["nbits"] - 1), g_lat,
                       g_lo, g_st)
        assert np.array_equal(N(g_lo), o_lo) and np.array_equal(N(g_st), o_st)
    assert np.array_equal(N(out), _oracle_stored(c)) and np.array_equal(N(out), c["stored"])
    assert np.array_equal(N(g_lat), want_lat) and np.array_equal(N(g_lat), c["g_latent"])
    for pre in (False, True):
        for cs in (c["col_scale"], None):
            y = torch.empty_like(out)
            mod.wht_scale(out, T(c["had"], dev), None if cs is None else _h(cs, dev), pre, y)
            assert np.array_equal(N(y), oracle.qad_wht_scale(N(out), c["had"], cs, pre))


def _fq(c, dev):
    """A duck-typed fake-quantised Linear (the fields hi2.qad.FakeQuantLinear exposes)."""
    groups = []
    for g in c["groups"]:
        groups.append(SimpleNamespace(
            rows=T(g["rows"], dev), consts=_h(g["consts"], dev), nbits=g["nbits"],
            block=g["block"], lo_u=torch.nn.Parameter(T(g["lo_u"], dev)),
            step_u=torch.nn.Parameter(T(g["st_u"], dev))))
    unit = T(c["unit"], dev) if c["unit"] is not None else torch.ones(0, device=dev)
    return SimpleNamespace(groups=groups, latent=torch.nn.Parameter(T(c["latent"], dev)),
                           unit=unit, had=T(c["had"], dev), col_scale=_h(c["col_scale"], dev),
                           has_had=bool(c["had"].any()), has_scale=True)


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_autograd_wrappers_end_to_end(case, dev):
    from hi2_amd.qad_kernel import original, stored

    tag, c = case
    print(f"qad autograd {tag}", flush=True)
    fq = _fq(c, dev)
    params = [fq.latent] + [p for g in fq.groups for p in (g.lo_u, g.step_u)]
    assert np.array_equal(N(stored(fq, False)), c["stored"])
    s = stored(fq, True)
    grads = torch.autograd.grad(s, params, T(c["grad"], dev))
    assert np.array_equal(N(grads[0]), c["g_latent"])
    _, per = _oracle_bwd(c, c["grad"])
    for gi, (o_lo, o_st) in enumerate(per):
        assert np.array_equal(N(grads[1 + 2 * gi]), o_lo)
        assert np.array_equal(N(grads[2 + 2 * gi]), o_st)
    w = original(fq)
    o_st = oracle.qad_wht_scale(c["stored"], c["had"], c["col_scale"], False)
    assert np.array_equal(N(w), o_st)
    scale = float(np.abs(c["original"]).max())
    assert float(np.abs(N(w) - c["original"]).max()) <= 1e-6 * scale  # torch path: matmul
    grads = torch.autograd.grad(w, params, T(c["grad2"], dev))
    g_in = oracle.qad_wht_scale(c["grad2"], c["had"], c["col_scale"], True)
    o_lat, per = _oracle_bwd(c, g_in)
    assert np.array_equal(N(grads[0]), o_lat)
    for gi, (o_lo, o_st) in enumerate(per):
        assert np.array_equal(N(grads[1 + 2 * gi]), o_lo)
        assert np.array_equal(N(grads[2 + 2 * gi]), o_st)
        ref = c["groups"][gi]["og_lo"]
        assert float(np.abs(N(grads[1 + 2 * gi]) - ref).max()) <= 2e-4 * (np.abs(ref).max() + 1e-12)


@pytest.mark.parametrize("k", [4096, 14336])
def test_configuration_widths_equal_the_oracle(k, dev):
    """Three groups (B = 16, 32, 64; INT2, INT4, INT8) over interleaved rows of a
    [192, K] latent in step units, every kernel bit-exact with the oracle."""
    from hi2_amd.qad_kernel import load

    print(f"qad width k={k}", flush=True)
    mod = load()
    rng = np.random.default_rng(k)
    r = 192
    latent = (rng.standard_normal((r, k)) * 3).astype(np.float32)
    unit = (rng.random((r, k)) * 0.5 + 0.5).astype(np.float32)
    grad = rng.standard_normal((r, k)).astype(np.float32)
    perm = rng.permutation(r)
    out = torch.zeros(r, k, device=dev)
    g_lat = torch.zeros(r, k, device=dev)
    want_out = np.zeros_like(latent)
    want_lat = np.zeros_like(latent)
    lt, ut, gt = T(latent, dev), T(unit, dev), T(grad, dev)
    for gi, (nbits, block) in enumerate(((2, 16), (4, 32), (8, 64))):
        rows = np.sort(perm[gi * 64:(gi + 1) * 64]).astype(np.int64)
        nb = k // block
        lo_u = (rng.random((64, nb)) * 255).astype(np.float32)
        st_u = (rng.random((64, nb)) * 255).astype(np.float32)
        st_u[::5, ::3] = 0.2  # zero step
        consts = np.stack([np.full(64, -3.0), np.full(64, 6.0 / 255), np.full(64, 0.1)], 1)
        consts = consts.astype(np.float16).view(np.uint16)
        args = (T(lo_u, dev), T(st_u, dev), _h(consts, dev), T(rows, dev))
        mod.decode_fwd(lt, ut, *args, block, float(2 ** nbits - 1), out)
        g_lo, g_st = torch.empty_like(args[0]), torch.empty_like(args[0])
        mod.decode_bwd(gt, lt, ut, *args, block, float(2 ** nbits - 1), g_lat, g_lo, g_st)
        oracle.qad_decode_fwd(latent, unit, lo_u, st_u, consts, rows, block, nbits, want_out)
        _, o_lo, o_st = oracle.qad_decode_bwd(grad, latent, unit, lo_u, st_u, consts, rows, block,
                                              nbits, want_lat)
        assert np.array_equal(N(g_lo), o_lo) and np.array_equal(N(g_st), o_st)
    assert np.array_equal(N(out), want_out) and np.array_equal(N(g_lat), want_lat)
    flags = (np.arange(k // 16) % 4 != 2).astype(np.uint8)
    cs = (rng.random(k) + 0.5).astype(np.float16).view(np.uint16)
    y = torch.empty_like(out)
    mod.wht_scale(out, T(flags, dev), _h(cs, dev), False, y)
    assert np.array_equal(N(y), oracle.qad_wht_scale(want_out, flags, cs, False))


def test_rows_outside_the_latent_are_skipped(dev):
    """A group row outside [0, R) is neither read nor written (no host check, no sync);
    its block gradients are 0, the other rows are decoded as usual."""
    from hi2_amd.qad_kernel import load

    mod = load()
    lat = torch.randn(4, 64, device=dev)
    n = 3
    lo_u = torch.full((n, 4), 10.0, device=dev)
    st_u = torch.full((n, 4), 20.0, device=dev)
    consts = torch.tensor([-1.0, 0.01, 0.01], device=dev).half().repeat(n, 1).contiguous()
    rows = torch.tensor([4, 1, -2], device=dev)
    out = torch.full_like(lat, 7.0)
    mod.decode_fwd(lat, torch.ones(0, device=dev), lo_u, st_u, consts, rows, 16, 3.0, out)
    g_lat = torch.full_like(lat, 7.0)
    g_lo, g_st = torch.full_like(lo_u, 7.0), torch.full_like(lo_u, 7.0)
    mod.decode_bwd(torch.ones_like(lat), lat, torch.ones(0, device=dev), lo_u, st_u, consts, rows,
                   16, 3.0, g_lat, g_lo, g_st)
    keep = [0, 2, 3]
    assert torch.equal(out[keep], torch.full_like(out[keep], 7.0))
    assert torch.equal(g_lat[keep], torch.full_like(g_lat[keep], 7.0))
    assert not bool((out[1] == 7.0).all()) and not bool((g_lat[1] == 7.0).all())
    assert torch.equal(g_lo[[0, 2]], torch.zeros(2, 4, device=dev))
    assert torch.equal(g_st[[0, 2]], torch.zeros(2, 4, device=dev))
