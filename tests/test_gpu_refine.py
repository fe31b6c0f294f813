"""Local code refinement on the MI355X (hi2x_refine_*) against the reference's golden
vectors and the oracle: codes bit-exact (the products are sequential fp32 FMA chains on
both sides), sse in the reference's reduction order, the device-side early stop, and
the block kernel of the ``refine_kernel`` mirror."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from golden_data import refine_cases

pytestmark = pytest.mark.gpu

CASES = list(refine_cases())


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.detach().cpu().numpy()


class _Enc:
    """The fields of hi2_amd.encode.Encoded that refine reads."""

    def __init__(self, codes, params, consts, sse=None, comp=None):
        self.codes, self.params, self.consts, self.sse, self.comp = codes, params, consts, sse, comp


def _groups(groups, dev):
    out = []
    for g in groups:
        enc = _Enc(T(g["codes_in"], dev), T(g["params"], dev),
                   T(g["consts"], dev).view(torch.float16))
        out.append((T(g["w"], dev), enc, g["nbits"], g["block"]))
    return out


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_refine_groups_equals_reference_golden(case, dev):
    from hi2_amd.refine import refine_groups

    tag, hs, passes, groups = case
    print(f"refine golden {tag} passes={passes}", flush=True)
    got = refine_groups(_groups(groups, dev), T(hs, dev), passes)
    for g, c in zip(groups, got):
        assert c.dtype == torch.uint8
        assert np.array_equal(N(c), g["codes"])


def test_refine_codes_and_expanded_entry_points(dev):
    from hi2_amd.refine import _expand, refine_codes, refine_expanded

    _, hs, passes, (g,) = next(c for c in CASES if c[0] == "a")
    w, hs_t = T(g["w"], dev), T(hs, dev)
    lo, st = T(g["lo"], dev), T(g["step"], dev)
    codes = T(g["codes_in"], dev)
    got = refine_codes(w, codes, lo, st, hs_t, g["nbits"], g["block"], passes)
    assert got.dtype == codes.dtype and np.array_equal(N(got), g["codes"])
    lo_x, st_x = _expand(lo, st, g["block"])
    top = torch.full((w.shape[0],), float(2 ** g["nbits"] - 1), device=dev)
    got = refine_expanded(w, codes.float(), lo_x, st_x, top, hs_t, passes)
    assert got.dtype == torch.float32 and np.array_equal(N(got), g["codes"].astype(np.float32))


def test_refine_encoded_recomputes_sse_in_the_reference_order(dev):
    from hi2_amd.refine import refine_encoded

    _, hs, passes, (g,) = next(c for c in CASES if c[0] == "b")
    (w, enc, nbits, block), = _groups([g], dev)
    out = refine_encoded(enc, w, T(hs, dev), nbits, block, passes)
    assert np.array_equal(N(out.codes), g["codes"])
    assert out.params is enc.params and out.consts is enc.consts
    _, _, sse = oracle.finish(g["codes"], None, None, block, g["lo"], g["step"], g["w"],
                              np.diag(hs).copy())
    assert np.array_equal(N(out.sse), sse)


def test_objective_is_the_hessian_error(dev):
    from hi2_amd.refine import objective

    _, hs, _, (g,) = next(c for c in CASES if c[0] == "e")
    idx = np.arange(g["w"].shape[1]) // g["block"]
    rec = (g["lo"][:, idx] + g["codes_in"].astype(np.float32) * g["step"][:, idx])
    e = rec.astype(np.float16).astype(np.float64) - g["w"].astype(np.float64)
    want = float(np.einsum("ij,jk,ik->", e, hs.astype(np.float64), e))
    got = objective(T(g["w"], dev), T(g["codes_in"], dev), T(g["lo"], dev), T(g["step"], dev),
                    T(hs, dev), g["block"])
    assert got == pytest.approx(want, rel=1e-5)


def _run_raw(dev, w, codes, lo, st, block, top, hs, passes):
    """hi2x_refine_run through the C ABI with the per-sweep move counters."""
    from hi2_amd import _lib

    n, k = w.shape
    wt, ct = T(w, dev), T(codes, dev).clone()
    lt, stt = T(lo, dev), T(st, dev)
    bt = T(np.broadcast_to(np.asarray(block, np.int32), (n,)), dev)
    tt = T(np.broadcast_to(np.asarray(top, np.float32), (n,)), dev)
    ht = T(hs, dev)
    moved = torch.full((max(passes, 1),), 7, dtype=torch.int64, device=dev)
    ws = _lib.workspace(dev, "hi2x_refine_workspace_bytes", n, k, passes)
    _lib.call("hi2x_refine_run", dev, _lib.ptr(wt), _lib.ptr(ct), n, k, _lib.ptr(lt),
              _lib.ptr(stt), lt.shape[1], _lib.ptr(bt), _lib.ptr(tt), _lib.ptr(ht), passes,
              _lib.ptr(moved), _lib.ptr(ws), ws.numel())
    return N(ct), N(moved)


def test_device_side_stop_counts_moves_per_sweep(dev):
    _, hs, _, (g,) = next(c for c in CASES if c[0] == "conv")
    top = 2 ** g["nbits"] - 1
    got, moved = _run_raw(dev, g["w"], g["codes_in"], g["lo"], g["step"], g["block"], top, hs, 40)
    want, mv_rows, sweeps = oracle.refine(g["w"], g["codes_in"], g["lo"], g["step"], g["block"],
                                          top, hs, 40)
    assert np.array_equal(got, want) and np.array_equal(got, g["codes"])
    assert sweeps < 40
    assert moved[: sweeps - 1].min() > 0 and moved[sweeps - 1:].max() == 0
    assert moved.sum() == mv_rows.sum()


def test_refine_block_mirror_is_the_first_block_of_a_sweep(dev):
    from hi2_amd import _lib
    from hi2_amd.refine import _expand
    from hi2_amd.refine_kernel import refine_block

    _, hs, _, (g,) = next(c for c in CASES if c[0] == "d")  # K = 128: one block
    _, hs2, _, (g2,) = next(c for c in CASES if c[0] == "zero")
    for gg, h in ((g, hs), (g2, hs2)):
        n, k = gg["w"].shape
        assert k == 128
        w, codes = T(gg["w"], dev), T(gg["codes_in"], dev)
        lo, st = T(gg["lo"], dev), T(gg["step"], dev)
        blk = torch.full((n,), gg["block"], dtype=torch.int32, device=dev)
        e = torch.empty(n, k, device=dev)
        gr = torch.empty(n, k, device=dev)
        ht = T(h, dev)  # held until the launch has run
        _lib.call("hi2x_refine_gradient", dev, _lib.ptr(w), _lib.ptr(codes), n, k, _lib.ptr(lo),
                  _lib.ptr(st), lo.shape[1], _lib.ptr(blk), _lib.ptr(ht), _lib.ptr(e),
                  _lib.ptr(gr))
        lo_x, st_x = _expand(lo, st, gg["block"])
        top = torch.full((n,), float(2 ** gg["nbits"] - 1), device=dev)
        c = codes.float().contiguous()
        dw = torch.zeros(n, k, device=dev)
        refine_block(gr.contiguous(), c, lo_x.contiguous(), st_x.contiguous(), top,
                     T(h, dev), 0, k, dw)
        want, _, _ = oracle.refine(gg["w"], gg["codes_in"], gg["lo"], gg["step"], gg["block"],
                                   2 ** gg["nbits"] - 1, h, 1)
        assert np.array_equal(N(c).astype(np.uint8), want)
        # dw is the change of the decoded value where a code moved, 0 elsewhere
        idx = np.arange(k) // gg["block"]
        dec = lambda cc: (gg["lo"][:, idx] + cc.astype(np.float32) * gg["step"][:, idx]).astype(  # noqa: E731
            np.float16).astype(np.float32)
        assert np.array_equal(N(dw), dec(want) - dec(gg["codes_in"]))


def _gptq_rows(dev, n, k, t, nbits, block, seed):
    """Realistic refinement input at width k: a damped Hessian of t outlier-scaled
    tokens and GPTQ codes of n heavy-tailed rows (all on the device)."""
    from hi2_amd.format import decode_params
    from hi2_amd.hessian import encode_rows_gptq, inverse_factor

    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(t, k, generator=g, device=dev)
    x[:, torch.randperm(k, generator=g, device=dev)[: (k + 99) // 100]] *= 20.0
    hs = (x.T @ x) / t
    hs = (hs + hs.T) * 0.5
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    w *= torch.exp(0.5 * torch.randn(n, 1, generator=g, device=dev))
    enc = encode_rows_gptq(w, hs.diagonal().clone(), inverse_factor(hs), nbits, block)
    lo, st = decode_params(enc.params[..., 0], enc.params[..., 1], enc.consts[:, 0:1],
                           enc.consts[:, 1:2], enc.consts[:, 2:3])
    return w, enc, hs, lo.float(), st.float()


@pytest.mark.parametrize("k,n,passes", [(4096, 48, 2), (14336, 16, 2), (960, 70, 3)])
def test_refine_at_configuration_widths_equals_the_oracle(k, n, passes, dev):
    """Mixed INT2/B32 and INT4/B64 rows at the q_proj (K=4096) and down_proj (K=14336)
    widths and at a width with a partial last block (K=960, three sweeps): codes equal
    the oracle's bit for bit."""
    from hi2_amd.refine import refine_groups

    print(f"refine width k={k} n={n} passes={passes}", flush=True)
    w2, e2, hs, lo2, st2 = _gptq_rows(dev, n // 2, k, 2048, 2, 32, seed=k)
    g = torch.Generator(device=dev).manual_seed(k + 1)
    w4 = torch.randn(n - n // 2, k, generator=g, device=dev) * 0.02
    from hi2_amd.format import decode_params
    from hi2_amd.hessian import encode_rows_gptq, inverse_factor

    e4 = encode_rows_gptq(w4, hs.diagonal().clone(), inverse_factor(hs), 4, 64)
    lo4, st4 = decode_params(e4.params[..., 0], e4.params[..., 1], e4.consts[:, 0:1],
                             e4.consts[:, 1:2], e4.consts[:, 2:3])
    got = refine_groups([(w2, e2, 2, 32), (w4, e4, 4, 64)], hs, passes)
    hs_h = N(hs)
    for w, enc, lo, st, nbits, block, c in ((w2, e2, lo2, st2, 2, 32, got[0]),
                                              (w4, e4, lo4.float(), st4.float(), 4, 64, got[1])):
        want, moved, _ = oracle.refine(N(w), N(enc.codes), N(lo), N(st), block, 2 ** nbits - 1,
                                       hs_h, passes)
        assert moved.sum() > 0
        assert np.array_equal(N(c), want)


@pytest.mark.parametrize("scaling", ["all_blocks", "one_block"])
def test_refine_blocks_outside_the_bounds_take_the_nan_aware_loop(scaling, dev):
    """The column loop runs the plain max of each move pair only when every gain of the
    block stays finite (|g| <= 2^60, |dw| <= 2^30, the block's Hessian within 2^30);
    otherwise the NaN-aware loop.  The Hessian scaled by 2^31 (every block outside) or
    one 128-column block's rows and columns by 2^16 (its diagonal block by 2^32, the
    others inside): codes equal the oracle's on the same inputs, bit for bit."""
    from hi2_amd.format import decode_params
    from hi2_amd.refine import refine_groups

    k, n, passes = 960, 40, 2
    w, enc, hs, lo, st = _gptq_rows(dev, n, k, 2048, 4, 64, seed=31)
    if scaling == "all_blocks":
        hs = hs * 2.0 ** 31
    else:
        sc = torch.ones(k, device=dev)
        sc[128:256] = 2.0 ** 16
        hs = sc[:, None] * hs * sc[None, :]
    assert hs[128:256, 128:256].abs().max() > 2.0 ** 30
    got = refine_groups([(w, enc, 4, 64)], hs, passes)[0]
    lo, st = decode_params(enc.params[..., 0], enc.params[..., 1], enc.consts[:, 0:1],
                           enc.consts[:, 1:2], enc.consts[:, 2:3])
    want, moved, _ = oracle.refine(N(w), N(enc.codes), N(lo.float()), N(st.float()), 64, 15,
                                   N(hs), passes)
    assert moved.sum() > 0
    assert np.array_equal(N(got), want)
