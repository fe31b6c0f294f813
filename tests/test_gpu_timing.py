"""The launch-timing hook (hi2x_timing_*) records the launches it is asked for, with
their algorithmic work, and leaves results unchanged (MI355X)."""

import pytest
import torch

from hi2_amd import _lib
from hi2_amd.hessian import HessianStats

pytestmark = pytest.mark.gpu


def _trailing(dev, wc, err, u, rg, up, n, k, c0):
    _lib.call("hi2x_gptq_trailing", dev, _lib.ptr(wc), n, k, 0, 128, _lib.ptr(err), 128, c0, k,
              _lib.ptr(rg), _lib.ptr(up))


def test_timing_records_trailing_launches_and_work(dev):
    n, k = 300, 512
    g = torch.Generator(device=dev).manual_seed(3)
    wc = torch.randn(n, k, device=dev, generator=g)
    err = torch.randn(n, 128, device=dev, generator=g)
    u = torch.triu(torch.randn(k, k, device=dev, generator=g))
    rg = torch.zeros(n, dtype=torch.int32, device=dev)
    up = torch.tensor([u.data_ptr()], dtype=torch.int64, device=dev)
    ref = wc.clone()
    _trailing(dev, ref, err, u, rg, up, n, k, 128)
    _lib.timing_enable([_lib.TIME_GPTQ_TRAILING])
    try:
        _trailing(dev, wc, err, u, rg, up, n, k, 128)
        _trailing(dev, wc, err, u, rg, up, n, k, 256)
        torch.cuda.synchronize()
        launches, ms, work = _lib.timing_query(_lib.TIME_GPTQ_TRAILING)
        other = _lib.timing_query(_lib.TIME_HESSIAN_SYRK)
    finally:
        _lib.timing_enable([])
    assert launches == 2
    assert ms > 0.0
    assert work == 2.0 * n * 128 * ((k - 128) + (k - 256))
    assert other == (0, 0.0, 0.0)
    # the first timed launch did what the untimed one did
    _trailing(dev, ref, err, u, rg, up, n, k, 256)
    assert torch.equal(wc, ref)


def test_timing_records_hessian_syrk(dev):
    t, k = 256, 384
    x = torch.randn(t, k, device=dev).to(torch.bfloat16)
    _lib.timing_enable([_lib.TIME_HESSIAN_SYRK])
    try:
        st = HessianStats(k, dev)
        st.update(x)
        torch.cuda.synchronize()
        launches, ms, work = _lib.timing_query(_lib.TIME_HESSIAN_SYRK)
    finally:
        _lib.timing_enable([])
    assert launches == 1 and ms > 0.0 and work == float(t * k * (k + 1))
    assert _lib.timing_query(_lib.TIME_HESSIAN_SYRK) == (0, 0.0, 0.0)


def test_timing_separates_the_factor_fp32_and_split_products(dev):
    """At K = 4096 the factor's top products run on the fp16 split planes (their own
    family, counting the three fp16 products) and the smaller ones on the fp32 MFMA GEMM:
    each family records its launches, and neither reports more than its peak."""
    from hi2_amd import _lib
    from hi2_amd.hessian import inverse_factor

    k = 4096
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(2 * k, k, generator=g, device=dev)
    hs = (x.T @ x) / (2 * k)
    inverse_factor(hs, 0.01)
    torch.cuda.synchronize()
    _lib.timing_enable([_lib.TIME_CHOL_GEMM, _lib.TIME_CHOL_SPLIT])
    try:
        inverse_factor(hs, 0.01)
        torch.cuda.synchronize()
        f32 = _lib.timing_query(_lib.TIME_CHOL_GEMM)
        f16 = _lib.timing_query(_lib.TIME_CHOL_SPLIT)
    finally:
        _lib.timing_enable([])
    assert f32[0] > 0 and f16[0] > 0
    assert f32[2] / (f32[1] / 1e3) < 157.3e12
    assert f16[2] / (f16[1] / 1e3) < 2.5e15
