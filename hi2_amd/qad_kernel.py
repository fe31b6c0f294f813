"""Fused ladder decode of QAD's fake-quantised Linears on MI355X, forward and backward.

Mirror of the reference's ``hi2/qad_kernel.py`` (``load`` 229-258, ``available`` 261-268,
``failure`` 271-272, ``_StoredDecode`` 275-318, ``_Transform`` 321-336, ``original``
339-348, ``stored`` 351-370), backed by ``hi2x_qad_decode_fwd``, ``hi2x_qad_decode_bwd``
and ``hi2x_qad_wht_scale`` of ``libhi2x.so``.  ``load()`` returns an object with the
extension's three functions (``decode_fwd``, ``decode_bwd``, ``wht_scale``, same
arguments), so code written against the reference's extension runs unchanged.  The
calls never wait for the device: a group row outside the latent is skipped by the
kernels (nothing read or written; its byte gradients are 0) instead of being checked on
the host.

The stored values equal the torch graph of ``hi2.qad.FakeQuantLinear._group`` bit for
bit; the latent gradients too; the per-block byte gradients are sums in the reference
kernel's pairwise-tree order, and the transform is the reference kernel's butterfly.
``HI2_QAD_BACKEND=torch`` makes :func:`available` False (the caller then runs its own
torch graph, as in the reference); ``=kernel`` makes a missing library an error.
"""

import os

import torch

from . import _lib
from .gptq_kernel import kernel_dir, supported  # noqa: F401  (re-exported as in the reference)


def _check(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if not t.is_contiguous() or t.dtype != dtype:
        raise RuntimeError(f"{name} must be contiguous {dtype}")


def _opt(t: torch.Tensor | None):
    return None if t is None or t.numel() == 0 else _lib.ptr(t)


def _group_args(latent, unit, lo_u, st_u, consts, rows, block):
    _check(latent, torch.float32, "latent")
    _check(lo_u, torch.float32, "lo_u")
    _check(st_u, torch.float32, "st_u")
    _check(consts, torch.float16, "consts")
    _check(rows, torch.int64, "rows")
    if unit is not None and unit.numel():
        _check(unit, torch.float32, "unit")
        if unit.shape != latent.shape:
            raise RuntimeError("unit must have the latent's shape")
    k, n = latent.shape[1], rows.shape[0]
    if block not in (16, 32, 64):
        raise RuntimeError("block must be 16, 32 or 64")
    if k % block or tuple(lo_u.shape) != (n, k // block) or tuple(st_u.shape) != (n, k // block):
        raise RuntimeError("lo_u / st_u must be [rows, K / block]")
    if tuple(consts.shape) != (n, 3):
        raise RuntimeError("consts must be [rows, 3]")
    return k, n


class _Kernels:
    """The three functions of the reference's extension (``hi2/qad_kernel.py:37-49``)."""

    @staticmethod
    def decode_fwd(latent, unit, lo_u, st_u, consts, rows, block, nmax, out):
        dev = _lib.require_gpu(latent, lo_u, st_u, consts, rows, out)
        k, n = _group_args(latent, unit, lo_u, st_u, consts, rows, block)
        _check(out, torch.float32, "out")
        if out.shape != latent.shape:
            raise RuntimeError("out must have the latent's shape")
        if n:
            _lib.call("hi2x_qad_decode_fwd", dev, _lib.ptr(latent), _opt(unit), _lib.ptr(lo_u),
                      _lib.ptr(st_u), _lib.ptr(consts), _lib.ptr(rows), n, latent.shape[0], k,
                      int(block), float(nmax), _lib.ptr(out))

    @staticmethod
    def decode_bwd(grad, latent, unit, lo_u, st_u, consts, rows, block, nmax, g_latent, g_lo,
                   g_st):
        dev = _lib.require_gpu(grad, latent, lo_u, st_u, consts, rows, g_latent, g_lo, g_st)
        k, n = _group_args(latent, unit, lo_u, st_u, consts, rows, block)
        for name, t in (("grad", grad), ("g_latent", g_latent), ("g_lo", g_lo), ("g_st", g_st)):
            _check(t, torch.float32, name)
        if grad.shape != latent.shape or g_latent.shape != latent.shape:
            raise RuntimeError("grad and g_latent must have the latent's shape")
        if g_lo.shape != lo_u.shape or g_st.shape != lo_u.shape:
            raise RuntimeError("g_lo / g_st must have the shape of lo_u")
        if n:
            _lib.call("hi2x_qad_decode_bwd", dev, _lib.ptr(grad), _lib.ptr(latent), _opt(unit),
                      _lib.ptr(lo_u), _lib.ptr(st_u), _lib.ptr(consts), _lib.ptr(rows), n,
                      latent.shape[0], k, int(block), float(nmax), _lib.ptr(g_latent),
                      _lib.ptr(g_lo), _lib.ptr(g_st))

    @staticmethod
    def wht_scale(x, flags, scale, pre_div, out):
        dev = _lib.require_gpu(x, flags, out)
        _check(x, torch.float32, "x")
        _check(out, torch.float32, "out")
        _check(flags, torch.uint8, "flags")
        n, k = x.shape
        if k % 16 or flags.numel() != k // 16:
            raise RuntimeError("K must be a multiple of 16 with one flag per 16 columns")
        if scale is not None and scale.numel():
            _check(scale, torch.float16, "scale")
            if scale.numel() != k:
                raise RuntimeError("scale must have K entries")
        if out.shape != x.shape:
            raise RuntimeError("out must have the shape of x")
        if n:
            _lib.call("hi2x_qad_wht_scale", dev, _lib.ptr(x), n, k, _lib.ptr(flags),
                      _opt(scale), int(bool(pre_div)), _lib.ptr(out))


_KERNELS = _Kernels()


def load():
    """The kernels (an object with ``decode_fwd``, ``decode_bwd``, ``wht_scale``), or None
    with :func:`failure` recorded."""
    if _lib.load() is None:
        if os.environ.get("HI2_QAD_BACKEND") == "kernel":
            raise RuntimeError(f"hi2x library unavailable: {_lib.failure()}")
        return None
    return _KERNELS


def available(dev: torch.device) -> bool:
    backend = os.environ.get("HI2_QAD_BACKEND", "auto")
    if backend == "torch":
        return False
    ok = supported(dev) and load() is not None
    if backend == "kernel" and not ok:
        raise RuntimeError(f"qad kernel unavailable on {dev}: {_lib.failure()}")
    return ok


def failure() -> str | None:
    return _lib.failure()


def _mod():
    mod = load()
    if mod is None:
        raise RuntimeError(f"hi2x library unavailable: {_lib.failure()}")
    return mod


class _StoredDecode(torch.autograd.Function):
    """``stored = decode(latent, unit, ladder bytes)`` over all groups of one tensor."""

    @staticmethod
    def forward(ctx, latent, unit, meta, *params):
        out = torch.empty_like(latent)
        mod = _mod()
        for gi, (rows, consts, nbits, block) in enumerate(meta):
            mod.decode_fwd(latent, unit, params[2 * gi], params[2 * gi + 1], consts, rows, block,
                           float(2 ** nbits - 1), out)
        ctx.meta = meta
        ctx.save_for_backward(latent, unit, *params)
        return out

    @staticmethod
    def backward(ctx, grad):
        latent, unit, *params = ctx.saved_tensors
        grad = grad.contiguous()
        g_latent = torch.empty_like(latent)
        grads = []
        mod = _mod()
        for gi, (rows, consts, nbits, block) in enumerate(ctx.meta):
            g_lo = torch.empty_like(params[2 * gi])
            g_st = torch.empty_like(params[2 * gi])
            mod.decode_bwd(grad, latent, unit, params[2 * gi], params[2 * gi + 1], consts, rows,
                           block, float(2 ** nbits - 1), g_latent, g_lo, g_st)
            grads += [g_lo, g_st]
        return (g_latent, None, None, *grads)


class _Transform(torch.autograd.Function):
    """``H(x) / scale`` over the flagged 16-column groups; the backward is ``H(grad / scale)``."""

    @staticmethod
    def forward(ctx, x, flags, scale):
        out = torch.empty_like(x)
        _mod().wht_scale(x.contiguous(), flags, scale, False, out)
        ctx.flags, ctx.scale = flags, scale
        return out

    @staticmethod
    def backward(ctx, grad):
        out = torch.empty_like(grad)
        _mod().wht_scale(grad.contiguous(), ctx.flags, ctx.scale, True, out)
        return out, None, None


def original(fq) -> torch.Tensor:
    """The weights of a fake-quantised Linear in the model's own basis, with the STE graph:
    the stored values, then the rotation of the flagged groups and the division by the
    smoothing vector, fused."""
    w = stored(fq, True)
    if not fq.has_had and not fq.has_scale:
        return w
    return _Transform.apply(w, fq.had, fq.col_scale if fq.has_scale else fq.col_scale[:0])


def stored(fq, grad: bool) -> torch.Tensor:
    """The stored-basis weights of a fake-quantised Linear (rows in the tensor's own order),
    with the STE graph when ``grad``."""
    meta = [(g.rows, g.consts, g.nbits, g.block) for g in fq.groups]
    params = [p for g in fq.groups for p in (g.lo_u, g.step_u)]
    latent = fq.latent
    if grad and torch.is_grad_enabled():
        return _StoredDecode.apply(latent, fq.unit, meta, *params)
    with torch.no_grad():
        out = torch.empty_like(latent)
        mod = _mod()
        for (rows, consts, nbits, block), lo_u, st_u in zip(meta, params[::2], params[1::2]):
            mod.decode_fwd(latent.detach(), fq.unit, lo_u.detach(), st_u.detach(), consts, rows,
                           block, float(2 ** nbits - 1), out)
        return out
