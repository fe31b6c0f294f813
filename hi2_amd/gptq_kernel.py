"""Fused GPTQ column loop for one lazy-update block on MI355X (gfx950).

Mirror of the reference's ``hi2/gptq_kernel.py`` (``BLOCK_COLUMNS`` 33, ``kernel_dir``
135-137, ``supported`` 140-145, ``load`` 148-174, ``available`` 177-180, ``failure``
183-184, ``gptq_block`` 187-196) backed by ``hi2x_gptq_block`` of ``libhi2x.so``.

The kernel gives each row 16 lanes (one DPP row of the wavefront), each lane holding 8
of the block's 128 columns in registers, so a wavefront works on 4 rows and a 256-thread
workgroup on 16; the row group's 128 x 128 ``U`` block sits in LDS.  Per column the
owner lane rounds and computes the error, a DPP row broadcast hands it to the row's
other 15 lanes, and every lane pushes it into its remaining columns with the reference's
operation order, so codes, errors and ``comp`` are bit-identical to the reference's
column loop.

The library is built ahead of time (``python -m hi2_amd.build``).  ``load()`` returns
None and records :func:`failure` when it is missing; ``HI2_GPTQ_BACKEND=kernel``
makes that an error at load time, as in the reference.  There is no torch fallback:
:func:`hi2_amd.hessian.encode_jobs_gptq` raises when the kernel is unavailable.
"""

import os
from pathlib import Path

import torch

from . import _lib

BLOCK_COLUMNS = 128
ARCH = "gfx950"


def kernel_dir() -> Path:
    """Directory of the built library (``$HI2_KERNEL_DIR`` overrides where it is
    looked up by tooling; the package loads ``hi2_amd/libhi2x.so``)."""
    d = os.environ.get("HI2_KERNEL_DIR")
    return Path(d) if d else Path(_lib.HERE)


def supported(dev: torch.device) -> bool:
    """A HIP device of the CDNA4 family the kernels are written for (gfx950)."""
    dev = torch.device(dev)
    if dev.type != "cuda" or not torch.version.hip or not torch.cuda.is_available():
        return False
    arch = torch.cuda.get_device_properties(dev).gcnArchName
    return arch.split(":")[0] == ARCH


def load():
    """The loaded library (ctypes handle), or None with :func:`failure` recorded."""
    mod = _lib.load()
    if mod is None and os.environ.get("HI2_GPTQ_BACKEND") == "kernel":
        raise RuntimeError(f"hi2x library unavailable: {_lib.failure()}")
    return mod


def available(dev: torch.device) -> bool:
    if os.environ.get("HI2_GPTQ_BACKEND", "auto") == "torch":
        return False
    return supported(dev) and load() is not None


def failure() -> str | None:
    return _lib.failure()


def gptq_block(
    wc, i1, length, err1, codes, lo, st, row_grp, u_ptrs, blk, nmax, comp=None
):
    """Launch the fused column loop for block ``[i1, i1 + length)``: ``wc [N, K]`` f32
    (read only), ``err1 [N, length]`` f32 out, ``codes [N, K]`` uint8 out (rounding
    order), ``lo``/``st [N, ldp]`` f32, ``row_grp [N]`` int32 (ascending), ``u_ptrs
    [G]`` int64 device addresses of contiguous ``[K, K]`` f32 factors, ``blk [G, K]``
    int32, ``nmax [G]`` f32, ``comp [N, K]`` f32 (optional) receives the value each
    code was rounded from."""
    dev = _lib.require_gpu(wc, err1, codes, lo, st, row_grp, u_ptrs, blk, nmax, comp)
    for name, t in (("wc", wc), ("err1", err1), ("codes", codes), ("lo", lo), ("st", st),
                    ("blk", blk)):
        if not t.is_contiguous():
            raise RuntimeError(f"gptq_block: {name} must be contiguous")
    if wc.dtype != torch.float32 or err1.dtype != torch.float32:
        raise RuntimeError("gptq_block: wc and err1 must be float32")
    if codes.dtype != torch.uint8 or blk.dtype != torch.int32:
        raise RuntimeError("gptq_block: codes must be uint8 and blk int32")
    if row_grp.dtype != torch.int32 or u_ptrs.dtype != torch.int64:
        raise RuntimeError("gptq_block: row_grp must be int32 and u_ptrs int64")
    if lo.dtype != torch.float32 or st.dtype != torch.float32 or nmax.dtype != torch.float32:
        raise RuntimeError("gptq_block: lo, st and nmax must be float32")
    length = int(length)
    if not (0 < length <= BLOCK_COLUMNS) or err1.shape[1] != length:
        raise RuntimeError(f"gptq_block: block length {length} (err1 {tuple(err1.shape)})")
    if comp is not None and comp.numel() and (
        not comp.is_contiguous() or comp.dtype != torch.float32 or comp.shape != wc.shape
    ):
        raise RuntimeError("gptq_block: comp must be a contiguous float32 [N, K] tensor")
    n, k = wc.shape
    if n == 0:
        return
    cp = comp if comp is not None and comp.numel() else None
    _lib.call("hi2x_gptq_block", dev, _lib.ptr(wc), n, k, int(i1), length, _lib.ptr(err1),
              _lib.ptr(codes), _lib.ptr(lo), _lib.ptr(st), lo.shape[1], _lib.ptr(row_grp),
              _lib.ptr(u_ptrs), _lib.ptr(blk), _lib.ptr(nmax), _lib.ptr(cp))
