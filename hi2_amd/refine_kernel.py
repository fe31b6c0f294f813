"""Column loop of one refinement block on MI355X.

Mirror of the reference's ``hi2/refine_kernel.py`` (``BLOCK_COLUMNS`` 27, ``load``
132-161, ``available`` 164-171, ``failure`` 174-175, ``refine_block`` 178-182,
``supported`` re-exported from the GPTQ module), backed by ``hi2x_refine_block`` of
``libhi2x.so``.  One launch handles a block of up to 128 columns for every row: 16 lanes
own a row, its ``g`` segment is held in registers and the block of ``hs`` in LDS; each
column's decision follows the reference torch loop's arithmetic, so codes and moves are
bit-identical to it.

:func:`hi2_amd.refine.refine_expanded` does not call this block by block: the whole
sweep loop runs in one ``hi2x_refine_run`` call.  ``HI2_REFINE_BACKEND=kernel`` makes a
missing library an error at load time, as in the reference; there is no torch loop to
fall back to.
"""

import os

import torch

from . import _lib
from .gptq_kernel import kernel_dir, supported  # noqa: F401  (re-exported as in the reference)

BLOCK_COLUMNS = 128


def load():
    """The loaded library (ctypes handle), or None with :func:`failure` recorded."""
    mod = _lib.load()
    if mod is None and os.environ.get("HI2_REFINE_BACKEND") == "kernel":
        raise RuntimeError(f"hi2x library unavailable: {_lib.failure()}")
    return mod


def available(dev: torch.device) -> bool:
    backend = os.environ.get("HI2_REFINE_BACKEND", "auto")
    if backend == "torch":
        return False
    ok = supported(dev) and load() is not None
    if backend == "kernel" and not ok:
        raise RuntimeError(f"refine kernel unavailable on {dev}: {_lib.failure()}")
    return ok


def failure() -> str | None:
    return _lib.failure()


def refine_block(gb, c, lo_x, st_x, top, hs, b0, length, dw_block) -> None:
    """The column loop for columns ``[b0, b0 + length)``: ``gb [N, length]`` is the block's
    slice of ``g``, ``c [N, K]`` float codes (updated in place), ``lo_x``/``st_x`` ``[N, K]``
    per-column ladders, ``top [N]`` the highest code of each row, ``hs [K, K]``;
    ``dw_block [N, length]`` receives the change of each decoded value."""
    n, k = c.shape
    dev = _lib.require_gpu(gb, c, lo_x, st_x, top, hs, dw_block)
    for name, t in (("gb", gb), ("c", c), ("lo_x", lo_x), ("st_x", st_x), ("top", top),
                    ("hs", hs), ("dw_block", dw_block)):
        if not t.is_contiguous() or t.dtype != torch.float32:
            raise RuntimeError(f"refine_block: {name} must be contiguous float32")
    cu = c.to(torch.uint8)
    blk = torch.ones(n, dtype=torch.int32, device=dev)
    if n:
        _lib.call("hi2x_refine_block", dev, _lib.ptr(gb), gb.shape[1], n, k, int(b0),
                  int(length), _lib.ptr(cu), _lib.ptr(lo_x), _lib.ptr(st_x), k, _lib.ptr(blk),
                  _lib.ptr(top), _lib.ptr(hs), _lib.ptr(dw_block), dw_block.shape[1], None)
        c.copy_(cu.float())
