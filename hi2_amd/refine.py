"""Local code refinement after GPTQ rounding, on MI355X (gfx950).

Mirror of the reference's ``hi2/refine.py`` (``BLOCK_COLUMNS`` 20, ``objective`` 23-36,
``_expand`` 39-41, ``refine_expanded`` 44-106, ``refine_codes`` 109-122,
``refine_groups`` 125-144, ``refine_encoded`` 147-162), backed by ``hi2x_refine_*`` of
``libhi2x.so``.

GPTQ rounds the columns of a row one after another and never goes back.  A sweep goes
back: for every column in turn it tries to move the code one level up or down and keeps
the move when the row's Hessian error ``e Hs e^T`` falls (``e`` is the row's error in the
stored basis).  The ladders stay as they are.  Given ``g = e Hs`` a move costs O(row);
the sweep works in 128-column blocks, and one GEMM per block brings ``g`` up to date.

The whole sweep loop runs on the device (``hi2x_refine_run``): the residual, the
gradient GEMM, the per-block column loops and the per-block GEMMs, with the reference's
stop after a sweep that moves nothing decided on the device.  Codes are bit-identical to
the reference's torch loop.  Ladders are not expanded to one value per column: each row
reads its ``[K / block]`` decoded ladder through its own block size, so rows of different
``(bits, block)`` candidates share one sweep without the ``[N, K]`` copies.
"""

import torch

from . import _lib
from .format import decode_params

BLOCK_COLUMNS = 128


def _rows_args(w, lo, step, block_rows, top_rows):
    dev = _lib.require_gpu(w)
    w = w.to(dev, torch.float32).contiguous()
    lo = lo.to(dev, torch.float32).contiguous()
    step = step.to(dev, torch.float32).contiguous()
    blk = block_rows.to(dev, torch.int32).contiguous()
    top = top_rows.to(dev, torch.float32).contiguous()
    return dev, w, lo, step, blk, top


def _gradient(w, codes, lo, step, block_rows, hs, want_g=True):
    """(e, g) of rows w with codes and per-row-block ladders ``lo/step [N, ldp]``."""
    n, k = w.shape
    dev, w, lo, step, blk, _ = _rows_args(w, lo, step, block_rows, block_rows)
    hs = hs.to(dev, torch.float32).contiguous()
    c = codes.to(dev, torch.uint8).contiguous()
    e = torch.empty(n, k, dtype=torch.float32, device=dev)
    g = torch.empty(n, k, dtype=torch.float32, device=dev) if want_g else None
    if n:
        _lib.call("hi2x_refine_gradient", dev, _lib.ptr(w), _lib.ptr(c), n, k, _lib.ptr(lo),
                  _lib.ptr(step), lo.shape[1], _lib.ptr(blk), _lib.ptr(hs), _lib.ptr(e),
                  _lib.ptr(g))
    return e, g


@torch.no_grad()
def objective(
    w: torch.Tensor,
    codes: torch.Tensor,
    lo: torch.Tensor,
    step: torch.Tensor,
    hs,
    block,
) -> float:
    """Sum over rows of ``e Hs e^T`` for the decoded codes (``hi2/refine.py:23-36``)."""
    n = w.shape[0]
    e, g = _gradient(w, codes, lo, step,
                     torch.full((n,), int(block), dtype=torch.int32, device=w.device), hs)
    return float((g * e).sum())


def _expand(lo: torch.Tensor, step: torch.Tensor, block: int):
    """Per-column ladders ``[N, K]`` from the per-block ones ``[N, K / block]``."""
    return lo.repeat_interleave(block, dim=1), step.repeat_interleave(block, dim=1)


def _run(w, codes_u8, lo, step, block_rows, top_rows, hs, passes) -> torch.Tensor:
    """hi2x_refine_run on rows ``w [N, K]``; returns the refined uint8 codes (a new tensor)."""
    n, k = w.shape
    dev, w, lo, step, blk, top = _rows_args(w, lo, step, block_rows, top_rows)
    hs = hs.to(dev, torch.float32).contiguous()
    if hs.shape != (k, k):
        raise RuntimeError(f"hs has shape {tuple(hs.shape)}, expected ({k}, {k})")
    c = codes_u8.to(dev, torch.uint8).clone().contiguous()
    if n == 0 or passes <= 0:
        return c
    ws = _lib.workspace(dev, "hi2x_refine_workspace_bytes", n, k, int(passes))
    _lib.call("hi2x_refine_run", dev, _lib.ptr(w), _lib.ptr(c), n, k, _lib.ptr(lo),
              _lib.ptr(step), lo.shape[1], _lib.ptr(blk), _lib.ptr(top), _lib.ptr(hs),
              int(passes), None, _lib.ptr(ws), ws.numel())
    return c


@torch.no_grad()
def refine_expanded(
    w: torch.Tensor,
    codes: torch.Tensor,
    lo_x: torch.Tensor,
    st_x: torch.Tensor,
    top: torch.Tensor,
    hs: torch.Tensor,
    passes: int,
) -> torch.Tensor:
    """Refined codes (float) of rows ``w[N, K]`` with per-column ladders ``lo_x``/``st_x``
    and the highest code of each row ``top[N]`` (``hi2/refine.py:44-106``)."""
    n, k = w.shape
    cf = codes.float()
    if bool(((cf < 0) | (cf > 255) | (cf != cf.round())).any()):
        raise RuntimeError("codes must be integers in [0, 255]")
    ones = torch.ones(n, dtype=torch.int32, device=w.device)
    out = _run(w, cf.to(torch.uint8), lo_x, st_x, ones, top.float(), hs, passes)
    return out.float()


def refine_codes(
    w: torch.Tensor,
    codes: torch.Tensor,
    lo: torch.Tensor,
    step: torch.Tensor,
    hs: torch.Tensor,
    nbits: int,
    block: int,
    passes: int,
) -> torch.Tensor:
    """:func:`refine_expanded` for rows rounded at one ``(nbits, block)`` with decoded
    ladders ``lo`` and ``step`` ``[N, K / block]``; returns codes of the dtype of ``codes``
    (``hi2/refine.py:109-122``)."""
    n = w.shape[0]
    out = _run(w, codes.to(torch.uint8), lo, step,
               torch.full((n,), int(block), dtype=torch.int32, device=w.device),
               torch.full((n,), float(2**nbits - 1), device=w.device), hs, passes)
    return out.to(codes.dtype)


def _decoded(enc):
    lo, step = decode_params(
        enc.params[..., 0],
        enc.params[..., 1],
        enc.consts[:, 0:1],
        enc.consts[:, 1:2],
        enc.consts[:, 2:3],
    )
    return lo.float(), step.float()


def refine_groups(groups, hs: torch.Tensor, passes: int) -> list[torch.Tensor]:
    """One sweep over the rows of every ``(w, enc, nbits, block)`` group of a tensor (the
    rows of different candidates share the column loop); returns the refined codes per
    group, uint8 like ``enc.codes`` (``hi2/refine.py:125-144``)."""
    if not groups:
        return []
    dev = _lib.require_gpu(groups[0][0])
    parts = []
    for w, enc, nbits, block in groups:
        lo, step = _decoded(enc)
        n = w.shape[0]
        parts.append((w, enc.codes, lo, step,
                      torch.full((n,), int(block), dtype=torch.int32, device=dev),
                      torch.full((n,), float(2**nbits - 1), device=dev)))
    ldp = max(p[2].shape[1] for p in parts)
    pad = lambda t: torch.nn.functional.pad(t.to(dev), (0, ldp - t.shape[1]))  # noqa: E731
    w = torch.cat([p[0].to(dev, torch.float32) for p in parts])
    codes = torch.cat([p[1].to(dev, torch.uint8) for p in parts])
    lo = torch.cat([pad(p[2]) for p in parts])
    step = torch.cat([pad(p[3]) for p in parts])
    blk = torch.cat([p[4] for p in parts])
    top = torch.cat([p[5] for p in parts])
    out = _run(w, codes, lo, step, blk, top, hs, passes)
    sizes = [p[0].shape[0] for p in parts]
    return [c.to(groups[i][1].codes.dtype) for i, c in enumerate(out.split(sizes))]


def refine_encoded(enc, w, hs, nbits: int, block: int, passes: int):
    """``enc`` (an :class:`hi2_amd.encode.Encoded`) with refined codes; the ladders are
    untouched.  The ``sse`` field is recomputed for the new codes with the ladder weights
    ``diag(hs)`` (``hi2/refine.py:147-162``), in the reference's reduction order."""
    (codes,) = refine_groups([(w, enc, nbits, block)], hs, passes)
    lo, step = _decoded(enc)
    dev = codes.device
    n, k = codes.shape
    wf = w.to(dev, torch.float32).contiguous()
    d = hs.to(dev, torch.float32).diagonal().contiguous()
    lo, step = lo.contiguous(), step.contiguous()
    c = codes.to(torch.uint8).contiguous()
    sse = torch.empty(n, dtype=torch.float32, device=dev)
    if n:
        _lib.call("hi2x_finish", dev, _lib.ptr(c), None, None, n, k, int(block), _lib.ptr(lo),
                  _lib.ptr(step), lo.shape[1], _lib.ptr(wf), _lib.ptr(d), _lib.ptr(c), None,
                  _lib.ptr(sse))
    return type(enc)(codes, enc.params, enc.consts, sse, enc.comp)
