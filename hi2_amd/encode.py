"""Block encoder for the v3.2 ladder on MI355X.

Mirror of the reference's ``hi2/encode.py`` (same names and meaning): ``EFFORT``
(18-22), ``CHUNK_ELEMS`` (23), ``_safe`` (26-27), ``fit_ladder`` (53-92),
``quantize_params`` (95-119), ``Encoded`` (122-130), ``encode_rows`` (133-173).
The ladder search and the 8-bit parameters run in the hi2x kernels
(``hi2x_ladder_fit``, ``hi2x_params``), bit-identical to the reference's torch code.
"""

from dataclasses import dataclass

import torch

from . import _lib

EFFORT = {
    "fast": dict(grid=(0.0, 0.06, 0.12), ls=1),
    "normal": dict(grid=(0.0, 0.04, 0.08, 0.12, 0.16, 0.20), ls=2),
    "max": dict(grid=(0.0, 0.025, 0.05, 0.075, 0.10, 0.125, 0.15, 0.20), ls=4),
}
CHUNK_ELEMS = 1 << 24  # rows per encode call are bounded so temporaries fit


def _safe(step: torch.Tensor) -> torch.Tensor:
    return torch.where(step == 0, torch.ones_like(step), step)


def _grid_array(grid) -> "ctypes.Array":
    import ctypes

    return (ctypes.c_float * len(grid))(*[float(g) for g in grid])


def _fit(wb: torch.Tensor, d: torch.Tensor, n: int, grid, ls: int, want_err: bool):
    rows, nb, b = wb.shape
    dev = _lib.require_gpu(wb, d)
    w = wb.to(torch.float32).contiguous()
    dv = d.to(dev, torch.float32).reshape(-1).contiguous()
    # the kernel reads 16-byte vectors
    if w.data_ptr() % 16:
        w = w.clone()
    if dv.data_ptr() % 16:
        dv = dv.clone()
    if dv.numel() != nb * b:
        raise ValueError(f"weights have {dv.numel()} entries, expected {nb * b}")
    lo = torch.empty(rows, nb, dtype=torch.float32, device=dev)
    st = torch.empty(rows, nb, dtype=torch.float32, device=dev)
    err = torch.empty(rows, nb, dtype=torch.float32, device=dev) if want_err else None
    if rows:
        _lib.call("hi2x_ladder_fit", dev, _lib.ptr(w), _lib.ptr(dv), rows, nb * b, b, int(n),
                  _grid_array(grid), len(grid), int(ls), _lib.ptr(lo), _lib.ptr(st),
                  _lib.ptr(err))
    return lo, st, err


def _block_weights(db: torch.Tensor, nb: int, b: int) -> torch.Tensor:
    if db.shape[-2:] != (nb, b) or any(s != 1 for s in db.shape[:-2]):
        raise ValueError(
            f"ladder weights must broadcast as [1, {nb}, {b}] (got {tuple(db.shape)})"
        )
    return db.reshape(nb * b)


def fit_ladder(wb: torch.Tensor, db: torch.Tensor, n: int, effort: str = "normal"):
    """Per-block ``(lo, step)`` minimising ``sum d * (w_hat - w)^2``: best of the grid
    of range shrinks of the min-max ladder, then ``ls`` weighted least-squares refits
    kept only where they lower the error.  ``wb`` is ``[N, nb, B]``, ``db`` is
    ``[1, nb, B]`` (the column weights)."""
    cfg = EFFORT[effort]
    nb, b = wb.shape[-2], wb.shape[-1]
    lo, st, _ = _fit(wb, _block_weights(db, nb, b), n, cfg["grid"], cfg["ls"], False)
    return lo, st


def quantize_params(lo: torch.Tensor, step: torch.Tensor):
    """8-bit block parameters relative to three fp16 row constants (spec 2.2):
    ``(lo_u8, step_u8, consts[N, 3])``, consts = (lo_min, lo_scale, step_scale)."""
    dev = _lib.require_gpu(lo, step)
    rows, nb = lo.shape
    l = lo.to(torch.float32).contiguous()
    s = step.to(torch.float32).contiguous()
    lo_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
    st_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
    consts = torch.empty(rows, 3, dtype=torch.float16, device=dev)
    if rows:
        _lib.call("hi2x_params", dev, _lib.ptr(l), _lib.ptr(s), rows, nb, _lib.ptr(lo_u8),
                  _lib.ptr(st_u8), _lib.ptr(consts), None, None, nb)
    return lo_u8, st_u8, consts


def params_decoded(lo: torch.Tensor, step: torch.Tensor, ldd: int | None = None):
    """:func:`quantize_params` plus the decoded fp32 ``lo_d``/``step_d`` ``[N, ldd]``
    (``hi2/format.py:45-60`` then ``.float()``) in one kernel."""
    dev = _lib.require_gpu(lo, step)
    rows, nb = lo.shape
    ldd = nb if ldd is None else ldd
    l = lo.to(torch.float32).contiguous()
    s = step.to(torch.float32).contiguous()
    lo_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
    st_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
    consts = torch.empty(rows, 3, dtype=torch.float16, device=dev)
    lo_d = torch.zeros(rows, ldd, dtype=torch.float32, device=dev)
    st_d = torch.zeros(rows, ldd, dtype=torch.float32, device=dev)
    if rows:
        _lib.call("hi2x_params", dev, _lib.ptr(l), _lib.ptr(s), rows, nb, _lib.ptr(lo_u8),
                  _lib.ptr(st_u8), _lib.ptr(consts), _lib.ptr(lo_d), _lib.ptr(st_d), ldd)
    return lo_u8, st_u8, consts, lo_d, st_d


@dataclass
class Encoded:
    codes: torch.Tensor  # uint8 [N, K]
    params: torch.Tensor  # uint8 [N, nb, 2]
    consts: torch.Tensor  # fp16 [N, 3]
    sse: torch.Tensor  # float32 [N], activation-weighted squared error
    # stored-basis values the codes are the nearest rounding of (GPTQ: the
    # error-compensated weights when each column was rounded); QAD initialisation
    comp: torch.Tensor | None = None


def encode_rows(
    w: torch.Tensor, d: torch.Tensor, nbits: int, block: int, effort: str = "normal"
) -> Encoded:
    """Quantise ``w[N, K]`` (already in the stored basis) at ``(nbits, block)`` with
    nearest rounding onto the fitted ladders; ``d[K]`` weights the error metric.

    Three kernels over the rows (``hi2/encode.py:133-173``): the ladder fit, the 8-bit
    parameters with their decode, and the codes; the weighted sse is the finish of the
    GPTQ path (the same sum).  No factor and no error propagation."""
    dev = _lib.require_gpu(w, d)
    n_rows, k = w.shape
    if k % block:
        raise ValueError(f"K={k} is not a multiple of the block {block}")
    nb = k // block
    cfg = EFFORT[effort]
    wf = w.to(torch.float32).contiguous()
    if wf.data_ptr() % 16:
        wf = wf.clone()
    dv = d.to(dev, torch.float32).reshape(-1).contiguous()
    lo, st, _ = _fit(wf.reshape(-1, nb, block), dv, 2 ** nbits, cfg["grid"], cfg["ls"], False)
    lo_u8, st_u8, consts, lo_d, st_d = params_decoded(lo, st)
    codes = torch.empty(n_rows, k, dtype=torch.uint8, device=dev)
    sse = torch.empty(n_rows, dtype=torch.float32, device=dev)
    if n_rows:
        _lib.call("hi2x_nearest_codes", dev, _lib.ptr(wf), n_rows, k, block, _lib.ptr(lo_d),
                  _lib.ptr(st_d), nb, int(nbits), _lib.ptr(codes))
        _lib.call("hi2x_finish", dev, _lib.ptr(codes), None, None, n_rows, k, block,
                  _lib.ptr(lo_d), _lib.ptr(st_d), nb, _lib.ptr(wf), _lib.ptr(dv),
                  _lib.ptr(codes), None, _lib.ptr(sse))
    return Encoded(codes, torch.stack([lo_u8, st_u8], dim=-1), consts, sse)
