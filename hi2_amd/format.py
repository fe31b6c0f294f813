"""HadamardINT2-FP16 v3.2 format helpers on the encode path (MI355X).

Mirror of the hot-path part of the reference's ``hi2/format.py`` (same names, argument
meaning and errors): ``GROUP``, ``hadamard16`` (22-27), ``fwht_groups`` (30-41),
``decode_params`` (45-60), ``ladder_dequantize`` (63-69), ``pack_codes`` (73-85),
``HI2Tensor`` / ``FIELDS`` (97-124) and ``assemble`` (127-184), plus ``rotate_rows`` (the
smoothing, rotation and row selection a tensor's weights go through before GPTQ, in one
pass) and ``assemble_many``.  The arithmetic runs in the hi2x HIP kernels; inputs must be device tensors (``assemble`` returns the flat
buffers on the host, as the reference does).  Decode/verification helpers
(``dequantize``, accounting) are not part of the encode path and are not provided.
"""

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

GROUP = 16


def hadamard16(dtype: torch.dtype = torch.float64, device="cpu") -> torch.Tensor:
    """Normalised order-16 Walsh-Hadamard matrix (Sylvester, entries +-1/4):
    symmetric, ``H @ H = I``.  A constant, built on the host."""
    i = torch.arange(GROUP)
    bits = torch.bitwise_and(i[:, None], i[None, :])
    parity = torch.zeros_like(bits)
    for b in range(4):
        parity ^= (bits >> b) & 1
    h = torch.where(parity.bool(), -1.0, 1.0).to(torch.float64) / math.sqrt(GROUP)
    return h.to(dtype=dtype, device=device)


def fwht_groups(x: torch.Tensor, flags: torch.Tensor) -> torch.Tensor:
    """Transform the flagged 16-column groups of ``x[..., K]`` (an involution).

    float32/float64 inputs are transformed in their own precision, other dtypes in
    float64 and cast back, as the reference does."""
    k = x.shape[-1]
    if k % GROUP:
        raise ValueError(f"K={k} must be a multiple of {GROUP}")
    if flags.numel() != k // GROUP:
        raise ValueError(f"flags has {flags.numel()} entries, expected {k // GROUP}")
    dev = _lib.require_gpu(x)
    work = x.dtype if x.dtype in (torch.float32, torch.float64) else torch.float64
    xi = x.to(work).contiguous()
    fl = _lib.to_device(flags.reshape(-1), dev, torch.uint8).contiguous()
    out = torch.empty_like(xi)
    rows = xi.numel() // k if k else 0
    _lib.call("hi2x_fwht16", dev, _lib.ptr(xi), _lib.ptr(out), 0 if work == torch.float32 else 1,
              rows, k, _lib.ptr(fl))
    return out.to(x.dtype)


def rotate_rows(w: torch.Tensor, flags: torch.Tensor | None, rows: torch.Tensor | None = None,
                col_scale: torch.Tensor | None = None) -> torch.Tensor:
    """``fwht_groups(w.float() * col_scale, flags)[rows]`` as float32 in one pass over the
    selected rows (``hi2x_rotate_rows``): the reference's smoothing, staging and
    rotation of a tensor's weights and its row selection per candidate
    (``hi2/calibrate.py:106-111, 329-330, 353-357``), bit for bit.  ``w`` is float32 or
    bfloat16 ``[N, K]``; ``rows`` device or host int64 indices (None: every row; host
    indices are range-checked here, a device index out of range yields a row of NaN)."""
    if w.dim() != 2 or w.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("rotate_rows takes a float32 or bfloat16 [N, K] matrix")
    n_all, k = w.shape
    if k % GROUP:
        raise ValueError(f"K={k} must be a multiple of {GROUP}")
    dev = _lib.require_gpu(w)
    if w.stride(1) != 1 or (w.stride(0) * w.element_size()) % 16:
        w = w.contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
    if rows is not None and rows.device.type == "cpu" and rows.numel():
        if int(rows.min()) < 0 or int(rows.max()) >= n_all:
            raise IndexError(f"row index out of range for {n_all} rows")
    fl = None
    if flags is not None:
        if flags.numel() != k // GROUP:
            raise ValueError(f"flags has {flags.numel()} entries, expected {k // GROUP}")
        fl = _lib.to_device(flags.reshape(-1), dev, torch.uint8).contiguous()
    idx = None if rows is None else _lib.to_device(rows.reshape(-1), dev, torch.int64).contiguous()
    n = n_all if idx is None else idx.numel()
    cs = None
    if col_scale is not None:
        cs = _lib.to_device(col_scale.reshape(-1), dev, torch.float32).contiguous()
        if cs.numel() != k:
            raise ValueError(f"col_scale has {cs.numel()} entries, expected {k}")
    out = torch.empty(n, k, dtype=torch.float32, device=dev)
    _lib.call("hi2x_rotate_rows", dev, _lib.ptr(w), 0 if w.dtype == torch.float32 else 2,
              w.stride(0), n_all, _lib.ptr(idx), n, k, _lib.ptr(cs), _lib.ptr(fl),
              _lib.ptr(out), k)
    return out


# ---- block parameters (spec 2.2) --------------------------------------------------------
def decode_params(
    lo_u8: torch.Tensor,
    step_u8: torch.Tensor,
    lo_min: torch.Tensor,
    lo_scale: torch.Tensor,
    step_scale: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fp16 ``lo``/``step`` of each block from its two bytes and the row constants
    (broadcast): ``lo = fp16(f32(f64(u) * f64(lo_scale) + f64(lo_min)))``,
    ``step = fp16(f32(u) * f32(step_scale))``."""
    dev = _lib.require_gpu(lo_u8, step_u8)
    shape = torch.broadcast_shapes(lo_u8.shape, step_u8.shape, lo_min.shape, lo_scale.shape,
                                   step_scale.shape)
    lu = lo_u8.to(dev, torch.uint8).expand(shape).contiguous().reshape(-1)
    su = step_u8.to(dev, torch.uint8).expand(shape).contiguous().reshape(-1)
    consts = torch.stack(
        [c.to(dev, torch.float16).expand(shape).reshape(-1) for c in (lo_min, lo_scale, step_scale)],
        dim=-1,
    ).contiguous()
    n = lu.numel()
    lo = torch.empty(n, dtype=torch.float16, device=dev)
    st = torch.empty(n, dtype=torch.float16, device=dev)
    if n:
        _lib.call("hi2x_decode_params", dev, _lib.ptr(lu), _lib.ptr(su), _lib.ptr(consts), n, 1,
                  _lib.ptr(lo), _lib.ptr(st))
    return lo.reshape(shape), st.reshape(shape)


def ladder_dequantize(
    codes: torch.Tensor, lo: torch.Tensor, step: torch.Tensor, dtype=torch.float64
) -> torch.Tensor:
    """``lo + code * step`` (codes ``[..., nb, B]``, lo/step ``[..., nb]``) with one
    rounding to fp16; evaluated in float64 (exact) or float32 (candidate search)."""
    if dtype not in (torch.float32, torch.float64):
        raise ValueError(f"dtype {dtype} (float32 or float64)")
    dev = _lib.require_gpu(codes)
    b = codes.shape[-1]
    lo_b = lo.to(dev, torch.float32).expand(codes.shape[:-1]).contiguous()
    st_b = step.to(dev, torch.float32).expand(codes.shape[:-1]).contiguous()
    c8 = codes.to(dev, torch.uint8).contiguous()
    out = torch.empty(codes.shape, dtype=torch.float16, device=dev)
    rows = lo_b.numel()
    if rows:
        _lib.call("hi2x_ladder_dequantize", dev, _lib.ptr(c8), _lib.ptr(lo_b), _lib.ptr(st_b),
                  rows, 1, b, int(dtype == torch.float64), _lib.ptr(out))
    return out


# ---- code packing (v3.1 6.2) --------------------------------------------------------------
def pack_codes(codes: torch.Tensor, nbits: int) -> torch.Tensor:
    """``[..., n]`` codes -> ``[..., n * nbits / 32]`` int32, LSB-first."""
    per_word = 32 // nbits
    n = codes.shape[-1]
    if n % per_word:
        raise ValueError(f"{n} codes is not a multiple of {per_word}")
    dev = _lib.require_gpu(codes)
    if codes.dtype != torch.uint8:
        if codes.numel() and (int(codes.max()) >= 2**nbits or int(codes.min()) < 0):
            raise ValueError("code outside the ladder")
        codes = codes.to(torch.uint8)
    c = codes.contiguous()
    rows = c.numel() // n if n else 0
    out = torch.empty(*codes.shape[:-1], n // per_word, dtype=torch.int32, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("hi2x_pack_codes", dev, _lib.ptr(c), rows, n, int(nbits), _lib.ptr(out),
              _lib.ptr(bad))
    if int(bad.item()):
        raise ValueError("code outside the ladder")
    return out


# ---- tensor container (2.4) ---------------------------------------------------------------
@dataclass
class HI2Tensor:
    """Flat per-tensor buffers of spec 2.4 (CPU tensors)."""

    codes: torch.Tensor  # int32 [sum words_per_row]
    code_off: torch.Tensor  # int32 [R+1]
    blk_params: torch.Tensor  # uint8 [2 * sum K/B_r]: (lo_u8, step_u8) per block
    param_off: torch.Tensor  # int32 [R+1], offsets in blocks
    row_consts: torch.Tensor  # fp16 [R, 3]: lo_min, lo_scale, step_scale
    row_nbits: torch.Tensor  # uint8 [R]
    row_block: torch.Tensor  # uint8 [R]
    had: torch.Tensor  # uint8 [K/16]
    shape: tuple[int, int]
    col_scale: torch.Tensor | None = None


FIELDS = (
    "codes",
    "code_off",
    "blk_params",
    "param_off",
    "row_consts",
    "row_nbits",
    "row_block",
    "had",
)


def assemble(
    pieces: list[tuple[torch.Tensor, ...]],
    row_nbits: torch.Tensor,
    row_block: torch.Tensor,
    had: torch.Tensor,
    k: int,
    col_scale: torch.Tensor | None = None,
    stager=None,
    bad: torch.Tensor | None = None,
) -> HI2Tensor:
    """Flat buffers from per-config row groups ``(rows, codes[r, K] uint8,
    params[r, nb, 2] uint8, consts[r, 3] fp16)``: packing and scatters run on the
    device of the first piece's codes, the result is returned on the host (through
    ``stager.to_host`` when given).

    The host never waits for the device when the pieces' row indices are host tensors
    and ``bad`` is given: ``bad`` (device int32 [1]) then counts codes outside their
    ladder for the caller to check later (several tensors can share one counter);
    without it the count is read here and a nonzero one raises ``ValueError``, as the
    reference does."""
    if not pieces:
        raise ValueError("assemble needs at least one piece on the device")
    dev = _lib.require_gpu(pieces[0][1])
    r = row_nbits.numel()
    nb = row_nbits.to(torch.int64).cpu()
    words = (k * nb) // 32
    blocks = k // row_block.to(torch.int64).cpu()
    code_off = torch.zeros(r + 1, dtype=torch.int64)
    code_off[1:] = torch.cumsum(words, 0)
    param_off = torch.zeros(r + 1, dtype=torch.int64)
    param_off[1:] = torch.cumsum(blocks, 0)
    code_off_d, param_off_d = _lib.h2d(code_off, dev), _lib.h2d(param_off, dev)
    codes = torch.zeros(int(code_off[-1]), dtype=torch.int32, device=dev)
    params = torch.zeros(int(param_off[-1]) * 2, dtype=torch.uint8, device=dev)
    consts = torch.zeros(r, 3, dtype=torch.float16, device=dev)
    own_bad = bad is None
    if own_bad:
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
    keep = []
    for rows, c, p, rc in pieces:
        if rows.device.type == "cpu":
            rows_c = rows
            rows_d = _lib.h2d(rows.to(torch.int64), dev)
        else:
            rows_c = rows[:1].cpu()
            rows_d = rows.to(torch.int64).contiguous()
        if rows.numel() == 0:
            continue
        nbits = int(nb[rows_c[0]])
        blk = k // int(blocks[rows_c[0]])
        c_d = c.to(dev, torch.uint8).contiguous()
        p_d = p.to(dev, torch.uint8).contiguous()
        rc_d = rc.to(dev, torch.float16).contiguous()
        keep += [rows_d, c_d, p_d, rc_d]
        _lib.call("hi2x_assemble_piece", dev, _lib.ptr(rows_d), rows_d.numel(), _lib.ptr(c_d),
                  _lib.ptr(p_d), _lib.ptr(rc_d), k, nbits, blk, _lib.ptr(code_off_d),
                  _lib.ptr(param_off_d), _lib.ptr(codes), _lib.ptr(params), _lib.ptr(consts),
                  _lib.ptr(bad))
    if own_bad and int(bad.item()):
        raise ValueError("code outside the ladder")
    to_host = stager.to_host if stager is not None else (lambda t: t.cpu())
    return HI2Tensor(
        codes=to_host(codes),
        code_off=code_off.to(torch.int32),
        blk_params=to_host(params),
        param_off=param_off.to(torch.int32),
        row_consts=to_host(consts),
        row_nbits=row_nbits.to(torch.uint8).cpu(),
        row_block=row_block.to(torch.uint8).cpu(),
        had=had.to(torch.uint8).reshape(-1).cpu(),
        shape=(r, k),
        col_scale=col_scale,
    )


def assemble_many(tensors: list[dict], stager=None, bad: torch.Tensor | None = None
                  ) -> list[HI2Tensor]:
    """:func:`assemble` of several tensors at once (every expert of an MoE layer): each
    entry of ``tensors`` holds the arguments of one call (``pieces``, ``row_nbits``,
    ``row_block``, ``had``, ``k``, optionally ``col_scale``).  The tensors' buffers are
    views of one allocation per field, the offsets and row lists go to the device in one
    copy, and every piece is packed through one ``hi2x_assemble_batch`` call, so the host
    cost does not grow with a call per piece.  Results equal :func:`assemble` on each; the
    pieces' row lists must be host tensors."""
    if not tensors:
        return []
    dev = _lib.require_gpu(tensors[0]["pieces"][0][1])
    metas, chunks = [], []
    n_words = n_blocks = n_rows = pos = 0
    for t in tensors:
        nb = t["row_nbits"].to(torch.int64).cpu().numpy()
        blocks = t["k"] // t["row_block"].to(torch.int64).cpu().numpy()
        r = nb.size
        code_off = np.zeros(r + 1, np.int64)
        code_off[1:] = np.cumsum((t["k"] * nb) // 32)
        param_off = np.zeros(r + 1, np.int64)
        param_off[1:] = np.cumsum(blocks)
        metas.append((r, nb, blocks, code_off, param_off, n_words, n_blocks, n_rows, pos))
        # device copies shifted into the shared buffers
        chunks += [code_off + n_words, param_off + n_blocks]
        pos += 2 * (r + 1)
        n_words += int(code_off[-1])
        n_blocks += int(param_off[-1])
        n_rows += r
    rows_at = []
    for t in tensors:
        for rows, *_ in t["pieces"]:
            if rows.device.type != "cpu":
                raise RuntimeError("assemble_many takes host row lists")
            rn = rows.numpy().astype(np.int64, copy=False)
            rows_at.append((pos, rn.size, int(rn[0]) if rn.size else 0))
            chunks.append(rn)
            pos += rn.size
    flat = _lib.h2d(torch.from_numpy(np.concatenate(chunks)), dev)
    base = flat.data_ptr()
    codes = torch.zeros(max(n_words, 1), dtype=torch.int32, device=dev)
    params = torch.zeros(max(n_blocks, 1) * 2, dtype=torch.uint8, device=dev)
    consts = torch.zeros(max(n_rows, 1), 3, dtype=torch.float16, device=dev)
    own_bad = bad is None
    if own_bad:
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
    pieces, keep = [], []
    pi = 0
    cbase, pbase, kbase = codes.data_ptr(), params.data_ptr(), consts.data_ptr()
    for t, (r, nb, blocks, code_off, param_off, w0, b0, r0, at0) in zip(tensors, metas):
        k = t["k"]
        co_ptr, po_ptr = base + 8 * at0, base + 8 * (at0 + r + 1)
        for _, c, p, rc in t["pieces"]:
            at, n, first = rows_at[pi]
            pi += 1
            if n == 0:
                continue
            if c.dtype != torch.uint8 or not c.is_contiguous() or c.device != dev:
                c = c.to(dev, torch.uint8).contiguous()
            if p.dtype != torch.uint8 or not p.is_contiguous() or p.device != dev:
                p = p.to(dev, torch.uint8).contiguous()
            if rc.dtype != torch.float16 or not rc.is_contiguous() or rc.device != dev:
                rc = rc.to(dev, torch.float16).contiguous()
            keep += [c, p, rc]
            pieces.append(_lib.Piece(base + 8 * at, n, c.data_ptr(), p.data_ptr(), rc.data_ptr(),
                                     k, int(nb[first]), 0, k // int(blocks[first]), co_ptr,
                                     po_ptr, cbase, pbase, kbase + 6 * r0))
    arr = (_lib.Piece * max(len(pieces), 1))(*pieces)
    _lib.call("hi2x_assemble_batch", dev, ctypes.cast(arr, ctypes.c_void_p), len(pieces),
              _lib.ptr(bad))
    if own_bad and int(bad.item()):
        raise ValueError("code outside the ladder")
    to_host = stager.to_host if stager is not None else (lambda x: x.cpu())
    out = []
    for t, (r, nb, blocks, code_off, param_off, w0, b0, r0, at0) in zip(tensors, metas):
        nw, nbk = int(code_off[-1]), int(param_off[-1])
        out.append(HI2Tensor(
            codes=to_host(codes[w0:w0 + nw]),
            code_off=torch.from_numpy(code_off.astype(np.int32)),
            blk_params=to_host(params[2 * b0:2 * (b0 + nbk)]),
            param_off=torch.from_numpy(param_off.astype(np.int32)),
            row_consts=to_host(consts[r0:r0 + r]),
            row_nbits=t["row_nbits"].to(torch.uint8).cpu(),
            row_block=t["row_block"].to(torch.uint8).cpu(),
            had=t["had"].to(torch.uint8).reshape(-1).cpu(),
            shape=(r, t["k"]),
            col_scale=t.get("col_scale"),
        ))
    return out
