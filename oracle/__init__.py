"""CPU oracle of the hi2 encode path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker / CPU baseline.  The product package
(``hi2_amd``) never imports, links or calls it.

``libhi2_oracle.so`` is the plain-C restatement in ``hi2_oracle.c`` (each function
cites the reference lines it follows); this module wraps it with numpy and composes
the per-tensor flow of the reference's ``encode_rows_gptq_reference``
(``hi2/hessian.py:89-175``): ladder fit -> 8-bit params -> decode -> GPTQ column loop
-> finish.

Pinning (what holds each function to the reference):

* ``f32_to_f16``: numpy's IEEE round-to-nearest-even ``astype(float16)``.
* ``fwht16``: closed form (Sylvester H16 / 4, involution, float64 matmul).
* ``fit_ladder``: golden vectors of the reference (``tests/golden/fit_ladder.npz``).
* ``params`` (quantize/decode): closed forms of ``hi2/encode.py:95-119`` and
  ``hi2/format.py:45-60`` evaluated independently with numpy, plus the reference's
  constant/zero-block KAT, plus the params inside the GPTQ golden vectors.
* ``gptq_rows`` / ``gptq_block`` / ``finish``: GPTQ golden vectors
  (``tests/golden/gptq_int*.npz``), the diagonal-Hessian special case (nearest
  rounding) and H-error decrease.
* ``hessian_update``: float64 brute force ``X^T X``.
* ``transform_sigma``: covariance of the transformed activation.
* ``inverse_factor``: golden vectors (``tests/golden/inverse_factor.npz``) and
  ``U^T U (Hs + lam I) = I``.
* ``pack_codes`` / ``assemble_piece``: LSB-first KATs and the mixed-row offsets KAT.
* ``refine``: golden vectors of ``refine_groups`` (``tests/golden/refine_*.npz``), the
  reference's sweep invariants and an unblocked float64 column loop.
* ``colstats_update`` / ``colstats_diag``: golden vectors of ``ColumnStats``
  (``tests/golden/colstats.npz``) and float64 brute force.
* ``qad_decode_fwd`` / ``qad_decode_bwd`` / ``qad_wht_scale``: the reference's torch
  graph (``tests/golden/qad.npz``, written from ``hi2.qad.FakeQuantLinear`` on the CPU):
  stored values and latent gradients bit-exact, block gradients and the transform within
  float32 summation rounding; exact sums on integer-valued inputs; the transform against
  the H16 product in float64.
* ``encode_many`` (a composition of the functions above): the golden output of the
  reference's ``encode_many`` (``tests/golden/encode_many.npz``), given the factors the
  reference computed there.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "libhi2_oracle.so")
_lib = None

EFFORT = {
    "fast": dict(grid=(0.0, 0.06, 0.12), ls=1),
    "normal": dict(grid=(0.0, 0.04, 0.08, 0.12, 0.16, 0.20), ls=2),
    "max": dict(grid=(0.0, 0.025, 0.05, 0.075, 0.10, 0.125, 0.15, 0.20), ls=4),
}


def build(force: bool = False) -> str:
    if force or not os.path.exists(_LIB) or (
        os.path.getmtime(_LIB) < os.path.getmtime(os.path.join(_HERE, "hi2_oracle.c"))
    ):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "-s"], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        _lib = ctypes.CDLL(_LIB)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        F = ctypes.c_float
        sig = {
            "or_f32_to_f16": (ctypes.c_uint16, [F]),
            "or_f16_to_f32": (F, [ctypes.c_uint16]),
            "or_fwht16": (None, [P, P, I64, I64, P]),
            "or_fit_ladder": (None, [P, P, I64, I64, I, I, P, I, I, P, P]),
            "or_params": (None, [P, P, I64, I64, P, P, P, P, P]),
            "or_gptq_rows": (None, [P, I64, I64, P, P, P, I64, P, I, P, P]),
            "or_gptq_block": (None, [P, I64, I64, I64, I, P, P, P, P, I64, P, P, P, P, P]),
            "or_finish": (None, [P, P, P, I64, I64, I64, P, P, P, P, P, P, P]),
            "or_hessian_update": (None, [P, I, I64, I64, P]),
            "or_transform_sigma": (None, [P, P, P, I64, P]),
            "or_inverse_factor": (I, [P, I64, F, P]),
            "or_torch_sum_strided": (F, [P, I64, I64]),
            "or_pack_codes": (I64, [P, I64, I64, I, P]),
            "or_assemble_piece": (I64, [P, I64, P, P, P, I64, I, I64, P, P, P, P, P]),
            "or_refine": (I, [P, P, I64, I64, P, P, I64, P, P, P, I, P]),
            "or_colstats_update": (None, [P, I, I64, I64, P]),
            "or_colstats_diag": (None, [P, I64, I64, P, P, P]),
            "or_qad_decode_fwd": (None, [P, P, P, P, P, P, I64, I64, I64, ctypes.c_float, P]),
            "or_qad_decode_bwd": (None, [P, P, P, P, P, P, P, I64, I64, I64, ctypes.c_float,
                                         P, P, P]),
            "or_qad_wht_scale": (None, [P, I64, I64, P, P, I, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16_bits(x):
    x = np.atleast_1d(_c(x, np.float32))
    return np.array([lib().or_f32_to_f16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def fwht16(x, flags):
    x = _c(x, np.float32)
    k = x.shape[-1]
    if k % 16:
        raise ValueError(f"K={k} must be a multiple of 16")
    flags = _c(flags, np.uint8).reshape(-1)
    if flags.size != k // 16:
        raise ValueError("flag count")
    y = np.empty_like(x)
    lib().or_fwht16(_p(x), _p(y), x.size // k, k, _p(flags))
    return y


def fit_ladder(wb, db, n, effort="normal"):
    """``hi2/encode.py:53-92``: wb [N, nb, B], db broadcastable to [nb, B]."""
    wb = _c(wb, np.float32)
    rows, nb, b = wb.shape
    db = _c(np.broadcast_to(np.asarray(db, np.float32).reshape(-1, nb, b)[0], (nb, b)), np.float32)
    cfg = EFFORT[effort]
    grid = np.array(cfg["grid"], np.float32)
    lo = np.empty((rows, nb), np.float32)
    st = np.empty((rows, nb), np.float32)
    lib().or_fit_ladder(_p(wb), _p(db), rows, nb, b, int(n), _p(grid), grid.size,
                        cfg["ls"], _p(lo), _p(st))
    return lo, st


def params(lo, step):
    """quantize_params + decode_params: returns lo_u8, step_u8, consts (fp16 bits
    [N, 3]), lo_d, step_d (fp32)."""
    lo = _c(lo, np.float32)
    step = _c(step, np.float32)
    rows, nb = lo.shape
    lo_u8 = np.empty((rows, nb), np.uint8)
    st_u8 = np.empty((rows, nb), np.uint8)
    consts = np.empty((rows, 3), np.uint16)
    lo_d = np.empty((rows, nb), np.float32)
    st_d = np.empty((rows, nb), np.float32)
    lib().or_params(_p(lo), _p(step), rows, nb, _p(lo_u8), _p(st_u8), _p(consts),
                    _p(lo_d), _p(st_d))
    return lo_u8, st_u8, consts, lo_d, st_d


def gptq_rows(wc, u, lo_d, step_d, blk_of, nbits, want_comp=True):
    wc = _c(wc, np.float32).copy()
    n, k = wc.shape
    u = _c(u, np.float32)
    lo_d = _c(lo_d, np.float32)
    step_d = _c(step_d, np.float32)
    blk_of = _c(blk_of, np.int64)
    codes = np.zeros((n, k), np.uint8)
    comp = np.zeros((n, k), np.float32) if want_comp else None
    lib().or_gptq_rows(_p(wc), n, k, _p(u), _p(lo_d), _p(step_d), lo_d.shape[1],
                       _p(blk_of), 2 ** int(nbits), _p(codes), _p(comp))
    return codes, comp


def gptq_block(wc, i1, length, lo, st, row_grp, us, blk, nmax, want_comp=True):
    """The one-block contract of ``hi2/gptq_kernel.py:59-101``."""
    wc = _c(wc, np.float32)
    n, k = wc.shape
    lo = _c(lo, np.float32)
    st = _c(st, np.float32)
    row_grp = _c(row_grp, np.int32)
    us = [_c(u, np.float32) for u in us]
    ptrs = (ctypes.c_void_p * len(us))(*[u.ctypes.data for u in us])
    blk = _c(blk, np.int32)
    nmax = _c(nmax, np.float32)
    err1 = np.zeros((n, length), np.float32)
    codes = np.zeros((n, k), np.uint8)
    comp = np.zeros((n, k), np.float32) if want_comp else None
    lib().or_gptq_block(_p(wc), n, k, int(i1), int(length), _p(err1), _p(codes), _p(lo),
                        _p(st), lo.shape[1], _p(row_grp), ctypes.cast(ptrs, ctypes.c_void_p),
                        _p(blk), _p(nmax), _p(comp))
    return err1, codes, comp


def finish(codes_ro, comp_ro, perm, block, lo_d, step_d, w, d):
    codes_ro = _c(codes_ro, np.uint8)
    n, k = codes_ro.shape
    comp_ro = None if comp_ro is None else _c(comp_ro, np.float32)
    perm = None if perm is None else _c(perm, np.int64)
    codes = np.zeros((n, k), np.uint8)
    comp = None if comp_ro is None else np.zeros((n, k), np.float32)
    sse = np.zeros(n, np.float32)
    lib().or_finish(_p(codes_ro), _p(comp_ro), _p(perm), n, k, int(block),
                    _p(_c(lo_d, np.float32)), _p(_c(step_d, np.float32)),
                    _p(_c(w, np.float32)), _p(_c(d, np.float32)), _p(codes), _p(comp), _p(sse))
    return codes, comp, sse


def encode_rows_gptq(w, d, u, nbits, block, effort="normal", perm=None, comp=True):
    """The reference flow of ``encode_rows_gptq_reference`` (``hi2/hessian.py:89-175``)
    on numpy arrays.  Returns dict(codes, params, consts (fp16 bits), sse, comp)."""
    w = _c(w, np.float32)
    n, k = w.shape
    d = _c(d, np.float32).reshape(-1)
    nb = k // block
    lo, st = fit_ladder(w.reshape(n, nb, block), d.reshape(1, nb, block), 2 ** nbits, effort)
    lo_u8, st_u8, consts, lo_d, st_d = params(lo, st)
    if perm is not None:
        perm = _c(perm, np.int64)
        wc = w[:, perm]
        blk_of = perm // block
    else:
        wc = w
        blk_of = np.arange(k, dtype=np.int64) // block
    codes_ro, comp_ro = gptq_rows(wc, u, lo_d, st_d, blk_of, nbits, comp)
    codes, compo, sse = finish(codes_ro, comp_ro, perm, block, lo_d, st_d, w, d)
    return dict(codes=codes, params=np.stack([lo_u8, st_u8], -1), consts=consts, sse=sse,
                comp=compo, lo_d=lo_d, step_d=st_d)


def encode_rows(w, d, nbits, block, effort="normal"):
    """``hi2/encode.py:133-173`` (nearest rounding): the ladder fit and params as above,
    then ``codes = clamp(where(step == 0, 0, rint((w - lo) / safe(step))), 0, 2^n - 1)``
    in float32 (IEEE division, half-to-even) and the weighted sse of the finish.
    Returns dict(codes, params, consts, sse, lo_d, step_d)."""
    w = _c(w, np.float32)
    n, k = w.shape
    d = _c(d, np.float32).reshape(-1)
    nb = k // block
    lo, st = fit_ladder(w.reshape(n, nb, block), d.reshape(1, nb, block), 2 ** nbits, effort)
    lo_u8, st_u8, consts, lo_d, st_d = params(lo, st)
    lo_e = np.repeat(lo_d, block, axis=1)
    st_e = np.repeat(st_d, block, axis=1)
    safe = np.where(st_e == 0, np.float32(1), st_e).astype(np.float32)
    with np.errstate(invalid="ignore"):
        q = np.rint((w - lo_e) / safe).astype(np.float32)
    q = np.where(st_e == 0, np.float32(0), q)
    q = np.clip(q, 0, 2 ** nbits - 1)
    codes = q.astype(np.uint8)
    codes, _, sse = finish(codes, None, None, block, lo_d, st_d, w, d)
    return dict(codes=codes, params=np.stack([lo_u8, st_u8], -1), consts=consts, sse=sse,
                lo_d=lo_d, step_d=st_d)


def hessian_update(s, x):
    """S += X^T X; x is float32 or bf16 given as uint16 bits."""
    s = _c(s, np.float32)
    x = np.ascontiguousarray(x)
    is_bf16 = x.dtype == np.uint16
    if not is_bf16:
        x = _c(x, np.float32)
    t, k = x.shape
    lib().or_hessian_update(_p(x), int(is_bf16), t, k, _p(s))
    return s


def transform_sigma(sigma, col_scale_bits, had):
    sigma = _c(sigma, np.float32)
    k = sigma.shape[0]
    out = np.empty_like(sigma)
    cs = None if col_scale_bits is None else _c(col_scale_bits, np.uint16)
    lib().or_transform_sigma(_p(sigma), _p(cs), _p(_c(had, np.uint8)), k, _p(out))
    return out


def damp_lambda(hs, damp=0.01, attempt=0):
    """The damping term of attempt ``attempt`` of inverse_factor (hi2/hessian.py:75-79):
    damp * max(mean(diag hs), 1e-12) * 10^attempt in fp32, the mean as torch's CPU
    reduction of the strided diagonal (hi2_oracle.c: or_torch_sum_strided)."""
    hs = np.ascontiguousarray(hs, dtype=np.float32)
    k = hs.shape[0]
    s = np.float32(lib().or_torch_sum_strided(_p(hs), k, k + 1))
    mean = np.float32(s / np.float32(k))
    mean = max(mean, np.float32(1e-12))
    p10 = np.float32(1.0)
    for _ in range(attempt):
        p10 = np.float32(p10 * np.float32(10.0))
    return np.float32(np.float32(np.float32(damp) * mean) * p10)


def torch_sum_strided(x, n, stride):
    """sum of x[0], x[stride], ..., x[(n-1) stride] in torch's CPU reduction order."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if n and (n - 1) * stride >= x.size:
        raise ValueError("strided vector exceeds the array")
    return np.float32(lib().or_torch_sum_strided(_p(x), n, stride))


def inverse_factor(hs, damp=0.01):
    """Returns (U, attempt); raises RuntimeError when every attempt fails."""
    hs = _c(hs, np.float32)
    k = hs.shape[0]
    u = np.zeros_like(hs)
    att = lib().or_inverse_factor(_p(hs), k, float(damp), _p(u))
    if att < 0:
        raise RuntimeError("Hessian is not factorisable even with heavy damping")
    return u, att


def pack_codes(codes, nbits):
    codes = _c(codes, np.uint8)
    k = codes.shape[-1]
    per = 32 // nbits
    if k % per:
        raise ValueError(f"{k} codes is not a multiple of {per}")
    rows = codes.size // k
    out = np.empty((rows, k // per), np.int32)
    bad = lib().or_pack_codes(_p(codes), rows, k, int(nbits), _p(out))
    if bad:
        raise ValueError("code outside the ladder")
    return out.reshape(*codes.shape[:-1], k // per)


def assemble(pieces, row_nbits, row_block, k):
    """Flat buffers of ``hi2/format.py:127-184`` from (rows, codes, params, consts
    fp16 bits) pieces."""
    row_nbits = np.asarray(row_nbits, np.int64)
    row_block = np.asarray(row_block, np.int64)
    r = row_nbits.size
    words = (k * row_nbits) // 32
    blocks = k // row_block
    code_off = np.zeros(r + 1, np.int64)
    code_off[1:] = np.cumsum(words)
    param_off = np.zeros(r + 1, np.int64)
    param_off[1:] = np.cumsum(blocks)
    codes = np.zeros(int(code_off[-1]), np.int32)
    params_ = np.zeros(int(param_off[-1]) * 2, np.uint8)
    consts = np.zeros((r, 3), np.uint16)
    for rows, c, p, rc in pieces:
        rows = _c(rows, np.int64)
        nbits = int(row_nbits[rows[0]])
        blk = int(row_block[rows[0]])
        bad = lib().or_assemble_piece(_p(rows), rows.size, _p(_c(c, np.uint8)),
                                      _p(_c(p, np.uint8)), _p(_c(rc, np.uint16)), k, nbits,
                                      blk, _p(code_off), _p(param_off), _p(codes), _p(params_),
                                      _p(consts))
        if bad:
            raise ValueError("code outside the ladder")
    return dict(codes=codes, code_off=code_off.astype(np.int32), blk_params=params_,
                param_off=param_off.astype(np.int32), row_consts=consts)


def refine(w, codes, lo, st, block, top, hs, passes):
    """Local code refinement (``hi2/refine.py:43-106``) of rows ``w [n, k]`` with codes
    ``[n, k]`` u8, decoded ladders ``lo/st [n, k / block]`` (``block`` and ``top`` scalars
    or per-row arrays), Hessian ``hs [k, k]``.  Returns (codes, moved per row, sweeps run)."""
    w = _c(w, np.float32)
    n, k = w.shape
    codes = _c(codes, np.uint8).copy()
    lo = _c(lo, np.float32)
    st = _c(st, np.float32)
    block = _c(np.broadcast_to(np.asarray(block), (n,)), np.int32)
    top = _c(np.broadcast_to(np.asarray(top, np.float32), (n,)), np.float32)
    moved = np.zeros(n, np.int64)
    sweeps = lib().or_refine(_p(w), _p(codes), n, k, _p(lo), _p(st), lo.shape[1] if lo.ndim == 2 else 0,
                             _p(block), _p(top), _p(_c(hs, np.float32)), int(passes), _p(moved))
    return codes, moved, sweeps


def colstats_update(s, x):
    """ColumnStats.update (``hi2/stats.py:26-33``) into ``s [K/16, 16, 16]`` float64 in
    place; ``x [t, K]`` float32, or bf16 bits as uint16."""
    x = np.ascontiguousarray(x)
    assert s.dtype == np.float64 and s.flags.c_contiguous
    lib().or_colstats_update(_p(x), 1 if x.dtype == np.uint16 else 0, x.shape[0], x.shape[1],
                             _p(s))
    return s


def colstats_diag(s, n, flags=None, inv_scale=None):
    """ColumnStats.diag (``hi2/stats.py:39-55``): float32 ``[K]``."""
    s = _c(s, np.float64)
    k = s.shape[0] * 16
    out = np.zeros(k, np.float32)
    fl = None if flags is None else _c(flags, np.uint8)
    inv = None if inv_scale is None else _c(inv_scale, np.float32)
    lib().or_colstats_diag(_p(s), k, int(n), _p(fl), _p(inv), _p(out))
    return out


def _f16_bits_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def encode_many(tensors, cands, cfg, factors=None):
    """The orchestration of ``encode_many`` (``hi2/calibrate.py:297-424``) on one device,
    composed of the functions above.  ``tensors``: dicts with ``w`` f32 [R, K]
    (original basis), ``had``, ``picks``, ``col_scale`` (fp16 bits) or None, ``sigma``
    or None, ``sigma_id`` or None, ``stats`` ``(S, n)`` or None, ``comp`` (bool).
    ``cfg``: dict(rounding, act_order, refine_passes, effort, damp=0.01).  ``factors``:
    the inverse factors to use, in the order the distinct inputs first appear
    (default: :func:`inverse_factor`).  Returns per tensor ``(packed dict, comp)``."""
    fac = None if factors is None else list(factors)
    damp = cfg.get("damp", 0.01)
    chains = {}
    out = []
    for i, t in enumerate(tensors):
        w = np.ascontiguousarray(t["w"], np.float32)
        r, k = w.shape
        cs = t["col_scale"]
        s = None if cs is None else _f16_bits_to_f32(cs)
        ws = w * s if s is not None else w  # one fp32 rounding, as torch's host multiply
        had = np.asarray(t["had"], np.uint8).reshape(-1)
        wt = fwht16(ws, had) if had.any() else ws
        gptq = cfg["rounding"] == "gptq" and t["sigma"] is not None
        perm = None
        if gptq:
            key = (t["sigma_id"] if t["sigma_id"] is not None else f"#{i}",
                   None if cs is None else np.asarray(cs, np.uint16).tobytes(), had.tobytes())
            if key not in chains:
                hs = transform_sigma(t["sigma"], cs, had)
                d = np.diag(hs).copy()
                if cfg["act_order"]:
                    p = np.argsort(-d, kind="stable")
                    hs = np.ascontiguousarray(hs[p][:, p])
                else:
                    p = None
                u = fac.pop(0) if fac is not None else inverse_factor(hs, damp)[0]
                chains[key] = (hs, d, u, p)
            hs, d, u, perm = chains[key]
        else:
            if t["stats"] is None:
                d = np.ones(k, np.float32)
            else:
                inv = None if s is None else (np.float32(1.0) / s).astype(np.float32)
                d = colstats_diag(t["stats"][0], t["stats"][1], had, inv)
            u = np.eye(k, dtype=np.float32)
        picks = np.asarray(t["picks"], np.int64)
        refine_rows = gptq and cfg["refine_passes"] and perm is None and not t["comp"]
        pieces = []
        comp = np.zeros((r, k), np.float32) if t["comp"] else None
        for ci, (nb, b) in enumerate(cands):
            rows = np.nonzero(picks == ci)[0]
            if rows.size == 0:
                continue
            e = encode_rows_gptq(wt[rows], d, u, nb, b, cfg["effort"], perm,
                                 comp=bool(gptq and t["comp"]))
            codes = e["codes"]
            if refine_rows:
                codes, _, _ = refine(wt[rows], codes, e["lo_d"], e["step_d"], b, 2 ** nb - 1,
                                     hs, cfg["refine_passes"])
            pieces.append((rows, codes, e["params"], e["consts"]))
            if comp is not None:
                comp[rows] = e["comp"] if gptq else wt[rows]
        nbits = np.array([cands[c][0] for c in picks], np.int64)
        block = np.array([cands[c][1] for c in picks], np.int64)
        packed = assemble(pieces, nbits, block, k)
        packed.update(row_nbits=nbits.astype(np.uint8), row_block=block.astype(np.uint8),
                      had=had)
        out.append((packed, comp))
    return out


def qad_decode_fwd(latent, unit, lo_u, st_u, consts_bits, rows, block, nbits, out=None):
    """decode_fwd (``hi2/qad_kernel.py:88-108``) into ``out`` [R, K] (rows of the group)."""
    latent = _c(latent, np.float32)
    r_all, k = latent.shape
    out = np.zeros_like(latent) if out is None else out
    rows = _c(rows, np.int64)
    lib().or_qad_decode_fwd(_p(latent), _p(None if unit is None else _c(unit, np.float32)),
                            _p(_c(lo_u, np.float32)), _p(_c(st_u, np.float32)),
                            _p(_c(consts_bits, np.uint16)), _p(rows), rows.size, k, int(block),
                            float(2 ** nbits - 1), _p(out))
    return out


def qad_decode_bwd(grad, latent, unit, lo_u, st_u, consts_bits, rows, block, nbits,
                   g_latent=None):
    """decode_bwd (``hi2/qad_kernel.py:110-159``): (g_latent [R, K], g_lo, g_st)."""
    latent = _c(latent, np.float32)
    k = latent.shape[1]
    rows = _c(rows, np.int64)
    g_latent = np.zeros_like(latent) if g_latent is None else g_latent
    nb = k // int(block)
    g_lo = np.zeros((rows.size, nb), np.float32)
    g_st = np.zeros((rows.size, nb), np.float32)
    lib().or_qad_decode_bwd(_p(_c(grad, np.float32)), _p(latent),
                            _p(None if unit is None else _c(unit, np.float32)),
                            _p(_c(lo_u, np.float32)), _p(_c(st_u, np.float32)),
                            _p(_c(consts_bits, np.uint16)), _p(rows), rows.size, k, int(block),
                            float(2 ** nbits - 1), _p(g_latent), _p(g_lo), _p(g_st))
    return g_latent, g_lo, g_st


def qad_wht_scale(x, flags, scale_bits, pre_div):
    """wht_scale (``hi2/qad_kernel.py:165-189``)."""
    x = _c(x, np.float32)
    n, k = x.shape
    out = np.zeros_like(x)
    lib().or_qad_wht_scale(_p(x), n, k, _p(_c(flags, np.uint8)),
                           _p(None if scale_bits is None else _c(scale_bits, np.uint16)),
                           int(bool(pre_div)), _p(out))
    return out


def moe_top_up(sums, counts, need):
    """The MoE token floor (``hi2/layerwise.py:241-257`` with ``blend``,
    ``hi2/moe.py:152-156``) on the experts' sums ``[E, K, K]`` (float32): with tot the
    float32 sum of all experts' sums in expert order (Python's ``sum``: ``0 + S_0``, then
    ``+ S_1`` ...), every expert with ``n_e < need`` (when any expert saw a token)
    becomes ``S_e + float32((need - n_e) / n_total) * tot`` and ``n_e = need``.  Returns
    ``(sums, counts)`` (new arrays)."""
    sums = np.asarray(sums, np.float32)
    counts = [int(c) for c in counts]
    tot_n = sum(counts)
    tot = np.float32(0) + sums[0]
    for e in range(1, len(sums)):
        tot = tot + sums[e]
    out, out_n = sums.copy(), list(counts)
    for e, n in enumerate(counts):
        if n >= need or tot_n == 0:
            continue
        fill = np.float32((need - n) / max(tot_n, 1))
        out[e] = sums[e] + fill * tot
        out_n[e] = need
    return out, out_n
