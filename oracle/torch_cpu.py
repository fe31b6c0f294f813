"""The reference's encode path restated in torch on the CPU (test infrastructure).

This is what ``bench.py``'s ``cpu_baseline`` times: the reference's own CPU path (hi2
runs these torch ops on the host when no HIP device is present), written here from the
reference's algorithm so that it can run on the GPU box, where the reference is absent.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it; the product path (``hi2_amd``) never does.

It restates, with the same torch operations in the same order (so that on one torch
build its results are the reference's bit for bit; ``tests/test_torch_cpu.py`` checks
that against the reference-written end-to-end fixtures):

* ``hi2/hessian.py:35-47``: ``HessianStats.update`` (4096-token fp32 chunks, ``S +=
  xc^T xc``) and ``mean``;
* ``hi2/hessian.py:50-68``: ``transform_sigma`` (two group einsums, symmetrised);
* ``hi2/hessian.py:71-86``: ``inverse_factor`` (LAPACK ``cholesky``,
  ``cholesky_inverse``, ``cholesky(upper)``; the damping retries);
* ``hi2/format.py:22-41``: ``hadamard16`` / ``fwht_groups``;
* ``hi2/encode.py:27-92``: ``fit_ladder`` on the torch path (grid of min-max shrinks,
  then ``ls`` weighted least-squares refits);
* ``hi2/encode.py:95-119`` and ``hi2/format.py:45-69``: ``quantize_params``,
  ``decode_params``, ``ladder_dequantize``;
* ``hi2/hessian.py:208-264, 318-345``: ``_prepare`` / ``_round_reference`` /
  ``_finish`` (the column loop with its BLAS trailing update, the weighted sse);
* ``hi2/format.py:73-85``: ``pack_codes``.
"""

import math

import torch

GROUP = 16
BLOCK_COLUMNS = 128
ROW_ELEMS = 1 << 26
GRIDS = {  # hi2/encode.py:18-22: grid of range shrinks and least-squares refits per effort
    "fast": ((0.0, 0.06, 0.12), 1),
    "normal": ((0.0, 0.04, 0.08, 0.12, 0.16, 0.20), 2),
    "max": ((0.0, 0.025, 0.05, 0.075, 0.10, 0.125, 0.15, 0.20), 4),
}


# ---- Hessian, rotation, factor ----------------------------------------------------------
def hessian_sum(x: torch.Tensor, chunk: int = 4096) -> torch.Tensor:
    """sum_t x_t x_t^T over fp32 chunks of ``chunk`` tokens (hi2/hessian.py:35-40)."""
    k = x.shape[-1]
    x = x.reshape(-1, k)
    s = torch.zeros(k, k, dtype=torch.float32)
    for t0 in range(0, x.shape[0], chunk):
        part = x[t0:t0 + chunk].to(torch.float32)
        s += part.T @ part
    return s


def h16(dtype=torch.float64) -> torch.Tensor:
    """Sylvester's order-16 Hadamard matrix over sqrt(16) (hi2/format.py:22-27)."""
    m = torch.ones(1, 1, dtype=torch.float64)
    for _ in range(4):
        m = torch.cat([torch.cat([m, m], 1), torch.cat([m, -m], 1)], 0)
    return (m / math.sqrt(GROUP)).to(dtype)


def rotate(x: torch.Tensor, flags: torch.Tensor) -> torch.Tensor:
    """fwht_groups (hi2/format.py:30-41): the flagged 16-column groups times h16."""
    k = x.shape[-1]
    dt = x.dtype if x.dtype in (torch.float32, torch.float64) else torch.float64
    groups = x.to(dt).reshape(*x.shape[:-1], k // GROUP, GROUP)
    mixed = groups @ h16(dt)
    keep = flags.bool().reshape(-1, 1)
    return torch.where(keep, mixed, groups).reshape(x.shape).to(x.dtype)


def transform_sigma(sigma, col_scale, flags) -> torch.Tensor:
    """hi2/hessian.py:50-68: Hs = M diag(1/s) Sigma diag(1/s) M^T, symmetrised."""
    k = sigma.shape[0]
    g = k // GROUP
    s = sigma.to(torch.float32)
    if col_scale is not None:
        inv = 1.0 / col_scale.to(torch.float32)
        s = s * inv[:, None] * inv[None, :]
    if bool(flags.any()):
        m = torch.where(flags.bool().reshape(-1, 1, 1), h16(torch.float32),
                        torch.eye(GROUP, dtype=torch.float32))
        blocks = s.reshape(g, GROUP, g, GROUP)
        blocks = torch.einsum("gij,gjhk->gihk", m, blocks)
        blocks = torch.einsum("gihk,hlk->gihl", blocks, m)
        s = blocks.reshape(k, k)
    return 0.5 * (s + s.T)


def inverse_factor(hs: torch.Tensor, damp: float = 0.01) -> torch.Tensor:
    """hi2/hessian.py:71-86: chol(H) -> cholesky_inverse -> chol(upper) of the
    symmetrised inverse, H = Hs + damp mean(diag) 10^a I for a = 0..5."""
    k = hs.shape[0]
    mean = hs.diagonal().mean().clamp_min(1e-12)
    eye = torch.eye(k, dtype=hs.dtype)
    for attempt in range(6):
        try:
            low = torch.linalg.cholesky(hs + (damp * mean * 10**attempt) * eye)
            inv = torch.cholesky_inverse(low)
            return torch.linalg.cholesky(0.5 * (inv + inv.T), upper=True)
        except RuntimeError:
            continue
    raise RuntimeError("Hessian is not factorisable even with heavy damping")


# ---- ladder fit and block parameters ------------------------------------------------------
def _nonzero(step):
    return torch.where(step == 0, torch.ones_like(step), step)


def _codes_of(wb, lo, step, levels):
    q = torch.round((wb - lo.unsqueeze(-1)) / _nonzero(step).unsqueeze(-1))
    q = q.clamp(0, levels - 1)
    return lo.unsqueeze(-1) + q * step.unsqueeze(-1), q


def _refit(q, wb, db):
    """Weighted least squares of wb ~ lo + q step per block (hi2/encode.py:32-50)."""
    sd = db.sum(-1)
    sq = (db * q).sum(-1)
    sqq = (db * q * q).sum(-1)
    sw = (db * wb).sum(-1)
    sqw = (db * q * wb).sum(-1)
    det = sd * sqq - sq * sq
    good = det.abs() > 1e-20
    step = torch.where(good, (sd * sqw - sq * sw) / torch.where(good, det, torch.ones_like(det)),
                       torch.zeros_like(det))
    lo = torch.where(good, (sw - step * sq) / sd.clamp_min(1e-20), wb.mean(-1))
    return lo, step


def fit_ladder(wb, db, levels: int, effort: str = "normal"):
    """hi2/encode.py:53-92 on the CPU path: the best (lo, step) of the grid of min-max
    shrinks (strict improvement keeps the earlier candidate), then the refits, each kept
    where it lowers the weighted error with a positive step."""
    grid, refits = GRIDS[effort]
    lo_min, hi_max = wb.amin(-1), wb.amax(-1)
    span = hi_max - lo_min
    best = None
    for a in grid:
        for b in grid:
            lo = lo_min + a * span
            step = (hi_max - b * span - lo) / (levels - 1)
            rec, _ = _codes_of(wb, lo, step, levels)
            err = (db * (rec - wb) ** 2).sum(-1)
            if best is None:
                best = [lo, step, err]
                continue
            better = err < best[2]
            best = [torch.where(better, lo, best[0]), torch.where(better, step, best[1]),
                    torch.where(better, err, best[2])]
    for _ in range(refits):
        _, q = _codes_of(wb, best[0], best[1], levels)
        lo, step = _refit(q, wb, db.expand_as(wb))
        rec, _ = _codes_of(wb, lo, step, levels)
        err = (db * (rec - wb) ** 2).sum(-1)
        better = (err < best[2]) & (step > 0)
        best = [torch.where(better, lo, best[0]), torch.where(better, step, best[1]),
                torch.where(better, err, best[2])]
    return best[0], best[1]


def quantize_params(lo, step):
    """hi2/encode.py:95-119: bytes against the fp16 row constants (lo_min, lo_scale,
    step_scale)."""
    step = step.clamp_min(0)
    s_scale = (step.amax(-1, keepdim=True) / 255).to(torch.float16)
    ss = s_scale.float()
    step_u8 = torch.where(ss > 0, torch.round(step / ss.clamp_min(1e-30)),
                          torch.zeros_like(step)).clamp(0, 255)
    l_min = lo.amin(-1, keepdim=True).to(torch.float16)
    l_scale = ((lo.amax(-1, keepdim=True) - l_min.float()).clamp_min(0) / 255).to(torch.float16)
    ls = l_scale.float()
    lo_u8 = torch.where(ls > 0, torch.round((lo - l_min.float()) / ls.clamp_min(1e-30)),
                        torch.zeros_like(lo)).clamp(0, 255)
    return lo_u8.to(torch.uint8), step_u8.to(torch.uint8), torch.cat([l_min, l_scale, s_scale], -1)


def decode_params(lo_u8, step_u8, consts):
    """hi2/format.py:45-60 with the row constants of ``consts [N, 3]``."""
    c = consts
    lo = (lo_u8.double() * c[:, 1:2].double() + c[:, 0:1].double()).float().to(torch.float16)
    step = (step_u8.float() * c[:, 2:3].float()).to(torch.float16)
    return lo, step


# ---- GPTQ -------------------------------------------------------------------------------
def gptq(w, d, u, nbits: int, block: int, effort: str = "normal"):
    """encode_rows_gptq on the CPU (hi2/hessian.py:208-264, 318-345): per row chunk of
    ROW_ELEMS weights the ladders fitted on the uncompensated rows, then the column loop
    with its per-block BLAS update, then the weighted sse.  Returns (codes uint8, params
    uint8 [N, nb, 2], consts fp16 [N, 3], sse f32 [N], comp f32)."""
    n_rows, k = w.shape
    levels = 2 ** nbits
    nb = k // block
    db = d.to(torch.float32).reshape(1, nb, block)
    out = []
    for r0 in range(0, n_rows, max(1, ROW_ELEMS // k)):
        wc = w[r0:r0 + max(1, ROW_ELEMS // k)].float().clone()
        lo, step = fit_ladder(wc.reshape(-1, nb, block), db, levels, effort)
        lo_u8, step_u8, consts = quantize_params(lo, step)
        lo_h, step_h = decode_params(lo_u8, step_u8, consts)
        lo_d, step_d = lo_h.float(), step_h.float()
        codes = torch.zeros_like(wc)
        comp = torch.zeros_like(wc)
        for i1 in range(0, k, BLOCK_COLUMNS):
            i2 = min(i1 + BLOCK_COLUMNS, k)
            seg = wc[:, i1:i2].clone()
            errs = torch.zeros_like(seg)
            ub = u[i1:i2, i1:i2]
            for i in range(i2 - i1):
                j = i1 + i
                b = j // block
                lo_j, st_j = lo_d[:, b], step_d[:, b]
                col = seg[:, i]
                q = torch.round((col - lo_j) / _nonzero(st_j)).clamp(0, levels - 1)
                q = torch.where(st_j == 0, torch.zeros_like(q), q)
                wq = (lo_j + q * st_j).to(torch.float16).float()
                codes[:, j] = q
                comp[:, j] = col
                e = (col - wq) / ub[i, i]
                seg[:, i:] -= e[:, None] * ub[i, i:][None, :]
                errs[:, i] = e
            wc[:, i2:] -= errs @ u[i1:i2, i2:]
        rec = (lo_d.unsqueeze(-1) + codes.reshape(-1, nb, block) * step_d.unsqueeze(-1))
        rec = rec.to(torch.float16).float().reshape(-1, k)
        diff = rec - w[r0:r0 + wc.shape[0]].float()
        sse = (d.to(torch.float32) * diff ** 2).sum(-1)
        out.append((codes.to(torch.uint8), torch.stack([lo_u8, step_u8], -1), consts, sse, comp))
    return tuple(torch.cat(f) for f in zip(*out))


def pack_codes(codes: torch.Tensor, nbits: int) -> torch.Tensor:
    """hi2/format.py:73-85: LSB-first int32 words."""
    per = 32 // nbits
    n = codes.shape[-1]
    if int(codes.max()) >= 2 ** nbits:
        raise ValueError("code outside the ladder")
    c = codes.to(torch.int64).reshape(*codes.shape[:-1], n // per, per)
    word = torch.zeros(c.shape[:-1], dtype=torch.int64)
    for i in range(per):
        word |= c[..., i] << (nbits * i)
    return torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)
