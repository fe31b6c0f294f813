"""Hessian-aware (error-compensated) rounding on MI355X, spec 8.3.

Mirror of the reference's ``hi2/hessian.py`` (same names, argument meaning, module
globals and errors): ``HessianStats`` (26-47), ``transform_sigma`` (50-68),
``inverse_factor`` (71-86), ``encode_rows_gptq_reference`` (89-175), ``GptqJob``
(178-188), ``_Unit`` / ``_prepare`` / ``_round_kernel`` / ``_finish`` (191-345),
``encode_jobs_gptq`` (359-416), ``encode_rows_gptq`` (419-443).  ``encode_jobs_gptq`` is
also offered in its two halves, ``prepare_jobs_gptq`` (copies, ladder fits, block
parameters: nothing that needs the factor) and ``round_prepared``, so that a caller can
fit a linear's ladders while its input's factor is still being computed.

Every arithmetic step runs in the hi2x HIP kernels (``libhi2x.so``):

* ``HessianStats.update``: ``hi2x_hessian_syrk_upper`` (bf16 / f32 MFMA), with
  ``hi2x_hessian_mirror`` when ``S`` is read (exactly symmetric);
* ``transform_sigma``: ``hi2x_sigma_transform`` (bit-identical to the reference einsums);
  ``HessianStats.transformed`` fuses the mean and the transform over the upper triangle
  (``hi2x_sigma_transform_upper``, the same bits);
* ``inverse_factor``: ``hi2x_chol_inv_upper`` (reversed blocked Cholesky + triangular
  inverse on f32 MFMA), the damping retry driven here as in the reference;
* the ladder fit / 8-bit params (``hi2x_ladder_fit``, ``hi2x_params``), the column loop
  with its cross-block updates (``hi2x_gptq_run``) and ``_finish`` (``hi2x_finish``),
  all bit-identical to the reference's torch CPU path for the same ``(w, d, u)``.

Inputs must be HIP device tensors; there is no CPU or torch fallback
(``backend="torch"`` raises).
"""

import os
from dataclasses import dataclass

import torch

from . import _lib
from .encode import EFFORT, Encoded, _fit, params_decoded
from .format import GROUP

BLOCK_COLUMNS = 128  # lazy-update block of GPTQ
ROW_ELEMS = 1 << 26  # rows per chunk are bounded so the working copies fit
# chunks of several jobs batched through one kernel launch sequence (weights per batch).
# 2^28 (a working copy of at most 1 GiB f32, so that every byte offset into a batch
# buffer stays below 2^30) where the reference takes 2^27: batching never changes a
# result, and bigger batches fill the chip in fewer sequential launch chains (the 70B
# layer's down_proj, 8192 rows at K = 28672, in one batch of 512 column-loop workgroups
# instead of two of 275 and 238: that layer 207.8-208.7 -> 202.4-203.5 ms; the 8B block
# and the MoE layer unchanged).
BATCH_ELEMS = int(os.environ.get("HI2_BATCH_ELEMS", 1 << 28))
# 128-column blocks whose far-column updates share one pass over the working copy
SUPER_BLOCKS = int(os.environ.get("HI2_SUPER_BLOCKS", 0))  # 0: by width (_super_blocks)


def _super_blocks(k: int) -> int:
    """Blocks per lazy super-block of the column loop: eight for the widest layers
    (K >= 8192: half the passes over the trailing columns, measured 8.87 -> 8.41 ms of
    trailing updates at 4096 x 14336), four below (eight measured slightly slower at
    14336 x 4096, where the near updates grow)."""
    if SUPER_BLOCKS > 0:
        return SUPER_BLOCKS
    return 8 if k >= 8192 else 4

__all__ = [
    "EFFORT",
    "GptqJob",
    "HessianStats",
    "PreparedJobs",
    "encode_jobs_gptq",
    "encode_rows_gptq",
    "encode_rows_gptq_reference",
    "finish_factor",
    "inverse_factor",
    "inverse_factor_async",
    "inverse_factors",
    "inverse_factors_batched",
    "inverse_factors_batched_async",
    "finish_factors_batched",
    "prepare_jobs_gptq",
    "round_prepared",
    "transform_sigma",
]


class HessianStats:
    """Full second moment ``sum x x^T`` of a Linear's input (fp32, ``[K, K]``) on a HIP
    device; ``update`` accumulates on MFMA (bf16 inputs exactly, fp32 inputs on f32
    MFMA, other dtypes converted to fp32 first as the reference does).

    ``update`` brings only the upper triangle up to date; the lower one is mirrored when
    ``S`` is read (``S``, ``mean``, ``merge``), and ``transformed`` reads the upper
    triangle directly, so the encode path never pays for the mirror."""

    def __init__(self, k: int, device="cuda"):
        self.k = k
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(
                f"hi2_amd.HessianStats accumulates on the MI355X; got device {dev}"
            )
        self._S = torch.zeros(k, k, dtype=torch.float32, device=dev)
        self._upper_only = False
        self.n = 0

    @property
    def S(self) -> torch.Tensor:
        if self._upper_only:
            _lib.call("hi2x_hessian_mirror", self._S.device, _lib.ptr(self._S), self.k)
            self._upper_only = False
        return self._S

    @S.setter
    def S(self, value: torch.Tensor) -> None:
        self._S = value
        self._upper_only = False

    @torch.no_grad()
    def update(self, x: torch.Tensor, chunk: int = 4096) -> None:
        """``S += x^T x`` over all rows of ``x[..., K]`` (``chunk`` is accepted for
        interface compatibility; the kernel streams the rows itself)."""
        x = x.reshape(-1, self.k)
        dev = self._S.device
        if x.dtype not in (torch.bfloat16, torch.float32):
            x = x.to(torch.float32)
        x = x.to(dev).contiguous()
        t = x.shape[0]
        if t:
            if self._S.dtype != torch.float32 or not self._S.is_contiguous():
                self._S = self.S.to(torch.float32).contiguous()
            dtype = 2 if x.dtype == torch.bfloat16 else 0
            ws = _lib.workspace(dev, "hi2x_hessian_workspace_bytes", dtype, t, self.k)
            _lib.call("hi2x_hessian_syrk_upper", dev, _lib.ptr(x), dtype, t, self.k,
                      _lib.ptr(self._S), _lib.ptr(ws), ws.numel())
            self._upper_only = True
        self.n += t

    def merge(self, other: "HessianStats") -> None:
        self.S += other.S.to(self.S.device)
        self.n += other.n

    def mean(self) -> torch.Tensor:
        # a device tensor divisor keeps this an IEEE division per element (a Python
        # scalar would turn into a multiplication by its reciprocal on the GPU)
        s = self.S
        return s / torch.tensor(float(max(self.n, 1)), dtype=s.dtype, device=s.device)

    def transformed(self, col_scale: torch.Tensor | None, had: torch.Tensor) -> torch.Tensor:
        """``transform_sigma(self.mean(), col_scale, had)`` in one pass over the upper
        triangle of ``S``, bit for bit."""
        k = self.k
        if k % GROUP:
            raise ValueError(f"K={k} must be a multiple of {GROUP}")
        s = self._S
        if s.dtype != torch.float32 or not s.is_contiguous():
            return transform_sigma(self.mean(), col_scale, had)
        dev = s.device
        fl = _lib.to_device(had.reshape(-1), dev, torch.uint8).contiguous()
        if fl.numel() != k // GROUP:
            raise ValueError(f"had has {fl.numel()} entries, expected {k // GROUP}")
        cs = None
        if col_scale is not None:
            cs = _lib.to_device(col_scale.reshape(-1), dev, torch.float16).contiguous()
        out = torch.empty_like(s)
        _lib.call("hi2x_sigma_transform_upper", dev, _lib.ptr(s), self.n, _lib.ptr(cs),
                  _lib.ptr(fl), k, _lib.ptr(out))
        return out


def transform_sigma(
    sigma: torch.Tensor, col_scale: torch.Tensor | None, had: torch.Tensor
) -> torch.Tensor:
    """``Hs = T Sigma T^T`` with ``T = R diag(1/s)`` (R block-diagonal, flagged groups),
    symmetrised."""
    k = sigma.shape[0]
    if k % GROUP:
        raise ValueError(f"K={k} must be a multiple of {GROUP}")
    dev = _lib.require_gpu(sigma)
    s = sigma.to(torch.float32).contiguous()
    fl = _lib.to_device(had.reshape(-1), dev, torch.uint8).contiguous()
    if fl.numel() != k // GROUP:
        raise ValueError(f"had has {fl.numel()} entries, expected {k // GROUP}")
    cs = None
    if col_scale is not None:
        cs = _lib.to_device(col_scale.reshape(-1), dev, torch.float16).contiguous()
    out = torch.empty_like(s)
    _lib.call("hi2x_sigma_transform", dev, _lib.ptr(s), _lib.ptr(cs), _lib.ptr(fl), k,
              _lib.ptr(out))
    return out


def inverse_factor(hs: torch.Tensor, damp: float = 0.01) -> torch.Tensor:
    """Upper Cholesky factor ``U`` of ``(Hs + damp * mean(diag) I)^-1``; the damping is
    raised tenfold (up to five times) if the factorisation fails."""
    dev = _lib.require_gpu(hs)
    k = hs.shape[0]
    h = hs.to(torch.float32).contiguous()
    u = torch.empty_like(h)
    ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", k)
    last = None
    for attempt in range(6):
        try:
            _lib.call("hi2x_chol_inv_upper", dev, _lib.ptr(h), k, float(damp), attempt,
                      _lib.ptr(u), _lib.ptr(ws), ws.numel())
            return u
        except _lib.NotPositiveDefinite as e:
            last = e
    raise RuntimeError(f"Hessian is not factorisable even with heavy damping: {last}")


_OK = 0x7FFFFFFF  # status word of a successful factorisation


def inverse_factor_async(hs: torch.Tensor, damp: float = 0.01):
    """First attempt of :func:`inverse_factor`, enqueued on the current stream without
    waiting for it: returns ``(u, status)`` with ``status`` a device int32 that reads
    0x7FFFFFFF once the factorisation has succeeded.  :func:`finish_factor` checks it
    (and retries with more damping) when the caller is ready to wait."""
    dev = _lib.require_gpu(hs)
    h = hs.to(torch.float32).contiguous()
    u = torch.empty_like(h)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", h.shape[0])
    _lib.call("hi2x_chol_inv_upper_async", dev, _lib.ptr(h), h.shape[0], float(damp), 0,
              _lib.ptr(u), _lib.ptr(status), _lib.ptr(ws), ws.numel())
    return u, status


def finish_factor(hs: torch.Tensor, u: torch.Tensor, status: torch.Tensor,
                  damp: float = 0.01) -> bool:
    """Wait for an :func:`inverse_factor_async` result; if that attempt failed, redo the
    reference's damping retries into ``u``.  Returns True when ``u`` was recomputed
    (work that consumed it must then be redone)."""
    if int(status.item()) == _OK:
        return False
    dev = u.device
    h = hs.to(torch.float32).contiguous()
    ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", h.shape[0])
    last = None
    for attempt in range(1, 6):
        try:
            _lib.call("hi2x_chol_inv_upper", dev, _lib.ptr(h), h.shape[0], float(damp),
                      attempt, _lib.ptr(u), _lib.ptr(ws), ws.numel())
            return True
        except _lib.NotPositiveDefinite as e:
            last = e
    raise RuntimeError(f"Hessian is not factorisable even with heavy damping: {last}")


def inverse_factors(hss: list[torch.Tensor], damp: float = 0.01) -> list[torch.Tensor]:
    """:func:`inverse_factor` of several Hessians (distinct calibration inputs) at once:
    the first attempt of every factor runs on its own stream, concurrently; the status
    words are read after one synchronisation and any factor that needs more damping is
    retried as :func:`inverse_factor` would.  Same results as calling it on each."""
    if not hss:
        return []
    dev = _lib.require_gpu(*hss)
    main = torch.cuda.current_stream(dev)
    hs32 = [h.to(torch.float32).contiguous() for h in hss]
    us = [torch.empty_like(h) for h in hs32]
    status = torch.empty(len(hss), dtype=torch.int32, device=dev)
    streams = [_lib.side_stream(dev, i) for i in range(len(hss))]
    for i, (h, u, st) in enumerate(zip(hs32, us, streams)):
        st.wait_stream(main)
        with torch.cuda.stream(st):
            ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", h.shape[0])
            _lib.call("hi2x_chol_inv_upper_async", dev, _lib.ptr(h), h.shape[0], float(damp), 0,
                      _lib.ptr(u), _lib.ptr(status[i:i + 1]), _lib.ptr(ws), ws.numel())
        for t in (h, u, status):
            t.record_stream(st)
    for st in streams:
        main.wait_stream(st)
    ok = status.cpu().tolist()
    out = []
    for h, u, stv in zip(hs32, us, ok):
        if stv == _OK:
            out.append(u)
            continue
        last = None
        ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", h.shape[0])
        for attempt in range(1, 6):
            try:
                _lib.call("hi2x_chol_inv_upper", dev, _lib.ptr(h), h.shape[0], float(damp),
                          attempt, _lib.ptr(u), _lib.ptr(ws), ws.numel())
                break
            except _lib.NotPositiveDefinite as e:
                last = e
        else:
            raise RuntimeError(f"Hessian is not factorisable even with heavy damping: {last}")
        out.append(u)
    return out


def inverse_factors_batched_async(hs: torch.Tensor, damp: float = 0.01):
    """First attempt of :func:`inverse_factor` for a batch of Hessians of one size
    (``hs [E, K, K]``, e.g. the experts of an MoE projection), enqueued as one launch
    sequence on the current stream (every kernel of the chain covers the whole batch):
    returns ``(u [E, K, K], status [E])``; :func:`finish_factors_batched` waits and redoes
    the reference's damping retries for the experts whose first attempt failed."""
    dev = _lib.require_gpu(hs)
    if hs.dim() != 3 or hs.shape[1] != hs.shape[2]:
        raise ValueError(f"hs must be [E, K, K], got {tuple(hs.shape)}")
    e, k = hs.shape[0], hs.shape[1]
    h = hs.to(torch.float32).contiguous()
    u = torch.empty_like(h)
    status = torch.empty(max(e, 1), dtype=torch.int32, device=dev)
    if e:
        ws = _lib.workspace(dev, "hi2x_chol_batched_workspace_bytes", k, e)
        _lib.call("hi2x_chol_inv_upper_batched_async", dev, _lib.ptr(h), k * k, k, e,
                  float(damp), 0, _lib.ptr(u), k * k, _lib.ptr(status), _lib.ptr(ws),
                  ws.numel())
    return u, status[:e]


def finish_factors_batched(hs: torch.Tensor, u: torch.Tensor, status: torch.Tensor,
                           damp: float = 0.01) -> list[int]:
    """Wait for :func:`inverse_factors_batched_async` and retry, as :func:`inverse_factor`
    does, every expert whose first attempt failed (its factor is rewritten in ``u``).
    Returns the experts that were retried."""
    bad = [i for i, v in enumerate(status.cpu().tolist()) if v != _OK]
    if not bad:
        return bad
    dev = u.device
    k = u.shape[1]
    ws = _lib.workspace(dev, "hi2x_chol_workspace_bytes", k)
    for i in bad:
        h = hs[i].to(torch.float32).contiguous()
        last = None
        for attempt in range(1, 6):
            try:
                _lib.call("hi2x_chol_inv_upper", dev, _lib.ptr(h), k, float(damp), attempt,
                          _lib.ptr(u[i]), _lib.ptr(ws), ws.numel())
                break
            except _lib.NotPositiveDefinite as e:
                last = e
        else:
            raise RuntimeError(f"Hessian is not factorisable even with heavy damping: {last}")
    return bad


def inverse_factors_batched(hs: torch.Tensor, damp: float = 0.01) -> torch.Tensor:
    """:func:`inverse_factor` of every matrix of ``hs [E, K, K]``: one batched launch
    sequence for the first attempts, the reference's retries per failing matrix.  Same
    results as :func:`inverse_factor` on each."""
    u, status = inverse_factors_batched_async(hs, damp)
    finish_factors_batched(hs, u, status, damp)
    return u


@dataclass
class GptqJob:
    """One call of :func:`encode_rows_gptq`: rows ``w[N, K]`` (stored basis), ladder
    weights ``d[K]``, factor ``u[K, K]`` (of the permuted Hessian when ``perm`` is set)."""

    w: torch.Tensor
    d: torch.Tensor
    u: torch.Tensor
    nbits: int
    block: int
    perm: torch.Tensor | None = None


@dataclass
class _Unit:
    """A row chunk of a job, exactly the unit the reference processes in one pass."""

    job: int
    s: int
    wc: torch.Tensor | None  # [n, K] fp32 working copy, columns in rounding order
    lo_u8: torch.Tensor
    step_u8: torch.Tensor
    consts: torch.Tensor
    lo_d: torch.Tensor  # [n, nb] fp32 decoded
    step_d: torch.Tensor
    blk_of: torch.Tensor  # [K] block of each column in rounding order
    codes: torch.Tensor | None = None  # uint8 [n, K] in rounding order
    comp: torch.Tensor | None = None  # fp32 [n, K] value each code was rounded from
    params: torch.Tensor | None = None  # uint8 [n, nb, 2] (prepared with its batch)
    sse: torch.Tensor | None = None  # fp32 [n] (finished with its batch)


def _prepare(ji: int, job: GptqJob, s: int, step_rows: int, effort: str,
             dest: torch.Tensor | None = None) -> _Unit:
    """The chunk's working copy (into ``dest``, a view of its batch's padded buffer, when
    given), its ladder fit and block parameters."""
    w, k = job.w, job.w.shape[1]
    if k % job.block:
        raise ValueError(f"K={k} is not a multiple of the block {job.block}")
    dev = w.device
    nb = k // job.block
    # always a fresh copy: the column loop writes its compensated columns into the
    # working copy, and a row slice of an fp32 job is otherwise a view of the caller's w
    # (at any chunk offset, not only the first)
    if dest is None:
        wc = w[s : s + step_rows].to(torch.float32, copy=True).contiguous()
    else:
        wc = dest
        wc.copy_(w[s : s + step_rows])
    cfg = EFFORT[effort]
    lo, step, _ = _fit(wc.reshape(-1, nb, job.block), job.d, 2**job.nbits, cfg["grid"],
                       cfg["ls"], False)
    lo_u8, step_u8, consts, lo_d, step_d = params_decoded(lo, step)
    cols = torch.arange(k, device=dev)
    if job.perm is not None:
        p = job.perm.to(dev)
        if dest is None:
            wc = wc.index_select(1, p)
        else:
            wc.copy_(wc.index_select(1, p))
        cols = p
    return _Unit(ji, s, wc, lo_u8, step_u8, consts, lo_d, step_d, cols // job.block)


# Batches of at least this many chunks (all without a column permutation, rows fp32 and
# contiguous) are prepared and finished as a whole: one ladder fit and one params launch
# per (block, bits) class and one sse launch per batch, instead of several launches and
# allocations per chunk (the many small jobs of an MoE layer's experts).  Results are
# the same: every row sees the same operations in the same order.
GROUPED_MIN = 4


def _groupable(jobs: list, specs: list, members: list[int]) -> bool:
    for t in members:
        job = jobs[specs[t][0]]
        if (job.perm is not None or job.w.dtype != torch.float32 or not job.w.is_contiguous()
                or job.w.shape[1] % job.block):
            return False
    return True


def _prepare_grouped(jobs: list, specs: list, members: list[int], effort: str,
                     dev: torch.device, k: int):
    """The chunks ``members`` of one batch (see GROUPED_MIN), ordered by (block, bits) so
    that each class's rows are contiguous: the padded working buffer, every row's ladder
    fit with its own job's d (``hi2x_ladder_fit_rows``) and params (``hi2x_params``) per
    class, the decoded ladders written straight into the batch's ``lo``/``st``
    (``ldp = K / 16``).  Padding rows are zero rows: they fit to lo = step = 0 and
    quantise to zero bytes, the zeros the per-chunk path leaves them.  Returns the units
    (in batch order), the buffer and (lo, st)."""
    order = sorted(members, key=lambda t: (jobs[specs[t][0]].block, jobs[specs[t][0]].nbits))
    sizes = [specs[t][2] for t in order]
    padded = _padded(sizes, _factor_keys(jobs, [specs[t][0] for t in order]))
    total = sum(padded)
    offs = [0]
    for pn in padded:
        offs.append(offs[-1] + pn)
    # padding rows must read zero: a whole-buffer fill for many units (one launch), the
    # padding slices alone for a few (no second pass over the rows)
    few = len(order) <= 16
    buf = (torch.empty if few else torch.zeros)(total, k, dtype=torch.float32, device=dev)
    d_at: dict[int, int] = {}
    dl, urow = [], []
    for t, o, pn in zip(order, offs, padded):
        ji, s0, n, _ = specs[t]
        job = jobs[ji]
        buf[o:o + n].copy_(job.w[s0:s0 + n])
        if few and pn > n:
            buf[o + n:o + pn].zero_()
        key = id(job.d)
        if key not in d_at:
            d_at[key] = len(dl)
            dl.append(job.d.to(dev, torch.float32).reshape(-1))
        urow.append(d_at[key])
    dtab = torch.stack(dl).contiguous()
    meta = _lib.h2d(torch.tensor(urow + padded, dtype=torch.int64), dev)
    d_row = torch.repeat_interleave(meta[:len(order)].to(torch.int32), meta[len(order):],
                                    output_size=total)
    ldp = k // 16
    lo = torch.zeros(total, ldp, dtype=torch.float32, device=dev)
    st = torch.zeros(total, ldp, dtype=torch.float32, device=dev)
    cfg = EFFORT[effort]
    from .encode import _grid_array

    units, i = [], 0
    while i < len(order):
        job0 = jobs[specs[order[i]][0]]
        j = i
        while j < len(order) and (jobs[specs[order[j]][0]].block,
                                  jobs[specs[order[j]][0]].nbits) == (job0.block, job0.nbits):
            j += 1
        r0, r1 = offs[i], offs[j]
        rows, b = r1 - r0, job0.block
        nb = k // b
        lo_c = torch.empty(rows, nb, dtype=torch.float32, device=dev)
        st_c = torch.empty(rows, nb, dtype=torch.float32, device=dev)
        _lib.call("hi2x_ladder_fit_rows", dev, _lib.ptr(buf[r0:r1]), _lib.ptr(dtab),
                  _lib.ptr(d_row[r0:r1]), rows, k, b, 2 ** job0.nbits,
                  _grid_array(cfg["grid"]), len(cfg["grid"]), int(cfg["ls"]), _lib.ptr(lo_c),
                  _lib.ptr(st_c), None)
        lo_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
        st_u8 = torch.empty(rows, nb, dtype=torch.uint8, device=dev)
        consts = torch.empty(rows, 3, dtype=torch.float16, device=dev)
        _lib.call("hi2x_params", dev, _lib.ptr(lo_c), _lib.ptr(st_c), rows, nb, _lib.ptr(lo_u8),
                  _lib.ptr(st_u8), _lib.ptr(consts), _lib.ptr(lo[r0:r1]), _lib.ptr(st[r0:r1]),
                  ldp)
        params = torch.stack([lo_u8, st_u8], dim=-1)
        blk_of = torch.arange(k, device=dev) // b
        for q in range(i, j):
            ji, s0, n, _ = specs[order[q]]
            o = offs[q] - r0
            units.append(_Unit(ji, s0, buf[offs[q]:offs[q] + n], lo_u8[o:o + n], st_u8[o:o + n],
                               consts[o:o + n], lo[offs[q]:offs[q] + n, :nb],
                               st[offs[q]:offs[q] + n, :nb], blk_of,
                               params=params[o:o + n]))
        i = j
    return order, units, buf, (lo, st)


def _finish_grouped(units: list[_Unit], jobs: list, total: int, k: int, row_grp: torch.Tensor,
                    codes: torch.Tensor, tabs, dev: torch.device) -> None:
    """Every unit's sse of a batch prepared by _prepare_grouped in one launch
    (``hi2x_finish_rows``); the units' rows are in batch order, laid out by ``_padded``."""
    sizes = [x.codes.shape[0] for x in units]
    padded = _padded(sizes, _factor_keys(jobs, [x.job for x in units]))
    tab, off = [], 0
    for x, n, pn in zip(units, sizes, padded):
        job = jobs[x.job]
        w = job.w[x.s:x.s + n]
        d = job.d.to(dev, torch.float32).reshape(-1)
        if not d.is_contiguous():
            d = d.contiguous()
        x._keep = (w, d)  # alive until the launch has run (the caller's stream holds it)
        tab += [w.data_ptr(), d.data_ptr(), off, n, job.block]
        off += pn
    groups = _lib.h2d(torch.tensor(tab, dtype=torch.int64), dev)
    sse = torch.empty(total, dtype=torch.float32, device=dev)
    lo, st = tabs
    _lib.call("hi2x_finish_rows", dev, _lib.ptr(codes), total, k, _lib.ptr(lo), _lib.ptr(st),
              lo.shape[1], _lib.ptr(row_grp), _lib.ptr(groups), _lib.ptr(sse))
    off = 0
    for x, n, pn in zip(units, sizes, padded):
        x.sse = sse[off:off + n]
        off += pn


def _padded(sizes: list[int], keys: list | None = None) -> list[int]:
    """Rows of each unit in a batch's working buffer.  In a multi-unit batch every run of
    consecutive units with one factor (equal ``keys``, the identity of each unit's job's
    ``u``; all different when None) starts on a 128-row boundary, so that no workgroup or
    tile of the kernels holds rows of two factors (it would run once per factor); the
    units inside a run follow each other without padding, since the kernels give a run's
    rows one pass (the row classes of one input: down_proj's 1229 + 2867 rows fill 4096,
    256 column-loop workgroups, instead of 4224)."""
    if len(sizes) <= 1:
        return list(sizes)
    keys = list(range(len(sizes))) if keys is None else keys
    out, off = [], 0
    for i, n in enumerate(sizes):
        end = off + n
        if i + 1 < len(sizes) and keys[i + 1] != keys[i]:
            end = -(-end // BLOCK_COLUMNS) * BLOCK_COLUMNS
        out.append(end - off)
        off = end
    return out


def _factor_keys(jobs: list, job_ids: list[int]) -> list[int]:
    """The factor identity of each unit (by its job index) for :func:`_padded`."""
    return [id(jobs[j].u) for j in job_ids]


def _round_kernel(
    units: list[_Unit], jobs: list[GptqJob], want_comp: bool = False, super_blocks=None,
    buf: torch.Tensor | None = None, tabs=None,
):
    """All ``units`` (same K, same device) through ``hi2x_gptq_run``: one intra-block
    launch per 128 columns for every row, the cross-block updates on MFMA with the
    reference's rounding.  ``buf``: the batch's working buffer when the units' working
    copies already sit in it (prepared in place); ``tabs``: the batch's decoded ladders
    (lo, st) when they are written there already (``_prepare_grouped``).  Returns
    (total rows, row -> unit map, codes)."""
    dev, k = units[0].wc.device, units[0].wc.shape[1]
    sizes = [x.wc.shape[0] for x in units]
    # Padding rows have w = lo = step = 0: they round to code 0 with zero error and
    # change nothing.
    padded = _padded(sizes, _factor_keys(jobs, [x.job for x in units]))
    total = sum(padded)
    if buf is not None:
        wc = buf
    elif len(units) > 1:
        wc = torch.zeros(total, k, dtype=torch.float32, device=dev)
    else:
        wc = units[0].wc
    ldp = k // 16
    if tabs is not None:
        lo, st = tabs
    else:
        lo = torch.zeros(total, ldp, dtype=torch.float32, device=dev)
        st = torch.zeros(total, ldp, dtype=torch.float32, device=dev)
    views, off = [], 0
    for x, n, pn in zip(units, sizes, padded):
        nb = x.lo_d.shape[1]
        if len(units) > 1 and buf is None:
            wc[off : off + n] = x.wc
        if tabs is None:
            lo[off : off + n, :nb] = x.lo_d
            st[off : off + n, :nb] = x.step_d
        views.append((off, n))
        off += pn
    # the batch's small tables (row counts, factor addresses, highest codes, blocks) in
    # one copy that does not block the host (other streams keep being fed while this
    # batch waits for its inputs); the row -> group map is expanded on the device
    # one device copy per distinct factor, so that units sharing a factor pass one address
    # (the kernels give such rows one pass)
    u_of: dict[int, torch.Tensor] = {}
    for x in units:
        u = jobs[x.job].u
        if id(u) not in u_of:
            u_of[id(u)] = u.to(dev, torch.float32).contiguous()
    uk = [u_of[id(jobs[x.job].u)] for x in units]
    for u in u_of.values():
        if u.shape != (k, k):
            raise ValueError(f"factor has shape {tuple(u.shape)}, expected ({k}, {k})")
    ng = len(units)
    meta = _lib.h2d(torch.tensor(
        padded + [u.data_ptr() for u in uk] + [2 ** jobs[x.job].nbits - 1 for x in units]
        + [jobs[x.job].block for x in units], dtype=torch.int64), dev)
    row_grp = torch.repeat_interleave(torch.arange(ng, dtype=torch.int32, device=dev),
                                      meta[:ng], output_size=total)
    u_ptrs = meta[ng:2 * ng]
    nmax = meta[2 * ng:3 * ng].to(torch.float32)
    if all(jobs[x.job].perm is None for x in units):
        blk = (torch.arange(k, dtype=torch.int32, device=dev)[None, :]
               // meta[3 * ng:4 * ng, None].to(torch.int32)).contiguous()
    else:
        blk = torch.stack([x.blk_of.to(dev, torch.int32) for x in units]).contiguous()
    codes = torch.zeros(total, k, dtype=torch.uint8, device=dev)
    comp = torch.zeros(total, k, dtype=torch.float32, device=dev) if want_comp else None
    sb = _super_blocks(k) if super_blocks is None else super_blocks
    sb = max(1, min(int(sb), (k + BLOCK_COLUMNS - 1) // BLOCK_COLUMNS))
    err_ws = torch.empty(total, BLOCK_COLUMNS * sb, dtype=torch.float32, device=dev)
    _lib.call("hi2x_gptq_run", dev, _lib.ptr(wc), total, k, _lib.ptr(codes), _lib.ptr(lo),
              _lib.ptr(st), ldp, _lib.ptr(row_grp), _lib.ptr(u_ptrs), _lib.ptr(blk),
              _lib.ptr(nmax), _lib.ptr(comp), _lib.ptr(err_ws), sb)
    for x, (o, n) in zip(units, views):
        x.codes = codes[o : o + n]
        x.comp = None if comp is None else comp[o : o + n]
    # Temporaries freed here (factor copies, index tensors, workspace) return to
    # torch's caching allocator, which reuses them only in order on this stream.
    return total, row_grp, codes


def _finish(unit: _Unit, job: GptqJob) -> Encoded:
    k = job.w.shape[1]
    dev = unit.codes.device
    n_rows = unit.codes.shape[0]
    w = job.w[unit.s : unit.s + n_rows].to(dev, torch.float32).contiguous()
    d = job.d.to(dev, torch.float32).reshape(-1).contiguous()
    perm = None if job.perm is None else job.perm.to(dev, torch.int64).contiguous()
    codes_ro = unit.codes.contiguous()
    comp_ro = None if unit.comp is None else unit.comp.contiguous()
    if perm is None:  # rounding order is storage order: the finish writes only sse
        codes, comp = codes_ro, comp_ro
    else:
        codes = torch.empty(n_rows, k, dtype=torch.uint8, device=dev)
        comp = None if comp_ro is None else torch.empty(n_rows, k, dtype=torch.float32,
                                                        device=dev)
    sse = torch.empty(n_rows, dtype=torch.float32, device=dev)
    lo_d, st_d = unit.lo_d.contiguous(), unit.step_d.contiguous()
    _lib.call("hi2x_finish", dev, _lib.ptr(codes_ro), _lib.ptr(comp_ro), _lib.ptr(perm), n_rows,
              k, job.block, _lib.ptr(lo_d), _lib.ptr(st_d), lo_d.shape[1], _lib.ptr(w),
              _lib.ptr(d), _lib.ptr(codes), _lib.ptr(comp), _lib.ptr(sse))
    return Encoded(
        codes,
        torch.stack([unit.lo_u8, unit.step_u8], dim=-1),
        unit.consts,
        sse,
        comp,
    )


def _use_kernel(dev: torch.device, backend: str) -> bool:
    from . import gptq_kernel

    if backend == "torch":
        raise RuntimeError(
            "hi2_amd has no torch backend: the encode path runs in the hi2x HIP kernels"
        )
    if not gptq_kernel.available(dev):
        raise RuntimeError(
            f"gptq kernel unavailable on {dev}: "
            f"{gptq_kernel.failure() or 'not a gfx950 HIP device'}"
        )
    return True


@dataclass
class PreparedJobs:
    """The factor-independent half of :func:`encode_jobs_gptq`: every job's row chunks
    copied into working copies, their ladders fitted and their block parameters
    quantised.  Nothing in it reads a job's ``u``, so it can be made before the factor
    exists (on any stream; see :meth:`record_stream`) and rounded with
    :func:`round_prepared` once it does."""

    jobs: list[GptqJob]
    units: list[_Unit]
    backend: str
    # the rounding batches: (device, K) -> [(units, working buffer or None, the batch's
    # decoded ladders (lo, st) when prepared as a whole, else None)]
    batches: dict

    def record_stream(self, stream: torch.cuda.Stream) -> None:
        """Mark every tensor made here as used on ``stream`` (for a rounding issued
        there while these were made on another stream)."""
        for x in self.units:
            for t in (x.wc, x.lo_u8, x.step_u8, x.consts, x.lo_d, x.step_d, x.blk_of):
                if t is not None:
                    t.record_stream(stream)
        for bl in self.batches.values():
            for _, buf, tabs in bl:
                for t in (buf,) + (tabs or ()):
                    if t is not None:
                        t.record_stream(stream)
            for x in self.units:
                if x.params is not None:
                    x.params.record_stream(stream)


@torch.no_grad()
def prepare_jobs_gptq(jobs: list[GptqJob], effort: str = "normal",
                      backend: str | None = None) -> PreparedJobs:
    """Cut the jobs into the reference's row chunks (``ROW_ELEMS``) and fit each
    chunk's ladder (``hi2/hessian.py:89-104``, the part of ``_prepare`` before the
    factor is used), on the current stream."""
    backend = backend or os.environ.get("HI2_GPTQ_BACKEND", "auto")
    for job in jobs:
        _lib.require_gpu(job.w)
    # the chunks, then their batches (same K and device, up to BATCH_ELEMS weights); a
    # batch of several chunks gets one working buffer that every chunk is copied into
    # (its padding rows zeroed), so that the rounding needs no gathering pass
    specs = []  # (job, row offset, rows, step_rows)
    for ji, job in enumerate(jobs):
        n_rows, k = job.w.shape
        step_rows = max(1, ROW_ELEMS // k)
        for s in range(0, n_rows, step_rows):
            specs.append((ji, s, min(step_rows, n_rows - s), step_rows))
    plan: dict[tuple, list[list[int]]] = {}
    for si, (ji, _s, n, _st) in enumerate(specs):
        w = jobs[ji].w
        key = (w.device, w.shape[1])
        bl = plan.setdefault(key, [[]])
        if bl[-1] and sum(specs[t][2] for t in bl[-1]) * w.shape[1] + n * w.shape[1] > BATCH_ELEMS:
            bl.append([])
        bl[-1].append(si)
    units: list[_Unit | None] = [None] * len(specs)
    batches: dict[tuple, list] = {}
    for (dev, k), bl in plan.items():
        for members in bl:
            if len(members) >= GROUPED_MIN and _groupable(jobs, specs, members):
                order, us, buf, tabs = _prepare_grouped(jobs, specs, members, effort, dev, k)
                for t, u in zip(order, us):
                    units[t] = u
                batches.setdefault((dev, k), []).append((us, buf, tabs))
                continue
            buf = None
            if len(members) > 1:
                sizes = [specs[t][2] for t in members]
                padded = _padded(sizes, _factor_keys(jobs, [specs[t][0] for t in members]))
                buf = torch.empty(sum(padded), k, dtype=torch.float32, device=dev)
            off = 0
            for j, t in enumerate(members):
                ji, s0, n, st = specs[t]
                dest = None
                if buf is not None:
                    pn = padded[j]
                    dest = buf[off : off + n]
                    if pn > n:
                        buf[off + n : off + pn].zero_()
                    off += pn
                units[t] = _prepare(ji, jobs[ji], s0, st, effort, dest)
            batches.setdefault((dev, k), []).append(([units[t] for t in members], buf, None))
    return PreparedJobs(jobs, units, backend, batches)


@torch.no_grad()
def encode_jobs_gptq(
    jobs: list[GptqJob],
    effort: str = "normal",
    backend: str | None = None,
    comp: bool = False,
    super_blocks: int | None = None,
) -> list[Encoded]:
    """:func:`encode_rows_gptq` for several jobs (tensors, experts, candidate groups)
    at once, bit-identical to calling it on each.  Jobs are cut into the reference's
    row chunks (``ROW_ELEMS``); chunks with the same K on the same device are batched
    (up to ``BATCH_ELEMS`` weights) through one ``hi2x_gptq_run``.  With ``comp`` every
    result carries ``Encoded.comp``.  Equal to
    ``round_prepared(prepare_jobs_gptq(jobs, effort, backend), comp, super_blocks)``."""
    return round_prepared(prepare_jobs_gptq(jobs, effort, backend), comp, super_blocks)


@torch.no_grad()
def round_prepared(prep: PreparedJobs, comp: bool = False,
                   super_blocks: int | None = None) -> list[Encoded]:
    """The rounding half of :func:`encode_jobs_gptq` on the current stream: the column
    loops and cross-block updates of every prepared chunk, then each job's finish.
    The working copies are consumed (a prepared set is rounded once)."""
    jobs, units, backend = prep.jobs, prep.units, prep.backend
    if any(x.wc is None for x in units):
        raise ValueError("these prepared jobs have already been rounded")
    batches = prep.batches
    # batches of different K are independent: each runs on its own stream
    side = []
    for bi, ((dev, k), bl) in enumerate(batches.items()):
        _use_kernel(dev, backend)
        main = torch.cuda.current_stream(dev)
        st = _lib.side_stream(dev, bi) if len(batches) > 1 else main
        if st is not main:
            st.wait_stream(main)
            side.append((main, st))
        with torch.cuda.stream(st):
            for batch, buf, tabs in bl:
                if st is not main:
                    for x in batch:
                        for t in (x.wc, x.lo_d, x.step_d, x.blk_of, jobs[x.job].u):
                            t.record_stream(st)
                    for t in (buf,) + (tabs or ()):
                        if t is not None:
                            t.record_stream(st)
                total, row_grp, codes = _round_kernel(batch, jobs, comp, super_blocks, buf,
                                                      tabs)
                if tabs is not None:
                    _finish_grouped(batch, jobs, total, k, row_grp, codes, tabs, dev)
                for x in batch:
                    if st is not main:
                        x.codes.record_stream(main)
                        if x.comp is not None:
                            x.comp.record_stream(main)
                        if x.sse is not None:
                            x.sse.record_stream(main)
                    x.wc = None  # free the working copy early
            bl[:] = [(batch, None, None) for batch, _, _ in bl]
    for main, st in side:
        main.wait_stream(st)
    per_job: list[list[Encoded]] = [[] for _ in jobs]
    for x in units:
        if x.sse is not None:  # finished with its batch
            per_job[x.job].append(Encoded(x.codes, x.params, x.consts, x.sse, x.comp))
        else:
            per_job[x.job].append(_finish(x, jobs[x.job]))
    out = []
    for encs in per_job:
        if len(encs) == 1:
            out.append(encs[0])
        else:
            out.append(
                Encoded(
                    *(
                        torch.cat([getattr(o, f) for o in encs])
                        for f in ("codes", "params", "consts", "sse")
                    ),
                    torch.cat([o.comp for o in encs]) if comp else None,
                )
            )
    return out


def encode_rows_gptq(
    w: torch.Tensor,
    d: torch.Tensor,
    u: torch.Tensor,
    nbits: int,
    block: int,
    effort: str = "normal",
    perm: torch.Tensor | None = None,
    backend: str | None = None,
    comp: bool = True,
) -> Encoded:
    """Quantise ``w[N, K]`` (stored basis) with error compensation; with ``perm`` the
    columns are rounded in that order (``u`` is then the factor of the permuted
    Hessian) and the blocks and stored codes keep their original positions.  ``d`` are
    the ladder-fit weights (``diag(Hs)``), ``u`` the factor from :func:`inverse_factor`."""
    return encode_jobs_gptq(
        [GptqJob(w, d, u, nbits, block, perm)], effort, backend, comp
    )[0]


def encode_rows_gptq_reference(
    w: torch.Tensor,
    d: torch.Tensor,
    u: torch.Tensor,
    nbits: int,
    block: int,
    effort: str = "normal",
    perm: torch.Tensor | None = None,
) -> Encoded:
    """The reference's per-block schedule (one cross-block update per 128 columns,
    ``hi2/hessian.py:132-150``) on the same kernels; bit-identical to
    :func:`encode_rows_gptq`, which batches the far-column updates."""
    return encode_jobs_gptq(
        [GptqJob(w, d, u, nbits, block, perm)], effort, comp=True, super_blocks=1
    )[0]
