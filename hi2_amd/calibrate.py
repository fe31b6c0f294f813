"""Encode orchestration on MI355X: ``encode_many``.

Mirror of the reference's per-tensor orchestration (``hi2/calibrate.py``): the request,
table and config types keep the reference's field names (``Config`` 36-69,
``TensorTable`` 72-81, ``EncodeRequest`` 273-287), so requests built by the reference's
pipeline can be handed over as they are (the functions here read fields only, duck
typed), and ``encode_many`` / ``encode_with_picks`` return the reference's packed
buffers bit for bit (``hi2/calibrate.py:297-443``).

Placement on the device:

* every distinct input (``_factor_key``: the Sigma id, the smoothing vector and the
  rotation flags) is one *chain* on its own stream: Sigma H2D -> ``transform_sigma``
  -> act-order permutation -> damped inverse factor (enqueued without a host wait) ->
  staging, smoothing and rotation of the rows of every tensor that reads that input ->
  one batched GPTQ call over all their candidate groups -> (when configured) the
  refinement, on a stream of the chain's own that is never marked background.  Chains
  run on a pool of ``LANES`` streams, so independent inputs overlap on the GPU;
* the host waits only after every chain is enqueued: for each chain's factor status
  (the reference's damping retries, which redo that chain's rounding and refinement),
  then per tensor for packing, whose range check and D2H copy end the chain;
* nearest-rounding rows (``cfg.rounding == "nearest"`` or no Sigma) go through
  :func:`hi2_amd.encode.encode_rows` (ladder fit, params, codes, sse) on a side stream
  of their own.

Weights and Sigma may come from the host in their stored dtype (staged through pinned
memory, cast and smoothed on the device, as exact as the reference's host cast and
multiply) or be on the device already.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .encode import encode_rows
from .format import GROUP, HI2Tensor, assemble, fwht_groups, rotate_rows
from .hessian import (
    GptqJob,
    encode_jobs_gptq,
    encode_rows_gptq_reference,
    finish_factor,
    inverse_factor,
    inverse_factor_async,
    transform_sigma,
)
from .refine import refine_groups
from .stats import ColumnStats

# the reference's candidate table (hi2/calibrate.py:28-31): (nbits, block)
ALL_CANDIDATES = [(nb, b) for nb in (2, 4) for b in (16, 32, 64)]
INT8_CANDIDATES = [(8, 32), (8, 64)]
SELECTABLE = ALL_CANDIDATES + INT8_CANDIDATES
LANES = 4  # streams the chains are spread over (one hardware queue each)


@dataclass
class Config:
    """The fields of ``hi2/calibrate.py:36-69`` that the encode reads (the others are
    kept so a reference config converts field by field)."""

    candidates: list[tuple[int, int]] = field(default_factory=lambda: list(ALL_CANDIDATES))
    rotation: str = "on"
    smooth: float = 0.5
    smooth_search: tuple[float, ...] = ()
    rounding: str = "gptq"  # gptq | nearest
    sequential: bool = False
    damp: float = 0.01
    act_order: bool = False
    refine_passes: int = 0
    effort: str = "normal"
    expert_min_tokens: float = 2.0


@dataclass
class TensorTable:
    """``hi2/calibrate.py:72-81``: per-tensor transform and candidate table."""

    name: str
    shape: tuple[int, int]
    had: torch.Tensor  # uint8 [K/16]
    sse: torch.Tensor  # float32 [C, R]
    candidates: list[tuple[int, int]]
    energy: float
    n_tokens: int
    col_scale: torch.Tensor | None = None  # fp16 [K]


@dataclass
class EncodeRequest:
    """``hi2/calibrate.py:273-287``: one tensor for :func:`encode_many`."""

    w: torch.Tensor  # [R, K] original basis
    stats: object | None  # ColumnStats (this package's or the reference's)
    table: TensorTable
    picks: torch.Tensor  # [R] candidate index per row
    sigma: torch.Tensor | None = None
    sigma_id: str | None = None
    comp_out: dict | None = None


class Executor:
    """Row placement of ``hi2/executor.py:49-67``: even contiguous row ranges, one per
    device.  The devices must be HIP devices."""

    def __init__(self, devices: list[str] | str | None = None):
        if devices is None:
            devices = [f"cuda:{torch.cuda.current_device()}"]
        if isinstance(devices, str):
            devices = [d for d in devices.split(",") if d]
        self.devices = [torch.device(d) for d in devices]
        if not self.devices:
            raise ValueError("no devices")

    @property
    def primary(self) -> torch.device:
        return self.devices[0]

    def shards(self, rows: int):
        n = min(len(self.devices), max(rows, 1))
        bounds = [rows * i // n for i in range(n + 1)]
        return [(self.devices[i], bounds[i], bounds[i + 1]) for i in range(n)]


def _device(dev) -> torch.device:
    dev = torch.device(dev)
    if dev.type != "cuda":
        raise RuntimeError(f"hi2_amd encodes on the MI355X only: executor device {dev}")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _to_device(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """A host tensor through pinned memory without a host wait, or a device tensor."""
    if t.device.type == "cuda":
        return t.to(dev)
    return _lib.h2d(t, dev)


def _inv_scale(col_scale: torch.Tensor | None) -> torch.Tensor | None:
    """``1 / s`` in float32, divided on the host as the reference does (``_smoothed``,
    ``hi2/calibrate.py:106-111``)."""
    if col_scale is None:
        return None
    return 1.0 / col_scale.detach().cpu().float()


def _row_source(w: torch.Tensor, col_scale, had: torch.Tensor, dev):
    """``rows -> fwht(W * s)[rows]`` in float32 on ``dev`` (``rows`` host int64).  The
    stored dtype crosses PCIe once; float32 and bfloat16 weights are then cast, scaled,
    rotated and gathered per candidate in one pass (``rotate_rows``), other dtypes
    through ``_stage_rows`` and a row gather."""
    if w.dtype in (torch.float32, torch.bfloat16):
        wd = _to_device(w, dev)
        cs = None if col_scale is None else _to_device(col_scale, dev).float()
        fl = _to_device(had.to(torch.uint8), dev) if bool(had.any()) else None
        return lambda rows: rotate_rows(wd, fl, _to_device(rows, dev), cs)
    wt = _stage_rows(w, col_scale, had, dev)
    return lambda rows: wt.index_select(0, _to_device(rows, dev))


def _stage_rows(w: torch.Tensor, col_scale, had: torch.Tensor, dev) -> torch.Tensor:
    """``fwht(W * s)`` in float32 on ``dev``: the stored dtype crosses PCIe, the cast
    (exact) and the fp32 product (one rounding, as on the host) run on the device."""
    wt = _to_device(w, dev)
    if wt.dtype != torch.float32:
        wt = wt.float()
    if col_scale is not None:
        wt = wt * _to_device(col_scale, dev).float()
    wt = wt.contiguous()
    return fwht_groups(wt, had) if bool(had.any()) else wt


def _weights(stats, k: int, had: torch.Tensor, dev, inv) -> torch.Tensor:
    """Ladder weights of nearest rounding (``hi2/calibrate.py:87-93``): ones without
    statistics, else ``E[x_j^2]`` in the stored basis from ``hi2x_colstats_diag``."""
    if stats is None:
        return torch.ones(k, device=dev)
    if not isinstance(stats, ColumnStats) or stats.S.device != dev:
        st = ColumnStats(k, dev)
        st.S = _to_device(stats.S.to(torch.float64) if stats.S.device.type == "cpu"
                          else stats.S, dev).to(torch.float64).contiguous()
        st.n = int(stats.n)
        stats = st
    return stats.diag(had, inv)


def _factor_key(req, i: int):
    """Requests that share this key share one transformed Hessian and one factor
    (``hi2/calibrate.py:290-294``)."""
    t = req.table
    cs = None if t.col_scale is None else t.col_scale.detach().cpu().numpy().tobytes()
    sid = req.sigma_id if req.sigma_id is not None else f"#{i}"
    return sid, cs, t.had.detach().cpu().numpy().tobytes()


def _factor(hs: torch.Tensor, damp: float):
    """The first factorisation attempt, enqueued: ``(u, status)``."""
    return inverse_factor_async(hs, damp)


@dataclass
class _Chain:
    stream: torch.cuda.Stream
    hs: torch.Tensor  # transformed (and permuted) Hessian
    d: torch.Tensor  # its diagonal before the permutation: the ladder weights
    u: torch.Tensor
    status: torch.Tensor
    perm: torch.Tensor | None
    jobs: list = field(default_factory=list)  # indices into the device's job list
    reqs: list = field(default_factory=list)  # the requests that read this input
    refine_stream: torch.cuda.Stream | None = None  # its refinement's (None: its own)


def _rows_of(picks_host: torch.Tensor, lo: int, hi: int, ci: int) -> torch.Tensor:
    return (picks_host[lo:hi] == ci).nonzero().flatten()


def _refine_chain(ch, reqs, jobs, job_at, encs, passes: int) -> None:
    """Enqueue the refinement of a chain's tensors: one column loop per tensor over all
    its candidate groups, with the unpermuted Hessian; never for a QAD start (comp_out).
    It runs on the chain's refinement stream, behind the chain's GPTQ, and the chain's
    stream waits for it: that stream is never marked background (the refinement is GEMM
    work throughout, which the background reservation only slows)."""
    by_tensor: dict[int, list[int]] = {}
    for x in ch.jobs:
        if reqs[job_at[x][0]].comp_out is None:
            by_tensor.setdefault(job_at[x][0], []).append(x)
    rst = ch.refine_stream or ch.stream
    if rst is not ch.stream:
        rst.wait_stream(ch.stream)
        ch.hs.record_stream(rst)
    with torch.cuda.stream(rst):
        for xs in by_tensor.values():
            if rst is not ch.stream:
                for x in xs:  # made on the chain's stream, read here
                    jobs[x].w.record_stream(rst)
                    for t in (encs[x].codes, encs[x].params, encs[x].consts):
                        t.record_stream(rst)
            new = refine_groups(
                [(jobs[x].w, encs[x], jobs[x].nbits, jobs[x].block) for x in xs], ch.hs, passes)
            for x, codes in zip(xs, new):
                e = encs[x]
                encs[x] = type(e)(codes, e.params, e.consts, e.sse, e.comp)
    if rst is not ch.stream:
        ch.stream.wait_stream(rst)


def _round_chain(ch, reqs, jobs, job_at, encs, cfg) -> None:
    """Enqueue a chain's GPTQ (one batched call over all its candidate groups) and, when
    configured, its refinement, without a host wait."""
    want = any(reqs[job_at[x][0]].comp_out is not None for x in ch.jobs)
    with torch.cuda.stream(ch.stream):
        for x, e in zip(ch.jobs, encode_jobs_gptq([jobs[x] for x in ch.jobs], cfg.effort,
                                                  comp=want)):
            encs[x] = e
    if cfg.refine_passes and ch.perm is None:
        _refine_chain(ch, reqs, jobs, job_at, encs, cfg.refine_passes)


def _on_device(reqs, cfg, ex, i: int, use_gptq, comp_full, pack=None):
    """Every request's shard ``i``.  Returns ``{request: [(rows, codes, params, consts),
    ...]}`` in candidate order, the stream each request's pieces were made on, the
    requests in the order their work was enqueued, and the streams to join.  With
    ``pack`` (one device), ``pack(ri, pieces, stream)`` is called for each request as soon
    as its chain is finished, while later chains still run."""
    dev = _device(ex.devices[i])
    main = torch.cuda.current_stream(dev)
    # lane 0 takes the widest input (the critical path) on the caller's stream, the others
    # persistent side streams.  HIP maps streams onto a few hardware queues and two streams
    # on one queue run in turn; the caller's stream had its queue to itself in every kernel
    # trace, while which queue a side stream lands on depends on what the process created
    # before it (the critical chain sharing one cost 20 % of the block's encode).  The
    # other lanes are marked background: their GPTQ updates leave room on the CUs for the
    # critical chain's latency-bound kernels.
    lanes = [main] + [_lib.side_stream(dev, 64 + j) for j in range(1, LANES)]
    for st in lanes[1:]:
        st.wait_stream(main)
        _lib.stream_background(st, True)
    try:
        return _enqueue(reqs, cfg, ex, i, use_gptq, comp_full, pack, dev, main, lanes)
    finally:
        # the marks are read when a launch is enqueued: every chain is enqueued now
        for st in lanes[1:LANES]:
            _lib.stream_background(st, False)


def _enqueue(reqs, cfg, ex, i, use_gptq, comp_full, pack, dev, main, lanes):
    """The body of :func:`_on_device` once its lane streams are set up."""
    groups: dict = {}  # factor key -> requests, in order of first appearance
    near: list[int] = []
    for ri, r in enumerate(reqs):
        if i >= len(ex.shards(r.table.shape[0])):
            continue
        if use_gptq[ri]:
            groups.setdefault(_factor_key(r, ri), []).append(ri)
        else:
            near.append(ri)
    # the widest input first: its chain (largest factor and rows) is the critical path,
    # and the host stages the other inputs while it runs
    order = sorted(groups, key=lambda fk: -reqs[groups[fk][0]].table.shape[1])
    jobs: list[GptqJob] = []
    job_at: list[tuple[int, torch.Tensor, int]] = []  # (request, global rows, piece slot)
    pieces: dict[int, list] = {}
    stream_of: dict[int, torch.cuda.Stream] = {}
    chains: list[_Chain] = []
    enqueued: list[int] = []
    encs: dict[int, object] = {}

    def stage(ri, st, emit):
        """Rows of request ri on stream st: smoothing, rotation, one job per candidate."""
        r = reqs[ri]
        t = r.table
        _, lo, hi = ex.shards(t.shape[0])[i]
        had = t.had.detach().cpu().to(torch.uint8)
        picks = r.picks.detach().cpu()
        stream_of[ri] = st
        out = pieces.setdefault(ri, [])
        enqueued.append(ri)
        with torch.cuda.stream(st):
            src = _row_source(r.w[lo:hi], t.col_scale, had, dev)
            ctx = emit(ri, r, had)
            for ci, (nb, b) in enumerate(t.candidates):
                rows = _rows_of(picks, lo, hi, ci)
                if rows.numel() == 0:
                    continue
                sub = src(rows)
                out.append(None)  # filled once encoded: keeps the candidate order
                ctx(sub, rows + lo, nb, b, len(out) - 1)

    with torch.cuda.device(dev):
        for j, fk in enumerate(order):
            st = lanes[j % LANES]
            r0 = reqs[groups[fk][0]]
            had0 = r0.table.had.detach().cpu().to(torch.uint8)
            with torch.cuda.stream(st):
                hs = transform_sigma(_to_device(r0.sigma, dev), r0.table.col_scale, had0)
                d = hs.diagonal().clone()
                perm = None
                if cfg.act_order:
                    perm = torch.argsort(d, descending=True, stable=True)
                    hs = hs[perm][:, perm].contiguous()
                u, status = _factor(hs, cfg.damp)
            ch = _Chain(st, hs, d, u, status, perm)
            ch.reqs = groups[fk]
            ch.refine_stream = _lib.side_stream(dev, 96 + j % LANES)
            chains.append(ch)

            def emit(ri, r, had, ch=ch):
                def add(sub, rows, nb, b, slot):
                    ch.jobs.append(len(jobs))
                    jobs.append(GptqJob(sub, ch.d, ch.u, nb, b, ch.perm))
                    job_at.append((ri, rows, slot))
                return add

            for ri in groups[fk]:
                stage(ri, st, emit)
            _round_chain(ch, reqs, jobs, job_at, encs, cfg)
        # nearest rows (hi2/encode.py:133-173: ladder fit, params, codes, sse) on a side
        # stream of their own (the caller's carries the critical chain)
        near_st = _lib.side_stream(dev, 64 + LANES)
        near_st.wait_stream(main)
        lanes.append(near_st)

        def emit_near(ri, r, had):
            k = r.table.shape[1]
            d = _weights(r.stats, k, had, dev, _inv_scale(r.table.col_scale))

            def add(sub, rows, nb, b, slot):
                e = encode_rows(sub, d, nb, b, cfg.effort)
                pieces[ri][slot] = (rows, e.codes, e.params, e.consts)
                if r.comp_out is not None:
                    comp_full[ri].index_copy_(0, _to_device(rows, dev), sub)
            return add

        for ri in near:
            stage(ri, near_st, emit_near)
        if pack is not None:
            for ri in near:
                pack(ri, pieces[ri], near_st)
        # the host waits for each chain's factor status only now, the chain enqueued last
        # (the first to end) first; a chain whose first attempt failed (the reference's
        # damping retries) is rounded and refined again; then its tensors are packed
        for ch in reversed(chains):
            with torch.cuda.stream(ch.stream):
                retried = finish_factor(ch.hs, ch.u, ch.status, cfg.damp)
            if retried:
                _round_chain(ch, reqs, jobs, job_at, encs, cfg)
            for x in ch.jobs:
                ri, rows, slot = job_at[x]
                e = encs[x]
                pieces[ri][slot] = (rows, e.codes, e.params, e.consts)
                if reqs[ri].comp_out is not None:
                    with torch.cuda.stream(ch.stream):
                        comp_full[ri].index_copy_(0, _to_device(rows, dev), e.comp)
            if pack is not None:
                for ri in ch.reqs:
                    pack(ri, pieces[ri], ch.stream)
    return pieces, stream_of, enqueued, lanes


def encode_many(reqs: list, cfg, ex=None) -> list[HI2Tensor]:
    """Encode several tensors with their allocator picks (``hi2/calibrate.py:297-424``):
    the same buffers as :func:`encode_with_picks` on each.  Rows are sharded over
    ``ex.devices`` as the reference shards them; the Hessian transform and the
    factorisation run once per distinct input and device."""
    ex = ex if ex is not None else Executor()
    use_gptq = [cfg.rounding == "gptq" and r.sigma is not None for r in reqs]
    n_dev = max((len(ex.shards(r.table.shape[0])) for r in reqs), default=1)
    first = _device(ex.devices[0])
    comp_full = {
        ri: torch.zeros(tuple(r.table.shape), dtype=torch.float32, device=first)
        for ri, r in enumerate(reqs) if r.comp_out is not None
    }
    main = torch.cuda.current_stream(first)
    out: list[HI2Tensor | None] = [None] * len(reqs)

    def pack(ri, pieces, st):
        """Packing (range check, D2H) of request ri on stream st: the host waits for st."""
        r = reqs[ri]
        t = r.table
        pieces = [p for p in pieces if p is not None]
        if not pieces:
            raise ValueError(f"{t.name}: no rows to encode")
        picks = r.picks.detach().cpu().tolist()
        nbits = torch.tensor([t.candidates[c][0] for c in picks])
        block = torch.tensor([t.candidates[c][1] for c in picks])
        with torch.cuda.stream(st):
            out[ri] = assemble(pieces, nbits, block, t.had, t.shape[1], t.col_scale,
                               stager=_Pinned)
            if r.comp_out is not None:
                r.comp_out["comp"] = _Pinned.to_host(comp_full[ri])

    if n_dev == 1:
        # one device: every tensor is packed on its chain's stream as soon as the chain ends
        per_dev = [_on_device(reqs, cfg, ex, 0, use_gptq, comp_full, pack)]
    else:
        per_dev = [_on_device(reqs, cfg, ex, i, use_gptq, comp_full) for i in range(n_dev)]
        for _, _, _, lanes in per_dev:
            for s in lanes:
                main.wait_stream(s)
        for ri in range(len(reqs)):
            pack(ri, [p for pd, _, _, _ in per_dev for p in pd.get(ri, [])], main)
    for _, _, _, lanes in per_dev:
        for s in lanes:
            main.wait_stream(s)
    main.synchronize()
    return out


class _Pinned:
    """assemble() stager: device buffers to page-locked host tensors, synchronously."""

    @staticmethod
    def to_host(t: torch.Tensor) -> torch.Tensor:
        out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        out.copy_(t)
        return out


def encode_with_picks(w, stats, table, picks, cfg, ex=None, sigma=None, comp_out=None):
    """``hi2/calibrate.py:427-443``: one tensor through :func:`encode_many`."""
    req = EncodeRequest(w, stats, table, picks, sigma, comp_out=comp_out)
    return encode_many([req], cfg, ex)[0]


def encode_with_picks_reference(w, stats, table, picks, cfg, ex=None, sigma=None,
                                comp_out=None):
    """``hi2/calibrate.py:446-520``: the per-tensor schedule (one factorisation and one
    rounding call per candidate group, the reference's per-block GPTQ schedule, no
    refinement), kept as the equality reference of :func:`encode_many`."""
    ex = ex if ex is not None else Executor()
    r, k = table.shape
    had = table.had.detach().cpu().to(torch.uint8)
    use_gptq = cfg.rounding == "gptq" and sigma is not None
    inv = _inv_scale(table.col_scale)
    pieces, comps = [], []
    for dev, lo, hi in ex.shards(r):
        dev = _device(dev)
        with torch.cuda.device(dev):
            src = _row_source(w[lo:hi], table.col_scale, had, dev)
            if use_gptq:
                hs = transform_sigma(_to_device(sigma, dev), table.col_scale, had)
                d = hs.diagonal().clone()
                perm = None
                if cfg.act_order:
                    perm = torch.argsort(d, descending=True, stable=True)
                    hs = hs[perm][:, perm].contiguous()
                u = inverse_factor(hs, cfg.damp)
            else:
                d = _weights(stats, k, had, dev, inv)
            for ci, (nb, b) in enumerate(table.candidates):
                rows = _rows_of(picks.detach().cpu(), lo, hi, ci)
                if rows.numel() == 0:
                    continue
                sub = src(rows)
                if use_gptq:
                    e = encode_rows_gptq_reference(sub, d, u, nb, b, cfg.effort, perm)
                else:
                    e = encode_rows(sub, d, nb, b, cfg.effort)
                pieces.append((rows + lo, e.codes, e.params, e.consts))
                if comp_out is not None:
                    comps.append((rows + lo, (e.comp if use_gptq else sub).cpu()))
    if comp_out is not None:
        full = torch.zeros(r, k, dtype=torch.float32)
        for rows, c in comps:
            full[rows] = c
        comp_out["comp"] = full
    pk = picks.detach().cpu().tolist()
    nbits = torch.tensor([table.candidates[c][0] for c in pk])
    block = torch.tensor([table.candidates[c][1] for c in pk])
    return assemble(pieces, nbits, block, had, k, table.col_scale, stager=_Pinned)


__all__ = [
    "ALL_CANDIDATES",
    "INT8_CANDIDATES",
    "SELECTABLE",
    "Config",
    "TensorTable",
    "EncodeRequest",
    "Executor",
    "encode_many",
    "encode_with_picks",
    "encode_with_picks_reference",
    "GROUP",
]
