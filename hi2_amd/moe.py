"""The encode path of a mixture-of-experts layer on the MI355X: every expert's Hessian
from one routed token batch, the token floor, and the batched factors.

The reference accumulates one ``HessianStats`` per expert Linear from the tokens its
router sends there (``hi2/moe.py:83-100``: a stable sort of the flat expert indices, a
gather of each expert's tokens; gate and up share their input), tops up the experts that
saw fewer than ``min_tokens`` x their widest input with the layer average
(``hi2/layerwise.py:230-257`` with ``blend``, ``hi2/moe.py:152-156``), and then encodes
every expert as an ordinary tensor: its own transformed Hessian and factor
(``hi2/calibrate.py:332-348``), GPTQ over all experts' rows in shared batches
(``hi2/hessian.py:267-315``, one factor pointer per row group).

Here the experts of one projection group are held together, ``S [E, K, K]``:

* :meth:`ExpertHessians.update_routed` is one grouped launch sequence over the routed
  batch (``hi2x_hessian_syrk_grouped``: the gather, the per-expert windows and every
  expert's tiles, largest expert first), with the token counts kept on the device;
* :meth:`ExpertHessians.top_up` applies the reference's token floor to every short
  expert in one pass (``hi2x_hessian_blend``);
* :meth:`ExpertHessians.transformed` and :func:`hi2_amd.hessian.inverse_factors_batched`
  transform and factor all experts in one launch sequence each.

Each result equals the reference's per-expert computation: the accumulation to the
Hessian GEMM's tolerance, everything after it bit for bit with this package's
per-expert entry points.
"""

import torch

from . import _lib
from .format import GROUP
from .hessian import inverse_factors_batched, inverse_factors_batched_async

__all__ = ["ExpertHessians", "route_order", "inverse_factors_batched",
           "inverse_factors_batched_async"]


def route_order(top_k_index: torch.Tensor, n_experts: int):
    """The routed batch of ``hi2/moe.py:83-100`` from the router's ``[T, k]`` expert
    indices: ``(rows, offs)`` with ``rows[j]`` the token of the j-th routed slot in
    expert order (a stable sort of the flat indices, so token order is kept inside an
    expert) and ``offs [E + 1]`` the experts' slot ranges, both on the device."""
    k = top_k_index.shape[-1]
    flat = top_k_index.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=n_experts)
    offs = torch.zeros(n_experts + 1, dtype=torch.int64, device=flat.device)
    offs[1:] = torch.cumsum(counts, 0)
    return (order // k).to(torch.int64).contiguous(), offs


class ExpertHessians:
    """The ``HessianStats`` of every expert of one projection group (same input width
    ``k``) of an MoE layer: ``S [E, k, k]`` fp32 (upper triangles, as
    :class:`hi2_amd.hessian.HessianStats` keeps them) and the token counts ``n [E]``
    (device int64)."""

    def __init__(self, n_experts: int, k: int, device="cuda"):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(f"hi2_amd.moe accumulates on the MI355X; got device {dev}")
        self.k = k
        self.S = torch.zeros(n_experts, k, k, dtype=torch.float32, device=dev)
        self.n = torch.zeros(n_experts, dtype=torch.int64, device=dev)

    @property
    def n_experts(self) -> int:
        return self.S.shape[0]

    @torch.no_grad()
    def update_routed(self, x: torch.Tensor, offs: torch.Tensor,
                      rows: torch.Tensor | None = None) -> None:
        """Every expert e accumulates the routed slots ``offs[e]:offs[e+1]``: token
        ``rows[j]`` of ``x [T, k]`` (bf16) for slot j, or row j of ``x`` itself when
        ``rows`` is None (a batch already in expert order, e.g. the down projection's
        inputs).  ``offs`` and ``rows`` stay on the device."""
        dev = self.S.device
        if x.dtype != torch.bfloat16:
            raise RuntimeError("update_routed takes bf16 tokens (the routed activations)")
        x = x.reshape(-1, self.k).to(dev).contiguous()
        offs = offs.to(dev, torch.int64).contiguous()
        if offs.numel() != self.n_experts + 1:
            raise ValueError(f"offs has {offs.numel()} entries, expected {self.n_experts + 1}")
        if rows is not None:
            rows = rows.to(dev, torch.int64).contiguous()
            t_total = rows.numel()
        else:
            t_total = x.shape[0]
        if t_total:
            ws = _lib.workspace(dev, "hi2x_hessian_grouped_workspace_bytes", t_total,
                                self.n_experts, self.k)
            _lib.call("hi2x_hessian_syrk_grouped", dev, _lib.ptr(x), x.shape[0], 2,
                      _lib.ptr(rows), _lib.ptr(offs), self.n_experts, t_total, self.k,
                      _lib.ptr(self.S), self.k * self.k, 1, _lib.ptr(ws), ws.numel())
        self.n += (offs[1:] - offs[:-1]).clamp_min(0)

    def counts(self) -> list[int]:
        return self.n.cpu().tolist()

    @torch.no_grad()
    def top_up(self, need: int) -> list[int]:
        """The reference's token floor (``hi2/layerwise.py:241-257``): every expert with
        fewer than ``need`` tokens becomes ``S_e + (need - n_e) / n_total * sum(S)`` with
        ``n_e = need`` (nothing when no expert saw a token).  ``need`` is
        ``int(min_tokens * widest input of the expert)``.  Returns the experts topped up."""
        counts = self.counts()
        tot_n = sum(counts)
        short = [e for e, c in enumerate(counts) if c < need and tot_n != 0]
        if not short:
            return short
        dev = self.S.device
        fill = torch.zeros(self.n_experts, dtype=torch.float32)
        mask = torch.zeros(self.n_experts, dtype=torch.uint8)
        for e in short:
            fill[e] = (need - counts[e]) / max(tot_n, 1)  # a double, rounded to fp32
            mask[e] = 1
        k = self.k
        # the device copies are held until the call has been enqueued: a temporary freed
        # earlier could be handed to the next copy and overwritten before the kernel runs
        fill_d, mask_d = _lib.h2d(fill, dev), _lib.h2d(mask, dev)
        _lib.call("hi2x_hessian_blend", dev, _lib.ptr(self.S), k * k, self.n_experts, k,
                  _lib.ptr(fill_d), _lib.ptr(mask_d), 1)
        idx = torch.tensor(short, dtype=torch.int64)
        self.n[_lib.h2d(idx, dev)] = need
        return short

    def full(self) -> torch.Tensor:
        """``S`` with both triangles (a copy)."""
        s = self.S.clone()
        k = self.k
        for e in range(self.n_experts):
            _lib.call("hi2x_hessian_mirror", s.device, _lib.ptr(s[e]), k)
        return s

    @torch.no_grad()
    def transformed(self, col_scale: torch.Tensor | None, had: torch.Tensor) -> torch.Tensor:
        """``transform_sigma(mean_e, col_scale, had)`` of every expert, ``[E, k, k]``, bit
        for bit as :meth:`hi2_amd.hessian.HessianStats.transformed` on each."""
        k = self.k
        if k % GROUP:
            raise ValueError(f"K={k} must be a multiple of {GROUP}")
        dev = self.S.device
        fl = _lib.to_device(had.reshape(-1), dev, torch.uint8).contiguous()
        if fl.numel() != k // GROUP:
            raise ValueError(f"had has {fl.numel()} entries, expected {k // GROUP}")
        cs = None
        if col_scale is not None:
            cs = _lib.to_device(col_scale.reshape(-1), dev, torch.float16).contiguous()
        out = torch.empty_like(self.S)
        _lib.call("hi2x_sigma_transform_upper_batched", dev, _lib.ptr(self.S), k * k,
                  _lib.ptr(self.n), self.n_experts, _lib.ptr(cs), _lib.ptr(fl), k,
                  _lib.ptr(out), k * k)
        return out
