"""Calibration statistics on MI355X: ``ColumnStats``.

Mirror of the reference's ``hi2/stats.py`` (``TOKEN_CHUNK`` 13, ``ColumnStats`` 16-62):
per linear, a 16 x 16 second-moment block per column group, ``S_g = E[x_g x_g^T]``,
enough for the exact diagonal of the activation's second moment in the rotated basis
without keeping activations.  ``update`` runs ``hi2x_colstats_update`` (each 4096-token
chunk's moments in fp32, added to the float64 state chunk by chunk, as the reference),
``diag`` runs ``hi2x_colstats_diag``.
"""

import torch

from . import _lib
from .format import GROUP

TOKEN_CHUNK = 4096


class ColumnStats:
    def __init__(self, k: int, device="cuda"):
        if k % GROUP:
            raise ValueError(f"K={k} must be a multiple of {GROUP}")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(
                f"hi2_amd.ColumnStats accumulates on the MI355X; got device {dev}"
            )
        self.k = k
        self.S = torch.zeros(k // GROUP, GROUP, GROUP, dtype=torch.float64, device=dev)
        self.n = 0

    @torch.no_grad()
    def update(self, x: torch.Tensor) -> None:
        """``S_g += x_g^T x_g`` over all rows of ``x[..., K]`` (``hi2/stats.py:26-33``)."""
        x = x.reshape(-1, self.k)
        dev = self.S.device
        if x.dtype not in (torch.bfloat16, torch.float32):
            x = x.to(torch.float32)
        x = x.to(dev).contiguous()
        t = x.shape[0]
        if t:
            if not self.S.is_contiguous() or self.S.dtype != torch.float64:
                self.S = self.S.to(torch.float64).contiguous()
            dtype = 2 if x.dtype == torch.bfloat16 else 0
            ws = _lib.workspace(dev, "hi2x_colstats_workspace_bytes", t, self.k)
            _lib.call("hi2x_colstats_update", dev, _lib.ptr(x), dtype, t, self.k,
                      _lib.ptr(self.S), _lib.ptr(ws), ws.numel())
        self.n += t

    def merge(self, other: "ColumnStats") -> None:
        self.S += other.S.to(self.S.device)
        self.n += other.n

    def diag(
        self, flags: torch.Tensor | None = None, inv_scale: torch.Tensor | None = None
    ) -> torch.Tensor:
        """``E[x_j^2]`` per column of the activation ``x * inv_scale`` (smoothed), in
        the rotated basis where ``flags`` is set (``hi2/stats.py:39-55``)."""
        dev = self.S.device
        s = self.S.to(torch.float64).contiguous()
        fl = None
        if flags is not None:
            fl = _lib.to_device(flags.reshape(-1), dev, torch.uint8).contiguous()
            if fl.numel() != self.k // GROUP:
                raise ValueError(f"flags has {fl.numel()} entries, expected {self.k // GROUP}")
        inv = None
        if inv_scale is not None:
            inv = _lib.to_device(inv_scale.reshape(-1), dev, torch.float32).contiguous()
        out = torch.empty(self.k, dtype=torch.float32, device=dev)
        _lib.call("hi2x_colstats_diag", dev, _lib.ptr(s), self.k, int(self.n), _lib.ptr(fl),
                  _lib.ptr(inv), _lib.ptr(out))
        return out

    def state(self) -> dict:
        return {"S": self.S.cpu(), "n": self.n, "k": self.k}

    @classmethod
    def from_state(cls, st: dict, device="cuda") -> "ColumnStats":
        c = cls(st["k"], device)
        c.S = st["S"].to(c.S.device)
        c.n = st["n"]
        return c
