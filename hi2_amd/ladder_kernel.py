"""Ladder grid search on MI355X.

Mirror of the reference's ``hi2/ladder_kernel.py`` (``ladder_grid`` 148-156,
``available`` 138-141, ``load`` 109-135, ``failure``, ``supported``): one thread per
``(row, block)`` evaluates the whole grid in registers (``hi2x_ladder_fit`` with no
refits).  Unlike the reference kernel, the weighted error is summed in the reference
torch path's own order, so the chosen ladder is bit-identical to ``fit_ladder``'s.
"""

import os

import torch

from . import _lib
from .gptq_kernel import kernel_dir, supported  # noqa: F401  (re-exported as in the reference)


def load():
    return _lib.load()


def available(dev: torch.device) -> bool:
    if os.environ.get("HI2_LADDER_BACKEND", "auto") == "torch":
        return False
    return supported(dev) and load() is not None


def failure() -> str | None:
    return _lib.failure()


def ladder_grid(wb: torch.Tensor, db: torch.Tensor, grid: tuple, n: int):
    """``(lo, step, err)`` per ``(row, block)``, all ``[N, nb]`` float32; ``wb`` is
    ``[N, nb, B]`` and ``db`` ``[nb, B]``."""
    from .encode import _fit

    nb, b = wb.shape[1], wb.shape[2]
    if db.numel() != nb * b:
        raise ValueError(f"db has {db.numel()} entries, expected {nb * b}")
    return _fit(wb, db.reshape(-1), n, grid, 0, True)
