"""The streaming writer's tensor contract: an encoded tensor as named checkpoint tensors.

Mirror of ``hi2/checkpoint.py:142-165`` (``to_tensors``, ``from_tensors``,
``read_tensors``) and ``docs/format-spec.md`` 2.4: the packed buffers of a weight
``<base>`` are stored as ``<base>.hi2_<field>`` for every field of the flat layout
(``codes``, ``code_off``, ``blk_params``, ``param_off``, ``row_consts``, ``row_nbits``,
``row_block``, ``had``) plus ``<base>.hi2_col_scale`` when the tensor is smoothed.  The
shape is implied: R = ``row_nbits`` entries, K = 16 x ``had`` entries.  Host tensors in,
host tensors out: ``encode_many`` already returns the packed buffers on the host (the
only D2H of the encode).
"""

from __future__ import annotations

import torch

from .format import FIELDS, HI2Tensor

PREFIX = "hi2_"


def to_tensors(t: HI2Tensor, base: str) -> dict[str, torch.Tensor]:
    """``{<base>.hi2_<field>: buffer}`` for a checkpoint writer."""
    out = {f"{base}.{PREFIX}{f}": getattr(t, f) for f in FIELDS}
    if t.col_scale is not None:
        out[f"{base}.{PREFIX}col_scale"] = t.col_scale
    return out


def from_tensors(d: dict[str, torch.Tensor], base: str) -> HI2Tensor:
    """The encoded tensor ``<base>`` back from checkpoint tensors."""
    g = {f: d[f"{base}.{PREFIX}{f}"] for f in FIELDS}
    return HI2Tensor(**g, shape=(g["row_nbits"].numel(), g["had"].numel() * 16),
                     col_scale=d.get(f"{base}.{PREFIX}col_scale"))


def read_tensors(f, base: str) -> dict[str, torch.Tensor]:
    """The ``<base>.hi2_*`` tensors (with the optional smoothing vector) from an open
    safetensors file."""
    names = [f"{base}.{PREFIX}{fld}" for fld in FIELDS]
    cs = f"{base}.{PREFIX}col_scale"
    if cs in f.keys():  # noqa: SIM118
        names.append(cs)
    return {n: f.get_tensor(n) for n in names}
