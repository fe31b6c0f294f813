"""The cached-Sigma file format on MI355X.

Mirror of the part of the reference's ``hi2/cache.py`` that touches the Hessian
(``_fname`` 258-259, ``_upper`` 262-263, ``sigma_payload`` 266-277, ``load_sigma``
280-290): a cached Sigma stores its upper triangle (row-major) when the matrix is
exactly symmetric, else the full matrix, in fp16 when ``fp16_above`` > 0 and K exceeds
it.  The symmetry check and the triangle packing run on the device
(``hi2x_sigma_pack_upper``), so only the triangle crosses PCIe.  The cache directory
logic (entries, locks, keys) is the reference's and is not rebuilt.
"""

from pathlib import Path

import torch

from . import _lib


def _fname(name: str) -> str:
    return name.replace("/", "_") + ".pt"


def _upper(k: int, device="cpu") -> torch.Tensor:
    return torch.ones(k, k, dtype=torch.bool, device=device).triu_()


def sigma_payload(sigma: torch.Tensor, n: int, fp16_above: int = 0) -> dict:
    """What a cached Sigma file stores (``hi2/cache.py:266-277``): the upper triangle
    (row-major) when ``sigma`` is exactly symmetric, else the full matrix; in fp16 when
    ``fp16_above`` > 0 and K exceeds it.  ``sigma`` must be on the device."""
    dev = _lib.require_gpu(sigma)
    s = sigma.detach().to(torch.float32).contiguous()
    k = s.shape[0]
    half = 0 < fp16_above < k
    tri = torch.empty(k * (k + 1) // 2, dtype=torch.float16 if half else torch.float32,
                      device=dev)
    asym = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("hi2x_sigma_pack_upper", dev, _lib.ptr(s), k, int(half), _lib.ptr(tri),
              _lib.ptr(asym))
    if int(asym.item()) == 0:
        return {"k": k, "n": n, "tri": _to_host(tri)}
    return {"k": k, "n": n, "full": _to_host(s.half() if half else s)}


def _to_host(t: torch.Tensor) -> torch.Tensor:
    """A host copy through page-locked memory (the DMA runs at full speed; a pageable
    destination is copied through bounce buffers several times slower)."""
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t)
    return out


def load_sigma(path: Path) -> torch.Tensor:
    """A cached Sigma back as the full fp32 matrix on the host (``hi2/cache.py:280-290``;
    file reading, the same as the reference's)."""
    obj = torch.load(path, weights_only=True)
    if isinstance(obj, torch.Tensor):  # legacy workdir file: the full matrix
        return obj
    if "full" in obj:
        return obj["full"].float()
    k = obj["k"]
    up = _upper(k)
    s = torch.zeros(k, k, dtype=torch.float32)
    s.masked_scatter_(up, obj["tri"].float())
    return torch.where(up, s, s.T)  # an exact copy of the upper triangle
