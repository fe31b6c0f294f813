"""Seeded inputs of the end-to-end fixtures (BASELINE configurations, some down-scaled).

Shared by ``tests/golden/make_golden.py`` (which runs the reference's own pipeline on
them) and the tests that run this build's pipeline on the same inputs.  numpy's PCG64
generator and its normal / Student-t samplers are plain scalar code, so the inputs are
the same on every machine of this image; the fixtures still record SHA-256 digests of
the inputs and the tests check them first.

Recipes (the BASELINE.json configurations):

* cfg1: W ~ N(0, 0.02^2) fp32; calibration X ~ N(0, 1) with 1 % of the channels (a
  seeded permutation) scaled x20, rounded to bf16; all rows INT4 with 64-column ladder
  blocks; every 16-column group rotated; damping 1 %.
* cfg2: rows with heavy-tailed scales (|t_4| normalised to median 1) times N(0, 0.02^2);
  X as cfg1; a seeded 30 % of the rows INT2 / 32-column blocks, the rest INT4 / 64.
"""

import hashlib

import numpy as np
import torch

# case -> (recipe, K, rows N, tokens T, seed)
CASES = {
    "cfg1_k512_t512": ("cfg1", 512, 512, 512, 101),  # cfg1 down-scaled (rank <= 512)
    "cfg1_k512_t2048": ("cfg1", 512, 512, 2048, 102),  # full-rank variant
    "cfg2_k512_t2048": ("cfg2", 512, 512, 2048, 103),  # mixed INT2/INT4, heavy tails
    "cfg1_full": ("cfg1", 2048, 2048, 512, 104),  # cfg1 at its own size (digests + slice)
}
# cases whose fixtures hold every output value (the others: digests and a row slice)
FULL_CASES = ("cfg1_k512_t512", "cfg1_k512_t2048", "cfg2_k512_t2048")
SLICE_ROWS = 64
CANDIDATES = [(2, 32), (4, 64)]  # the cfg2 allocation's two candidates
DAMP = 0.01


def sha(a) -> str:
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.view(np.uint8).reshape(-1).tobytes()).hexdigest()


def inputs(case: str):
    """(x_bf16 torch [T, K] bfloat16, w float32 [N, K], picks int64 [N] index into
    CANDIDATES, had uint8 [K / 16]) of a case."""
    recipe, k, n, t, seed = CASES[case]
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((t, k)).astype(np.float32)
    x[:, rng.permutation(k)[: -(-k // 100)]] *= 20.0
    xb = torch.from_numpy(x).to(torch.bfloat16)
    if recipe == "cfg1":
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        picks = np.ones(n, np.int64)  # INT4 / B64
    else:
        s = np.abs(rng.standard_t(4, (n, 1)))
        s /= np.median(s)
        w = (0.02 * s * rng.standard_normal((n, k))).astype(np.float32)
        picks = np.ones(n, np.int64)
        picks[rng.permutation(n)[: (3 * n) // 10]] = 0  # 30 % INT2 / B32
    had = np.ones(k // 16, np.uint8)
    return xb, w, picks, had


def input_digests(case: str) -> dict:
    xb, w, picks, had = inputs(case)
    return {"x": sha(xb.view(torch.int16).numpy()), "w": sha(w), "picks": sha(picks)}


def upper(a: np.ndarray) -> np.ndarray:
    """The upper triangle (i <= j) of a square matrix, row-major."""
    return a[np.triu_indices(a.shape[0])]


def from_upper(tri: np.ndarray, k: int, symmetric: bool) -> np.ndarray:
    """Inverse of :func:`upper`: the full matrix (mirrored, or zero below)."""
    out = np.zeros((k, k), tri.dtype)
    out[np.triu_indices(k)] = tri
    if symmetric:
        il = np.tril_indices(k, -1)
        out[il] = out.T[il]
    return out
