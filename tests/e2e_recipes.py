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
* cfg3: W ~ N(0, 0.02^2); X as cfg1; a seeded 30 % of the rows INT2 / 32, the rest
  INT4 / 64 (the bench's block allocation).

The wide cases run at the benchmark's own widths, where the factor's large products take
the fp16 split-plane path: cfg3's q_proj (K = 4096, 8192 tokens, full rank) and cfg2's
down_proj (K = 14336, 4096 tokens: rank 4096, definite through the damping alone).
"""

import hashlib

import numpy as np
import torch

from oracle.parity import row_digests  # noqa: F401  (8-byte digests of rows)

# case -> (recipe, K, rows N, tokens T, seed)
CASES = {
    "cfg1_k512_t512": ("cfg1", 512, 512, 512, 101),  # cfg1 down-scaled (rank <= 512)
    "cfg1_k512_t2048": ("cfg1", 512, 512, 2048, 102),  # full-rank variant
    "cfg2_k512_t2048": ("cfg2", 512, 512, 2048, 103),  # mixed INT2/INT4, heavy tails
    "cfg1_full": ("cfg1", 2048, 2048, 512, 104),  # cfg1 at its own size (digests + slice)
    "cfg3_q_proj": ("cfg3", 4096, 4096, 8192, 105),  # the bench's K = 4096 input
    "cfg2_down_proj": ("cfg2", 14336, 4096, 4096, 106),  # cfg2's down_proj at K = 14336
}
# cases whose fixtures hold every output value (the others: digests and a row slice)
FULL_CASES = ("cfg1_k512_t512", "cfg1_k512_t2048", "cfg2_k512_t2048")
SLICE_ROWS = 64
# wide cases: every row's sse and per-row digests of its codes and ladder bytes, a slice
# of rows in full, and a few rows of Sigma and U (the fixture files stay near 1 MB)
WIDE_CASES = ("cfg3_q_proj", "cfg2_down_proj")
WIDE_SLICE_ROWS = {"cfg3_q_proj": 48, "cfg2_down_proj": 16}
WIDE_FACTOR_ROWS = {"cfg3_q_proj": 16, "cfg2_down_proj": 6}
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
    elif recipe == "cfg3":
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        picks = np.ones(n, np.int64)
        picks[rng.permutation(n)[: (3 * n) // 10]] = 0  # 30 % INT2 / B32
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


SEGMENT = 512  # columns per segment digest


def segment_digests(codes: np.ndarray) -> np.ndarray:
    """A 4-byte BLAKE2b digest of every SEGMENT-column segment of every row of a codes
    matrix [rows, K] (K a multiple of SEGMENT), uint32 [rows, K / SEGMENT]: a lower bound
    on the share of equal codes of two encodings is the share of segments whose digests
    are equal."""
    n, k = codes.shape
    seg = np.ascontiguousarray(codes).reshape(n * (k // SEGMENT), SEGMENT)
    return np.array([int.from_bytes(hashlib.blake2b(r.tobytes(), digest_size=4).digest(),
                                    "little") for r in seg], np.uint32).reshape(n, -1)


def factor_rows(case: str) -> np.ndarray:
    """The rows of Sigma and U a wide fixture stores: spread evenly over the matrix."""
    k = CASES[case][1]
    return np.linspace(0, k - 1, WIDE_FACTOR_ROWS[case]).round().astype(np.int64)


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
