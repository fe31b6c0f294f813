"""The oracle's ColumnStats (``or_colstats_update``, ``or_colstats_diag``) pinned against
the reference's ``hi2.stats.ColumnStats`` golden vectors and a float64 brute force —
CPU only."""

import numpy as np
import pytest
import torch

import oracle
from golden_data import colstats_case

G = colstats_case()


def _inputs(tag):
    xb = G["x_bf16"].view(np.uint16)
    if tag == "bf16":
        return xb
    return (xb.astype(np.uint32) << 16).view(np.float32)  # the same values as float32


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_update_matches_reference_golden_and_brute_force(tag):
    x = _inputs(tag)
    t1, t2 = (int(v) for v in G["split"])
    k = x.shape[1]
    s = np.zeros((k // 16, 16, 16))
    oracle.colstats_update(s, x[:t1])
    oracle.colstats_update(s, x[t1:])
    ref = G[f"{tag}_S"]
    # the reference forms each 4096-token chunk's moments with torch's fp32 einsum, the
    # oracle with its own fp32 order: they agree to fp32 summation rounding
    assert np.abs(s - ref).max() <= 1e-6 * np.abs(ref).max()
    xf = (x.astype(np.uint32) << 16).view(np.float32) if tag == "bf16" else x
    x64 = xf.astype(np.float64).reshape(-1, k // 16, 16)
    brute = np.einsum("tgi,tgj->gij", x64, x64)
    assert np.abs(s - brute).max() <= 1e-6 * np.abs(brute).max()
    assert np.array_equal(s, np.transpose(s, (0, 2, 1)))  # (i, j) and (j, i): same chain
    assert int(G[f"{tag}_n"]) == t1 + t2


@pytest.mark.parametrize("tag", ["bf16", "f32"])
@pytest.mark.parametrize("variant", ["diag", "diag_rot", "diag_inv", "diag_rot_inv"])
def test_diag_equals_reference_golden_bit_for_bit(tag, variant):
    s = G[f"{tag}_S"]
    flags = G["flags"] if "rot" in variant else None
    inv = G["inv_scale"] if "inv" in variant else None
    got = oracle.colstats_diag(s, int(G[f"{tag}_n"]), flags, inv)
    assert np.array_equal(got, G[f"{tag}_{variant}"])


def test_rotated_diag_is_the_second_moment_of_the_rotated_activation():
    # the reference's tests/test_encode.py:58-73 property, against fwht16 in float64
    x = _inputs("f32")
    k = x.shape[1]
    s = np.zeros((k // 16, 16, 16))
    oracle.colstats_update(s, x)
    flags = np.array([1, 0, 1, 1], np.uint8)
    xr = oracle.fwht16(x, flags)
    want = (xr.astype(np.float64) ** 2).mean(0)
    got = oracle.colstats_diag(s, x.shape[0], flags, None)
    assert np.allclose(got, want, rtol=1e-4)
    # a plant: the rotation's sign pattern transposed would still give a symmetric H
    # (Sylvester H16 is symmetric), so also check one group against an explicit H16
    h = np.array([[(-1.0) ** bin(i & j).count("1") / 4 for j in range(16)] for i in range(16)])
    g0 = h @ (s[0] / x.shape[0]) @ h.T
    assert np.allclose(got[:16], np.diag(g0), rtol=1e-6)
