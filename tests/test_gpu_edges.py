"""Edge cases of the encode path on the GPU, each against what the reference does with
it (hi2/hessian.py, hi2/encode.py):

- a Hessian update with no tokens changes nothing (the reference's chunk loop does not
  run), and the mean of an empty accumulator is zero (``S / max(n, 1)``);
- a one-row GPTQ job, and a job whose K is not a multiple of the 128-column block (the
  last block shorter), bit for bit against the oracle;
- a job with no rows fails as the reference's ``torch.cat`` of no chunks does
  (``ValueError``, from the same ``torch.cat``);
- a ladder fit over no rows returns empty (lo, step).
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def N(t):
    return t.detach().cpu().numpy()


def test_hessian_update_with_no_tokens(dev):
    from hi2_amd.hessian import HessianStats

    k = 256
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(300, k, device=dev, generator=g).to(torch.bfloat16)
    a = HessianStats(k, dev)
    a.update(x[:0])
    assert a.n == 0
    assert not bool(a.mean().any())
    a.update(x)
    b = HessianStats(k, dev)
    b.update(x)
    assert a.n == b.n == 300
    assert torch.equal(a.S, b.S)


@pytest.mark.parametrize("n,k", [(1, 256), (3, 320), (37, 1088)])
def test_gptq_small_and_ragged_jobs_equal_oracle(dev, n, k):
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq

    rng = np.random.default_rng(n * k)
    x = rng.standard_normal((2 * k, k)).astype(np.float32)
    hs = (x.T @ x / x.shape[0]).astype(np.float32)
    u, _ = oracle.inverse_factor(hs, 0.01)
    d = np.diag(hs).copy()
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    for nbits, block in ((2, 32), (4, 64), (8, 64)):
        got = encode_jobs_gptq([GptqJob(T(w), T(d), T(u), nbits, block)], "normal",
                               comp=True)[0]
        want = oracle.encode_rows_gptq(w, d, u, nbits, block, "normal")
        assert np.array_equal(N(got.codes), want["codes"]), nbits
        assert np.array_equal(N(got.params), want["params"]), nbits
        assert np.array_equal(N(got.consts).view(np.int16), want["consts"].view(np.int16))
        assert np.array_equal(N(got.sse), want["sse"]), nbits
        assert np.array_equal(N(got.comp), want["comp"]), nbits


def test_gptq_job_without_rows_fails_like_the_reference(dev):
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq

    k = 256
    u = torch.eye(k, device=dev)
    d = torch.ones(k, device=dev)
    w = torch.zeros(0, k, device=dev)
    with pytest.raises(ValueError, match="non-empty list"):
        encode_jobs_gptq([GptqJob(w, d, u, 4, 64)], "normal")


def test_fit_ladder_without_rows(dev):
    from hi2_amd.encode import fit_ladder

    wb = torch.zeros(0, 4, 64, device=dev)
    db = torch.ones(1, 4, 64, device=dev)
    lo, st = fit_ladder(wb, db, 16, "normal")
    assert tuple(lo.shape) == (0, 4) and tuple(st.shape) == (0, 4)
