"""The torch-CPU restatement that bench.py's cpu_baseline times (oracle/torch_cpu.py)
against the reference-written end-to-end fixtures (CPU test): on one thread (as the
fixtures were written) every stage equals the reference's output bit for bit, so the
baseline times the reference's own CPU path."""

import numpy as np
import pytest
import torch

from e2e_recipes import CANDIDATES, FULL_CASES, inputs, sha, upper
from golden_data import e2e_case
from oracle import torch_cpu as R


@pytest.mark.parametrize("case", ["cfg1_k512_t512", "cfg2_k512_t2048"])
def test_torch_cpu_pipeline_is_the_reference(case):
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        g = e2e_case(case)
        xb, w, picks, had = inputs(case)
        flags = torch.from_numpy(had)
        sigma = R.hessian_sum(xb) / xb.shape[0]
        assert np.array_equal(upper(sigma.numpy()), upper(g["sigma"]))
        hs = R.transform_sigma(sigma, None, flags)
        assert sha(hs.numpy()) == g["hs_sha"]
        u = R.inverse_factor(hs, 0.01)
        assert np.array_equal(u.numpy(), g["u"])
        wt = R.rotate(torch.from_numpy(w), flags)
        d = hs.diagonal().clone()
        for ci, rows, params, consts in g["groups"]:
            nb, b = CANDIDATES[ci]
            codes, prm, cst, sse, comp = R.gptq(wt[torch.from_numpy(rows)], d, u, nb, b)
            assert np.array_equal(codes.numpy(), g["codes"][rows]), ci
            assert np.array_equal(prm.numpy(), params)
            assert np.array_equal(cst.view(torch.int16).numpy().view(np.uint16), consts)
            assert np.array_equal(sse.numpy(), g["sse"][rows])
            assert np.array_equal(comp.numpy(), g["comp"][rows])
            words = R.pack_codes(codes, nb).reshape(-1).numpy()
            off = g["packed_code_off"]
            got = np.concatenate([g["packed_codes"][off[r]:off[r + 1]] for r in rows])
            assert np.array_equal(words, got)
    finally:
        torch.set_num_threads(threads)


@pytest.mark.parametrize("case", ["cfg3_q_proj", "cfg2_down_proj"])
def test_torch_cpu_pipeline_is_the_reference_at_the_benchmark_widths(case):
    """K = 4096 with 8192 tokens and K = 14336 with 4096 tokens (the wide fixtures, written
    by the reference on 8 threads): Sigma, Hs and U by digest; every row's codes and
    ladder bytes by their digests, every row's sse and consts bit for bit.  LAPACK's
    blocking follows the thread count (3 or 16 threads give another U), so the check runs
    on the fixture's own count."""
    from e2e_recipes import row_digests

    threads = torch.get_num_threads()
    g = e2e_case(case)
    torch.set_num_threads(int(g["threads"]))
    try:
        xb, w, picks, had = inputs(case)
        flags = torch.from_numpy(had)
        sigma = R.hessian_sum(xb) / xb.shape[0]
        assert sha(sigma.numpy()) == g["sigma_sha"]
        hs = R.transform_sigma(sigma, None, flags)
        assert sha(hs.numpy()) == g["hs_sha"]
        u = R.inverse_factor(hs, 0.01)
        assert sha(u.numpy()) == g["u_sha"]
        wt = R.rotate(torch.from_numpy(w), flags)
        d = hs.diagonal().clone()
        assert np.array_equal(d.numpy(), g["d"])
        for ci, (nb, b) in enumerate(CANDIDATES):
            rows = np.nonzero(picks == ci)[0]
            codes, prm, cst, sse, comp = R.gptq(wt[torch.from_numpy(rows)], d, u, nb, b)
            assert np.array_equal(row_digests(codes.numpy()), g["codes_digest"][rows]), ci
            assert np.array_equal(row_digests(prm.numpy()), g["params_digest"][rows]), ci
            assert np.array_equal(cst.view(torch.int16).numpy().view(np.uint16),
                                  g["consts_all"][rows]), ci
            assert np.array_equal(sse.numpy(), g["sse"][rows]), ci
            r = len(g["comp_slice"])
            head = rows[rows < r]
            assert np.array_equal(comp.numpy()[:head.size], g["comp_slice"][head]), ci
    finally:
        torch.set_num_threads(threads)
