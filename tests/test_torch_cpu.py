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
