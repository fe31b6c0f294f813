"""The cfg3 block exactly as ``bench.py`` times it (Llama-3-8B-shaped: 8192 tokens, seven
linears over four inputs, 30/70 INT2/INT4 rows): the packed tensors the bench step
produces, checked against the oracle, and independent of how the chains are scheduled.

- rows of down_proj (K = 14336) and q_proj (K = 4096), both allocations, re-encoded by
  the oracle from the step's own rotated weights, ladder-fit weights and factor: codes,
  block parameters, constants and sse bit for bit (hi2/hessian.py:89-175);
- the step with the critical chain's rotations and ladder fits moved to another chain's
  stream equals the step with every chain doing its own, field for field.
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def N(t):
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def block(dev):
    import bench

    print("cfg3 block inputs", flush=True)
    xs, ws, masks = bench.make_inputs(dev)
    return bench, xs, ws, masks


def _run(bench, xs, ws, masks, offload):
    keep = {}
    saved = bench.OFFLOAD_PREP
    bench.OFFLOAD_PREP = offload
    try:
        out = bench.encode_block(xs, ws, masks, keep=keep)
    finally:
        bench.OFFLOAD_PREP = saved
    torch.cuda.synchronize()
    return out, keep


def test_block_rows_equal_the_oracle(block):
    bench, xs, ws, masks = block
    print("cfg3 block step", flush=True)
    _, keep = _run(bench, xs, ws, masks, True)
    for inp, name in (("down", "down_proj"), ("attn", "q_proj")):
        _, _, jobs, where, encs = keep[inp]
        for job, (nm, _rows), enc in zip(jobs, where, encs):
            if nm != name:
                continue
            print(f"oracle rows of {name} nbits={job.nbits}", flush=True)
            sl = slice(0, 4)
            want = oracle.encode_rows_gptq(N(job.w[sl]), N(job.d), N(job.u), job.nbits,
                                           job.block, bench.EFFORT)
            assert np.array_equal(N(enc.codes[sl]), want["codes"]), (name, job.nbits)
            assert np.array_equal(N(enc.params[sl]), want["params"]), (name, job.nbits)
            assert np.array_equal(N(enc.consts[sl]).view(np.int16),
                                  want["consts"].view(np.int16)), (name, job.nbits)
            assert np.array_equal(N(enc.sse[sl]), want["sse"]), (name, job.nbits)


def test_block_independent_of_the_schedule(block):
    from hi2_amd.format import FIELDS

    bench, xs, ws, masks = block
    print("cfg3 block, offloaded and in-place preparation", flush=True)
    a, _ = _run(bench, xs, ws, masks, True)
    b, _ = _run(bench, xs, ws, masks, False)
    assert a.keys() == b.keys()
    for name in a:
        for f in FIELDS:
            x, y = getattr(a[name], f), getattr(b[name], f)
            assert torch.equal(x.cpu(), y.cpu()), (name, f)
