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


def test_cfg4_layer_rows_equal_the_oracle(dev):
    """The cfg4 layer (Llama-3-70B-shaped: 8192 tokens, q/o 8192 x 8192, gate/up 28672 x
    8192, down 8192 x 28672; 25 / 72 / 3 % INT2/B32, INT4/B64, INT8/B64 rows) as the
    bench's cfg4 leg encodes it, all chains concurrent: two rows of every allocation class
    of down_proj (K = 28672) and gate_proj (K = 8192, the 57344-row batch of one input)
    re-encoded by the oracle from the step's own rotated weights, ladder-fit weights and
    factor, bit for bit; every packed tensor's codes within its ladders."""
    import bench

    print("cfg4 layer inputs", flush=True)
    xs, ws, masks = bench.make_inputs(dev, 1, bench.CFG4)
    keep = {}
    print("cfg4 layer step", flush=True)
    out = bench.encode_block(xs, ws, masks, keep=keep, cfg=bench.CFG4)
    torch.cuda.synchronize()
    del xs, ws
    assert sorted(out) == sorted(n for n, *_ in bench.CFG4["linears"])
    seen = set()
    for inp, name in (("down", "down_proj"), ("mlp", "gate_proj")):
        _, _, jobs, where, encs = keep[inp]
        u_h = None
        for job, (nm, _rows), enc in zip(jobs, where, encs):
            if nm != name:
                continue
            if u_h is None:
                u_h, d_h = N(job.u), N(job.d)
            print(f"oracle rows of {name} nbits={job.nbits}", flush=True)
            sl = slice(0, 2)
            want = oracle.encode_rows_gptq(N(job.w[sl]), d_h, u_h, job.nbits, job.block,
                                           bench.EFFORT)
            assert np.array_equal(N(enc.codes[sl]), want["codes"]), (name, job.nbits)
            assert np.array_equal(N(enc.params[sl]), want["params"]), (name, job.nbits)
            assert np.array_equal(N(enc.consts[sl]).view(np.int16),
                                  want["consts"].view(np.int16)), (name, job.nbits)
            assert np.array_equal(N(enc.sse[sl]), want["sse"]), (name, job.nbits)
            seen.add((name, job.nbits))
        del u_h
    assert seen == {(n, b) for n in ("down_proj", "gate_proj") for b in (2, 4, 8)}
