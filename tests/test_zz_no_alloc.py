"""hi2x_gptq_run_noalloc (the column loop with its error workspace in the library's
per-device scratch array) against hi2x_gptq_run with a caller workspace, through the C
ABI: codes, comp and the updated working copy bit for bit, on two calls in a row (the
second with fewer rows and another width, so it runs over the first call's leftovers),
plus the size limit refused before any launch."""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _inputs(dev, n, k, seed, groups=2):
    """A batch of `groups` row groups (own factor, 4-bit and 2-bit ladders) laid out as
    hi2_amd.hessian._round_kernel hands them to the column loop."""
    rng = np.random.default_rng(seed)
    us = []
    for _ in range(groups):
        x = rng.standard_normal((2 * k, k)) * np.exp(0.5 * rng.standard_normal(k))
        hs = (x.T @ x / (2 * k)).astype(np.float32)
        us.append(torch.from_numpy(oracle.inverse_factor(hs, 0.01)[0]).to(dev))
    w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
    ldp = k // 16
    lo = torch.from_numpy(rng.uniform(-0.06, -0.03, (n, ldp)).astype(np.float32)).to(dev)
    st = torch.from_numpy(rng.uniform(0.002, 0.01, (n, ldp)).astype(np.float32)).to(dev)
    grp = np.sort(rng.integers(0, groups, n)).astype(np.int32)
    row_grp = torch.from_numpy(grp).to(dev)
    u_ptrs = torch.tensor([u.data_ptr() for u in us], dtype=torch.int64, device=dev)
    blk = torch.stack([torch.arange(k, device=dev, dtype=torch.int32) // b
                       for b in (64, 32)[:groups]]).contiguous()
    nmax = torch.tensor([15.0, 3.0][:groups], dtype=torch.float32, device=dev)
    return dict(w=w, lo=lo, st=st, ldp=ldp, row_grp=row_grp, u_ptrs=u_ptrs, blk=blk,
                nmax=nmax, us=us)


def _run(dev, inp, noalloc, sb):
    from hi2_amd import _lib

    wc = inp["w"].clone()
    n, k = wc.shape
    codes = torch.zeros(n, k, dtype=torch.uint8, device=dev)
    comp = torch.zeros(n, k, dtype=torch.float32, device=dev)
    args = [_lib.ptr(wc), n, k, _lib.ptr(codes), _lib.ptr(inp["lo"]), _lib.ptr(inp["st"]),
            inp["ldp"], _lib.ptr(inp["row_grp"]), _lib.ptr(inp["u_ptrs"]), _lib.ptr(inp["blk"]),
            _lib.ptr(inp["nmax"]), _lib.ptr(comp)]
    if noalloc:
        _lib.call("hi2x_gptq_run_noalloc", dev, *args, sb)
    else:
        ws = torch.empty(n, 128 * sb, dtype=torch.float32, device=dev)
        _lib.call("hi2x_gptq_run", dev, *args, _lib.ptr(ws), sb)
    torch.cuda.synchronize(dev)
    return wc, codes, comp


def test_noalloc_column_loop_equals_the_workspace_entry_point(dev):
    for n, k, sb, seed in ((1000, 1024, 4, 1), (300, 640, 2, 2)):
        print(f"gptq_run_noalloc n={n} k={k} super_blocks={sb}", flush=True)
        inp = _inputs(dev, n, k, seed)
        want = _run(dev, inp, False, sb)
        got = _run(dev, inp, True, sb)
        for g, w, name in zip(got, want, ("wc", "codes", "comp")):
            assert torch.equal(g, w), (n, k, name)


def test_noalloc_refuses_a_batch_beyond_its_scratch(dev):
    from hi2_amd import _lib

    inp = _inputs(dev, 16, 256, 3, groups=1)
    args = [None, 40000, 4096, None, None, None, 256, None, None, None, None, None, 4]
    with pytest.raises(RuntimeError, match="64 MiB"):
        _lib.call("hi2x_gptq_run_noalloc", dev, *args)
    del inp
