"""hi2x_gptq_run_noalloc (the column loop with its error workspace in the library's
per-device scratch array) against hi2x_gptq_run with a caller workspace, through the C
ABI: codes, comp and the updated working copy bit for bit, on two calls in a row (the
second with fewer rows and another width, so it runs over the first call's leftovers),
plus the size limit refused before any launch, and a fresh process whose first library
call is the no-allocation entry point: device memory changes only by the library's code
objects (with their 64 MiB array) on that first call and not at all on the next."""

import os
import subprocess
import sys
import textwrap

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


_FRESH = textwrap.dedent("""
    import sys, torch
    sys.path[:0] = [{root!r}, {tests!r}]
    from hi2_amd import _lib
    from test_zz_no_alloc import _inputs
    dev = torch.device("cuda", 0)
    assert _lib.load() is not None, _lib.failure()
    shapes = ((1000, 1024, 4, 1), (300, 640, 2, 2))
    bufs = []
    for n, k, sb, seed in shapes:
        inp = _inputs(dev, n, k, seed)
        wc = inp["w"].clone()
        codes = torch.zeros(n, k, dtype=torch.uint8, device=dev)
        comp = torch.zeros(n, k, dtype=torch.float32, device=dev)
        bufs.append((inp, wc, codes, comp, sb))
    torch.cuda.synchronize(dev)
    free = [torch.cuda.mem_get_info(dev)[0]]
    for inp, wc, codes, comp, sb in bufs:  # the library's first calls in this process
        n, k = wc.shape
        _lib.call("hi2x_gptq_run_noalloc", dev, _lib.ptr(wc), n, k, _lib.ptr(codes),
                  _lib.ptr(inp["lo"]), _lib.ptr(inp["st"]), inp["ldp"],
                  _lib.ptr(inp["row_grp"]), _lib.ptr(inp["u_ptrs"]), _lib.ptr(inp["blk"]),
                  _lib.ptr(inp["nmax"]), _lib.ptr(comp), sb)
        torch.cuda.synchronize(dev)
        free.append(torch.cuda.mem_get_info(dev)[0])
    print("FREE", *free, flush=True)
    for inp, wc, codes, comp, sb in bufs:  # against the workspace entry, allocated now
        n, k = wc.shape
        w2 = inp["w"].clone()
        c2 = torch.zeros_like(codes)
        p2 = torch.zeros_like(comp)
        ws = torch.empty(n, 128 * sb, dtype=torch.float32, device=dev)
        _lib.call("hi2x_gptq_run", dev, _lib.ptr(w2), n, k, _lib.ptr(c2),
                  _lib.ptr(inp["lo"]), _lib.ptr(inp["st"]), inp["ldp"],
                  _lib.ptr(inp["row_grp"]), _lib.ptr(inp["u_ptrs"]), _lib.ptr(inp["blk"]),
                  _lib.ptr(inp["nmax"]), _lib.ptr(p2), _lib.ptr(ws), sb)
        torch.cuda.synchronize(dev)
        assert torch.equal(w2, wc) and torch.equal(c2, codes) and torch.equal(p2, comp)
    print("EQUAL", flush=True)
""")


def test_noalloc_first_in_a_fresh_process_allocates_only_its_code_objects(dev):
    """Call the no-allocation entry point first in a new process: the first call may load
    the library's code objects (the 64 MiB array and a few MiB of code, in the device's
    allocation granules) but nothing that scales with the launch, such as the scratch
    memory the runtime allocates for a kernel with a private segment (hundreds of MiB
    over the whole chip); the second call changes nothing."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = _FRESH.format(root=root, tests=os.path.join(root, "tests"))
    print("fresh process: hi2x_gptq_run_noalloc first", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       timeout=240, cwd=root)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    line = next(ln for ln in r.stdout.splitlines() if ln.startswith("FREE"))
    f0, f1, f2 = (int(v) for v in line.split()[1:])
    mib = 1 << 20
    assert f0 - f1 <= 64 * mib + 32 * mib, f"first call took {(f0 - f1) / mib:.1f} MiB"
    assert f1 == f2, f"second call took {(f1 - f2) / mib:.1f} MiB"
    assert "EQUAL" in r.stdout
