"""Encode benchmark on one MI355X: the Llama-3-8B-shaped decoder block (cfg3).

A step is one full encode of the block with every input resident in HBM:
4 calibration Hessians (q/k/v share one input, gate/up another; 8192 bf16 tokens)
-> transform to the rotated basis -> damped factor -> Hadamard rotation of the 7
weight matrices -> GPTQ of every row (30 % INT2/B32, 70 % INT4/B64, seeded mask) ->
rdna_hint_flex packing into device buffers.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--refine-steps R]
                    [--many-steps M]
    python bench.py --micro {trailing,syrk,factor,refine,stats,qad} [--steps R]  # one kernel alone
"""

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HIDDEN, INTER, KV = 4096, 14336, 1024
TOKENS = 8192
LINEARS = [  # name, rows N, cols K, input
    ("q_proj", HIDDEN, HIDDEN, "attn"),
    ("k_proj", KV, HIDDEN, "attn"),
    ("v_proj", KV, HIDDEN, "attn"),
    ("o_proj", HIDDEN, HIDDEN, "o"),
    ("gate_proj", INTER, HIDDEN, "mlp"),
    ("up_proj", INTER, HIDDEN, "mlp"),
    ("down_proj", HIDDEN, INTER, "down"),
]
INPUTS = {"attn": HIDDEN, "o": HIDDEN, "mlp": HIDDEN, "down": INTER}
INT2_FRAC = 0.30
DAMP = 0.01
EFFORT = "normal"
PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s
PEAK_F32 = 157.3e12  # MI355X dense fp32 MFMA, FLOP/s
PEAK_HBM = 8.0e12  # B/s


class _DeviceStager:
    """assemble() stager that keeps the packed buffers on the device."""

    @staticmethod
    def to_host(t):
        return t


def make_inputs(dev, seed=0):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    xs = {}
    for name, k in INPUTS.items():
        x = torch.randn(TOKENS, k, generator=g, device=dev)
        idx = torch.randperm(k, generator=g, device=dev)[: (k + 99) // 100]
        x[:, idx] *= 20.0  # 1 % outlier channels
        xs[name] = x.to(torch.bfloat16)
    ws, masks = {}, {}
    for name, n, k, _ in LINEARS:
        w = torch.randn(n, k, generator=g, device=dev) * 0.02
        ws[name] = w.to(torch.bfloat16)
        perm = torch.randperm(n, generator=g, device=dev)
        m = torch.zeros(n, dtype=torch.bool, device=dev)
        m[perm[: int(round(INT2_FRAC * n))]] = True
        # the allocation (fixed input of the encode): INT2 rows, INT4 rows, per-row tables
        masks[name] = {
            "r2": m.nonzero().flatten(),
            "r4": (~m).nonzero().flatten(),
            "nbits": torch.where(m, 2, 4).cpu(),
            "block": torch.where(m, 32, 64).cpu(),
        }
    return xs, ws, masks


ORDER = ["down", "mlp", "attn", "o"]  # calibration inputs, longest chain first
# streams and the inputs each one encodes in turn (one stream per input measured best:
# the short chains fill the GPU around the long chain's latency-bound steps)
LANES = [["down"], ["mlp"], ["attn"], ["o"]]
_CHAIN_STREAMS = {}
HEAD_START = os.environ.get("HI2_HEAD_START", "transform")


def _chain_stream(dev, i):
    """One persistent stream per chain (reused every step, so each keeps its cached
    device blocks; the library's own side streams are separate)."""
    import torch

    key = (dev.index, i)
    if key not in _CHAIN_STREAMS:
        _CHAIN_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _CHAIN_STREAMS[key]


def encode_block(xs, ws, masks, timer=None, lanes=None, keep=None):
    """Encode the whole block.  Each calibration input runs its own chain on its own
    stream (Hessian -> transform -> factor -> rotation -> GPTQ -> packing of the linears
    it feeds); the chains are independent, so they overlap on the GPU.  The host waits
    only after every chain has been enqueued (factor status, packing's range check).
    keep (a dict) receives each input's (stream, hs, jobs, where, encs)."""
    import torch

    from hi2_amd.format import assemble, fwht_groups
    from hi2_amd.hessian import GptqJob, HessianStats, encode_jobs_gptq
    from hi2_amd.hessian import finish_factor, inverse_factor_async, transform_sigma

    dev = next(iter(xs.values())).device
    main = torch.cuda.current_stream(dev)
    lanes = LANES if lanes is None else lanes
    lane_of = {inp: li for li, lane in enumerate(lanes) for inp in lane}
    order = [inp for lane in zip(*[l + [None] * (4 - len(l)) for l in lanes]) for inp in lane
             if inp is not None]
    chains = {}
    for li in range(len(lanes)):
        _chain_stream(dev, li).wait_stream(main)
    lead = None  # the first chain's head start: the others wait for its Hessian stages
    for inp in order:
        k = INPUTS[inp]
        st = _chain_stream(dev, lane_of[inp])
        mark = (lambda stage, inp=inp: timer.mark(inp, stage)) if timer else (lambda stage: None)
        with torch.cuda.stream(st):
            if lead is not None and lane_of[inp] != 0:
                st.wait_event(lead)
            had = torch.ones(k // 16, dtype=torch.uint8, device=dev)
            mark("hessian")
            hst = HessianStats(k, dev)
            hst.update(xs[inp])
            if HEAD_START == "hessian" and lane_of[inp] == 0 and lead is None:
                lead = torch.cuda.Event()
                lead.record(st)
            mark("transform")
            hs = hst.transformed(None, had)  # == transform_sigma(hst.mean(), None, had)
            d = hs.diagonal().clone()
            if HEAD_START == "transform" and lane_of[inp] == 0 and lead is None:
                lead = torch.cuda.Event()
                lead.record(st)
            mark("factor")
            u, status = inverse_factor_async(hs, DAMP)
            mark("rotate")
            jobs, where = [], []
            for name, n, kk, i in LINEARS:
                if i != inp:
                    continue
                wt = fwht_groups(ws[name].float(), had)
                r2, r4 = masks[name]["r2"], masks[name]["r4"]
                jobs.append(GptqJob(wt.index_select(0, r2), d, u, 2, 32))
                where.append((name, r2))
                jobs.append(GptqJob(wt.index_select(0, r4), d, u, 4, 64))
                where.append((name, r4))
            mark("gptq")
            encs = encode_jobs_gptq(jobs, EFFORT)
            mark("end")
        chains[inp] = (st, hs, u, status, had, jobs, where, encs)
    out = {}
    for inp in reversed(order):  # the long chain last: the others are packed meanwhile
        st, hs, u, status, had, jobs, where, encs = chains[inp]
        with torch.cuda.stream(st):
            if finish_factor(hs, u, status, DAMP):  # more damping was needed: redo the rounding
                encs = encode_jobs_gptq(jobs, EFFORT)
            for name, n, k, i in LINEARS:
                if i != inp:
                    continue
                pieces = [(rows, e.codes, e.params, e.consts)
                          for (nm, rows), e in zip(where, encs) if nm == name]
                out[name] = assemble(pieces, masks[name]["nbits"], masks[name]["block"], had, k,
                                     stager=_DeviceStager)
        main.wait_stream(st)
        if keep is not None:
            keep[inp] = (st, hs, jobs, where, encs)
    return out


REFINE_PASSES = 2  # the reference's default for a calibrated GPTQ run without QAD


def refine_linears(kept):
    """Local code refinement of every linear of the block (hi2/calibrate.py:374-391: one
    sweep per tensor over all its candidate groups, with the input's transformed Hessian),
    each calibration input's linears on that input's stream.  Returns the refined codes."""
    import torch

    from hi2_amd.refine import refine_groups

    dev = next(iter(kept.values()))[1].device
    main = torch.cuda.current_stream(dev)
    out = {}
    for inp in ORDER:
        st, hs, jobs, where, encs = kept[inp]
        st.wait_stream(main)
        with torch.cuda.stream(st):
            for name, n, k, i in LINEARS:
                if i != inp:
                    continue
                xs = [x for x, (nm, _) in enumerate(where) if nm == name]
                out[name] = refine_groups(
                    [(jobs[x].w, encs[x], jobs[x].nbits, jobs[x].block) for x in xs], hs,
                    REFINE_PASSES)
    for inp in ORDER:
        main.wait_stream(kept[inp][0])
    return out


def many_requests(xs, ws, masks):
    """The block as the reference's pipeline hands it to ``encode_many``
    (hi2/calibrate.py:297): bf16 weights and the cached fp32 Sigma of each input on the
    host (pageable, as loaded), picks of the fixed allocation over the candidates
    (INT2/B32, INT4/B64), two refinement sweeps."""
    import torch

    from hi2_amd.calibrate import Config, EncodeRequest, TensorTable
    from hi2_amd.hessian import HessianStats

    dev = next(iter(xs.values())).device
    sigma = {}
    for inp, k in INPUTS.items():
        hst = HessianStats(k, dev)
        hst.update(xs[inp])
        sigma[inp] = hst.mean().cpu()
    cands = [(2, 32), (4, 64)]
    reqs = []
    for name, n, k, inp in LINEARS:
        picks = (masks[name]["nbits"] == 4).to(torch.int64)
        table = TensorTable(name, (n, k), torch.ones(k // 16, dtype=torch.uint8),
                            torch.zeros(1), cands, 0.0, TOKENS, None)
        reqs.append(EncodeRequest(ws[name].cpu(), None, table, picks, sigma[inp], inp))
    cfg = Config(candidates=cands, refine_passes=REFINE_PASSES, effort=EFFORT, damp=DAMP)
    return reqs, cfg


class StageTimer:
    """Events on each chain's stream at its stage boundaries."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}

    def mark(self, chain, stage):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.events.setdefault(chain, []).append((stage, e))

    def summary(self):
        self.torch.cuda.synchronize()
        out = {}
        for chain, evs in self.events.items():
            out[chain] = {n0: round(e0.elapsed_time(e1), 3)
                          for (n0, e0), (_, e1) in zip(evs, evs[1:])}
        return out


# kernel families timed by the library (hi2x_timing_*), with the peak that bounds each
KERNELS = {  # kind -> (kernel, bound, peak FLOP/s, work unit)
    0: ("gptq_trailing_kernel", "mfma", PEAK_F32, "2*rows*rank*cols"),
    1: ("syrk2_bf16_kernel", "mfma", PEAK_BF16, "T*K*(K+1) (upper triangle, 2 flops per product)"),
    2: ("tri_gemm_kernel", "mfma", PEAK_F32, "M*N*rank (one triangular operand)"),
    3: ("leaf_kernel", "latency", PEAK_F32, "2*n^3/3"),
    4: ("gptq_block_kernel", "latency", PEAK_F32, "rows*L*(L-1)"),
    5: ("refine GEMMs (refine_gradient_kernel + gptq_trailing_kernel)", "mfma", PEAK_F32,
        "2*rows*rank*cols"),
    6: ("refine_block_kernel", "latency", PEAK_F32, "rows*L (column decisions)"),
}
DOMINANT = 0  # the GPTQ trailing-update GEMM: the metric's MFMA kernel with the most time


def traffic_per_launch(kernel):
    """HBM bytes per launch of ``kernel`` from the committed PMC summary (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), or None when not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("bytes_per_launch")


def kernel_stats(kind):
    """Event-timed launches of one kernel family since hi2x_timing_enable."""
    from hi2_amd import _lib

    name, bound, peak, unit = KERNELS[kind]
    n, ms, work = _lib.timing_query(kind)
    if n == 0 or ms <= 0.0:
        return None
    rate = work / (ms / 1e3)
    return {"kernel": name, "bound": bound, "launches": n, "avg_ms": ms / n,
            "total_ms": ms, "work_per_launch": work / n, "work_unit": unit,
            "tflops": rate / 1e12, "frac_of_peak": rate / peak}


def roofline(kind):
    st = kernel_stats(kind)
    name, bound, peak, unit = KERNELS[kind]
    return {"bound": bound, "achieved": st["tflops"], "peak": peak / 1e12, "unit": "TFLOP/s",
            "frac": st["frac_of_peak"], "traffic": traffic_per_launch(name), "kernel": name,
            "launches": st["launches"], "avg_ms": st["avg_ms"],
            "flops_per_launch": st["work_per_launch"], "work": unit}


def cpu_baseline(seed=0):
    """The oracle (plain-C restatement of the reference path, OpenMP) timed on this host
    on a bounded sample of cfg3, scaled to ms per linear of the whole block:
      Hessian: 256 of 8192 tokens of each input (x32); transform: full K=4096 (the
      K=14336 one scaled by (14336/4096)^2); factor: K=1024 scaled by (K/1024)^3 per
      input; rotation + GPTQ + pack: 32 rows of every linear (scaled by N/32)."""
    import numpy as np

    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(seed)
    total = 0.0
    parts = {}
    t_tok = 256
    for name, k in INPUTS.items():
        x = rng.standard_normal((t_tok, k)).astype(np.float32)
        s = np.zeros((k, k), np.float32)
        t0 = time.perf_counter()
        oracle.hessian_update(s, x)
        dt = (time.perf_counter() - t0) * (TOKENS / t_tok)
        parts["hessian"] = parts.get("hessian", 0.0) + dt
    k0 = 4096
    a = rng.standard_normal((k0, k0)).astype(np.float32)
    t0 = time.perf_counter()
    oracle.transform_sigma(a, None, np.ones(k0 // 16, np.uint8))
    dt = time.perf_counter() - t0
    parts["transform"] = sum(dt * (k / k0) ** 2 for k in INPUTS.values())
    kf = 1024
    xf = rng.standard_normal((2 * kf, kf)).astype(np.float32)
    hf = (xf.T @ xf / (2 * kf)).astype(np.float32)
    t0 = time.perf_counter()
    oracle.inverse_factor(hf, DAMP)
    dt = time.perf_counter() - t0
    parts["factor"] = sum(dt * (k / kf) ** 3 for k in INPUTS.values())
    rows = 32
    gptq = 0.0
    for name, n, k, inp in LINEARS:
        w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
        d = (rng.random(k) + 0.5).astype(np.float32)
        xu = rng.standard_normal((k, k)).astype(np.float32) * 0.01
        u = np.triu(xu) + np.eye(k, dtype=np.float32)  # any upper factor: same op count
        t0 = time.perf_counter()
        wt = oracle.fwht16(w, np.ones(k // 16, np.uint8))
        n2 = int(rows * INT2_FRAC)
        o2 = oracle.encode_rows_gptq(wt[:n2], d, u, 2, 32, EFFORT, comp=False)
        o4 = oracle.encode_rows_gptq(wt[n2:], d, u, 4, 64, EFFORT, comp=False)
        oracle.pack_codes(o2["codes"], 2)
        oracle.pack_codes(o4["codes"], 4)
        gptq += (time.perf_counter() - t0) * (n / rows)
    parts["gptq"] = gptq
    total = sum(parts.values())
    return {
        "value": total * 1e3 / len(LINEARS),
        "unit": "ms per linear",
        "cores": threads,
        "kind": "port",
        "sample": "oracle (C, OpenMP) on a cfg3 sample: 256/8192 tokens per Hessian, "
                  "transform at K=4096, factor at K=1024, 32 rows per linear for "
                  "rotation+GPTQ+pack, each scaled to the full block",
        "stages_s": {k: round(v, 2) for k, v in parts.items()},
    }


# ---- kernel microbenchmarks (for profiling single kernels; not the contract line) --------
def micro(which, reps=3):
    """One kernel family at the cfg3 shapes, alone on the GPU, event-timed; prints one
    JSON line per shape.  trailing: hi2x_gptq_run (column loop + cross-block updates) on
    4096 x 14336 and 14336 x 4096; syrk: HessianStats.update of 8192 bf16 tokens at
    K = 4096 and 14336; factor: inverse_factor at K = 14336 and 4096; refine: two
    refinement sweeps of GPTQ codes at 4096 x 4096, 4096 x 14336 and 14336 x 4096;
    stats: ColumnStats.update of 8192 bf16 tokens and the cached-Sigma payload at
    K = 4096 and 14336; qad: the QAD decode forward, backward and transform over the
    latents of q_proj, gate_proj and down_proj (30 % INT2/B32, 70 % INT4/B64 rows, step
    units)."""
    import torch

    from hi2_amd import _lib
    from hi2_amd.hessian import HessianStats, encode_rows_gptq, inverse_factor

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    def hessian(k, seed=0):
        g = torch.Generator(device=dev).manual_seed(seed)
        x = torch.randn(TOKENS, k, generator=g, device=dev)
        x[:, torch.randperm(k, generator=g, device=dev)[: (k + 99) // 100]] *= 20.0
        st = HessianStats(k, dev)
        st.update(x.to(torch.bfloat16))
        return st.transformed(None, torch.ones(k // 16, dtype=torch.uint8, device=dev)), x

    def timed(fn, kinds):
        fn()
        torch.cuda.synchronize()
        _lib.timing_enable(kinds)
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        stats = {}
        for kd in kinds:
            n, kms, work = _lib.timing_query(kd)
            name, bound, peak, unit = KERNELS[kd]
            stats[name] = {"launches": n // reps, "ms": kms / reps,
                           "tflops": work / kms / 1e9 if kms > 0 and work > 0 else None,
                           "frac_of_peak": work / kms / 1e9 / (peak / 1e12)
                           if kms > 0 and work > 0 else None}
        _lib.timing_enable([])
        return ms, stats

    if which == "trailing":
        for n, k in ((HIDDEN, INTER), (INTER, HIDDEN)):
            g = torch.Generator(device=dev).manual_seed(0)
            u = torch.triu(torch.randn(k, k, generator=g, device=dev) * (0.1 / k ** 0.5))
            u += torch.eye(k, device=dev)
            w = torch.randn(n, k, generator=g, device=dev) * 0.02
            lo = torch.full((n, k // 16), -0.05, device=dev)
            st = torch.full((n, k // 16), 0.1 / 15, device=dev)
            row_grp = torch.zeros(n, dtype=torch.int32, device=dev)
            u_ptrs = torch.tensor([u.data_ptr()], dtype=torch.int64, device=dev)
            blk = (torch.arange(k, device=dev) // 64).to(torch.int32).reshape(1, k)
            nmax = torch.tensor([15.0], device=dev)
            codes = torch.zeros(n, k, dtype=torch.uint8, device=dev)
            from hi2_amd.hessian import _super_blocks

            sb = _super_blocks(k)
            err = torch.empty(n, 128 * sb, device=dev)

            def run():
                wc = w.clone()
                _lib.call("hi2x_gptq_run", dev, _lib.ptr(wc), n, k, _lib.ptr(codes),
                          _lib.ptr(lo), _lib.ptr(st), k // 16, _lib.ptr(row_grp),
                          _lib.ptr(u_ptrs), _lib.ptr(blk), _lib.ptr(nmax), None, _lib.ptr(err),
                          sb)

            ms, stats = timed(run, [0, 4])
            print(json.dumps({"micro": "trailing", "rows": n, "k": k, "super_blocks": sb,
                              "ms": ms, "kernels": stats}), flush=True)
    elif which == "syrk":
        for k in (HIDDEN, INTER):
            g = torch.Generator(device=dev).manual_seed(0)
            x = torch.randn(TOKENS, k, generator=g, device=dev).to(torch.bfloat16)
            st = HessianStats(k, dev)
            ms, stats = timed(lambda: st.update(x), [1])
            print(json.dumps({"micro": "syrk", "tokens": TOKENS, "k": k, "ms": ms,
                              "kernels": stats}), flush=True)
    elif which == "factor":
        for k in (INTER, HIDDEN):
            hs, _ = hessian(k)
            ms, stats = timed(lambda: inverse_factor(hs, DAMP), [2, 3])
            print(json.dumps({"micro": "factor", "k": k, "ms": ms, "kernels": stats}),
                  flush=True)
    elif which == "refine":
        from hi2_amd.refine import refine_groups

        for n, k in ((HIDDEN, HIDDEN), (HIDDEN, INTER), (INTER, HIDDEN)):
            hs, _ = hessian(k)
            g = torch.Generator(device=dev).manual_seed(1)
            w = torch.randn(n, k, generator=g, device=dev) * 0.02
            enc = encode_rows_gptq(w, hs.diagonal().clone(), inverse_factor(hs, DAMP), 4, 64)
            ms, stats = timed(lambda: refine_groups([(w, enc, 4, 64)], hs, REFINE_PASSES),
                              [5, 6])
            print(json.dumps({"micro": "refine", "rows": n, "k": k, "sweeps": REFINE_PASSES,
                              "ms": ms, "kernels": stats}), flush=True)
    elif which == "stats":
        from hi2_amd.cache import sigma_payload
        from hi2_amd.stats import ColumnStats

        for k in (HIDDEN, INTER):
            g = torch.Generator(device=dev).manual_seed(0)
            x = torch.randn(TOKENS, k, generator=g, device=dev).to(torch.bfloat16)
            cs = ColumnStats(k, dev)
            ms, _ = timed(lambda: cs.update(x), [])
            nsub = (TOKENS + 255) // 256
            # X read once; the fp32 partials written and read back; S read and written
            hbm = TOKENS * k * 2 + 2 * nsub * k * 16 * 4 + 2 * k * 16 * 8
            print(json.dumps({"micro": "colstats_update", "tokens": TOKENS, "k": k, "ms": ms,
                              "hbm_bytes": hbm, "gb_per_s": hbm / ms / 1e6,
                              "frac_of_hbm_peak": hbm / ms / 1e6 / (PEAK_HBM / 1e9)}),
                  flush=True)
            hs = HessianStats(k, dev)
            hs.update(x)
            sig = hs.mean()
            ms, _ = timed(lambda: sigma_payload(sig, hs.n), [])
            hbm = k * k * 4 + k * (k + 1) // 2 * 4  # the matrix read, the triangle written
            print(json.dumps({"micro": "sigma_payload", "k": k, "ms_incl_d2h": ms,
                              "hbm_bytes": hbm, "d2h_bytes": k * (k + 1) // 2 * 4}),
                  flush=True)
    elif which == "qad":
        from hi2_amd.qad_kernel import load

        mod = load()

        def events(fn, n=20):
            fn()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(n):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / n

        for name, r, k, _ in LINEARS:
            if name not in ("q_proj", "down_proj", "gate_proj"):
                continue
            g = torch.Generator(device=dev).manual_seed(1)
            latent = torch.randn(r, k, generator=g, device=dev)
            unit = torch.rand(r, k, generator=g, device=dev) * 0.5 + 0.5
            grad = torch.randn(r, k, generator=g, device=dev)
            out, g_lat = torch.empty_like(latent), torch.empty_like(latent)
            perm = torch.randperm(r, generator=g, device=dev)
            n2 = int(round(INT2_FRAC * r))
            groups = []
            for rows, nbits, block in ((perm[:n2].sort().values, 2, 32),
                                       (perm[n2:].sort().values, 4, 64)):
                nb = k // block
                lo_u = torch.rand(rows.numel(), nb, generator=g, device=dev) * 255
                st_u = torch.rand(rows.numel(), nb, generator=g, device=dev) * 255
                c = torch.tensor([-3.0, 6.0 / 255, 0.1], device=dev).half().repeat(rows.numel(), 1)
                groups.append((lo_u, st_u, c.contiguous(), rows.contiguous(), block,
                               float(2 ** nbits - 1), torch.empty_like(lo_u),
                               torch.empty_like(lo_u)))

            def fwd():
                for lo_u, st_u, c, rows, block, nmax, _, _ in groups:
                    mod.decode_fwd(latent, unit, lo_u, st_u, c, rows, block, nmax, out)

            def bwd():
                for lo_u, st_u, c, rows, block, nmax, g_lo, g_st in groups:
                    mod.decode_bwd(grad, latent, unit, lo_u, st_u, c, rows, block, nmax, g_lat,
                                   g_lo, g_st)

            flags = torch.ones(k // 16, dtype=torch.uint8, device=dev)
            cs = (torch.rand(k, generator=g, device=dev) + 0.5).half()
            y = torch.empty_like(latent)
            elems = r * k
            # algorithmic HBM bytes: fwd latent + unit in, values out; bwd grad + latent +
            # unit in, latent gradient out; the transform x in, out (block bytes negligible)
            for kern, fn, per in (("decode_fwd", fwd, 12), ("decode_bwd", bwd, 16),
                                  ("wht_scale", lambda: mod.wht_scale(out, flags, cs, False, y),
                                   8)):
                ms = events(fn)
                gbs = elems * per / ms / 1e6
                print(json.dumps({"micro": f"qad_{kern}", "linear": name, "rows": r, "k": k,
                                  "ms": ms, "hbm_bytes": elems * per, "gb_per_s": gbs,
                                  "frac_of_hbm_peak": gbs / (PEAK_HBM / 1e9)}), flush=True)
    else:
        raise SystemExit(f"unknown --micro {which}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--refine-steps", type=int, default=2,
                    help="timed steps of the separate refinement leg (0: skip it)")
    ap.add_argument("--many-steps", type=int, default=2,
                    help="timed calls of the drop-in encode_many leg on host inputs "
                         "(0: skip it)")
    ap.add_argument("--micro", choices=["trailing", "syrk", "factor", "refine", "stats", "qad"],
                    help="instead of the block step: one kernel family alone at the cfg3 "
                         "shapes (for single-kernel profiles; prints one line per shape)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run 3 plain device copies of MIB MiB (f32), the known-size "
                         "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (--gpus 1); the "
                          "multi-GPU design is documented, not run"}))
        sys.exit(2)
    if args.micro:
        micro(args.micro, max(1, args.steps))
        return
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.ones(args.copy_probe << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    xs, ws, masks = make_inputs(dev)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        encode_block(xs, ws, masks)
    torch.cuda.synchronize()
    from hi2_amd import _lib

    timer = StageTimer(torch)
    _lib.timing_enable([DOMINANT])  # HIP events around each launch of the dominant kernel
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        encode_block(xs, ws, masks, timer if i == args.steps - 1 else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    stages = timer.summary()
    roof = roofline(DOMINANT)
    # one more, untimed step with every kernel family event-timed and the chains run one
    # after another on one stream: per-kernel rates without other chains sharing the GPU
    _lib.timing_enable(list(KERNELS))
    encode_block(xs, ws, masks, lanes=[ORDER])
    torch.cuda.synchronize()
    kernels = {KERNELS[k][0]: kernel_stats(k) for k in KERNELS}
    roof_iso = roofline(DOMINANT)
    _lib.timing_enable([])
    refine = None
    if args.refine_steps:
        kept = {}
        encode_block(xs, ws, masks, keep=kept)
        refine_linears(kept)  # warm-up
        torch.cuda.synchronize()
        _lib.timing_enable([5])
        t0 = time.perf_counter()
        for _ in range(args.refine_steps):
            refine_linears(kept)
        torch.cuda.synchronize()
        r_ms = (time.perf_counter() - t0) * 1e3 / args.refine_steps
        r_roof = roofline(5)
        _lib.timing_enable([5, 6])
        refine_linears({k: (torch.cuda.current_stream(dev),) + v[1:] for k, v in kept.items()})
        torch.cuda.synchronize()
        refine = {
            "what": f"local code refinement, {REFINE_PASSES} sweeps, of all 7 linears' GPTQ "
                    "codes (hi2/refine.py; the reference's default after calibrated GPTQ "
                    "without QAD); not part of value",
            "steps": args.refine_steps,
            "ms_per_step": r_ms,
            "ms_per_linear": r_ms / len(LINEARS),
            "roofline": r_roof,
            "kernels_one_step_serial": {KERNELS[k][0]: kernel_stats(k) for k in (5, 6)},
        }
        _lib.timing_enable([])
        del kept
    many = None
    if args.many_steps:
        from hi2_amd.calibrate import Executor, encode_many

        reqs, cfg = many_requests(xs, ws, masks)
        ex = Executor([str(dev)])
        encode_many(reqs, cfg, ex)  # warm-up
        t0 = time.perf_counter()
        for _ in range(args.many_steps):
            packed = encode_many(reqs, cfg, ex)
        m_ms = (time.perf_counter() - t0) * 1e3 / args.many_steps
        srcs = [r.w for r in reqs] + list({id(r.sigma): r.sigma for r in reqs}.values())
        h2d = sum(t.numel() * t.element_size() for t in srcs)
        # the staging floor: the same host tensors to the device, nothing else
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        staged = [_lib.h2d(t, dev) for t in srcs]
        torch.cuda.synchronize()
        stage_ms = (time.perf_counter() - t0) * 1e3
        del staged
        d2h = sum(sum(getattr(p, f).numel() * getattr(p, f).element_size()
                      for f in ("codes", "blk_params", "row_consts")) for p in packed)
        many = {
            "what": "drop-in hi2_amd.calibrate.encode_many on the block's 7 requests with "
                    "bf16 weights and cached fp32 Sigma on the host: H2D, transform, "
                    "factor, rotation, GPTQ, 2 refinement sweeps, packing, D2H of the "
                    "packed buffers (PCIe-inclusive; the Hessian is not in it, the "
                    "refinement is); not part of value",
            "steps": args.many_steps,
            "ms_per_step": m_ms,
            "ms_per_linear": m_ms / len(LINEARS),
            "h2d_bytes": h2d,
            "h2d_staging_ms": stage_ms,
            "d2h_bytes": d2h,
        }
        del reqs, packed
    res = {
        "metric": "encode ms per linear layer (Llama-3-8B-shaped block, 7 linears)",
        "value": ms_step / len(LINEARS),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded normal X with 1% x20 outlier channels, W ~ N(0, 0.02^2))",
        "config": {"workload": "cfg3: Llama-3-8B-shaped decoder block, 8192 calibration "
                               "tokens, 30% INT2/B32 + 70% INT4/B64 rows, order-16 Hadamard, "
                               "damp 0.01, effort normal", "linears": len(LINEARS),
                   "hessian_input_dtype": "bf16 (f32 accumulation)"},
        "chain_stages_ms": stages,
        "roofline": roof,
        "roofline_isolated": roof_iso,
        "kernels_one_step": kernels,
    }
    if refine is not None:
        res["refine"] = refine
    if many is not None:
        res["encode_many"] = many
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
