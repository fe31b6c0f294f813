"""Encode benchmark on one MI355X: the Llama-3-8B-shaped decoder block (cfg3).

A step is one full encode of the block with every input resident in HBM:
4 calibration Hessians (q/k/v share one input, gate/up another; 8192 bf16 tokens)
-> transform to the rotated basis -> damped factor -> Hadamard rotation of the 7
weight matrices -> GPTQ of every row (30 % INT2/B32, 70 % INT4/B64, seeded mask) ->
rdna_hint_flex packing into device buffers.  Prints one JSON line, which also carries:

* a per-linear stage breakdown of one serial step (Hessian, transform, factor per
  input; rotation, ladder fit, column loop, trailing update, finish, packing per linear)
  and the HBM rates of the rotation and packing kernels;
* the cfg4 leg (Llama-3-70B-shaped layer, K = 28672, 25/72/3 % INT2/INT4/INT8 rows) and
  the cfg5 leg (OLMoE-shaped MoE layer: 64 experts, top-8 of 16384 Zipf-routed tokens),
  each timed whole;
* the refinement and encode_many legs, and the CPU baseline (the reference's CPU path
  restated in torch, oracle/torch_cpu.py, on cfg1 and cfg3 in full).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--refine-steps R]
                    [--many-steps M] [--cfg4-steps S] [--cfg5-steps S]
    python bench.py --micro {trailing,syrk,factor,refine,stats,qad,ladder} [--steps R]  # one kernel alone
"""

import argparse
import contextlib
import ctypes
import gc
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
PEAK_BF16 = 2.5e15  # MI355X dense bf16 (and fp16) MFMA, FLOP/s
PEAK_F32 = 157.3e12  # MI355X dense fp32 MFMA, FLOP/s
PEAK_HBM = 8.0e12  # B/s

# a configuration: its linears, calibration inputs (width), tokens and the allocation
# (fraction of rows, bits, ladder block) of every linear
CFG3 = dict(name="cfg3", linears=LINEARS, inputs=INPUTS, tokens=TOKENS,
            alloc=[(INT2_FRAC, 2, 32), (1 - INT2_FRAC, 4, 64)],
            order=["down", "mlp", "attn", "o"])
H70, I70 = 8192, 28672
CFG4 = dict(name="cfg4", tokens=8192,
            linears=[("q_proj", H70, H70, "attn"), ("o_proj", H70, H70, "o"),
                     ("gate_proj", I70, H70, "mlp"), ("up_proj", I70, H70, "mlp"),
                     ("down_proj", H70, I70, "down")],
            inputs={"attn": H70, "o": H70, "mlp": H70, "down": I70},
            alloc=[(0.25, 2, 32), (0.72, 4, 64), (0.03, 8, 64)],
            order=["down", "mlp", "attn", "o"])


class _DeviceStager:
    """assemble() stager that keeps the packed buffers on the device."""

    @staticmethod
    def to_host(t):
        return t



@contextlib.contextmanager
def quiet_host():
    """Python's cyclic garbage collector off for a timed GPU loop (collected once before).
    The step is enqueued from Python with host synchronisations inside it, so a full
    collection falling inside a step stalls the GPU: runs of 20-40 steps measured 35.9 ms
    at the median, two of four processes with the collector on a single step of 48.5 or
    58.5 ms, the two with it off none above 38.8 ms."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()

def make_inputs(dev, seed=0, cfg=CFG3, host=False):
    """Calibration tokens (bf16, 1 % x20 outlier channels) per input, bf16 weights
    ~N(0, 0.02^2), and each linear's allocation: a seeded permutation of the rows cut by
    the configuration's fractions; the row lists are kept on the device (rounding) and
    the host (packing).  With ``host`` every tensor is drawn on the host (torch's CPU
    generator) and copied to the device once, before anything is timed; the host tensors
    are returned as a fourth value, so that the CPU baseline and the parity check run on
    exactly the GPU step's inputs."""
    import torch

    gdev = torch.device("cpu") if host else dev
    g = torch.Generator(device=gdev).manual_seed(seed)
    xs, hx, hw = {}, {}, {}
    for name, k in cfg["inputs"].items():
        x = torch.randn(cfg["tokens"], k, generator=g, device=gdev)
        idx = torch.randperm(k, generator=g, device=gdev)[: (k + 99) // 100]
        x[:, idx] *= 20.0  # 1 % outlier channels
        xb = x.to(torch.bfloat16)
        del x
        if host:
            hx[name] = xb
            xb = xb.to(dev)
        xs[name] = xb
    ws, masks = {}, {}
    for name, n, k, _ in cfg["linears"]:
        w = torch.randn(n, k, generator=g, device=gdev) * 0.02
        wb = w.to(torch.bfloat16)
        del w
        if host:
            hw[name] = wb
            wb = wb.to(dev)
        ws[name] = wb
        perm = torch.randperm(n, generator=g, device=gdev)
        nbits = torch.empty(n, dtype=torch.int64)
        block = torch.empty(n, dtype=torch.int64)
        groups, lo = [], 0
        for gi, (frac, nb, b) in enumerate(cfg["alloc"]):
            hi = n if gi == len(cfg["alloc"]) - 1 else lo + int(round(frac * n))
            rows = perm[lo:hi].sort().values
            rows_h = rows.cpu()
            nbits[rows_h] = nb
            block[rows_h] = b
            groups.append((nb, b, rows.to(dev), rows_h))
            lo = hi
        masks[name] = {"groups": groups, "nbits": nbits, "block": block}
    if host:
        return xs, ws, masks, (hx, hw)
    return xs, ws, masks


# streams and the inputs each one encodes in turn (one stream per input measured best:
# the short chains fill the GPU around the long chain's latency-bound steps)
_CHAIN_STREAMS = {}
HEAD_START = os.environ.get("HI2_HEAD_START", "transform")
# the critical chain's rotations and ladder fits on the last chain's stream (0: in place)
OFFLOAD_PREP = os.environ.get("HI2_OFFLOAD_PREP", "1") != "0"
# the other chains' streams marked background (hi2x_stream_background; 0: not marked)
BACKGROUND = os.environ.get("HI2_BACKGROUND", "1") != "0"


def _chain_stream(dev, i):
    """The stream of chain lane i: lane 0 (the critical chain) runs on the caller's
    current stream, every other lane on a persistent stream of its own (reused every step,
    so each keeps its cached device blocks; the library's own side streams are separate).
    HIP maps streams onto a few hardware queues (four here), and two streams on one queue
    run in turn: the critical chain measured 24 ms for its factor alone on a queue and
    29 ms sharing one with another chain, and which pool stream lands on which queue
    depends on what the process created before.  The current stream's queue held no other
    stream in every kernel trace, so the critical chain takes it."""
    import torch

    if i == 0:
        return torch.cuda.current_stream(dev)
    key = (dev.index, i)
    if key not in _CHAIN_STREAMS:
        _CHAIN_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _CHAIN_STREAMS[key]


def encode_block(xs, ws, masks, timer=None, lanes=None, keep=None, cfg=CFG3):
    """Encode the whole block (see _encode_block).  Every chain's stream but the first
    (the critical path) is marked background while the step's work is enqueued, and the
    marks are cleared once it is (they are read when a launch is enqueued)."""
    from hi2_amd import _lib

    dev = next(iter(xs.values())).device
    n_lanes = len(cfg["order"]) if lanes is None else len(lanes)
    marked = [_chain_stream(dev, i) for i in range(1, n_lanes)] if BACKGROUND else []
    for st in marked:
        _lib.stream_background(st, True)
    try:
        return _encode_block(xs, ws, masks, timer, lanes, keep, cfg)
    finally:
        for st in marked:
            _lib.stream_background(st, False)


def _encode_block(xs, ws, masks, timer=None, lanes=None, keep=None, cfg=CFG3):
    """Encode the whole block.  Each calibration input runs its own chain on its own
    stream (Hessian -> transform -> factor -> rotation -> GPTQ -> packing of the linears
    it feeds); the chains are independent, so they overlap on the GPU.  The first chain
    (the widest input: the critical path) hands its rotations and ladder fits, which need
    only its Hessian's diagonal, to the head of the last chain's stream, where they run
    while its factor is computed; its rounding waits for them.  Once every chain has ended,
    one launch packs all linears; the host builds its tables while the chains run.  The
    host waits once, for the packing's range counter, and then reads the factor statuses:
    an input whose first factor attempt failed gets the damping retries, its rounding is
    redone and the block is packed again.  keep (a dict) receives each input's (stream, hs,
    jobs, where, encs)."""
    import torch

    from hi2_amd.format import assemble_many, rotate_rows
    from hi2_amd.hessian import GptqJob, HessianStats, encode_jobs_gptq, prepare_jobs_gptq
    from hi2_amd.hessian import finish_factor, inverse_factor_async, round_prepared

    dev = next(iter(xs.values())).device
    main = torch.cuda.current_stream(dev)
    order_in = cfg["order"]
    lanes = [[inp] for inp in order_in] if lanes is None else lanes
    lane_of = {inp: li for li, lane in enumerate(lanes) for inp in lane}
    width = max(len(l) for l in lanes)
    order = [inp for lane in zip(*[l + [None] * (width - len(l)) for l in lanes]) for inp in lane
             if inp is not None]
    # the critical chain's preparation moves to the last chain's stream (with one lane
    # there is nowhere to move it)
    crit = order[0] if len(lanes) > 1 and OFFLOAD_PREP else None
    helper = lanes[-1][0] if crit is not None else None  # first chain of the last lane
    chains = {}
    point = timer.point if timer else (lambda name: None)
    point("start")
    for li in range(1, len(lanes)):  # lane 0 is main itself
        _chain_stream(dev, li).wait_stream(main)
    lead = None  # the first chain's head start: the others wait for its Hessian stages

    def prepare(inp, had, d, u):
        """Rotation and ladder fits of the linears fed by inp, on the current stream."""
        jobs, where = [], []
        for name, n, kk, i in cfg["linears"]:
            if i != inp:
                continue
            for nb, b, rows_d, rows_h in masks[name]["groups"]:
                # == fwht_groups(ws[name].float(), had).index_select(0, rows_d)
                jobs.append(GptqJob(rotate_rows(ws[name], had, rows_d), d, u, nb, b))
                where.append((name, rows_h))
        return jobs, where, prepare_jobs_gptq(jobs, EFFORT)

    crit_d = None  # (event after the critical chain's d, had, d, u)
    for inp in order:
        k = cfg["inputs"][inp]
        st = _chain_stream(dev, lane_of[inp])
        mark = (lambda stage, inp=inp: timer.mark(inp, stage)) if timer else (lambda stage: None)
        with torch.cuda.stream(st):
            if lead is not None and lane_of[inp] != 0:
                st.wait_event(lead)
            if inp == helper:  # first the critical chain's rotations and fits
                ev, chad, cd, cu = crit_d
                st.wait_event(ev)
                for t in (chad, cd, cu):
                    t.record_stream(st)
                cjobs, cwhere, cprep = prepare(crit, chad, cd, cu)
                cprep.record_stream(_chain_stream(dev, lane_of[crit]))
                for j in cjobs:
                    j.w.record_stream(_chain_stream(dev, lane_of[crit]))
                done = torch.cuda.Event()
                done.record(st)
                chains[crit][5:7] = [cjobs, cwhere]
                crit_prep = (done, cprep)
            had = torch.ones(k // 16, dtype=torch.uint8, device=dev)
            mark("hessian")
            hst = HessianStats(k, dev)
            hst.update(xs[inp])
            if HEAD_START == "hessian" and lane_of[inp] == 0 and lead is None:
                lead = torch.cuda.Event()
                lead.record(st)
            mark("transform")
            hs = hst.transformed(None, had)  # == transform_sigma(hst.mean(), None, had)
            del hst
            d = hs.diagonal().clone()
            if HEAD_START == "transform" and lane_of[inp] == 0 and lead is None:
                lead = torch.cuda.Event()
                lead.record(st)
            if inp == crit:  # d is what the ladder fits need
                ev = torch.cuda.Event()
                ev.record(st)
            mark("factor")
            u, status = inverse_factor_async(hs, DAMP)
            if inp == crit:
                crit_d = (ev, had, d, u)
                chains[inp] = [st, hs, u, status, had, None, None, None]
                continue
            mark("rotate")
            jobs, where, prep = prepare(inp, had, d, u)
            mark("gptq")
            encs = round_prepared(prep)
            mark("end")
        chains[inp] = [st, hs, u, status, had, jobs, where, encs]
    if crit is not None:
        st = chains[crit][0]
        mark = (lambda stage: timer.mark(crit, stage)) if timer else (lambda stage: None)
        with torch.cuda.stream(st):
            done, cprep = crit_prep
            mark("prep_wait")
            st.wait_event(done)
            mark("gptq")
            chains[crit][7] = round_prepared(cprep)
            mark("end")
    point("enqueued")

    def pack():
        """Every linear of the block packed by one launch, on the main stream once every
        chain has ended (the host builds the launch's tables while the chains run)."""
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        tensors, names = [], []
        for inp in order:
            st, hs, u, status, had, jobs, where, encs = chains[inp]
            if st != main:
                main.wait_stream(st)
            for name, n, k, i in cfg["linears"]:
                if i != inp:
                    continue
                pieces = [(rows, e.codes, e.params, e.consts)
                          for (nm, rows), e in zip(where, encs) if nm == name]
                tensors.append(dict(pieces=pieces, row_nbits=masks[name]["nbits"],
                                    row_block=masks[name]["block"],
                                    had=torch.ones(k // 16, dtype=torch.uint8), k=k))
                names.append(name)
        return dict(zip(names, assemble_many(tensors, stager=_DeviceStager, bad=bad))), bad

    out, bad = pack()
    point("packed")
    if int(bad.item()):  # waits for every chain and the packing
        raise ValueError("code outside the ladder")
    point("end")
    # the factor statuses are final now: an input whose first attempt failed gets the
    # reference's damping retries, its rounding redone, and the block is packed again
    redo = False
    for inp in order:
        st, hs, u, status, had, jobs, where, encs = chains[inp]
        with torch.cuda.stream(st):
            if finish_factor(hs, u, status, DAMP):
                chains[inp][7] = encode_jobs_gptq(jobs, EFFORT)
                redo = True
    if redo:
        out, bad = pack()
        if int(bad.item()):
            raise ValueError("code outside the ladder")
    if keep is not None:
        for inp in order:
            st, hs, u, status, had, jobs, where, encs = chains[inp]
            keep[inp] = (st, hs, jobs, where, encs)
    return out


def trailing_flops(cfg) -> float:
    """Algorithmic flops of every cross-block update of a step: per linear,
    sum over 128-column blocks of 2 N 128 (K - i2) on the real rows (no padding)."""
    total = 0.0
    for _, n, k, _ in cfg["linears"]:
        for i1 in range(0, k, 128):
            i2 = min(i1 + 128, k)
            total += 2.0 * n * (i2 - i1) * (k - i2)
    return total


def stage_breakdown(xs, ws, masks, cfg=CFG3):
    """One step run serially on one stream with every stage timed: per input its Hessian,
    transform and factor (stream events), per linear its rotation, ladder fit, column
    loop, trailing update, finish and packing (the library's per-launch events summed by
    kernel family).  Returns (per_input, per_linear, hbm) in ms and the HBM rates of the
    rotation and packing kernels."""
    import torch

    from hi2_amd import _lib
    from hi2_amd.format import assemble_many, rotate_rows
    from hi2_amd.hessian import GptqJob, HessianStats, encode_jobs_gptq, inverse_factor

    dev = next(iter(xs.values())).device
    per_input, per_linear = {}, {}
    hbm = {7: [0.0, 0.0], 9: [0.0, 0.0]}  # kind -> [bytes, ms]
    tensors = []  # every linear's pieces, packed by one launch at the end (as the step does)

    def ev():
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    for inp in cfg["order"]:
        k = cfg["inputs"][inp]
        had = torch.ones(k // 16, dtype=torch.uint8, device=dev)
        e0 = ev()
        hst = HessianStats(k, dev)
        hst.update(xs[inp])
        e1 = ev()
        hs = hst.transformed(None, had)
        del hst
        e2 = ev()
        u = inverse_factor(hs, DAMP)
        e3 = ev()
        torch.cuda.synchronize()
        per_input[inp] = {"hessian": e0.elapsed_time(e1), "transform": e1.elapsed_time(e2),
                          "factor": e2.elapsed_time(e3)}
        d = hs.diagonal().clone()
        for name, n, kk, i in cfg["linears"]:
            if i != inp:
                continue
            kinds = [7, 8, 4, 0, 10]
            _lib.timing_enable(kinds)
            jobs = [GptqJob(rotate_rows(ws[name], had, rows_d), d, u, nb, b)
                    for nb, b, rows_d, _ in masks[name]["groups"]]
            encs = encode_jobs_gptq(jobs, EFFORT)
            tensors.append(dict(pieces=[(g[3], e.codes, e.params, e.consts)
                                        for g, e in zip(masks[name]["groups"], encs)],
                                row_nbits=masks[name]["nbits"], row_block=masks[name]["block"],
                                had=torch.ones(kk // 16, dtype=torch.uint8), k=kk))
            torch.cuda.synchronize()
            row = {}
            for kind, label in ((7, "rotate"), (8, "ladder_fit"), (4, "column_loop"),
                                (0, "trailing"), (10, "finish")):
                cnt, ms, work = _lib.timing_query(kind)
                row[label] = round(ms, 3)
                if kind in hbm:
                    hbm[kind][0] += work
                    hbm[kind][1] += ms
            per_linear[name] = row
            _lib.timing_enable([])
            del jobs, encs
        del hs, u, d
    _lib.timing_enable([9])
    assemble_many(tensors, stager=_DeviceStager)
    torch.cuda.synchronize()
    cnt, ms, work = _lib.timing_query(9)
    _lib.timing_enable([])
    hbm[9] = [work, ms]
    del tensors
    rates = {}
    for kind, kname in ((7, "rotate_rows_kernel"), (9, "assemble_kernel")):
        b, ms = hbm[kind]
        if ms > 0:
            gbs = b / ms / 1e6
            rates[kname] = {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM / 1e9,
                            "unit": "GB/s", "frac": gbs / (PEAK_HBM / 1e9),
                            "bytes_per_step": b, "ms_per_step": ms,
                            "work": "rotation: 2 B read (bf16) + 4 B written (f32) per weight "
                            "of the selected rows" if kind == 7
                            else "pack (all linears of the step in one launch): code bytes "
                            "read + packed words written + ladder bytes read and written + "
                            "consts"}
    return per_input, per_linear, rates


def block_leg(cfg, dev, steps, warmup):
    """A whole configuration (cfg4) timed like the main step, plus its serial stage
    breakdown and trailing roofline; the inputs are freed afterwards."""
    import torch

    from hi2_amd import _lib

    xs, ws, masks = make_inputs(dev, 1, cfg)
    torch.cuda.synchronize()
    for _ in range(warmup):
        encode_block(xs, ws, masks, cfg=cfg)
    torch.cuda.synchronize()
    with quiet_host():
        t0 = time.perf_counter()
        for i in range(steps):
            if i == steps - 1:  # launch events in the last timed step only
                _lib.timing_enable([0, 1, 2, 11])
            encode_block(xs, ws, masks, cfg=cfg)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    tr = _lib.timing_query(0)
    sy = _lib.timing_query(1)
    ch = _lib.timing_query(2)
    sp = _lib.timing_query(11)
    _lib.timing_enable([])
    per_input, per_linear, rates = stage_breakdown(xs, ws, masks, cfg)
    flops = trailing_flops(cfg)
    trail_ms = tr[1]  # one step's launches
    res = {
        "workload": f"{cfg['name']}: " + ", ".join(f"{n} {r}x{k}" for n, r, k, _ in cfg["linears"])
                    + f"; {cfg['tokens']} tokens; "
                    + " / ".join(f"{int(round(f * 100))}% INT{nb}/B{b}" for f, nb, b in cfg["alloc"]),
        "steps": steps,
        "ms_per_step": ms,
        "ms_per_linear": ms / len(cfg["linears"]),
        "trailing_roofline": {"bound": "mfma", "achieved": flops / trail_ms / 1e9,
                              "peak": PEAK_F32 / 1e12, "unit": "TFLOP/s",
                              "frac": flops / trail_ms / 1e9 / (PEAK_F32 / 1e12),
                              "flops_per_step": flops, "launches_per_step": tr[0],
                              "timing": "event-timed launches in the last timed step (chains "
                                        "concurrent)"},
        "syrk_tflops_executed": sy[2] / sy[1] / 1e9 if sy[1] > 0 else None,
        "factor_fp32_gemm_tflops": ch[2] / ch[1] / 1e9 if ch[1] > 0 else None,
        "factor_split_fp16_tflops_executed": sp[2] / sp[1] / 1e9 if sp[1] > 0 else None,
        "stages_serial_ms": {"per_input": per_input, "per_linear": per_linear},
        "hbm_kernels": rates,
    }
    del xs, ws, masks
    torch.cuda.empty_cache()
    return res


# ---- cfg5: the OLMoE-shaped MoE layer ------------------------------------------------------
E5, T5, TOP5, H5, I5 = 64, 16384, 8, 2048, 1024
ALLOC5 = [(0.30, 2, 32), (0.70, 4, 64)]
FLOOR5 = 2.0  # expert_min_tokens (hi2/calibrate.py:69) x the widest input


def moe_inputs(dev, seed=5):
    """Router indices [T, 8] (Zipf(1.1), Gumbel-top-8), hidden tokens [T, 2048], the down
    projection's inputs [8 T, 1024] in expert order (act(gate) * up of the routed slots,
    synthesised), bf16 weights of gate/up [E, 2 I, H] and down [E, H, I], and per expert
    tensor its allocation rows (30 % INT2/B32, 70 % INT4/B64)."""
    import torch

    from hi2_amd.workloads import activations, zipf_topk

    idx = zipf_topk(T5, E5, TOP5, 1.1, seed, dev)
    x = activations(T5, H5, seed + 1, dev)
    xd = activations(T5 * TOP5, I5, seed + 2, dev)
    g = torch.Generator(device=dev).manual_seed(seed + 3)
    wgu = (torch.randn(E5, 2 * I5, H5, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E5, H5, I5, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    masks = {}
    for e in range(E5):
        for name, n in (("gate", I5), ("up", I5), ("down", H5)):
            perm = torch.randperm(n, generator=g, device=dev)
            n2 = int(round(ALLOC5[0][0] * n))
            groups = []
            nbits = torch.full((n,), ALLOC5[1][1], dtype=torch.int64)
            block = torch.full((n,), ALLOC5[1][2], dtype=torch.int64)
            for (frac, nb, b), rows in zip(ALLOC5, (perm[:n2].sort().values,
                                                    perm[n2:].sort().values)):
                rh = rows.cpu()
                nbits[rh] = nb
                block[rh] = b
                groups.append((nb, b, rows, rh))
            masks[(e, name)] = {"groups": groups, "nbits": nbits, "block": block}
    return idx, x, xd, wgu, wdn, masks


def encode_moe(idx, x, xd, wgu, wdn, masks, timer=None):
    """One MoE layer: the routed batch, every expert's gate/up (K = 2048) and down
    (K = 1024) Hessians in one grouped launch each, the token floor, the batched
    transforms and factors, the rotation, GPTQ of all experts' rows (one factor per
    expert), and packing of the 192 expert tensors into device buffers."""
    import torch

    from hi2_amd.format import assemble_many, rotate_rows
    from hi2_amd.hessian import (GptqJob, encode_jobs_gptq, finish_factors_batched,
                                 inverse_factors_batched_async)
    from hi2_amd.moe import ExpertHessians, route_order

    dev = x.device
    mark = timer.mark if timer else (lambda *a: None)
    mark("moe", "route")
    rows, offs = route_order(idx, E5)
    mark("moe", "hessian")
    gu = ExpertHessians(E5, H5, dev)
    gu.update_routed(x, offs, rows)
    dn = ExpertHessians(E5, I5, dev)
    dn.update_routed(xd, offs)
    mark("moe", "floor")
    need = int(FLOOR5 * H5)
    gu.top_up(need)
    dn.top_up(need)
    mark("moe", "transform")
    had_h = torch.ones(H5 // 16, dtype=torch.uint8, device=dev)
    had_i = torch.ones(I5 // 16, dtype=torch.uint8, device=dev)
    hs_g = gu.transformed(None, had_h)
    hs_d = dn.transformed(None, had_i)
    del gu, dn
    mark("moe", "factor")
    u_g, st_g = inverse_factors_batched_async(hs_g, DAMP)
    u_d, st_d = inverse_factors_batched_async(hs_d, DAMP)
    mark("moe", "rotate")
    d_g = torch.diagonal(hs_g, dim1=1, dim2=2).contiguous()
    d_d = torch.diagonal(hs_d, dim1=1, dim2=2).contiguous()
    # one job per expert, projection input and allocation class: gate and up rows of one
    # class share the expert's Hessian, so they are rounded together (fewer, larger
    # units); where[j] lists the (tensor, rows, slice of the job) it holds
    jobs, where = [], []
    for e in range(E5):
        for ci, (nb, b) in enumerate((g[0], g[1]) for g in masks[(e, "gate")]["groups"]):
            rg = masks[(e, "gate")]["groups"][ci]
            ru = masks[(e, "up")]["groups"][ci]
            rows = torch.cat([rg[2], ru[2] + I5])
            jobs.append(GptqJob(rotate_rows(wgu[e], had_h, rows), d_g[e], u_g[e], nb, b))
            where.append([((e, "gate"), rg[3], 0, rg[3].numel()),
                          ((e, "up"), ru[3], rg[3].numel(), rows.numel())])
        for nb, b, rows_d, rows_h in masks[(e, "down")]["groups"]:
            jobs.append(GptqJob(rotate_rows(wdn[e], had_i, rows_d), d_d[e], u_d[e], nb, b))
            where.append([((e, "down"), rows_h, 0, rows_h.numel())])
    mark("moe", "gptq")
    encs = encode_jobs_gptq(jobs, EFFORT)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    flags = {H5: torch.ones(H5 // 16, dtype=torch.uint8), I5: torch.ones(I5 // 16, dtype=torch.uint8)}

    def pack(encs):
        """The 192 expert tensors' packing, enqueued behind the rounding (the host builds
        its tables while the GPU rounds)."""
        by = {}
        for parts, enc in zip(where, encs):
            for key, rows_h, a, z in parts:
                by.setdefault(key, []).append((rows_h, enc.codes[a:z], enc.params[a:z],
                                               enc.consts[a:z]))
        keys = list(by)
        packed = assemble_many([dict(pieces=by[key], row_nbits=masks[key]["nbits"],
                                     row_block=masks[key]["block"],
                                     had=flags[H5 if key[1] != "down" else I5],
                                     k=H5 if key[1] != "down" else I5) for key in keys],
                               stager=_DeviceStager, bad=bad)
        return dict(zip(keys, packed))

    mark("moe", "pack")
    out = pack(encs)
    mark("moe", "end")
    # the factor statuses are read only now (the read waits for the work enqueued so far)
    redo = finish_factors_batched(hs_g, u_g, st_g, DAMP) + finish_factors_batched(hs_d, u_d, st_d,
                                                                                   DAMP)
    if redo:  # an expert needed more damping: its rows again (the reference's retry)
        bad.zero_()
        out = pack(encode_jobs_gptq(jobs, EFFORT))
    if int(bad.item()):
        raise ValueError("code outside the ladder")
    return out


def moe_leg(dev, steps, warmup):
    import torch

    from hi2_amd import _lib

    inp = moe_inputs(dev)
    torch.cuda.synchronize()
    for _ in range(warmup):
        encode_moe(*inp)
    torch.cuda.synchronize()
    with quiet_host():
        t0 = time.perf_counter()
        for i in range(steps):
            if i == steps - 1:  # launch events in the last timed step only
                _lib.timing_enable([0, 1, 2, 3, 11])
            encode_moe(*inp)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    tr, sy, ch, lf, sp = (_lib.timing_query(k) for k in (0, 1, 2, 3, 11))
    _lib.timing_enable([])
    timer = StageTimer(torch)
    encode_moe(*inp, timer=timer)
    stages = timer.summary()["moe"]
    counts = torch.bincount(inp[0].reshape(-1), minlength=E5).cpu().tolist()
    # trailing flops on the real rows: per expert gate/up 2048 rows at K = 2048, down
    # 2048 rows at K = 1024
    flops = 0.0
    for n, k in ((2 * I5, H5), (H5, I5)):
        for i1 in range(0, k, 128):
            i2 = min(i1 + 128, k)
            flops += E5 * 2.0 * n * (i2 - i1) * (k - i2)
    trail_ms = tr[1]  # one step's launches
    res = {
        "workload": "cfg5: OLMoE-shaped MoE layer, 64 experts (gate/up 1024x2048 sharing a "
                    "Hessian, down 2048x1024), top-8 of 16384 tokens routed by Zipf(1.1) "
                    "Gumbel-top-k, token floor 2 x 2048, 30% INT2/B32 + 70% INT4/B64 rows",
        "steps": steps,
        "ms_per_layer": ms,
        "ms_per_expert_linear": ms / (3 * E5),
        "routed_tokens_per_expert": {"min": min(counts), "median": sorted(counts)[E5 // 2],
                                     "max": max(counts)},
        "experts_below_floor": sum(c < int(FLOOR5 * H5) for c in counts),
        "stages_ms": stages,
        "trailing_roofline": {"bound": "mfma", "achieved": flops / trail_ms / 1e9,
                              "peak": PEAK_F32 / 1e12, "unit": "TFLOP/s",
                              "frac": flops / trail_ms / 1e9 / (PEAK_F32 / 1e12),
                              "flops_per_step": flops, "launches_per_step": tr[0]},
        "grouped_syrk": {"launches_per_step": sy[0], "ms_per_step": sy[1],
                         "tflops_executed": sy[2] / sy[1] / 1e9 if sy[1] > 0 else None},
        "factor_ms_per_step_kernels": ch[1] + lf[1] + sp[1],
    }
    del inp
    torch.cuda.empty_cache()
    return res


REFINE_PASSES = 2  # the reference's default for a calibrated GPTQ run without QAD


_REFINE_STREAMS = {}


def refine_linears(kept, serial=False):
    """Local code refinement of every linear of the block (hi2/calibrate.py:374-391: one
    sweep per tensor over all its candidate groups, with the input's transformed Hessian),
    each calibration input's linears on a refinement stream of that input's own.  Own
    streams, not the encode chains' (the down_proj input's is the caller's), and none
    marked background: 78 against 86 ms per block measured in one process (the
    refinement is GEMM-bound throughout, so the background reservation only costs).
    With ``serial`` everything runs on the caller's stream, one linear after another.
    Returns the refined codes."""
    import torch

    from hi2_amd.refine import refine_groups

    dev = next(iter(kept.values()))[1].device
    main = torch.cuda.current_stream(dev)
    out = {}
    streams = []
    for li, inp in enumerate(CFG3["order"]):
        _, hs, jobs, where, encs = kept[inp]
        key = (dev.index, li)
        if key not in _REFINE_STREAMS:
            _REFINE_STREAMS[key] = torch.cuda.Stream(device=dev)
        st = main if serial else _REFINE_STREAMS[key]
        if st != main:
            streams.append(st)
            st.wait_stream(main)
        if kept[inp][0] != st:
            st.wait_stream(kept[inp][0])
        with torch.cuda.stream(st):
            for name, n, k, i in LINEARS:
                if i != inp:
                    continue
                xs = [x for x, (nm, _) in enumerate(where) if nm == name]
                out[name] = refine_groups(
                    [(jobs[x].w, encs[x], jobs[x].nbits, jobs[x].block) for x in xs], hs,
                    REFINE_PASSES)
    for st in streams:
        main.wait_stream(st)
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
    """Events on each chain's stream at its stage boundaries, and host points of the
    step: each a host clock reading and an event on the caller's stream, so the report
    shows how far the host's enqueueing ran ahead of the GPU."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}
        self.points = []

    def mark(self, chain, stage):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.events.setdefault(chain, []).append((stage, e))

    def point(self, name):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.points.append((name, time.perf_counter(), e))

    def summary(self):
        self.torch.cuda.synchronize()
        out = {}
        for chain, evs in self.events.items():
            out[chain] = {n0: round(e0.elapsed_time(e1), 3)
                          for (n0, e0), (_, e1) in zip(evs, evs[1:])}
        return out

    def host_points(self):
        """{point: (host ms, GPU ms)} since the step's first point: the host clock when
        the point was reached, and the time its event ran on the caller's stream (behind
        all work enqueued there before it)."""
        self.torch.cuda.synchronize()
        if not self.points:
            return {}
        _, h0, e0 = self.points[0]
        return {n: [round((h - h0) * 1e3, 3), round(e0.elapsed_time(e), 3)]
                for n, h, e in self.points}


# kernel families timed by the library (hi2x_timing_*), with the peak that bounds each
KERNELS = {  # kind -> (kernel, bound, peak FLOP/s, work unit)
    0: ("gptq_trailing_kernel", "mfma", PEAK_F32, "2*rows*rank*cols"),
    1: ("syrk2_bf16_kernel", "mfma", PEAK_BF16, "T*K*(K+1) (upper triangle, 2 flops per product)"),
    2: ("tri_gemm_kernel", "mfma", PEAK_F32, "M*N*rank (one triangular operand; the "
        "factor's fp32 MFMA products)"),
    11: ("gemm3_kernel/gemm3x_kernel (split planes)", "mfma", PEAK_BF16,
         "3*M*N*rank fp16 MFMA flops executed (three fp16 products per fp32-equivalent "
         "product of one triangular operand)"),
    3: ("leaf_kernel", "latency", PEAK_F32, "2*n^3/3"),
    4: ("gptq_block_kernel", "latency", PEAK_F32, "rows*L*(L-1)"),
    5: ("refine GEMMs (refine_gradient_kernel + gptq_trailing_kernel)", "mfma", PEAK_F32,
        "2*rows*rank*cols"),
    6: ("refine_block_kernel", "latency", PEAK_F32, "rows*L (column decisions)"),
    8: ("ladder_fit_kernel", "valu", PEAK_HBM, "bytes of w read (rows*k*4)"),
}
DOMINANT = 0  # the GPTQ trailing-update GEMM: the metric's MFMA kernel with the most time


def kernel_stats(kind):
    """Event-timed launches of one kernel family since hi2x_timing_enable.  The SYRK also
    carries the algorithmic rate: the reference's Hessian is a full fp32 GEMM, 2 T K^2
    flops per input (its executed work here is the upper triangle, T K (K + 1))."""
    from hi2_amd import _lib

    name, bound, peak, unit = KERNELS[kind]
    n, ms, work = _lib.timing_query(kind)
    if n == 0 or ms <= 0.0:
        return None
    rate = work / (ms / 1e3)
    out = {"kernel": name, "bound": bound, "launches": n, "avg_ms": ms / n,
           "total_ms": ms, "work_per_launch": work / n, "work_unit": unit,
           "tflops": rate / 1e12, "frac_of_peak": rate / peak}
    if kind == 1:  # T K (K + 1) executed -> 2 T K^2 algorithmic: a factor 2 K / (K + 1)
        k = max(CFG3["inputs"].values())
        alg = rate * 2.0 * k / (k + 1)
        out["algorithmic"] = {"work_unit": "2*T*K^2 (the reference's full GEMM)",
                              "tflops": alg / 1e12, "frac_of_peak": alg / peak}
    return out


def pmc_traffic(kernel):
    """HBM bytes per launch of ``kernel`` (read + write) from the committed counter
    summary (profiles/traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE passes over this
    bench's step, each scaled by what the counter reads for a 1 GiB device copy), with the
    split; None when the summary or the kernel is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            e = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None, None
    if not e:
        return None, None
    rd, wr = e["fetch_bytes_per_launch"], e["write_bytes_per_launch"]
    return rd + wr, {"read_bytes": rd, "write_bytes": wr, "dispatches": e["dispatches"],
                     "source": "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE, then "
                               "WRITE_SIZE, averaged over the step's launches)"}


def trailing_roofline(steps, basis):
    """The trailing update's roofline over the last timing window: the algorithmic flops
    of the block's cross-block updates on real rows (trailing_flops) divided by the summed
    event-timed durations of its launches; ``traffic`` from the committed PMC summary."""
    from hi2_amd import _lib

    n, ms, work = _lib.timing_query(DOMINANT)
    flops = trailing_flops(CFG3) * steps
    rate = flops / (ms / 1e3)
    traffic, split = pmc_traffic(KERNELS[DOMINANT][0])
    return {"bound": "mfma", "achieved": rate / 1e12, "peak": PEAK_F32 / 1e12,
            "unit": "TFLOP/s", "frac": rate / PEAK_F32, "traffic": traffic,
            "traffic_split": split,
            "kernel": KERNELS[DOMINANT][0], "launches": n, "avg_ms": ms / n,
            "flops_per_launch": flops / n,
            "work": "2*rows*rank*cols summed over the block's cross-block updates, real rows "
                    "only (the launches also run the zero rows that align factor runs to "
                    "128)", "timing": basis}


def _cpu_info():
    import torch

    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    par = torch.__config__.parallel_info()
    return {"nproc": os.cpu_count(), "model": model, "torch_threads": torch.get_num_threads(),
            "parallel_info": [l.strip() for l in par.splitlines() if l.strip()][:8]}


def _torch_cpu_block(R, cfg, seed, host=None, keep=None):
    """The reference's CPU path (oracle/torch_cpu.py) on a whole configuration: per input
    its Hessian (fp32 chunks), transform and factor; per linear rotation, GPTQ of every
    allocation group and packing.  Returns seconds per stage.  ``host`` = (calibration
    tokens, weights, allocation) runs it on given host tensors (the GPU step's own
    inputs); otherwise it draws its own from ``seed``.  ``keep`` (a dict) receives, per
    input, Sigma, Hs and U, and per linear and allocation group its rotated rows, codes,
    ladder bytes, consts, sse and comp (numpy), for the parity check."""
    import torch

    g = torch.Generator().manual_seed(seed)
    parts = {"hessian": 0.0, "transform": 0.0, "factor": 0.0, "rotate": 0.0, "gptq": 0.0,
             "pack": 0.0}
    for inp, k in cfg["inputs"].items():
        if host is None:
            x = torch.randn(cfg["tokens"], k, generator=g)
            x[:, torch.randperm(k, generator=g)[: (k + 99) // 100]] *= 20.0
            x = x.to(torch.bfloat16)
        else:
            x = host[0][inp]
        flags = torch.ones(k // 16, dtype=torch.uint8)
        t0 = time.perf_counter()
        sigma = R.hessian_sum(x) / x.shape[0]
        t1 = time.perf_counter()
        hs = R.transform_sigma(sigma, None, flags)
        t2 = time.perf_counter()
        u = R.inverse_factor(hs, DAMP)
        t3 = time.perf_counter()
        parts["hessian"] += t1 - t0
        parts["transform"] += t2 - t1
        parts["factor"] += t3 - t2
        d = hs.diagonal().clone()
        if keep is not None:
            keep.setdefault("inputs", {})[inp] = {"sigma": sigma.numpy(), "hs": hs.numpy(),
                                                  "u": u.numpy()}
        del x, sigma
        for name, n, kk, i in cfg["linears"]:
            if i != inp:
                continue
            if host is None:
                w = (torch.randn(n, kk, generator=g) * 0.02).to(torch.bfloat16)
                perm = torch.randperm(n, generator=g)
                rows_of, lo = [], 0
                for gi, (frac, nb, b) in enumerate(cfg["alloc"]):
                    hi = n if gi == len(cfg["alloc"]) - 1 else lo + int(round(frac * n))
                    rows_of.append((nb, b, perm[lo:hi].sort().values))
                    lo = hi
            else:
                w = host[1][name]
                rows_of = [(nb, b, rows_h) for nb, b, _, rows_h in host[2][name]["groups"]]
            t0 = time.perf_counter()
            wt = R.rotate(w.float(), flags)
            t1 = time.perf_counter()
            tg = tp = 0.0
            for nb, b, rows in rows_of:
                s0 = time.perf_counter()
                codes, prm, cst, sse, comp = R.gptq(wt[rows], d, u, nb, b, EFFORT)
                s1 = time.perf_counter()
                R.pack_codes(codes, nb)
                s2 = time.perf_counter()
                tg += s1 - s0
                tp += s2 - s1
                if keep is not None:
                    keep.setdefault("linears", {}).setdefault(name, []).append({
                        "nb": nb, "b": b, "rows": rows.numpy(), "wt": wt[rows].numpy(),
                        "codes": codes.numpy(), "params": prm.numpy(),
                        "consts": cst.view(torch.int16).numpy().view("uint16"),
                        "sse": sse.numpy(), "comp": comp.numpy()})
            parts["rotate"] += t1 - t0
            parts["gptq"] += tg
            parts["pack"] += tp
        del hs, u
    return parts


CFG1 = dict(name="cfg1", tokens=512, linears=[("linear", 2048, 2048, "x")],
            inputs={"x": 2048}, alloc=[(1.0, 4, 64)])


def cpu_baseline(seed=0, which=("cfg1", "cfg3"), host=None, keep=None):
    """The reference's own CPU path (restated in torch: oracle/torch_cpu.py, bit-identical
    to the reference on its fixtures) timed on this host's cores, on cfg1 and cfg3 in
    full.  value: cfg3 ms per linear (the metric of the GPU line).  ``host``: cfg3's
    inputs as the GPU step drew them (see make_inputs); ``keep`` receives cfg3's outputs
    (see _torch_cpu_block)."""
    import torch

    from oracle import torch_cpu as R

    out = {"unit": "ms per linear", "kind": "port", "cores": torch.get_num_threads(),
           "host": _cpu_info()}
    for name, cfg in (("cfg1", CFG1), ("cfg3", CFG3)):
        if name not in which:
            continue
        t0 = time.perf_counter()
        parts = _torch_cpu_block(R, cfg, seed, host if name == "cfg3" else None,
                                 keep if name == "cfg3" else None)
        wall = time.perf_counter() - t0
        out[name] = {"s_total": round(wall, 2),
                     "ms_per_linear": wall * 1e3 / len(cfg["linears"]),
                     "stages_s": {k: round(v, 2) for k, v in parts.items()}}
    main = out.get("cfg3") or out.get("cfg1")
    out["value"] = main["ms_per_linear"]
    out["sample"] = ("the reference's CPU path (torch ops of hi2/hessian.py, hi2/encode.py, "
                     "hi2/format.py restated in oracle/torch_cpu.py) on "
                     + " and ".join(w for w in which) + " in full, no extrapolation"
                     + ("; cfg3 on the GPU step's own inputs (drawn on the host, copied to "
                        "the device before the timed region)" if host is not None else "")
                     + "; value is " + ("cfg3" if "cfg3" in out else "cfg1")
                     + " ms per linear")
    return out


def gpu_outputs(xs, ws, masks, cfg=CFG3):
    """The step's outputs for the parity check, on the host: one more (untimed) step with
    every chain's Hs, factor and encodings kept, the rounding run again with comp on (the
    same codes: comp only records the values the codes were rounded from), and each
    input's Sigma."""
    import torch

    from hi2_amd.hessian import HessianStats, encode_jobs_gptq

    dev = next(iter(xs.values())).device
    kept = {}
    encode_block(xs, ws, masks, keep=kept, cfg=cfg)
    out = {"inputs": {}, "linears": {}}
    for inp, k in cfg["inputs"].items():
        _, hs, jobs, where, encs = kept.pop(inp)
        hst = HessianStats(k, dev)
        hst.update(xs[inp])
        out["inputs"][inp] = {"sigma": hst.mean().cpu().numpy(), "hs": hs.cpu().numpy(),
                              "u": jobs[0].u.cpu().numpy()}
        del hst
        with_comp = encode_jobs_gptq(jobs, EFFORT, comp=True)
        for (name, rows_h), job, e, ec in zip(where, jobs, encs, with_comp):
            if not torch.equal(e.codes, ec.codes):
                raise RuntimeError(f"{name}: codes changed with comp on")
            out["linears"].setdefault(name, []).append({
                "nb": job.nbits, "b": job.block, "rows": rows_h.numpy(),
                "codes": e.codes.cpu().numpy(), "params": e.params.cpu().numpy(),
                "consts": e.consts.view(torch.int16).cpu().numpy().view("uint16"),
                "sse": e.sse.cpu().numpy(), "comp": ec.comp.cpu().numpy()})
        del hs, jobs, encs, with_comp
    torch.cuda.synchronize()
    return out


def parity(gpu, cpu, cfg=CFG3):
    """The GPU step's cfg3 encoding against the reference's CPU path on the same inputs:
    Sigma, Hs and U relative to the largest entry, and per linear the share of equal
    codes, every departing row classified as a ladder or a rounding tie with its distance,
    and the sse (oracle/parity.py: compare_groups)."""
    import numpy as np

    from oracle.parity import compare_groups

    res = {"against": "the reference's CPU path (oracle/torch_cpu.py; bit-identical to the "
                      "reference on its fixtures at their thread count) on the same "
                      "host-drawn inputs, with this host's torch threads",
           "inputs": {}, "linears": {}}
    for inp in cfg["inputs"]:
        o, r = gpu["inputs"][inp], cpu["inputs"][inp]
        res["inputs"][inp] = {
            f"{m}_rel": float(np.abs(o[m] - r[m]).max() / np.abs(r[m]).max())
            for m in ("sigma", "hs", "u")}
    equal = total = dep = nl = nr = 0
    tie_q = tie_d = 0.0
    stay = 0.0
    sse_o = sse_r = 0.0
    for name, n, k, inp in cfg["linears"]:
        d_o = np.diag(gpu["inputs"][inp]["hs"]).copy()
        d_r = np.diag(cpu["inputs"][inp]["hs"]).copy()
        groups = []
        for go, gr in zip(gpu["linears"][name], cpu["linears"][name]):
            if (go["nb"], go["b"]) != (gr["nb"], gr["b"]) or not np.array_equal(go["rows"],
                                                                               gr["rows"]):
                raise RuntimeError(f"{name}: allocation groups differ")
            groups.append({"wt": gr["wt"], "o": go, "r": gr, "d_o": d_o, "d_r": d_r,
                           "nbits": go["nb"], "block": go["b"]})
        c = compare_groups(groups)
        res["linears"][name] = c
        equal += c["codes_equal"] * c["codes"]
        total += c["codes"]
        dep += c["rows_departing"]
        nl += c["ladder"]["rows"]
        nr += c["rounding"]["rows"]
        tie_q = max(tie_q, c["rounding"]["max_quotient_distance_steps"])
        tie_d = max(tie_d, c["ladder"]["max_d_rel"])
        stay = max(stay, c["sse_rel_max_rows_that_stay"])
        so = sum(float(x["sse"].astype(np.float64).sum()) for x in gpu["linears"][name])
        sr = sum(float(x["sse"].astype(np.float64).sum()) for x in cpu["linears"][name])
        sse_o += so
        sse_r += sr
    res["codes_equal"] = equal / total
    res["rows"] = sum(n for _, n, _, _ in cfg["linears"])
    res["rows_departing"] = dep
    res["ladder_rows"] = nl
    res["rounding_rows"] = nr
    res["max_rounding_tie_steps"] = tie_q
    res["max_ladder_d_rel"] = tie_d
    res["sse_rel_total"] = abs(sse_o / sse_r - 1)
    res["sse_rel_max_rows_that_stay"] = stay
    return res


def micro(which, reps=3):
    """One kernel family at the cfg3 shapes, alone on the GPU, event-timed; prints one
    JSON line per shape.  trailing: hi2x_gptq_run (column loop + cross-block updates) on
    4096 x 14336 and 14336 x 4096; syrk: HessianStats.update of 8192 bf16 tokens at
    K = 4096 and 14336; factor: inverse_factor at K = 14336 and 4096; refine: two
    refinement sweeps of GPTQ codes at 4096 x 4096, 4096 x 14336 and 14336 x 4096;
    stats: ColumnStats.update of 8192 bf16 tokens and the cached-Sigma payload at
    K = 4096 and 14336; qad: the QAD decode forward, backward and transform over the
    latents of q_proj, gate_proj and down_proj (30 % INT2/B32, 70 % INT4/B64 rows, step
    units); ladder: the ladder fits of down_proj's and q_proj's rows (30 % INT2/B32,
    70 % INT4/B64, effort "normal")."""
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
        """Wall milliseconds per call with no timing events (events around every launch
        add gaps that fall hardest on many-launch schedules), then the kernels' event
        statistics over the same number of calls in a second pass."""
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        _lib.timing_enable(kinds)
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
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

    if which == "ladder":
        from hi2_amd.encode import EFFORT as EFFORTS
        from hi2_amd.encode import _fit

        cfg = EFFORTS[EFFORT]
        for n, k in ((HIDDEN, INTER), (HIDDEN, HIDDEN)):
            g = torch.Generator(device=dev).manual_seed(0)
            w = torch.randn(n, k, generator=g, device=dev) * 0.02
            d = torch.rand(k, generator=g, device=dev) + 0.5
            for frac, nbits, b in CFG3["alloc"]:
                rows = int(round(frac * n))
                wb = w[:rows].reshape(rows, k // b, b)
                ms, stats = timed(lambda: _fit(wb, d, 2 ** nbits, cfg["grid"], cfg["ls"],
                                               False), [8])
                print(json.dumps({"micro": "ladder", "rows": rows, "k": k, "nbits": nbits,
                                  "block": b, "ms": ms, "kernels": stats}), flush=True)
    elif which == "trailing":
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
            ms, stats = timed(lambda: inverse_factor(hs, DAMP), [2, 3, 11])
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
    ap.add_argument("--cfg4-steps", type=int, default=2,
                    help="timed steps of the cfg4 (Llama-3-70B-shaped layer) leg (0: skip)")
    ap.add_argument("--cfg5-steps", type=int, default=2,
                    help="timed steps of the cfg5 (OLMoE-shaped MoE layer) leg (0: skip)")
    ap.add_argument("--micro", choices=["trailing", "syrk", "factor", "refine", "stats", "qad",
                                        "ladder"],
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
    # cfg3's inputs drawn once on the host and copied to the device before anything is
    # timed: the CPU baseline and the parity check run on these same tensors
    xs, ws, masks, host = make_inputs(dev, host=True)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        encode_block(xs, ws, masks)
    torch.cuda.synchronize()
    from hi2_amd import _lib

    timer = StageTimer(torch)
    torch.cuda.synchronize()
    with quiet_host():
        t0 = time.perf_counter()
        for i in range(args.steps):
            last = i == args.steps - 1
            if last:  # HIP events around each launch of the dominant kernel (~1 ms per step)
                _lib.timing_enable([DOMINANT])
            encode_block(xs, ws, masks, timer if last else None)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    stages = timer.summary()
    host_points = timer.host_points()
    roof = trailing_roofline(1, "contended: event-timed launches of the last timed step, "
                             "where the four input chains run concurrently")
    # one more, untimed step with every kernel family event-timed and the chains run one
    # after another on one stream: per-kernel rates without other chains sharing the GPU
    _lib.timing_enable(list(KERNELS))
    encode_block(xs, ws, masks, lanes=[CFG3["order"]])
    torch.cuda.synchronize()
    kernels = {KERNELS[k][0]: kernel_stats(k) for k in KERNELS}
    roof_iso = trailing_roofline(1, "isolated: one step with the chains run one after "
                                 "another on one stream")
    _lib.timing_enable([])
    per_input, per_linear, hbm = stage_breakdown(xs, ws, masks)
    gpu_out = None if args.no_cpu else gpu_outputs(xs, ws, masks)
    refine = None
    if args.refine_steps:
        kept = {}
        encode_block(xs, ws, masks, keep=kept)
        refine_linears(kept)  # warm-up
        torch.cuda.synchronize()
        with quiet_host():
            t0 = time.perf_counter()
            for i in range(args.refine_steps):
                if i == args.refine_steps - 1:  # launch events in the last timed step only
                    _lib.timing_enable([5])
                refine_linears(kept)
            torch.cuda.synchronize()
            r_ms = (time.perf_counter() - t0) * 1e3 / args.refine_steps
        r_stats = kernel_stats(5)
        _lib.timing_enable([5, 6])
        refine_linears(kept, serial=True)
        torch.cuda.synchronize()
        refine = {
            "what": f"local code refinement, {REFINE_PASSES} sweeps, of all 7 linears' GPTQ "
                    "codes (hi2/refine.py; the reference's default after calibrated GPTQ "
                    "without QAD); not part of value",
            "steps": args.refine_steps,
            "ms_per_step": r_ms,
            "ms_per_linear": r_ms / len(LINEARS),
            "gemm_contended": r_stats,
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
        with quiet_host():
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
    del xs, ws
    torch.cuda.empty_cache()
    cfg4 = block_leg(CFG4, dev, args.cfg4_steps, 1) if args.cfg4_steps else None
    cfg5 = moe_leg(dev, args.cfg5_steps, 1) if args.cfg5_steps else None
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
        "data": "synthetic (seeded normal X with 1% x20 outlier channels, W ~ N(0, 0.02^2), "
                "drawn on the host and resident in HBM before the timed region)",
        "config": {"workload": "cfg3: Llama-3-8B-shaped decoder block, 8192 calibration "
                               "tokens, 30% INT2/B32 + 70% INT4/B64 rows, order-16 Hadamard, "
                               "damp 0.01, effort normal", "linears": len(LINEARS),
                   "hessian_input_dtype": "bf16 (f32 accumulation)"},
        "chain_stages_ms": stages,
        "step_points_ms": {"what": "the last timed step: [host clock, GPU time of an event "
                           "on the caller's stream] at each point, ms since its start",
                           **host_points},
        "roofline": roof,
        "roofline_isolated": roof_iso,
        "kernels_one_step": kernels,
        "stages_serial_ms": {"per_input": per_input, "per_linear": per_linear},
        "hbm_kernels": hbm,
    }
    if refine is not None:
        res["refine"] = refine
    if many is not None:
        res["encode_many"] = many
    if cfg4 is not None:
        res["cfg4"] = cfg4
    if cfg5 is not None:
        res["cfg5"] = cfg5
    if not args.no_cpu:
        cpu_out = {}
        res["cpu_baseline"] = cpu_baseline(host=(host[0], host[1], masks), keep=cpu_out)
        res["parity"] = parity(gpu_out, cpu_out)
        del cpu_out, gpu_out
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
