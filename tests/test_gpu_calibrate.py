"""Encode orchestration on the MI355X (``hi2_amd.calibrate.encode_many``) against the
reference's own ``encode_many`` output and the oracle: packed buffers and ``comp`` bit
for bit.  The factor is the one quantity of the path that is not bit-identical to the
reference's LAPACK chain (it is pinned to tolerance elsewhere), so the golden tests feed
the reference's factors through the orchestration's factor hook; the other tests use the
device's own factors on both sides."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from golden_data import encode_many_case

pytestmark = pytest.mark.gpu

CANDS, TENSORS, CONFIGS = encode_many_case()
FIELDS = ("codes", "code_off", "blk_params", "param_off", "row_consts", "row_nbits",
          "row_block", "had")
OK = 0x7FFFFFFF


def _requests(dev, on_device=False, ref_stats_for=("n",)):
    """EncodeRequests of the fixture: bf16 weights stay bf16 (host or device), the
    statistics are this package's ColumnStats, or a reference-shaped object (S, n, k on
    the host) for the tensors named in ``ref_stats_for``."""
    from hi2_amd.calibrate import EncodeRequest, TensorTable
    from hi2_amd.stats import ColumnStats

    reqs = []
    for t in TENSORS:
        if t["w_bf16"] is not None:
            w = torch.from_numpy(t["w_bf16"].view(np.int16).copy()).view(torch.bfloat16)
        else:
            w = torch.from_numpy(t["w"].copy())
        cs = None
        if t["col_scale"] is not None:
            cs = torch.from_numpy(t["col_scale"].view(np.int16).copy()).view(torch.float16)
        sigma = None if t["sigma"] is None else torch.from_numpy(t["sigma"].copy())
        stats = None
        if t["stats"] is not None:
            S, n = t["stats"]
            if t["name"] in ref_stats_for:
                stats = SimpleNamespace(S=torch.from_numpy(S.copy()), n=n, k=S.shape[0] * 16)
            else:
                stats = ColumnStats.from_state({"S": torch.from_numpy(S.copy()), "n": n,
                                                "k": S.shape[0] * 16}, dev)
        if on_device:
            w = w.to(dev)
            sigma = None if sigma is None else sigma.to(dev)
        r, k = t["w"].shape
        table = TensorTable(t["name"], (r, k), torch.from_numpy(t["had"].copy()),
                            torch.zeros(len(CANDS), r), list(CANDS), 0.0, 0, cs)
        reqs.append(EncodeRequest(w, stats, table, torch.from_numpy(t["picks"].copy()), sigma,
                                  t["sigma_id"], {} if t["comp"] else None))
    return reqs


def _cfg(tag):
    from hi2_amd.calibrate import Config

    c = CONFIGS[tag]
    return Config(candidates=list(CANDS), rounding=c["rounding"], act_order=c["act_order"],
                  refine_passes=c["refine_passes"], effort=c["effort"])


def _expected_hessians(tag):
    """The transformed (and, under act-order, permuted) Hessian of every distinct input of
    the fixture, by the oracle, in the order the reference factored them."""
    out, keys = [], []
    if CONFIGS[tag]["rounding"] != "gptq":
        return out
    for i, t in enumerate(TENSORS):
        if t["sigma"] is None:
            continue
        key = (t["sigma_id"] or f"#{i}", None if t["col_scale"] is None else
               t["col_scale"].tobytes(), t["had"].tobytes())
        if key in keys:
            continue
        keys.append(key)
        hs = oracle.transform_sigma(t["sigma"], t["col_scale"], t["had"])
        if CONFIGS[tag]["act_order"]:
            p = np.argsort(-np.diag(hs), kind="stable")
            hs = hs[p][:, p]
        out.append(hs)
    return out


def _inject(monkeypatch, tag):
    """Make the orchestration use the reference's factors: each factorisation gets the
    reference's factor of the Hessian it is handed, which must equal the oracle's
    transform of one of the fixture's inputs bit for bit.  Returns the list of inputs
    (indices in the reference's order) factored."""
    import hi2_amd.calibrate as C

    hss, us = _expected_hessians(tag), CONFIGS[tag]["factors"]
    assert len(hss) == len(us)
    calls = []

    def fake(hs, damp):
        h = hs.cpu().numpy()
        j = next((j for j, e in enumerate(hss) if e.shape == h.shape and np.array_equal(e, h)),
                 None)
        assert j is not None, "a Hessian that is not the oracle's transform of any input"
        calls.append(j)
        u = torch.from_numpy(np.ascontiguousarray(us[j])).to(hs.device)
        return u, torch.full((1,), OK, dtype=torch.int32, device=hs.device)

    monkeypatch.setattr(C, "_factor", fake)
    return calls


def _check_golden(got, reqs, tag):
    for t, o, r in zip(TENSORS, got, reqs):
        want = CONFIGS[tag]["out"][t["name"]]
        for f in FIELDS:
            g = getattr(o, f)
            g = g.view(torch.int16) if g.dtype == torch.float16 else g
            assert np.array_equal(g.numpy().reshape(-1).view(want[f].dtype)
                                  if g.dtype == torch.int16 else g.numpy().reshape(-1),
                                  want[f].reshape(-1)), (tag, t["name"], f)
        if t["comp"]:
            assert np.array_equal(r.comp_out["comp"].numpy(), want["comp"]), (tag, t["name"])


@pytest.mark.parametrize("tag", list(CONFIGS))
def test_encode_many_equals_reference_golden(tag, dev, monkeypatch):
    from hi2_amd.calibrate import Executor, encode_many

    print(f"encode_many golden {tag}", flush=True)
    calls = _inject(monkeypatch, tag)
    reqs = _requests(dev)
    got = encode_many(reqs, _cfg(tag), Executor([str(dev)]))
    # one factorisation per distinct input, as the reference (the widest input first)
    assert sorted(calls) == list(range(len(CONFIGS[tag]["factors"])))
    _check_golden(got, reqs, tag)


def test_device_resident_inputs_and_two_shards_give_the_same_buffers(dev, monkeypatch):
    from hi2_amd.calibrate import Executor, encode_many

    tag = "gr"
    n = len(CONFIGS[tag]["factors"])
    calls = _inject(monkeypatch, tag)
    reqs = _requests(dev, on_device=True, ref_stats_for=())
    _check_golden(encode_many(reqs, _cfg(tag), Executor([str(dev)])), reqs, tag)
    assert sorted(calls) == list(range(n))
    # two shards on one device: every shard factors its inputs again (as the reference
    # does per device); rows are independent, so the buffers are the same
    calls.clear()
    reqs = _requests(dev)
    _check_golden(encode_many(reqs, _cfg(tag), Executor([str(dev), str(dev)])), reqs, tag)
    assert sorted(calls) == sorted(list(range(n)) * 2)


@pytest.mark.parametrize("shards", [1, 2])
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("rounding", ["gptq", "nearest"])
def test_encode_many_equals_per_tensor_reference(shards, act_order, rounding, dev):
    """The reference's tests/test_cache.py:599-653 equality on the device's own factors:
    encode_many == encode_with_picks_reference per tensor, including comp."""
    from hi2_amd.calibrate import Config, Executor, encode_many, encode_with_picks_reference

    print(f"encode_many vs per-tensor shards={shards} ao={act_order} {rounding}", flush=True)
    cfg = Config(candidates=list(CANDS), rounding=rounding, act_order=act_order, effort="fast")
    ex = Executor([str(dev)] * shards)
    reqs = _requests(dev)
    got = encode_many(reqs, cfg, ex)
    for r, o in zip(reqs, got):
        co = {} if r.comp_out is not None else None
        ref = encode_with_picks_reference(r.w, r.stats, r.table, r.picks, cfg, ex, r.sigma, co)
        for f in FIELDS:
            assert torch.equal(getattr(o, f), getattr(ref, f)), (r.table.name, f)
        if co is not None:
            assert torch.equal(r.comp_out["comp"], co["comp"])


def test_encode_many_at_width_1024_equals_the_oracle(dev, monkeypatch):
    """Three tensors on one input at K=1024 (bf16 weights, smoothing, mixed rotation,
    every candidate, two refinement sweeps) and one on another input: the device's
    packed buffers equal the oracle's composition given the device's factors."""
    import hi2_amd.calibrate as C
    from hi2_amd.calibrate import Config, EncodeRequest, Executor, TensorTable

    g = torch.Generator().manual_seed(41)
    k, k2 = 1024, 512
    us = {}
    orig = C._factor

    def record(hs, damp):
        u, st = orig(hs, damp)
        us[hs.shape[0]] = u
        return u, st

    monkeypatch.setattr(C, "_factor", record)
    x = (torch.randn(3000, k, generator=g) * torch.exp(0.5 * torch.randn(k, generator=g)))
    sig = (x.T @ x) / 3000
    x2 = torch.randn(2000, k2, generator=g)
    sig2 = (x2.T @ x2) / 2000
    cs = (torch.rand(k, generator=g) * 1.5 + 0.5).half()
    had = (torch.arange(k // 16) % 4 != 3).to(torch.uint8)
    had2 = torch.ones(k2 // 16, dtype=torch.uint8)
    tensors, reqs = [], []
    for name, rows, kk, s, sid, c, h, comp in (
            ("q", 96, k, sig, "a", cs, had, False), ("k", 40, k, sig, "a", cs, had, True),
            ("v", 40, k, sig, "a", cs, had, False), ("o", 64, k2, sig2, "b", None, had2, False)):
        w = (torch.randn(rows, kk, generator=g) * 0.02).to(torch.bfloat16)
        picks = torch.randint(0, len(CANDS), (rows,), generator=g)
        table = TensorTable(name, (rows, kk), h, torch.zeros(1), list(CANDS), 0.0, 0, c)
        reqs.append(EncodeRequest(w, None, table, picks, s, sid, {} if comp else None))
        tensors.append(dict(name=name, w=w.float().numpy(), had=h.numpy(), picks=picks.numpy(),
                            col_scale=None if c is None else c.view(torch.int16).numpy()
                            .view(np.uint16), sigma=s.numpy(), sigma_id=sid, stats=None,
                            comp=comp))
    cfg = Config(candidates=list(CANDS), refine_passes=2)
    got = C.encode_many(reqs, cfg, Executor([str(dev)]))
    assert len(us) == 2
    want = oracle.encode_many(tensors, CANDS, dict(rounding="gptq", act_order=False,
                                                  refine_passes=2, effort="normal"),
                              [us[k].cpu().numpy(), us[k2].cpu().numpy()])
    for r, o, (wp, wc) in zip(reqs, got, want):
        for f in FIELDS:
            gv = getattr(o, f)
            gv = gv.view(torch.int16).numpy().view(np.uint16) if gv.dtype == torch.float16 \
                else gv.numpy()
            assert np.array_equal(gv.reshape(-1), np.asarray(wp[f]).reshape(-1)), (r.table.name, f)
        if wc is not None:
            assert np.array_equal(r.comp_out["comp"].numpy(), wc)



def test_encode_many_at_the_configuration_widths_equals_per_tensor_reference(dev):
    """cfg3 widths: a down_proj-shaped tensor (1024 x 14336 rows of the 4096) and a q/k
    pair on one K=4096 input (k with comp), INT2/B32 and INT4/B64 rows, smoothing and
    rotation: encode_many equals the per-tensor reference path bit for bit."""
    from hi2_amd.calibrate import (Config, EncodeRequest, Executor, TensorTable, encode_many,
                                   encode_with_picks_reference)

    print("encode_many cfg3 widths", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    cands = [(2, 32), (4, 64)]
    reqs = []
    for inp, k, tensors in (("down", 14336, (("down_proj", 1024, False),)),
                            ("attn", 4096, (("q_proj", 512, False), ("k_proj", 256, True)))):
        x = torch.randn(2048, k, generator=g, device=dev)
        x[:, torch.randperm(k, generator=g, device=dev)[: k // 100]] *= 20.0
        sigma = (x.T @ x) / 2048
        sigma = ((sigma + sigma.T) * 0.5).cpu()
        cs = (torch.rand(k, generator=g, device=dev) + 0.5).half().cpu()
        had = (torch.arange(k // 16) % 5 != 0).to(torch.uint8)
        for name, rows, comp in tensors:
            w = (torch.randn(rows, k, generator=g, device=dev) * 0.02).to(torch.bfloat16).cpu()
            picks = (torch.rand(rows, generator=g, device=dev) > 0.3).long().cpu()
            table = TensorTable(name, (rows, k), had, torch.zeros(1), cands, 0.0, 2048, cs)
            reqs.append(EncodeRequest(w, None, table, picks, sigma, inp, {} if comp else None))
    cfg = Config(candidates=cands)
    ex = Executor([str(dev)])
    got = encode_many(reqs, cfg, ex)
    for r, o in zip(reqs, got):
        co = {} if r.comp_out is not None else None
        ref = encode_with_picks_reference(r.w, r.stats, r.table, r.picks, cfg, ex, r.sigma, co)
        for f in FIELDS:
            assert torch.equal(getattr(o, f), getattr(ref, f)), (r.table.name, f)
        if co is not None:
            assert torch.equal(r.comp_out["comp"], co["comp"])


def test_act_order_skips_refinement_as_the_reference(dev):
    """refine_passes under act_order: the reference refines only unpermuted factors
    (hi2/calibrate.py:339-341), so the buffers equal the unrefined per-tensor path."""
    from hi2_amd.calibrate import Config, Executor, encode_many, encode_with_picks_reference

    cfg = Config(candidates=list(CANDS), act_order=True, refine_passes=2, effort="fast")
    ex = Executor([str(dev)])
    reqs = _requests(dev)
    got = encode_many(reqs, cfg, ex)
    for r, o in zip(reqs, got):
        ref = encode_with_picks_reference(r.w, r.stats, r.table, r.picks, cfg, ex, r.sigma)
        for f in FIELDS:
            assert torch.equal(getattr(o, f), getattr(ref, f)), (r.table.name, f)


@pytest.mark.parametrize("passes", [0, 2])
def test_damping_retry_reencodes_the_chain(passes, dev, monkeypatch):
    """An indefinite Sigma (smallest eigenvalue -5 % of the mean diagonal): the first,
    asynchronous factor attempt (damping 1 %) fails, the reference's retry ladder
    (hi2/hessian.py:76-86) succeeds at 10 %, and encode_many rounds (and refines) the
    chain again.  Row chunks are cut small, so chunks at an offset run alone in a batch.
    Without refinement the buffers equal encode_with_picks_reference (synchronous
    inverse_factor) bit for bit; with two refinement sweeps they equal the oracle's
    composition given the retried factor."""
    import hi2_amd.calibrate as C
    import hi2_amd.hessian as hm
    from hi2_amd.calibrate import (Config, EncodeRequest, Executor, TensorTable,
                                   encode_with_picks_reference)

    monkeypatch.setattr(hm, "ROW_ELEMS", 256 * 24)
    monkeypatch.setattr(hm, "BATCH_ELEMS", 256 * 24)
    k, t = 256, 2000
    rng = np.random.default_rng(17)
    x = rng.standard_normal((t, k)) * np.exp(0.5 * rng.standard_normal(k))
    sig = x.T @ x / t
    ev, vec = np.linalg.eigh(sig)
    m = np.trace(sig) / k
    sig = sig - (ev[0] + 0.05 * m) * np.outer(vec[:, 0], vec[:, 0])
    sig = ((sig + sig.T) / 2).astype(np.float32)
    statuses, factors = [], []
    orig = C._factor

    def record(hs, damp):
        u, st = orig(hs, damp)
        statuses.append(st)
        factors.append(u)
        return u, st

    monkeypatch.setattr(C, "_factor", record)
    cands = [(2, 32), (4, 64)]
    had = np.ones(k // 16, np.uint8)
    w = (rng.standard_normal((70, k)) * 0.02).astype(np.float32)
    picks = (rng.random(70) > 0.3).astype(np.int64)
    table = TensorTable("t", (70, k), torch.from_numpy(had), torch.zeros(1), cands, 0.0, t,
                        None)
    req = EncodeRequest(torch.from_numpy(w), None, table, torch.from_numpy(picks),
                        torch.from_numpy(sig), "in")
    cfg = Config(candidates=cands, refine_passes=passes)
    ex = Executor([str(dev)])
    got = C.encode_many([req], cfg, ex)[0]
    assert len(statuses) == 1 and int(statuses[0].item()) != OK, "first attempt succeeded"
    if passes == 0:
        ref = encode_with_picks_reference(req.w, None, table, req.picks, cfg, ex, req.sigma)
        for f in FIELDS:
            assert torch.equal(getattr(got, f), getattr(ref, f)), f
    else:
        tensor = dict(name="t", w=w, had=had, picks=picks, col_scale=None, sigma=sig,
                      sigma_id="in", stats=None, comp=False)
        (want, _), = oracle.encode_many([tensor], cands, dict(
            rounding="gptq", act_order=False, refine_passes=passes, effort="normal"),
            [factors[0].cpu().numpy()])
        for f in FIELDS:
            gv = getattr(got, f)
            gv = gv.view(torch.int16).numpy().view(np.uint16) if gv.dtype == torch.float16 \
                else gv.numpy()
            assert np.array_equal(gv.reshape(-1), np.asarray(want[f]).reshape(-1)), f
