"""cfg5, the OLMoE-shaped MoE layer, on the MI355X: every expert's Hessian from one
routed token batch, the token floor, the batched transform and factors, and GPTQ of the
experts' rows with one factor per expert (hi2/moe.py:83-100, hi2/layerwise.py:241-257,
hi2/calibrate.py:332-348, hi2/hessian.py:267-315).

- grouped accumulation: each expert's S against its float64 X_e^T X_e (bf16 products
  are exact; fp32 sums in another order: within 1e-5 of the largest entry), empty and
  one-token experts included; deterministic; the gather equals a pre-gathered batch bit
  for bit;
- token floor: bit for bit with the oracle (which equals the reference's blend);
- batched transform and factors: bit for bit with the per-expert entry points,
  including an expert whose first factor attempt fails (the reference's retries);
- GPTQ on expert factors: bit for bit with the oracle given the same factors;
- the full cfg5 layer (16384 tokens, 64 experts, top-8 of Zipf(1.1)): Hessians (with the
  floor) of sampled experts against float64, and sampled experts' GPTQ against the oracle.
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def N(t):
    return t.detach().cpu().numpy()


def _upper(a):
    return np.triu(a)


def _grouped(dev, x, rows, offs, e, k, upper_only=1):
    from hi2_amd import _lib

    s = torch.zeros(e, k, k, device=dev)
    t_total = rows.numel() if rows is not None else x.shape[0]
    ws = _lib.workspace(dev, "hi2x_hessian_grouped_workspace_bytes", t_total, e, k)
    _lib.call("hi2x_hessian_syrk_grouped", dev, _lib.ptr(x), x.shape[0], 2, _lib.ptr(rows),
              _lib.ptr(offs), e, t_total, k, _lib.ptr(s), k * k, upper_only, _lib.ptr(ws),
              ws.numel())
    return s


def test_grouped_accumulation_matches_float64_per_expert(dev):
    from hi2_amd.workloads import activations

    print("moe grouped syrk", flush=True)
    k = 1024
    sizes = [300, 0, 2048, 1, 7, 0, 129, 5000]
    offs_h = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    t_total = int(offs_h[-1])
    x = activations(3000, k, 21, dev)
    g = torch.Generator(device=dev).manual_seed(3)
    rows = torch.randint(0, 3000, (t_total,), generator=g, device=dev)
    offs = torch.from_numpy(offs_h).to(dev)
    s = _grouped(dev, x, rows, offs, len(sizes), k, upper_only=0)
    again = _grouped(dev, x, rows, offs, len(sizes), k, upper_only=0)
    assert torch.equal(s, again), "not deterministic"
    pre = _grouped(dev, x[rows].contiguous(), None, offs, len(sizes), k, upper_only=0)
    assert torch.equal(s, pre), "the gather differs from a pre-gathered batch"
    up = _grouped(dev, x, rows, offs, len(sizes), k, upper_only=1)
    for e, t in enumerate(sizes):
        se = N(s[e])
        assert np.array_equal(se, se.T), e
        assert np.array_equal(np.triu(N(up[e])), np.triu(se)), e
        xe = x[rows[offs_h[e]:offs_h[e + 1]]].double()
        want = N(xe.T @ xe)
        if t == 0:
            assert not se.any(), e
            continue
        err = np.abs(se - want).max() / np.abs(want).max()
        assert err < 1e-5, (e, t, err)


def test_top_up_equals_the_oracle(dev):
    from hi2_amd.moe import ExpertHessians

    print("moe top-up", flush=True)
    rng = np.random.default_rng(4)
    e, k = 7, 256
    counts = [5000, 300, 0, 4096, 1200, 70, 9000]
    sums = []
    for n in counts:
        a = rng.standard_normal((k, k)).astype(np.float32)
        sums.append(((a + a.T) * np.float32(n / 8)).astype(np.float32))
    sums = np.stack(sums)
    eh = ExpertHessians(e, k, dev)
    eh.S.copy_(torch.from_numpy(sums))
    eh.n.copy_(torch.tensor(counts))
    short = eh.top_up(4096)
    want, want_n = oracle.moe_top_up(sums, counts, 4096)
    assert short == [1, 2, 4, 5]
    assert eh.counts() == want_n
    got = N(eh.S)
    for i in range(e):
        assert np.array_equal(np.triu(got[i]), np.triu(want[i])), i


def test_batched_transform_and_factors_equal_per_expert(dev):
    from hi2_amd import _lib
    from hi2_amd.hessian import inverse_factor, inverse_factors_batched
    from hi2_amd.moe import ExpertHessians

    print("moe batched transform + factors", flush=True)
    e, k = 6, 1024
    rng = np.random.default_rng(8)
    eh = ExpertHessians(e, k, dev)
    for i in range(e):
        x = rng.standard_normal((1500 + 300 * i, k)) * np.exp(0.5 * rng.standard_normal(k))
        s = (x.T @ x).astype(np.float32)
        if i == 3:  # indefinite: the first attempt fails, a later damping succeeds
            ev, vec = np.linalg.eigh(s.astype(np.float64))
            s = (s - (ev[0] + 0.05 * np.trace(s) / k) * np.outer(vec[:, 0], vec[:, 0]))
            s = ((s + s.T) / 2).astype(np.float32)
        eh.S[i] = torch.from_numpy(s).to(dev)
        eh.n[i] = 1500 + 300 * i
    had = torch.ones(k // 16, dtype=torch.uint8)
    had_d = had.to(dev)
    hs = eh.transformed(None, had)
    for i in range(e):
        one = torch.empty(k, k, device=dev)
        _lib.call("hi2x_sigma_transform_upper", dev, _lib.ptr(eh.S[i]), 1500 + 300 * i, None,
                  _lib.ptr(had_d), k, _lib.ptr(one))
        assert torch.equal(hs[i], one), i
    u = inverse_factors_batched(hs)
    for i in range(e):
        assert torch.equal(u[i], inverse_factor(hs[i])), i


def test_gptq_on_expert_factors_equals_the_oracle(dev):
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq, inverse_factors_batched

    print("moe gptq", flush=True)
    rng = np.random.default_rng(12)
    jobs, want = [], []
    for k, ne in ((2048, 3), (1024, 3)):
        hs = []
        for i in range(ne):
            x = rng.standard_normal((3000, k)) * np.exp(0.5 * rng.standard_normal(k))
            hs.append((x.T @ x / 3000).astype(np.float32))
        u = inverse_factors_batched(torch.from_numpy(np.stack(hs)).to(dev))
        for i in range(ne):
            d = np.diag(hs[i]).copy()
            for nbits, block, n in ((2, 32, 40), (4, 64, 90)):
                w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
                jobs.append(GptqJob(torch.from_numpy(w).to(dev), torch.from_numpy(d).to(dev),
                                    u[i], nbits, block))
                want.append(oracle.encode_rows_gptq(w, d, N(u[i]), nbits, block, "normal"))
    got = encode_jobs_gptq(jobs, "normal", comp=True)
    for j, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(N(g.codes), w["codes"]), j
        assert np.array_equal(N(g.sse), w["sse"]), j
        assert np.array_equal(N(g.comp), w["comp"]), j


def test_cfg5_layer_hessians_floor_factors_and_gptq(dev):
    """The whole cfg5 layer at its size: 16384 tokens, 64 experts, top-8 of Zipf(1.1);
    gate/up inputs (K = 2048) gathered by the route, the down inputs (K = 1024) one per
    routed slot; floor 2 x 2048 tokens."""
    from hi2_amd.hessian import GptqJob, encode_jobs_gptq, inverse_factors_batched
    from hi2_amd.moe import ExpertHessians, route_order
    from hi2_amd.workloads import activations, zipf_topk

    print("moe cfg5 layer", flush=True)
    E, T, TOP, H, I = 64, 16384, 8, 2048, 1024
    idx = zipf_topk(T, E, TOP, 1.1, 0, dev)
    rows, offs = route_order(idx, E)
    counts = (offs[1:] - offs[:-1]).cpu().tolist()
    assert sum(counts) == T * TOP and max(counts) <= T
    x = activations(T, H, 1, dev)
    xd = activations(T * TOP, I, 2, dev)
    had_h, had_i = torch.ones(H // 16, dtype=torch.uint8), torch.ones(I // 16, dtype=torch.uint8)
    gu = ExpertHessians(E, H, dev)
    gu.update_routed(x, offs, rows)
    dn = ExpertHessians(E, I, dev)
    dn.update_routed(xd, offs)
    raw = {"gu": gu.S.clone(), "dn": dn.S.clone()}
    need = int(2.0 * H)
    short = gu.top_up(need)
    assert short == dn.top_up(need) and len(short) > 0
    order = sorted(range(E), key=lambda e: -counts[e])
    sample = [order[0], order[E // 2], order[-1]]
    offs_h = offs.cpu().numpy()
    for name, eh, xs, rr in (("gu", gu, x, rows), ("dn", dn, xd, None)):
        tot = raw[name].double().sum(0)
        for e in sample:
            sl = slice(int(offs_h[e]), int(offs_h[e + 1]))
            xe = (xs[rr[sl]] if rr is not None else xs[sl]).double()
            want = xe.T @ xe
            if counts[e] < need:
                want = want + (need - counts[e]) / (T * TOP) * tot
            err = (torch.triu(eh.S[e].double()) - torch.triu(want)).abs().max() / want.abs().max()
            assert err.item() < 2e-5, (name, e, counts[e], err.item())
    hs_gu = gu.transformed(None, had_h)
    hs_dn = dn.transformed(None, had_i)
    u_gu = inverse_factors_batched(hs_gu)
    u_dn = inverse_factors_batched(hs_dn)
    rng = np.random.default_rng(3)
    jobs, want = [], []
    for e in sample:
        for hs, u, k in ((hs_gu, u_gu, H), (hs_dn, u_dn, I)):
            d = torch.diagonal(hs[e]).clone()
            w = (rng.standard_normal((48, k)) * 0.02).astype(np.float32)
            for nbits, block, sl in ((2, 32, slice(0, 16)), (4, 64, slice(16, 48))):
                jobs.append(GptqJob(torch.from_numpy(w[sl]).to(dev), d, u[e], nbits, block))
                want.append(oracle.encode_rows_gptq(w[sl], N(d), N(u[e]), nbits, block,
                                                    "normal"))
    got = encode_jobs_gptq(jobs, "normal", comp=True)
    for j, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(N(g.codes), w["codes"]), j
        assert np.array_equal(N(g.comp), w["comp"]), j


def test_grouped_preparation_equals_per_chunk_preparation(dev, monkeypatch):
    """A batch of many small jobs (an MoE layer's experts: each job its own d and factor,
    INT2/B32 and INT4/B64 rows, K = 512 and 256) prepared and finished as a whole (one
    ladder fit and params launch per class, one sse launch per batch) equals the
    per-chunk path (GROUPED_MIN above the chunk count) in every output, bit for bit, with
    and without comp."""
    import hi2_amd.hessian as H

    rng = np.random.default_rng(11)
    jobs = []
    for e in range(10):
        for k in (512, 256):
            x = rng.standard_normal((2 * k, k)) * np.exp(0.4 * rng.standard_normal(k))
            hs = (x.T @ x / (2 * k)).astype(np.float32)
            u = torch.from_numpy(oracle.inverse_factor(hs, 0.01)[0]).to(dev)
            d = torch.from_numpy(np.diag(hs).copy()).to(dev)
            for nb, b in ((2, 32), (4, 64)):
                n = int(rng.integers(20, 150))
                w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
                jobs.append(H.GptqJob(w.to(dev), d, u, nb, b))
    for comp in (False, True):
        print(f"grouped vs per-chunk, comp={comp}", flush=True)
        got = H.encode_jobs_gptq(jobs, "normal", comp=comp)
        monkeypatch.setattr(H, "GROUPED_MIN", 10 ** 9)
        want = H.encode_jobs_gptq(jobs, "normal", comp=comp)
        monkeypatch.setattr(H, "GROUPED_MIN", 4)
        for j, (g, w) in enumerate(zip(got, want)):
            for f in ("codes", "params", "sse") + (("comp",) if comp else ()):
                assert torch.equal(getattr(g, f), getattr(w, f)), (j, f)
            assert torch.equal(g.consts.view(torch.int16), w.consts.view(torch.int16)), j
