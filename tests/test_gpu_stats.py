"""Calibration statistics on the MI355X (hi2x_colstats_*, hi2x_sigma_pack_upper) against
the oracle (bit-exact: same fp32 chunk order, same f64 sums), the reference's golden
vectors and closed forms of the cached-Sigma format."""

import numpy as np
import pytest
import torch

import oracle
from golden_data import colstats_case

pytestmark = pytest.mark.gpu

G = colstats_case()


def _x(tag, dev):
    xb = torch.from_numpy(G["x_bf16"].copy()).view(torch.bfloat16).to(dev)
    return xb if tag == "bf16" else xb.float()


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_update_equals_oracle_and_reference(tag, dev):
    from hi2_amd.stats import ColumnStats

    x = _x(tag, dev)
    t1 = int(G["split"][0])
    st = ColumnStats(x.shape[1], dev)
    st.update(x[:t1])
    st.update(x[t1:])
    got = st.S.cpu().numpy()
    want = np.zeros_like(got)
    xn = x.cpu().view(torch.int16).numpy().view(np.uint16) if tag == "bf16" else x.cpu().numpy()
    oracle.colstats_update(want, xn[:t1])
    oracle.colstats_update(want, xn[t1:])
    assert np.array_equal(got, want)
    ref = G[f"{tag}_S"]
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    assert st.n == int(G[f"{tag}_n"])


@pytest.mark.parametrize("variant", ["diag", "diag_rot", "diag_inv", "diag_rot_inv"])
def test_diag_equals_reference_golden(variant, dev):
    from hi2_amd.stats import ColumnStats

    st = ColumnStats.from_state({"S": torch.from_numpy(G["bf16_S"]), "n": int(G["bf16_n"]),
                                 "k": 64}, dev)
    flags = torch.from_numpy(G["flags"]) if "rot" in variant else None
    inv = torch.from_numpy(G["inv_scale"]) if "inv" in variant else None
    got = st.diag(flags, inv).cpu().numpy()
    assert np.array_equal(got, G[f"bf16_{variant}"])


def test_merge_and_state_roundtrip(dev):
    from hi2_amd.stats import ColumnStats

    x = _x("bf16", dev)
    a, b, whole = ColumnStats(64, dev), ColumnStats(64, dev), ColumnStats(64, dev)
    a.update(x[:1000])
    b.update(x[1000:])
    a.merge(b)
    whole.update(x[:1000])
    whole.update(x[1000:])
    assert torch.equal(a.S, whole.S) and a.n == whole.n
    c = ColumnStats.from_state(a.state(), dev)
    assert torch.equal(c.S, a.S) and c.n == a.n


@pytest.mark.parametrize("k", [4096, 14336])
def test_update_at_configuration_widths_equals_the_oracle(k, dev):
    """8192 bf16 tokens at the cfg3 widths (two 4096-token chunks)."""
    from hi2_amd.stats import ColumnStats

    print(f"colstats width k={k}", flush=True)
    g = torch.Generator(device=dev).manual_seed(k)
    x = (torch.randn(8192, k, generator=g, device=dev) * 3.0).to(torch.bfloat16)
    st = ColumnStats(k, dev)
    st.update(x)
    want = np.zeros((k // 16, 16, 16))
    oracle.colstats_update(want, x.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(st.S.cpu().numpy(), want)


@pytest.mark.parametrize("fp16_above", [0, 32])
def test_sigma_payload_is_the_exact_upper_triangle(fp16_above, tmp_path, dev):
    from hi2_amd.cache import load_sigma, sigma_payload
    from hi2_amd.hessian import HessianStats

    k = 48
    g = torch.Generator(device=dev).manual_seed(5)
    hst = HessianStats(k, dev)
    hst.update(torch.randn(300, k, generator=g, device=dev))
    s = hst.mean()
    obj = sigma_payload(s, hst.n, fp16_above)
    sh = s.cpu().numpy()
    iu = np.triu_indices(k)
    assert set(obj) == {"k", "n", "tri"} and obj["k"] == k and obj["n"] == 300
    tri = obj["tri"].numpy()
    if fp16_above:
        assert tri.dtype == np.float16 and np.array_equal(tri, sh[iu].astype(np.float16))
    else:
        assert tri.dtype == np.float32 and np.array_equal(tri, sh[iu])
        torch.save(obj, tmp_path / "a.weight.pt")
        assert torch.equal(load_sigma(tmp_path / "a.weight.pt"), s.cpu())
    asym = s.clone()
    asym[0, 1] += 1e-3  # not symmetric: stored in full
    obj = sigma_payload(asym, hst.n, fp16_above)
    assert set(obj) == {"k", "n", "full"}
    full = asym.half() if fp16_above else asym
    assert torch.equal(obj["full"], full.cpu())
