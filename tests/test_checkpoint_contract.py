"""The writer's ``hi2_*`` tensor contract (``hi2/checkpoint.py:142-165``,
``docs/format-spec.md`` 2.4) on the reference's own packed ``encode_many`` output: key
names and dtypes, and a round trip through a safetensors file — CPU only."""

import numpy as np
import torch

from golden_data import encode_many_case

CANDS, TENSORS, CONFIGS = encode_many_case()


def _packed(name, tag="g"):
    from hi2_amd.format import HI2Tensor

    o = CONFIGS[tag]["out"][name]
    t = next(t for t in TENSORS if t["name"] == name)
    cs = None
    if t["col_scale"] is not None:
        cs = torch.from_numpy(t["col_scale"].view(np.int16).copy()).view(torch.float16)
    f = {k: torch.from_numpy(np.ascontiguousarray(o[k])) for k in
         ("codes", "code_off", "blk_params", "param_off", "row_nbits", "row_block", "had")}
    f["row_consts"] = torch.from_numpy(o["row_consts"].view(np.int16).reshape(-1, 3).copy()
                                       ).view(torch.float16)
    return HI2Tensor(**f, shape=(f["row_nbits"].numel(), f["had"].numel() * 16), col_scale=cs)


def test_names_and_dtypes_follow_the_format_spec():
    from hi2_amd.checkpoint import to_tensors

    d = to_tensors(_packed("q"), "model.layers.0.self_attn.q_proj.weight")
    base = "model.layers.0.self_attn.q_proj.weight.hi2_"
    want = {"codes": torch.int32, "code_off": torch.int32, "blk_params": torch.uint8,
            "param_off": torch.int32, "row_consts": torch.float16, "row_nbits": torch.uint8,
            "row_block": torch.uint8, "had": torch.uint8, "col_scale": torch.float16}
    assert {k: v.dtype for k, v in d.items()} == {base + k: v for k, v in want.items()}
    o = to_tensors(_packed("o"), "o")  # not smoothed: no col_scale entry
    assert "o.hi2_col_scale" not in o and len(o) == 8
    r = _packed("q")
    assert d[base + "code_off"].numel() == d[base + "param_off"].numel() == r.shape[0] + 1
    assert d[base + "blk_params"].numel() == 2 * int(d[base + "param_off"][-1])
    assert d[base + "codes"].numel() == int(d[base + "code_off"][-1])


def test_round_trip_through_safetensors(tmp_path):
    from safetensors import safe_open
    from safetensors.torch import save_file

    from hi2_amd.checkpoint import from_tensors, read_tensors, to_tensors
    from hi2_amd.format import FIELDS

    tensors = {}
    for t in TENSORS:
        tensors.update(to_tensors(_packed(t["name"]), f"layer.{t['name']}.weight"))
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path))
    with safe_open(str(path), "pt") as f:
        for t in TENSORS:
            base = f"layer.{t['name']}.weight"
            back = from_tensors(read_tensors(f, base), base)
            ref = _packed(t["name"])
            assert back.shape == ref.shape == t["w"].shape
            for fld in FIELDS:
                assert torch.equal(getattr(back, fld), getattr(ref, fld)), (t["name"], fld)
            assert (back.col_scale is None) == (ref.col_scale is None)
            if ref.col_scale is not None:
                assert torch.equal(back.col_scale, ref.col_scale)
