"""The C ABI library loads and exports every entry point include/hi2x.h declares, and
the Python mirror keeps the reference's call surface — CPU only (no compute calls)."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "hi2x.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hi2x_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from hi2_amd import _lib

    lib = _lib.lib()
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert lib.hi2x_version() >= 100
    assert set(_lib.SIGNATURES) | set(_lib.SIZES) | {
        "hi2x_version", "hi2x_last_error", "hi2x_timing_enable", "hi2x_timing_query"
    } == set(names)


def test_raw_symbols_resolve_without_ctypes_wrappers():
    from hi2_amd import _lib

    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert ctypes.cast(getattr(raw, name), ctypes.c_void_p).value


def test_argument_errors_come_back_as_status_without_a_gpu():
    # argument checks run before any HIP call, so they work on a host without a GPU
    from hi2_amd import _lib

    lib = _lib.lib()
    rc = lib.hi2x_gptq_block(None, 4, 64, 0, 200, None, None, None, None, 4, None, None,
                             None, None, None, None)
    assert rc == _lib.EINVAL and "block length" in _lib.last_error()
    rc = lib.hi2x_fwht16(None, None, 0, 1, 24, None, None)
    assert rc == _lib.EINVAL and "multiple of 16" in _lib.last_error()
    rc = lib.hi2x_pack_codes(None, 1, 30, 4, None, None, None)
    assert rc == _lib.EINVAL
    rc = lib.hi2x_refine_block(None, 128, 4, 256, 0, 200, None, None, None, 4, None, None,
                               None, None, 128, None, None)
    assert rc == _lib.EINVAL and "outside" in _lib.last_error()
    rc = lib.hi2x_refine_run(None, None, 4, 256, None, None, 0, None, None, None, 2, None, None,
                             0, None)
    assert rc == _lib.EINVAL and "bad shape" in _lib.last_error()
    assert lib.hi2x_refine_workspace_bytes(4, 256, 2) >= 2 * 4 * 256 * 4
    assert lib.hi2x_refine_workspace_bytes(-1, 256, 2) == -1
    rc = lib.hi2x_qad_decode_fwd(None, None, None, None, None, None, 4, 4, 128, 24, 3.0, None,
                                 None)
    assert rc == _lib.EINVAL and "16, 32 or 64" in _lib.last_error()
    rc = lib.hi2x_qad_decode_bwd(None, None, None, None, None, None, None, 4, 4, 96, 64, 3.0,
                                 None, None, None, None)
    assert rc == _lib.EINVAL and "multiple of the block" in _lib.last_error()
    rc = lib.hi2x_qad_wht_scale(None, 2, 24, None, None, 0, None, None)
    assert rc == _lib.EINVAL and "multiple of 16" in _lib.last_error()
    rc = lib.hi2x_qad_wht_scale(ctypes.c_void_p(8), 2, 32, None, None, 0, ctypes.c_void_p(16),
                                None)
    assert rc == _lib.EINVAL and "aligned" in _lib.last_error()
    # the allocation-free column loop refuses a batch beyond its 64 MiB scratch first
    rc = lib.hi2x_gptq_run_noalloc(None, 40000, 4096, None, None, None, 256, None, None, None,
                                   None, None, 4, None)
    assert rc == _lib.EINVAL and "64 MiB" in _lib.last_error()
    rc = lib.hi2x_timing_query(0, None, None, None)
    assert rc == _lib.EINVAL and "null" in _lib.last_error()
    _lib.timing_enable([])  # nothing recorded yet: no HIP call is made
    assert _lib.timing_query(_lib.TIME_GPTQ_TRAILING) == (0, 0.0, 0.0)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERANGE, "x")
    with pytest.raises(_lib.NotPositiveDefinite):
        _lib.check(_lib.ENOTPD, "x")


def test_python_surface_matches_the_reference_modules():
    import hi2_amd.encode as enc
    import hi2_amd.format as fmt
    import hi2_amd.gptq_kernel as gk
    import hi2_amd.hessian as hs
    import hi2_amd.ladder_kernel as lk

    for name in ("BLOCK_COLUMNS", "kernel_dir", "supported", "load", "available", "failure",
                 "gptq_block"):
        assert hasattr(gk, name), name
    for name in ("BLOCK_COLUMNS", "ROW_ELEMS", "BATCH_ELEMS", "HessianStats", "transform_sigma",
                 "inverse_factor", "GptqJob", "encode_jobs_gptq", "encode_rows_gptq",
                 "encode_rows_gptq_reference", "EFFORT", "Encoded"):
        assert hasattr(hs, name), name
    for name in ("EFFORT", "CHUNK_ELEMS", "_safe", "fit_ladder", "quantize_params", "Encoded",
                 "encode_rows"):
        assert hasattr(enc, name), name
    for name in ("ladder_grid", "available", "load", "failure", "supported"):
        assert hasattr(lk, name), name
    for name in ("GROUP", "hadamard16", "fwht_groups", "decode_params", "ladder_dequantize",
                 "pack_codes", "HI2Tensor", "FIELDS", "assemble"):
        assert hasattr(fmt, name), name
    import hi2_amd.refine as rf
    import hi2_amd.refine_kernel as rk

    for name in ("BLOCK_COLUMNS", "objective", "_expand", "refine_expanded", "refine_codes",
                 "refine_groups", "refine_encoded"):
        assert hasattr(rf, name), name
    for name in ("BLOCK_COLUMNS", "load", "available", "failure", "refine_block", "supported",
                 "kernel_dir"):
        assert hasattr(rk, name), name
    assert rf.BLOCK_COLUMNS == rk.BLOCK_COLUMNS == 128
    import hi2_amd.cache as ch
    import hi2_amd.stats as sts

    for name in ("TOKEN_CHUNK", "ColumnStats"):
        assert hasattr(sts, name), name
    for name in ("update", "merge", "diag", "state", "from_state"):
        assert hasattr(sts.ColumnStats, name), name
    for name in ("_fname", "_upper", "sigma_payload", "load_sigma"):
        assert hasattr(ch, name), name
    assert sts.TOKEN_CHUNK == 4096
    import hi2_amd.qad_kernel as qk

    for name in ("load", "available", "failure", "original", "stored", "supported",
                 "kernel_dir", "_StoredDecode", "_Transform"):
        assert hasattr(qk, name), name
    for name in ("decode_fwd", "decode_bwd", "wht_scale"):
        assert hasattr(qk._Kernels, name), name
    import hi2_amd.calibrate as cal

    for name in ("ALL_CANDIDATES", "INT8_CANDIDATES", "SELECTABLE", "Config", "TensorTable",
                 "EncodeRequest", "Executor", "encode_many", "encode_with_picks",
                 "encode_with_picks_reference", "_factor_key"):
        assert hasattr(cal, name), name
    assert cal.SELECTABLE == [(2, 16), (2, 32), (2, 64), (4, 16), (4, 32), (4, 64), (8, 32),
                              (8, 64)]
    c = cal.Config()
    assert (c.rounding, c.damp, c.act_order, c.refine_passes, c.effort) == \
        ("gptq", 0.01, False, 0, "normal")
    assert cal.Executor(["cuda:0", "cuda:1"]).shards(5) == [
        (torch.device("cuda:0"), 0, 2), (torch.device("cuda:1"), 2, 5)]
    assert hs.BLOCK_COLUMNS == gk.BLOCK_COLUMNS == 128
    assert enc.EFFORT["normal"]["grid"] == (0.0, 0.04, 0.08, 0.12, 0.16, 0.20)


def test_cpu_tensors_are_refused_not_computed():
    import hi2_amd.format as fmt
    import hi2_amd.hessian as hs

    with pytest.raises(RuntimeError, match="MI355X"):
        fmt.fwht_groups(torch.zeros(2, 32), torch.ones(2, dtype=torch.uint8))
    with pytest.raises(RuntimeError):
        hs.HessianStats(16, "cpu")
    with pytest.raises(RuntimeError, match="MI355X"):
        hs.encode_rows_gptq(torch.zeros(4, 32), torch.ones(32), torch.eye(32), 2, 16)
    with pytest.raises(ValueError):
        fmt.fwht_groups(torch.zeros(2, 24), torch.ones(1))
    import hi2_amd.refine as rf

    import hi2_amd.stats as sts

    with pytest.raises(RuntimeError, match="MI355X"):
        sts.ColumnStats(32, "cpu")
    with pytest.raises(ValueError):
        sts.ColumnStats(24, "cuda")
    with pytest.raises(RuntimeError, match="MI355X"):
        rf.refine_codes(torch.zeros(4, 32), torch.zeros(4, 32, dtype=torch.uint8),
                        torch.zeros(4, 1), torch.ones(4, 1), torch.eye(32), 2, 32, 1)
    import hi2_amd.calibrate as cal

    table = cal.TensorTable("t", (4, 32), torch.ones(2, dtype=torch.uint8), torch.zeros(1),
                            [(2, 16)], 0.0, 0)
    req = cal.EncodeRequest(torch.zeros(4, 32), None, table, torch.zeros(4, dtype=torch.long),
                            torch.eye(32))
    with pytest.raises(RuntimeError, match="MI355X"):
        cal.encode_many([req], cal.Config(candidates=[(2, 16)]), cal.Executor(["cpu"]))


def test_hadamard16_constant():
    import hi2_amd.format as fmt

    h = fmt.hadamard16()
    assert torch.allclose(h @ h, torch.eye(16, dtype=torch.float64))
    assert torch.equal(h, h.T)


def test_stream_background_marks_and_clears_without_a_gpu():
    # the background mark is a host-side registry keyed by the stream handle: no HIP call
    from hi2_amd import _lib

    lib = _lib.lib()
    handle = ctypes.c_void_p(0x1234560)
    assert lib.hi2x_stream_background(handle, 1) == _lib.OK
    assert lib.hi2x_stream_background(handle, 1) == _lib.OK  # marking twice is harmless
    assert lib.hi2x_stream_background(handle, 0) == _lib.OK
    assert lib.hi2x_stream_background(handle, 0) == _lib.OK  # so is clearing twice
