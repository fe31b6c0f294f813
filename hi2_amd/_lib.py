"""ctypes binding of ``libhi2x.so`` (the C ABI declared in ``include/hi2x.h``).

The library is the only compute path of this package: if it is missing or fails to
load, every entry point raises ``RuntimeError`` naming the problem — there is no CPU
or torch fallback.  Tensors are passed as raw device pointers with the caller's
current HIP stream, and the library never keeps them beyond the call.
"""

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhi2x.so")

OK, EINVAL, ENOTPD, ELAUNCH, ERANGE = 0, -1, -2, -3, -4

_lock = threading.Lock()
_lib = None
_failed: str | None = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (all return int status except the two identity calls)
SIGNATURES = {
    "hi2x_gptq_block": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P],
    "hi2x_gptq_trailing": [_P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P],
    "hi2x_gptq_run": [_P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _P],
    "hi2x_gptq_run_noalloc": [_P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P],
    "hi2x_stream_background": [_P, _I],
    "hi2x_ladder_fit": [_P, _P, _I64, _I64, _I64, _I, _P, _I, _I, _P, _P, _P, _P],
    "hi2x_ladder_fit_rows": [_P, _P, _P, _I64, _I64, _I64, _I, _P, _I, _I, _P, _P, _P, _P],
    "hi2x_finish_rows": [_P, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P],
    "hi2x_params": [_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P],
    "hi2x_decode_params": [_P, _P, _P, _I64, _I64, _P, _P, _P],
    "hi2x_nearest_codes": [_P, _I64, _I64, _I64, _P, _P, _I64, _I, _P, _P],
    "hi2x_finish": [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P],
    "hi2x_ladder_dequantize": [_P, _P, _P, _I64, _I64, _I64, _I, _P, _P],
    "hi2x_fwht16": [_P, _P, _I, _I64, _I64, _P, _P],
    "hi2x_rotate_rows": [_P, _I, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _P],
    "hi2x_pack_codes": [_P, _I64, _I64, _I, _P, _P, _P],
    "hi2x_assemble_piece": [_P, _I64, _P, _P, _P, _I64, _I, _I64, _P, _P, _P, _P, _P, _P, _P],
    "hi2x_hessian_syrk": [_P, _I, _I64, _I64, _P, _P, _I64, _P],
    "hi2x_hessian_syrk_grouped": [_P, _I64, _I, _P, _P, _I64, _I64, _I64, _P, _I64, _I, _P,
                                  _I64, _P],
    "hi2x_hessian_syrk_upper": [_P, _I, _I64, _I64, _P, _P, _I64, _P],
    "hi2x_hessian_mirror": [_P, _I64, _P],
    "hi2x_hessian_blend": [_P, _I64, _I64, _I64, _P, _P, _I, _P],
    "hi2x_sigma_transform_upper_batched": [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P],
    "hi2x_sigma_transform": [_P, _P, _P, _I64, _P, _P],
    "hi2x_sigma_transform_upper": [_P, _I64, _P, _P, _I64, _P, _P],
    "hi2x_chol_lambda": [_P, _I64, _F, _I, _P, _P],
    "hi2x_chol_inv_upper": [_P, _I64, _F, _I, _P, _P, _I64, _P],
    "hi2x_chol_inv_upper_async": [_P, _I64, _F, _I, _P, _P, _P, _I64, _P],
    "hi2x_chol_inv_upper_batched_async": [_P, _I64, _I64, _I64, _F, _I, _P, _I64, _P, _P, _I64,
                                          _P],
    "hi2x_refine_run": [_P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P],
    "hi2x_refine_gradient": [_P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P],
    "hi2x_refine_block": [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P,
                          _I64, _P, _P],
    "hi2x_colstats_update": [_P, _I, _I64, _I64, _P, _P, _I64, _P],
    "hi2x_colstats_diag": [_P, _I64, _I64, _P, _P, _P, _P],
    "hi2x_sigma_pack_upper": [_P, _I64, _I, _P, _P, _P],
    "hi2x_qad_decode_fwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _F, _P],
    "hi2x_qad_decode_bwd": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _F, _P, _P,
                            _P],
    "hi2x_qad_wht_scale": [_P, _I64, _I64, _P, _P, _I, _P],
}
class Piece(ctypes.Structure):
    """hi2x_piece (include/hi2x.h): one piece of hi2x_assemble_batch."""

    _fields_ = [("rows", _P), ("r", _I64), ("codes", _P), ("params", _P), ("consts", _P),
                ("k", _I64), ("nbits", ctypes.c_int32), ("pad_", ctypes.c_int32),
                ("block", _I64), ("code_off", _P), ("param_off", _P), ("out_codes", _P),
                ("out_params", _P), ("out_consts", _P)]


SIGNATURES["hi2x_assemble_batch"] = [_P, _I64, _P, _P]

# workspace sizes (int64 bytes, -1 for bad arguments): name -> argtypes
SIZES = {
    "hi2x_hessian_workspace_bytes": [_I, _I64, _I64],
    "hi2x_hessian_grouped_workspace_bytes": [_I64, _I64, _I64],
    "hi2x_chol_workspace_bytes": [_I64],
    "hi2x_chol_batched_workspace_bytes": [_I64, _I64],
    "hi2x_refine_workspace_bytes": [_I64, _I64, _I64],
    "hi2x_colstats_workspace_bytes": [_I64, _I64],
}


def _bind(lib):
    lib.hi2x_version.restype = ctypes.c_int
    lib.hi2x_version.argtypes = []
    lib.hi2x_timing_enable.restype = ctypes.c_int
    lib.hi2x_timing_enable.argtypes = [ctypes.c_uint]
    lib.hi2x_timing_query.restype = ctypes.c_int
    lib.hi2x_timing_query.argtypes = [_I, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_double)]
    lib.hi2x_last_error.restype = ctypes.c_char_p
    lib.hi2x_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    for name, args in SIZES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int64
        fn.argtypes = args
    return lib


def load():
    """The loaded library, or None with :func:`failure` set (thread-safe, idempotent)."""
    global _lib, _failed
    if _lib is not None or _failed is not None:
        return _lib
    with _lock:
        if _lib is not None or _failed is not None:
            return _lib
        try:
            if not os.path.exists(LIB_PATH):
                raise FileNotFoundError(
                    f"{LIB_PATH} is not built (run `python -m hi2_amd.build`)"
                )
            _lib = _bind(ctypes.CDLL(LIB_PATH))
        except (OSError, AttributeError) as e:
            _failed = f"{type(e).__name__}: {e}"
        return _lib


def failure() -> str | None:
    return _failed


def lib():
    """The library; raises RuntimeError if it cannot be loaded (no fallback exists)."""
    handle = load()
    if handle is None:
        raise RuntimeError(f"hi2x HIP library unavailable: {_failed}")
    return handle


# launch-timing kinds (HI2X_TIME_* in include/hi2x.h)
(TIME_GPTQ_TRAILING, TIME_HESSIAN_SYRK, TIME_CHOL_GEMM, TIME_CHOL_LEAF, TIME_GPTQ_BLOCK,
 TIME_REFINE_GEMM, TIME_REFINE_BLOCK, TIME_FWHT, TIME_LADDER_FIT, TIME_PACK,
 TIME_FINISH, TIME_CHOL_SPLIT) = range(12)


def timing_enable(kinds) -> None:
    """Start recording event-timed launches of the given kinds (empty: stop)."""
    mask = 0
    for k in kinds:
        mask |= 1 << k
    check(lib().hi2x_timing_enable(mask), "hi2x_timing_enable")


def timing_query(kind: int) -> tuple[int, float, float]:
    """(launches, summed event milliseconds, summed algorithmic work) of ``kind``."""
    n, ms, work = _I64(0), ctypes.c_double(0.0), ctypes.c_double(0.0)
    check(lib().hi2x_timing_query(kind, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(work)),
          "hi2x_timing_query")
    return n.value, ms.value, work.value


def stream_background(st: torch.cuda.Stream, on: bool = True) -> None:
    """Mark (or unmark) ``st`` as a background stream: the GPTQ cross-block updates
    launched on it leave room on each CU for the latency-bound kernels of other streams
    (``hi2x_stream_background``; results are unchanged)."""
    check(lib().hi2x_stream_background(ctypes.c_void_p(st.cuda_stream), int(bool(on))),
          "hi2x_stream_background")


def last_error() -> str:
    return lib().hi2x_last_error().decode(errors="replace")


class NotPositiveDefinite(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    """Map a status to the reference's exception types."""
    if rc == OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == ERANGE:
        raise ValueError(msg)
    if rc == ENOTPD:
        raise NotPositiveDefinite(msg)
    raise RuntimeError(msg)


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"hi2_amd runs on the MI355X only: got a tensor on {t.device} "
                "(move inputs to a 'cuda' device)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


_streams: dict = {}


def side_stream(dev: torch.device, i: int) -> torch.cuda.Stream:
    """The i-th persistent side stream of ``dev`` (default priority).  Reusing the same
    streams keeps torch's per-stream cached blocks warm: a fresh stream per call would
    make the caching allocator go back to the driver, which can synchronise the device."""
    key = (torch.device(dev).index, i)
    st = _streams.get(key)
    if st is None:
        with _lock:
            st = _streams.get(key)
            if st is None:
                st = torch.cuda.Stream(device=dev)
                _streams[key] = st
    return st


H2D_CHUNK = 64 << 20  # bytes per pinned staging chunk of a large host tensor


def h2d(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """Host tensor to the device without waiting for the copy: staged through pinned
    memory (torch's pinned allocator keeps each buffer until its copy has run).  Large
    tensors go in chunks of ``H2D_CHUNK`` bytes, so the DMA of one chunk overlaps the
    host's copy of the next into pinned memory."""
    t = t.contiguous()
    nbytes = t.numel() * t.element_size()
    if t.dim() == 0 or nbytes <= H2D_CHUNK:
        return t.pin_memory().to(dev, non_blocking=True)
    out = torch.empty(t.shape, dtype=t.dtype, device=dev)
    step = max(1, H2D_CHUNK // max(1, t[0].numel() * t.element_size()))
    for i in range(0, t.shape[0], step):
        out[i:i + step].copy_(t[i:i + step].pin_memory(), non_blocking=True)
    return out


def to_device(t: torch.Tensor, dev: torch.device, dtype: torch.dtype | None = None
              ) -> torch.Tensor:
    """``t.to(dev, dtype)`` without a host wait: a host tensor goes through :func:`h2d`
    (torch's pageable copy would synchronise the current stream)."""
    if t.device.type == "cpu":
        return h2d(t if dtype is None else t.to(dtype), dev)
    return t.to(dev) if dtype is None else t.to(dev, dtype)


def workspace(dev: torch.device, size_fn: str, *args) -> torch.Tensor:
    """A device workspace for an entry point, from torch's caching allocator on the
    current stream (so concurrent streams never share a block): ``size_fn`` is the
    library's size query for that entry point."""
    n = getattr(lib(), size_fn)(*args)
    if n < 0:
        raise RuntimeError(f"{size_fn}{args}: bad arguments")
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=dev)


def call(name: str, dev: torch.device, *args) -> None:
    """Call ``name`` with ``args`` + the current stream of ``dev`` (device made current)."""
    fn = getattr(lib(), name)
    with torch.cuda.device(dev):
        rc = fn(*args, stream(dev))
    check(rc, name)
