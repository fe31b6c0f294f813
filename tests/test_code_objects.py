"""The gfx950 kernels of the library need no private segment: every kernel descriptor in
the code objects built into hi2_amd/libhi2x.so states a fixed private (scratch) size of
0 bytes and no dynamic stack.  A kernel that needs scratch makes the HIP runtime allocate
device memory at its first dispatch in a process, which the no-allocation entry point
(hi2x_gptq_run_noalloc) promises not to do — CPU only: reads the metadata notes of the
library's own build with the ROCm LLVM tools."""

import os
import re
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _code_objects(tmp_path):
    """The gfx950 code objects of the library's offload bundles (one per source file)."""
    lib = os.path.join(ROOT, "hi2_amd", "libhi2x.so")
    if not os.path.exists(lib):
        pytest.skip("libhi2x.so not built")
    objcopy = os.path.join(LLVM, "llvm-objcopy")
    if not os.path.exists(objcopy):
        pytest.skip("llvm-objcopy not available")
    fat = tmp_path / "fatbin.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", lib, str(tmp_path / "x.so")],
                   check=True, capture_output=True)
    blob = fat.read_bytes()
    out, i = [], 0
    while (j := blob.find(MAGIC, i)) >= 0:
        (count,) = struct.unpack_from("<Q", blob, j + len(MAGIC))
        p = j + len(MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", blob, p)
            triple = blob[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple and size:
                co = tmp_path / f"co{len(out)}.elf"
                co.write_bytes(blob[j + off:j + off + size])
                out.append(co)
        i = j + 1
    return out


def test_no_kernel_needs_a_private_segment(tmp_path):
    readelf = os.path.join(LLVM, "llvm-readelf")
    if not os.path.exists(readelf) or shutil.which("true") is None:
        pytest.skip("llvm-readelf not available")
    cos = _code_objects(tmp_path)
    assert len(cos) >= 8, "one gfx950 code object per kernel source"
    kernels = 0
    for co in cos:
        notes = subprocess.run([readelf, "--notes", str(co)], check=True, capture_output=True,
                               text=True).stdout
        names = re.findall(r"^\s+\.name:\s+(\S+)", notes, re.M)
        priv = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)]
        dyn = re.findall(r"\.uses_dynamic_stack:\s+(\w+)", notes)
        kern = [n for n in names if not n.endswith(".kd")]
        assert len(priv) == len(kern) > 0, co
        for name, size in zip(kern, priv):
            assert size == 0, f"{name} needs {size} B of scratch per lane"
        assert all(d == "false" for d in dyn), co
        kernels += len(kern)
    assert kernels >= 40
