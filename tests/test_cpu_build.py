"""The built gfx950 code object: no kernel spills registers to scratch memory.

A spill is silent in every numerics test and costs the hot kernels several
times their time (an exit inside the q4 GEMM's K-step pair once moved its
accumulators out of the matrix registers and made the prefill 3.4x slower), so
the kernel metadata of the code object this repository built is checked:
`.private_segment_fixed_size` must be 0 for every kernel."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from _lisa import load_pkg

READELF = Path("/opt/rocm/llvm/bin/llvm-readelf")


def kernel_notes():
    blob = Path(load_pkg().HSACO_PATH).read_bytes()
    start = blob.find(b"\x7fELF")  # the gfx950 code object inside the offload bundle
    assert start >= 0
    elf = Path(load_pkg().PKG_DIR) / "_build_notes.elf"
    try:
        elf.write_bytes(blob[start:])
        return subprocess.run([str(READELF), "--notes", str(elf)], capture_output=True, text=True, check=True).stdout
    finally:
        elf.unlink(missing_ok=True)


def kernel_field(out, field):
    names = re.findall(r"^\s+\.name:\s+(\S+)", out, re.M)
    vals = [int(x) for x in re.findall(r"\." + field + r":\s+(\d+)", out)]
    assert len(names) == len(vals) and names
    return dict(zip(names, vals))


def kernel_metadata():
    return kernel_field(kernel_notes(), "private_segment_fixed_size")


@pytest.mark.skipif(not READELF.exists() or shutil.which("true") is None, reason="llvm-readelf not installed")
def test_no_kernel_spills_to_scratch():
    meta = kernel_metadata()
    for k in ("lisa_q4_gemm", "lisa_q4_gemm_wide", "lisa_qmv_k5120_m1_prenorm_gateup", "lisa_qmv_k17408_m1_x",
              "lisa_gdn_recurrence_m1", "lisa_attn_partial_m1"):
        assert k in meta
    spilled = {k: v for k, v in meta.items() if v}
    assert not spilled, spilled


@pytest.mark.skipif(not READELF.exists(), reason="llvm-readelf not installed")
def test_python_launch_sizes_match_the_kernels():
    """The workgroup sizes the Python mirror launches with are the ones the
    kernels were built for (their __launch_bounds__)."""
    pkg = load_pkg()
    wg = kernel_field(kernel_notes(), "max_flat_workgroup_size")
    for m in (1, 3):
        assert wg[f"lisa_attn_partial_m{m}"] == pkg.ATT_PARTIAL_THREADS[m]
    assert wg["lisa_q4_gemm_wide"] == pkg.GEMM_THREADS_WIDE
