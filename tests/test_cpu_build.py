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


def kernel_metadata():
    blob = Path(load_pkg().HSACO_PATH).read_bytes()
    start = blob.find(b"\x7fELF")  # the gfx950 code object inside the offload bundle
    assert start >= 0
    elf = Path(load_pkg().PKG_DIR) / "_build_notes.elf"
    try:
        elf.write_bytes(blob[start:])
        out = subprocess.run([str(READELF), "--notes", str(elf)], capture_output=True, text=True, check=True).stdout
    finally:
        elf.unlink(missing_ok=True)
    names = re.findall(r"^\s+\.name:\s+(\S+)", out, re.M)
    scratch = [int(x) for x in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", out)]
    assert len(names) == len(scratch) and names
    return dict(zip(names, scratch))


@pytest.mark.skipif(not READELF.exists() or shutil.which("true") is None, reason="llvm-readelf not installed")
def test_no_kernel_spills_to_scratch():
    meta = kernel_metadata()
    for k in ("lisa_q4_gemm", "lisa_q4_gemm_wide", "lisa_qmv_k5120_m1_prenorm_gateup", "lisa_qmv_k17408_m1_x",
              "lisa_gdn_recurrence_m1", "lisa_attn_partial_m1"):
        assert k in meta
    spilled = {k: v for k, v in meta.items() if v}
    assert not spilled, spilled
