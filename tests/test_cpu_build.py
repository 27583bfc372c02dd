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
              "lisa_gdn_recurrence_m1", "lisa_attn_partial_m1", "lisa_qmv_k5120_m1_prenorm_gateup_wide",
              "lisa_qmv_k5120_m3_prenorm_gateup_wide"):
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
        assert wg[f"lisa_qmv_k5120_m{m}_prenorm_gateup_wide"] == pkg.QMV_WIDE_THREADS
    assert wg["lisa_q4_gemm_wide"] == pkg.GEMM_THREADS_WIDE
    hdr = (Path(pkg.PKG_DIR).parent / "include" / "lisa_kernels.h").read_text()
    assert int(re.search(r"#define LISA_QMV_WIDE_TILES (\d+)", hdr).group(1)) == pkg.QMV_WIDE_TILES
    assert int(re.search(r"#define LISA_QMV_WIDE_THREADS (\d+)", hdr).group(1)) == pkg.QMV_WIDE_THREADS


STRUCTS = {  # Python mirror -> C typedef (include/lisa_kernels.h, include/lisa_hip.h)
    "Q4Mat": "LisaQ4Mat", "QmvParams": "LisaQmvParams", "GdnParams": "LisaGdnParams",
    "AttnParams": "LisaAttnParams", "GemmParams": "LisaGemmParams", "RowsParams": "LisaRowsParams",
    "ConvRowsParams": "LisaConvRowsParams", "SynthParams": "LisaSynthParams", "CopyParams": "LisaCopyParams",
    "AttnDecodeArgs": "LisaAttnDecodeArgs", "RunnerConfig": "LisaRunnerConfig", "WeightSlotStruct": "LisaWeightSlot",
    "Acceptance": "LisaAcceptance", "ReconcilePlan": "LisaReconcilePlan", "SpecStats": "LisaSpecStats",
}


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_python_structs_match_the_headers(tmp_path):
    """Every argument block the Python package passes by value has the C
    header's size and field offsets (a kernel reads its block by those
    offsets, so a field the mirror lacks would be read from past the end)."""
    pkg = load_pkg()
    inc = Path(pkg.PKG_DIR).parent / "include"
    lines = ['#include <cstdio>', '#include <cstddef>', '#include "lisa_kernels.h"', '#include "lisa_hip.h"',
             "int main() {"]
    want = {}
    for py, c in STRUCTS.items():
        cls = getattr(pkg, py)
        lines.append(f'  std::printf("{py} size %zu\\n", sizeof({c}));')
        want[f"{py} size"] = pkg.C.sizeof(cls)
        for name, _ in cls._fields_:
            if name.startswith("pad"):
                continue
            lines.append(f'  std::printf("{py}.{name} %zu\\n", offsetof({c}, {name}));')
            want[f"{py}.{name}"] = getattr(cls, name).offset
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "layout.cpp", tmp_path / "layout"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["g++", "-std=c++17", f"-I{inc}", str(src), "-o", str(exe)], check=True, capture_output=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        key, val = line.rsplit(" ", 1)
        got[key] = int(val)
    assert got == want
