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
              "lisa_qmv_k5120_m3_prenorm_gateup_wide", "lisa_qmv_k5120_m1_prenorm_wide7",
              "lisa_qmv_k5120_m1_prenorm_wide8", "lisa_qmv_k5120_m3_prenorm_wide7", "lisa_qmv_k5120_m3_prenorm_wide8",
              "lisa_qmv_k5120_m1_x_wide9", "lisa_q4_gemm_m128"):
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
        for nw in (7, 8):
            assert wg[f"lisa_qmv_k5120_m{m}_prenorm_wide{nw}"] == 64 * nw
    assert wg["lisa_qmv_k5120_m1_x_wide9"] == 64 * pkg.QMV_X_WIDE_WAVES
    assert wg["lisa_attn_partial_rows"] == pkg.ATT_ROWS_THREADS
    assert wg["lisa_q4_gemm_m128"] == 256
    assert wg["lisa_q4_gemm_wide"] == pkg.GEMM_THREADS_WIDE
    hdr = (Path(pkg.PKG_DIR).parent / "include" / "lisa_kernels.h").read_text()
    assert int(re.search(r"#define LISA_QMV_WIDE_TILES (\d+)", hdr).group(1)) == pkg.QMV_WIDE_TILES
    assert int(re.search(r"#define LISA_QMV_WIDE_THREADS (\d+)", hdr).group(1)) == pkg.QMV_WIDE_THREADS
    assert int(re.search(r"#define LISA_QMV_WIDE_GROUPS (\d+)", hdr).group(1)) == pkg.QMV_WIDE_GROUPS
    assert int(re.search(r"#define LISA_QMV_X_WIDE_WAVES (\d+)", hdr).group(1)) == pkg.QMV_X_WIDE_WAVES
    assert int(re.search(r"#define LISA_ATT_ROWS_THREADS (\d+)", hdr).group(1)) == pkg.ATT_ROWS_THREADS
    assert int(re.search(r"#define LISA_GEMM_TILE_M_SMALL (\d+)", hdr).group(1)) == pkg.GEMM_TILE_M_SMALL


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


ENUMS = {"PRO_": "LISA_PRO_", "EPI_": "LISA_EPI_", "FILL_": "LISA_FILL_"}


def test_python_enums_match_the_headers(tmp_path):
    """The package's prologue, epilogue and fill-kind constants equal the C
    enums (a fill kind off by one writes 4-byte elements into a buffer sized
    for 2-byte ones)."""
    pkg = load_pkg()
    inc = Path(pkg.PKG_DIR).parent / "include"
    lines = ['#include <cstdio>', '#include "lisa_kernels.h"', '#include "lisa_synth.h"', "int main() {"]
    want = {}
    for py, c in ENUMS.items():
        for name in dir(pkg):
            if name.startswith(py) and isinstance(getattr(pkg, name), int):
                lines.append(f'  std::printf("{name} %d\\n", (int){c}{name[len(py):]});')
                want[name] = getattr(pkg, name)
    for name in ("DIST_BITS", "DIST_UNIFORM", "DIST_NORMAL"):
        lines.append(f'  std::printf("{name} %d\\n", (int)LISA_{name});')
        want[name] = getattr(pkg, name)
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "enums.cpp", tmp_path / "enums"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["g++", "-std=c++17", f"-I{inc}", str(src), "-o", str(exe)], check=True, capture_output=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        key, val = line.rsplit(" ", 1)
        got[key] = int(val)
    assert len(want) >= 20 and got == want


def test_synth_fill_refuses_overruns():
    """Device.synth_fill checks the element count against the buffer on the
    host before any dispatch."""
    pkg = load_pkg()

    class Dev:  # the check runs before self.dispatch
        dispatch = None

    class Buf:
        nbytes, ptr = 1024, 0

    fill = pkg.Device.synth_fill
    with pytest.raises(ValueError):
        fill(Dev(), Buf(), 512, pkg.FILL_SB, 1)  # 2048 bytes
    with pytest.raises(ValueError):
        fill(Dev(), Buf(), 513, pkg.FILL_BF16, 1)
    with pytest.raises(ValueError):
        fill(Dev(), Buf(), 4 * 256, pkg.FILL_KV, 1, capacity=1, filled=1)  # 2048 bytes
    with pytest.raises(ValueError):
        fill(Dev(), Buf(), 4 * 256, pkg.FILL_KV, 1, capacity=0, filled=1)
    with pytest.raises(ValueError):
        fill(Dev(), Buf(), 4, 7, 1)


def test_python_launch_rule_matches_the_runner(tmp_path):
    """tests/_lisa.py's qmv_shape (the launch shape the GPU tests dispatch)
    equals lisa_qmv_shape of csrc/qmv_launch.h, which the runner applies, on
    the model's q4 launches and the edges of each rule."""
    import _lisa
    pkg = load_pkg()
    root = Path(pkg.PKG_DIR).parent
    S, G, C, A, R = pkg.EPI_STORE, pkg.EPI_GATEUP, pkg.EPI_CONV, pkg.EPI_ARGMAX, pkg.EPI_RESID
    cases = []
    for m in (1, 3):
        cases += [(5120, m, pkg.PRO_PRENORM, [G], 4352, 0, 0), (5120, m, pkg.PRO_PRENORM, [G], 251, 0, 0),
                  (5120, m, pkg.PRO_PRENORM, [G], 4352, 1, 0), (5120, m, pkg.PRO_RESNORM, [G], 4352, 0, 0),
                  (5120, m, pkg.PRO_PRENORM, [C, S], 2048, 1, 0), (5120, m, pkg.PRO_PRENORM, [S, S, S], 1792, 0, 0),
                  (5120, m, pkg.PRO_PRENORM, [S], 2047, 0, 0), (5120, m, pkg.PRO_PRENORM, [S], 1536, 0, 0),
                  (5120, m, pkg.PRO_PRENORM, [A], 31040, 0, 1), (5120, m, pkg.PRO_PRENORM, [R, S], 2048, 0, 0),
                  (5120, m, pkg.PRO_EMBED, [C, S], 2048, 1, 0), (5120, m, pkg.PRO_CAST, [S, S, S], 1792, 0, 0),
                  (5120, m, pkg.PRO_LOADX, [S], 2176, 0, 0), (5120, m, pkg.PRO_LOADX, [S], 2048, 0, 0),
                  (5120, m, pkg.PRO_LOADX, [S], 2049, 0, 0), (5120, m, pkg.PRO_LOADX, [S], 2304, 0, 0),
                  (5120, m, pkg.PRO_LOADX, [S], 2305, 0, 0), (5120, m, pkg.PRO_LOADX, [S, S], 2176, 0, 0),
                  (5120, m, pkg.PRO_LOADX, [C], 2176, 0, 0), (17408, m, pkg.PRO_LOADX, [R], 640, 0, 0),
                  (6144, m, pkg.PRO_LOADX, [R], 640, 0, 0), (10240, m, pkg.PRO_MTPFC, [S], 640, 0, 0),
                  (1024, m, pkg.PRO_LOADX, [S], 3, 0, 0), (5120, m, pkg.PRO_PRENORM, [S, S], 6, 0, 0)]
    lines = ["#include <cstdio>", '#include "qmv_launch.h"', "int main() {"]
    for K, m, pro, kinds, tiles, gab, amv in cases:
        ks = ", ".join(str(k) for k in kinds)
        lines.append(f"  {{ const uint32_t k[] = {{{ks}}}; const LisaQmvShape s = lisa_qmv_shape({K}, {m}, {pro}, k, "
                     f"{len(kinds)}, {tiles}, {'true' if gab else 'false'}, {'true' if amv else 'false'}); "
                     'std::printf("%d %u %u %u\\n", s.family, s.grid, s.block, s.nw); }')
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "shape.cpp", tmp_path / "shape"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["g++", "-std=c++17", f"-I{root / 'include'}", f"-I{root / 'lisa-rs_amd' / 'csrc'}", str(src),
                    "-o", str(exe)], check=True, capture_output=True)
    got = [tuple(int(v) for v in line.split())
           for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()]
    want = [_lisa.qmv_shape(pkg, K, m, pro, kinds, tiles, bool(gab), bool(amv)) for K, m, pro, kinds, tiles, gab, amv in cases]
    assert got == want
    families = {w[0] for w in want}
    assert families == {0, 1, 2, 3}
