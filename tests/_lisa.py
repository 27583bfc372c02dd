"""Shared helpers for the tests: package/oracle loading, random q4 tensors,
and a Python restatement of the runner's q4 launch rule (tile ranges, ksplit,
grid) for kernel-level dispatches."""
import ctypes as C
import importlib.util
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def load_pkg():
    if "lisa_rs_amd" in sys.modules:
        return sys.modules["lisa_rs_amd"]
    pkg_dir = ROOT / "lisa-rs_amd"
    spec = importlib.util.spec_from_file_location("lisa_rs_amd", pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lisa_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    if "lisa_oracle" in sys.modules:
        return sys.modules["lisa_oracle"]
    spec = importlib.util.spec_from_file_location("lisa_oracle", ROOT / "oracle" / "oracle.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lisa_oracle"] = mod
    spec.loader.exec_module(mod)
    return mod


def bf16(x):
    return load_oracle().f32_to_bf16_bits(x)


def f32(h):
    return load_oracle().bf16_bits_to_f32(h)


def rand_q4(rng, n, k):
    """MLX-affine q4 of BASELINE config 0: nibbles U{0..15}, scales U(0.005,0.02),
    biases U(-0.1,0.1), both bf16."""
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16(rng.uniform(0.005, 0.02, size=(n, k // 64)).astype(np.float32))
    b = bf16(rng.uniform(-0.1, 0.1, size=(n, k // 64)).astype(np.float32))
    return w, s, b


def pack_sb(s, b):
    return (s.astype(np.uint32) | (b.astype(np.uint32) << 16)).astype(np.uint32)


class DevQ4:
    def __init__(self, dev, w, s, b):
        self.n, self.k = w.shape[0], w.shape[1] * 8
        self.wbuf = dev.upload(w)
        self.sbbuf = dev.upload(pack_sb(s, b))
        self.w, self.s, self.b = w, s, b


PROLOGUE_NAMES = ["x", "resnorm", "embed", "cast", "norm", "mtpfc", "prenorm"]


def launch_qmv(pkg, dev, K, M, params, mats, wide=True):
    """Restates launch_qmv of lisa-rs_amd/csrc/runner.cpp. mats: list of
    (DevQ4, DevQ4-or-None, out_ptr, kind). One 8-row tile per wave (K = 5120,
    four tiles per workgroup) or per workgroup with the group iterations split
    over its four waves (every other K); unless wide=False, the MLP gate/up
    alone under PRENORM runs on the 16-wave kernel, a PRENORM launch of
    STORE/CONV matrices of 256 x 7 or 256 x 8 tiles on the 7- or 8-wave one,
    and a one-row LOADX launch of STORE matrices of 2049..2304 tiles on the
    9-wave one."""
    tiles = 0
    for e, (q, q2, out, kind) in enumerate(mats):
        m = params.mats[e]
        m.w, m.sb = q.wbuf.ptr, q.sbbuf.ptr
        m.w2 = q2.wbuf.ptr if q2 else 0
        m.sb2 = q2.sbbuf.ptr if q2 else 0
        m.out = out
        m.rows = q.n
        m.kind = kind
        params.tile_start[e] = tiles
        pair = kind == pkg.EPI_GATEUP
        tiles += (q.n + 3) // 4 if pair else (q.n + 7) // 8
    params.tile_start[len(mats)] = tiles
    params.n_mats = len(mats)
    params.ksplit = 1 if K == 5120 else 4
    grid = max(1, tiles if params.ksplit == 4 else (tiles + 3) // 4)
    name = f"lisa_qmv_k{K}_m{M}_{PROLOGUE_NAMES[params.pro_mode]}"
    kinds = {kind for _, _, _, kind in mats}
    if K == 5120 and params.pro_mode in (pkg.PRO_RESNORM, pkg.PRO_PRENORM) and kinds in ({pkg.EPI_GATEUP},
                                                                                    {pkg.EPI_ARGMAX}):
        name += "_gateup" if kinds == {pkg.EPI_GATEUP} else "_argmax"  # the runner's specialized kernels
    if (wide and K == 5120 and len(mats) == 1 and kinds == {pkg.EPI_GATEUP} and params.pro_mode == pkg.PRO_PRENORM
            and not params.gate_ab and not params.am_val):
        # the runner's 16-wave gate/up: LISA_QMV_WIDE_TILES tiles per workgroup
        grid = max(1, (tiles + pkg.QMV_WIDE_TILES - 1) // pkg.QMV_WIDE_TILES)
        dev.dispatch(name + "_wide", params, (grid,), (pkg.QMV_WIDE_THREADS,))
        return params.ksplit, grid
    nw = tiles // pkg.QMV_WIDE_GROUPS
    if (wide and K == 5120 and params.pro_mode == pkg.PRO_PRENORM and kinds <= {pkg.EPI_STORE, pkg.EPI_CONV}
            and not params.am_val and tiles % pkg.QMV_WIDE_GROUPS == 0 and nw in (7, 8)):
        # the runner's in-projection launch: one tile per wave, one workgroup per CU
        dev.dispatch(f"{name}_wide{nw}", params, (pkg.QMV_WIDE_GROUPS,), (64 * nw,))
        return params.ksplit, pkg.QMV_WIDE_GROUPS
    xw = pkg.QMV_X_WIDE_WAVES
    if (wide and K == 5120 and M == 1 and params.pro_mode == pkg.PRO_LOADX and kinds == {pkg.EPI_STORE}
            and not params.am_val and not params.gate_ab
            and (xw - 1) * pkg.QMV_WIDE_GROUPS < tiles <= xw * pkg.QMV_WIDE_GROUPS):
        # the runner's one-row plain-x launch of a 17408-row projection
        grid = (tiles + xw - 1) // xw
        dev.dispatch(f"{name}_wide{xw}", params, (grid,), (64 * xw,))
        return params.ksplit, grid
    dev.dispatch(name, params, (grid,), (256,))
    return params.ksplit, grid
