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


QMV_FOUR_WAVE, QMV_GATEUP_WIDE, QMV_INPROJ_WIDE, QMV_X_WIDE = range(4)  # csrc/qmv_launch.h LisaQmvFamily


def qmv_shape(pkg, K, M, pro_mode, kinds, tiles, gate_ab, am_val, wide=True):
    """Restates lisa_qmv_shape of lisa-rs_amd/csrc/qmv_launch.h (the runner's
    rule): (family, grid, block, waves per workgroup). With wide=False every
    launch takes the four-wave kernel."""
    kinds = list(kinds)
    all_store = bool(kinds) and all(k == pkg.EPI_STORE for k in kinds)
    store_conv = bool(kinds) and all(k in (pkg.EPI_STORE, pkg.EPI_CONV) for k in kinds)
    if wide and K == 5120:
        if (kinds == [pkg.EPI_GATEUP] and pro_mode == pkg.PRO_PRENORM and not gate_ab and not am_val):
            return QMV_GATEUP_WIDE, max(1, -(-tiles // pkg.QMV_WIDE_TILES)), pkg.QMV_WIDE_THREADS, pkg.QMV_WIDE_THREADS // 64
        nw = tiles // pkg.QMV_WIDE_GROUPS
        if (pro_mode == pkg.PRO_PRENORM and store_conv and not am_val and tiles % pkg.QMV_WIDE_GROUPS == 0
                and nw in (7, 8)):
            return QMV_INPROJ_WIDE, pkg.QMV_WIDE_GROUPS, 64 * nw, nw
        xw = pkg.QMV_X_WIDE_WAVES
        if (M == 1 and pro_mode == pkg.PRO_LOADX and all_store and not am_val and not gate_ab
                and (xw - 1) * pkg.QMV_WIDE_GROUPS < tiles <= xw * pkg.QMV_WIDE_GROUPS):
            return QMV_X_WIDE, -(-tiles // xw), 64 * xw, xw
    return QMV_FOUR_WAVE, max(1, -(-tiles // 4) if K == 5120 else tiles), 256, 4


def launch_qmv(pkg, dev, K, M, params, mats, wide=True):
    """Restates launch_qmv of lisa-rs_amd/csrc/runner.cpp. mats: list of
    (DevQ4, DevQ4-or-None, out_ptr, kind). The launch shape follows qmv_shape;
    the four-wave kernel owns one 8-row tile per wave (K = 5120, four tiles
    per workgroup) or one per workgroup with its group iterations split over
    the four waves (every other K)."""
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
    kinds = [kind for _, _, _, kind in mats]
    family, grid, block, nw = qmv_shape(pkg, K, M, params.pro_mode, kinds, tiles, bool(params.gate_ab),
                                        bool(params.am_val), wide)
    name = f"lisa_qmv_k{K}_m{M}_{PROLOGUE_NAMES[params.pro_mode]}"
    if family == QMV_GATEUP_WIDE:
        name += "_gateup_wide"
    elif family == QMV_INPROJ_WIDE:
        name += f"_wide{nw}"
    elif family == QMV_X_WIDE:
        name += f"_wide{nw}"
    elif K == 5120 and params.pro_mode in (pkg.PRO_RESNORM, pkg.PRO_PRENORM) and set(kinds) in ({pkg.EPI_GATEUP},
                                                                                          {pkg.EPI_ARGMAX}):
        name += "_gateup" if set(kinds) == {pkg.EPI_GATEUP} else "_argmax"  # the runner's specialized kernels
    dev.dispatch(name, params, (grid,), (block,))
    return params.ksplit, grid


def top2(logits):
    """(top-1 index, top-1 value, top-2 value) of a logit row, ties to the
    lowest index as the argmax kernels break them."""
    v = np.asarray(logits, np.float32)
    i1 = int(np.argmax(v))
    rest = v.copy()
    rest[i1] = -np.inf
    return i1, float(v[i1]), float(rest.max())


def mismatch_diagnostic(step, gpu_token, oracle_logits):
    """The report of a greedy mismatch (tests/spec_diag.rs:79-103): the step,
    both tokens, the oracle's top-2 logit margin, and how far below the
    oracle's top logit the GPU's token scored."""
    i1, v1, v2 = top2(oracle_logits)
    return (f"greedy mismatch at step {step}: gpu token {gpu_token}, oracle token {i1}; "
            f"oracle top-2 margin {v1 - v2:.6g}; oracle logit of the gpu token "
            f"{float(oracle_logits[gpu_token]):.6g} ({v1 - float(oracle_logits[gpu_token]):.6g} below the top)")
