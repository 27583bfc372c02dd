"""lisa-rs_amd — MI355X (gfx950) decode path of lisa-rs behind a C ABI.

This module is a thin ctypes binding of ``liblisa_hip.so`` (include/lisa_hip.h)
that mirrors the reference's Rust interfaces for the decode path:

* ``Runner``  — ``QwenRunner`` + ``MtpRunner`` (src/model/runner.rs): load,
  forward_token_decode / forward_token_with_hidden, verify_block3_decode,
  commit_verified_prefix, checkpoint/restore/reset, and the MTP drafter's
  forward_position_decode_device / trim_state.
* ``accept_greedy``, ``mtp_reconcile_plan``, ``Runner.generate_greedy_block3``
  — src/speculative/mod.rs.
* ``Device`` / ``Buffer`` / ``Function`` — the device bridge that replaces
  src/device/metal.rs, used by kernel-level tests the way the reference's
  tests drive ``MetalDevice`` directly.

Errors are raised as ``LisaError`` carrying ``lisa_last_error()``, where the
reference returns ``Err(String)`` or panics. There is no CPU fallback: when
the shared library or the kernel code object is missing, loading fails.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "liblisa_hip.so"
HSACO_PATH = PKG_DIR / "lisa_kernels.hsaco"

HIDDEN = 5120
INTER = 17408
VOCAB = 248320
LAYERS = 64
GDN_KH, GDN_VH, GDN_HD = 16, 48, 128
GDN_CONV_DIM = 10240
GDN_STATE = GDN_VH * GDN_HD * GDN_HD
ATT_QH, ATT_KVH, ATT_HD = 24, 4, 256

# launch kinds of lisa_runner_profile_step (lisa_hip.h LISA_KIND_*)
KINDS = ["gdn_in_proj", "gdn_recurrence", "gdn_out_proj", "attn_in_proj", "attn_partial", "attn_merge",
         "attn_o_proj", "mlp_gate_up", "mlp_down", "lm_head", "finalize"]

# lisa_kernels.h enums
PRO_LOADX, PRO_RESNORM, PRO_EMBED, PRO_CAST, PRO_NORM, PRO_MTPFC, PRO_PRENORM = range(7)
EPI_STORE, EPI_GATEUP, EPI_CONV, EPI_ARGMAX, EPI_RESID = range(5)
FILL_WORDS, FILL_BF16, FILL_F32, FILL_SB, FILL_KV = range(5)
DIST_BITS, DIST_UNIFORM, DIST_NORMAL = range(3)  # lisa_synth.h LISA_DIST_*


class LisaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


# ---------------------------------------------------------------------------
# kernel argument blocks (include/lisa_kernels.h)
# ---------------------------------------------------------------------------
class Q4Mat(C.Structure):
    _fields_ = [("w", C.c_uint64), ("sb", C.c_uint64), ("w2", C.c_uint64), ("sb2", C.c_uint64),
                ("out", C.c_uint64), ("rows", C.c_uint32), ("kind", C.c_uint32)]


class QmvParams(C.Structure):
    _fields_ = [("x_in", C.c_uint64), ("h_in", C.c_uint64), ("o_in", C.c_uint64), ("tokens", C.c_uint64),
                ("emb_w", C.c_uint64), ("emb_sb", C.c_uint64), ("norm_w", C.c_uint64), ("norm_w2", C.c_uint64),
                ("r_out", C.c_uint64), ("x_out", C.c_uint64),
                ("conv_w", C.c_uint64), ("conv_state", C.c_uint64), ("conv_slots", C.c_uint64),
                ("conv_slot_stride", C.c_uint64),
                ("am_val", C.c_uint64), ("am_idx", C.c_uint64),
                ("mats", Q4Mat * 4), ("tile_start", C.c_uint32 * 5),
                ("n_mats", C.c_uint32), ("pro_mode", C.c_uint32), ("capture", C.c_uint32), ("ksplit", C.c_uint32),
                ("gate_a_w", C.c_uint64), ("gate_a_sb", C.c_uint64), ("gate_b_w", C.c_uint64),
                ("gate_b_sb", C.c_uint64), ("gate_ab", C.c_uint64)]


class GdnParams(C.Structure):
    _fields_ = [("conv_out", C.c_uint64), ("z", C.c_uint64), ("a", C.c_uint64), ("b", C.c_uint64),
                ("a_log", C.c_uint64), ("dt_bias", C.c_uint64), ("norm_w", C.c_uint64),
                ("state", C.c_uint64), ("slots", C.c_uint64), ("slot_stride", C.c_uint64),
                ("gated", C.c_uint64), ("y_out", C.c_uint64), ("q_scale", C.c_float), ("k_scale", C.c_float),
                ("capture", C.c_uint32), ("m_rows", C.c_uint32), ("qk", C.c_uint64), ("gates", C.c_uint64),
                ("gate_ab", C.c_uint64), ("pf_w", C.c_uint64), ("pf_sb", C.c_uint64), ("pf_sink", C.c_uint64),
                ("pf_tiles", C.c_uint32), ("pf_k", C.c_uint32), ("pf_delay", C.c_uint32), ("pad0", C.c_uint32)]


class AttnParams(C.Structure):
    _fields_ = [("q_proj", C.c_uint64), ("k_raw", C.c_uint64), ("v_raw", C.c_uint64),
                ("q_norm_w", C.c_uint64), ("k_norm_w", C.c_uint64), ("key_cache", C.c_uint64),
                ("value_cache", C.c_uint64), ("part_o", C.c_uint64), ("part_ml", C.c_uint64),
                ("pos", C.c_uint64), ("gated", C.c_uint64), ("capacity", C.c_uint32), ("s_max", C.c_uint32),
                ("query", C.c_uint64), ("m_rows", C.c_uint32), ("pad0", C.c_uint32)]


class GemmParams(C.Structure):
    _fields_ = [("a", C.c_uint64), ("w", C.c_uint64), ("sb", C.c_uint64), ("c", C.c_uint64),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32), ("ldc", C.c_uint32),
                ("w2", C.c_uint64), ("sb2", C.c_uint64), ("act", C.c_uint64)]


ROWS_EMBED, ROWS_NORM, ROWS_RESNORM, ROWS_SILU, ROWS_ARGMAX = range(5)
GEMM_TILE_M, GEMM_TILE_N = 256, 128  # lisa_q4_gemm output tile (LISA_GEMM_TILE_M/N)
GEMM_TILE_M_SMALL = 128  # lisa_q4_gemm_m128 output tile rows (LISA_GEMM_TILE_M_SMALL)
GEMM_TILE_N_WIDE = 256  # lisa_q4_gemm_wide (LISA_GEMM_TILE_N_WIDE)
GEMM_THREADS_WIDE = 512  # lisa_q4_gemm_wide workgroup size (LISA_GEMM_THREADS_WIDE)
QMV_MAX_MATS = 4  # matrices per q4 launch (LISA_QMV_MAX_MATS)
ATT_ROWS_PER_WG = 16  # lisa_attn_partial_rows rows per workgroup (LISA_ATT_ROWS_PER_WG)
ATT_PARTIAL_THREADS = {1: 1024, 3: 1024}  # lisa_attn_partial_m{1,3} workgroup size (LISA_ATT_PARTIAL_THREADS)
QMV_WIDE_THREADS = 1024  # lisa_qmv_k5120_m{1,3}_prenorm_gateup_wide workgroup size (LISA_QMV_WIDE_THREADS)
QMV_WIDE_TILES = 17  # 8-row tiles per workgroup of that kernel (LISA_QMV_WIDE_TILES)
QMV_WIDE_GROUPS = 256  # workgroups of a lisa_qmv_k5120_m{1,3}_prenorm_wide{7,8} launch (LISA_QMV_WIDE_GROUPS)
QMV_X_WIDE_WAVES = 9  # waves of lisa_qmv_k5120_m1_x_wide9 (LISA_QMV_X_WIDE_WAVES)
ATT_ROWS_THREADS = 1024  # workgroup size of lisa_attn_partial_rows (LISA_ATT_ROWS_THREADS)


class RowsParams(C.Structure):
    _fields_ = [("h_in", C.c_uint64), ("o_in", C.c_uint64), ("norm_w", C.c_uint64), ("r_out", C.c_uint64),
                ("x_out", C.c_uint64), ("tokens", C.c_uint64), ("emb_w", C.c_uint64), ("emb_sb", C.c_uint64),
                ("g_in", C.c_uint64), ("u_in", C.c_uint64), ("act_out", C.c_uint64), ("logits", C.c_uint64),
                ("argmax_out", C.c_uint64), ("width", C.c_uint32), ("mode", C.c_uint32),
                ("x_stride", C.c_uint32), ("pad0", C.c_uint32)]


class ConvRowsParams(C.Structure):
    _fields_ = [("qkv", C.c_uint64), ("conv_w", C.c_uint64), ("conv_state", C.c_uint64), ("conv_out", C.c_uint64),
                ("m_rows", C.c_uint32), ("pad0", C.c_uint32)]


class SynthParams(C.Structure):
    _fields_ = [("out", C.c_uint64), ("n", C.c_uint64), ("key", C.c_uint64), ("key2", C.c_uint64),
                ("kind", C.c_uint32), ("dist", C.c_uint32), ("a", C.c_float), ("b", C.c_float),
                ("capacity", C.c_uint32), ("filled", C.c_uint32)]


class CopyParams(C.Structure):
    _fields_ = [("src", C.c_uint64), ("dst", C.c_uint64), ("n16", C.c_uint64)]


class AttnDecodeArgs(C.Structure):
    _fields_ = [("q_proj", C.c_uint64), ("k_raw", C.c_uint64), ("v_raw", C.c_uint64), ("q_norm_w", C.c_uint64),
                ("k_norm_w", C.c_uint64), ("key_cache", C.c_uint64), ("value_cache", C.c_uint64), ("pos", C.c_uint64),
                ("gated", C.c_uint64), ("capacity", C.c_uint32), ("m_rows", C.c_uint32), ("max_pos", C.c_uint32),
                ("pad0", C.c_uint32)]


class RunnerConfig(C.Structure):
    _fields_ = [("layers", C.c_int32), ("vocab", C.c_int32), ("capacity", C.c_int32), ("with_mtp", C.c_int32),
                ("seed", C.c_uint64), ("use_graph", C.c_int32), ("device", C.c_int32)]


MAX_DIMS = 8
DTYPES = ["BOOL", "U8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "F64"]


class WeightSlotStruct(C.Structure):
    _fields_ = [("shard", C.c_int32), ("dtype", C.c_int32), ("ndim", C.c_int32), ("pad0", C.c_int32),
                ("offset", C.c_uint64), ("data_start", C.c_uint64), ("len", C.c_uint64),
                ("shape", C.c_uint64 * MAX_DIMS)]


class Acceptance(C.Structure):
    _fields_ = [("accepted_drafts", C.c_int32), ("emitted_count", C.c_int32), ("emitted", C.c_uint32 * 3),
                ("target_trim", C.c_int32)]


class ReconcilePlan(C.Structure):
    _fields_ = [("trim", C.c_int32), ("replay_count", C.c_int32), ("replay", C.c_int32 * 3)]


class SpecStats(C.Structure):
    _fields_ = [("rounds", C.c_int32), ("accepted_drafts", C.c_int32), ("drafted_tokens", C.c_int32),
                ("target_forwards", C.c_int32)]


# ---------------------------------------------------------------------------
# library loading
# ---------------------------------------------------------------------------
_LIB = None

_P = C.c_void_p
_SIGS = {
    "lisa_last_error": (C.c_char_p, []),
    "lisa_device_create": (C.c_int, [C.c_int, C.POINTER(_P)]),
    "lisa_device_free": (None, [_P]),
    "lisa_device_name": (C.c_int, [_P, C.c_char_p, C.c_size_t]),
    "lisa_device_max_working_set": (C.c_uint64, [_P]),
    "lisa_device_synchronize": (C.c_int, [_P]),
    "lisa_buffer_alloc": (C.c_int, [_P, C.c_size_t, C.POINTER(_P)]),
    "lisa_buffer_free": (None, [_P]),
    "lisa_buffer_device_ptr": (C.c_uint64, [_P]),
    "lisa_buffer_len": (C.c_size_t, [_P]),
    "lisa_buffer_write": (C.c_int, [_P, C.c_size_t, _P, C.c_size_t]),
    "lisa_buffer_read": (C.c_int, [_P, C.c_size_t, _P, C.c_size_t]),
    "lisa_buffer_copy": (C.c_int, [_P, C.c_size_t, _P, C.c_size_t, C.c_size_t]),
    "lisa_module_load": (C.c_int, [_P, C.c_char_p, C.POINTER(_P)]),
    "lisa_module_load_data": (C.c_int, [_P, _P, C.c_size_t, C.POINTER(_P)]),
    "lisa_module_load_default": (C.c_int, [_P, C.POINTER(_P)]),
    "lisa_module_free": (None, [_P]),
    "lisa_function_get": (C.c_int, [_P, C.c_char_p, C.POINTER(_P)]),
    "lisa_encoder_begin": (C.c_int, [_P, C.POINTER(_P)]),
    "lisa_encoder_set_function": (C.c_int, [_P, _P]),
    "lisa_encoder_set_buffer": (C.c_int, [_P, C.c_uint32, _P, C.c_uint64]),
    "lisa_encoder_set_bytes": (C.c_int, [_P, C.c_uint32, _P, C.c_size_t]),
    "lisa_encoder_dispatch_groups": (C.c_int, [_P] + [C.c_uint32] * 6),
    "lisa_encoder_dispatch_threads": (C.c_int, [_P] + [C.c_uint32] * 6),
    "lisa_encoder_end": (C.c_int, [_P, C.c_int]),
    "lisa_capture_begin": (C.c_int, [_P]),
    "lisa_capture_end": (C.c_int, [_P, C.POINTER(_P)]),
    "lisa_graph_launch": (C.c_int, [_P, _P]),
    "lisa_graph_free": (None, [_P]),
    "lisa_event_create": (C.c_int, [C.POINTER(_P)]),
    "lisa_event_free": (None, [_P]),
    "lisa_event_record": (C.c_int, [_P, _P]),
    "lisa_event_elapsed_ms": (C.c_int, [_P, _P, C.POINTER(C.c_float)]),
    "lisa_attention_workspace_bytes": (C.c_uint64, [C.c_uint32, C.c_uint32]),
    "lisa_attention_decode": (C.c_int, [_P, _P, C.POINTER(AttnDecodeArgs), _P]),
    "lisa_attention_decode_noalloc": (C.c_int, [_P, _P, C.POINTER(AttnDecodeArgs)]),
    "lisa_runner_create": (C.c_int, [C.POINTER(RunnerConfig), C.POINTER(_P)]),
    "lisa_runner_free": (None, [_P]),
    "lisa_runner_load": (C.c_int, [C.c_char_p, C.c_char_p, C.POINTER(RunnerConfig), C.POINTER(_P)]),
    "lisa_mtp_load": (C.c_int, [_P, C.c_char_p, C.c_int32]),
    "lisa_weight_index_open": (C.c_int, [C.POINTER(C.c_char_p), C.c_int32, C.POINTER(_P)]),
    "lisa_weight_index_open_snapshot": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "lisa_weight_index_free": (None, [_P]),
    "lisa_weight_index_len": (C.c_int32, [_P]),
    "lisa_weight_index_shard_count": (C.c_int32, [_P]),
    "lisa_weight_index_slot": (C.c_int, [_P, C.c_char_p, C.POINTER(WeightSlotStruct)]),
    "lisa_weight_index_validate": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32]),
    "lisa_runner_device": (_P, [_P]),
    "lisa_runner_position": (C.c_uint32, [_P]),
    "lisa_runner_weight_bytes": (C.c_uint64, [_P]),
    "lisa_runner_reset_state": (C.c_int, [_P]),
    "lisa_runner_fill_state": (C.c_int, [_P, C.c_uint32, C.c_uint64]),
    "lisa_runner_forward_token_decode": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_uint32), _P]),
    "lisa_runner_forward_token_with_hidden": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_uint32), _P, _P]),
    "lisa_runner_decode_greedy": (C.c_int, [_P, C.c_uint32, C.c_int32, _P]),
    "lisa_runner_forward_prefill": (C.c_int, [_P, _P, C.c_int32, C.c_int32, _P, _P]),
    "lisa_runner_profile_step": (C.c_int, [_P, C.c_uint32, C.c_int32, _P, _P]),
    "lisa_runner_profile_block3": (C.c_int, [_P, _P, _P, _P]),
    "lisa_runner_verify_block3": (C.c_int, [_P, _P, _P, _P, _P]),
    "lisa_runner_commit_verified_prefix": (C.c_int, [_P, C.c_int32]),
    "lisa_runner_checkpoint_state": (C.c_int, [_P, C.POINTER(_P)]),
    "lisa_runner_restore_state": (C.c_int, [_P, _P]),
    "lisa_checkpoint_free": (None, [_P]),
    "lisa_runner_upload_hidden": (C.c_int, [_P, C.c_int32, _P]),
    "lisa_runner_vocab": (C.c_int32, [_P]),
    "lisa_runner_read_gdn_state": (C.c_int, [_P, C.c_int32, _P]),
    "lisa_runner_read_conv_state": (C.c_int, [_P, C.c_int32, _P]),
    "lisa_mtp_forward": (C.c_int, [_P, C.c_uint32, C.c_int32, C.c_int32, C.POINTER(C.c_uint32)]),
    "lisa_mtp_upload_normalized": (C.c_int, [_P, _P]),
    "lisa_mtp_upload_cond": (C.c_int, [_P, _P]),
    "lisa_mtp_read_normalized": (C.c_int, [_P, _P]),
    "lisa_mtp_position": (C.c_uint32, [_P]),
    "lisa_mtp_trim_state": (C.c_int, [_P, C.c_int32]),
    "lisa_mtp_reset_state": (C.c_int, [_P]),
    "lisa_runner_hidden_offset": (C.c_uint64, [C.c_int32]),
    "lisa_mtp_normalized_offset": (C.c_uint64, []),
    "lisa_mtp_resolve_cond": (C.c_int, [C.c_int32, C.c_uint64, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "lisa_mtp_forward_device": (C.c_int, [_P, C.c_uint32, C.c_int32, C.c_uint64, C.POINTER(C.c_uint32),
                                          C.POINTER(C.c_uint64)]),
    "lisa_mtp_forward_position_decode": (C.c_int, [_P, C.c_uint32, _P, C.POINTER(C.c_uint32), _P]),
    "lisa_mtp_forward_batch": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P, _P]),
    "lisa_prefill_prompt": (C.c_int, [_P, _P, C.c_int32, C.c_int32, C.POINTER(C.c_uint32), _P,
                                      C.POINTER(C.c_uint32), _P]),
    "lisa_mtp_checkpoint_state": (C.c_int, [_P, C.POINTER(_P)]),
    "lisa_mtp_restore_state": (C.c_int, [_P, _P]),
    "lisa_mtp_checkpoint_free": (None, [_P]),
    "lisa_accept_greedy": (C.c_int, [_P, C.c_int32, _P, C.POINTER(Acceptance)]),
    "lisa_mtp_reconcile_plan": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.POINTER(ReconcilePlan)]),
    "lisa_generate_greedy_block3": (C.c_int, [_P, C.c_uint32, _P, C.c_uint32, _P, C.c_int32, _P, C.c_int32,
                                              C.c_uint64, C.c_float, _P, C.POINTER(SpecStats)]),
}


def exported_symbols() -> list[str]:
    """Every entry point declared in include/lisa_hip.h."""
    return sorted(_SIGS)


def lib() -> C.CDLL:
    """Load liblisa_hip.so (built by __graft_entry__.build()); fails loudly."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        if not HSACO_PATH.exists():
            raise FileNotFoundError(f"{HSACO_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _check(rc: int) -> None:
    if rc != 0:
        raise LisaError(rc, lib().lisa_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# device bridge (src/device/metal.rs)
# ---------------------------------------------------------------------------
class Buffer:
    def __init__(self, dev: "Device", nbytes: int):
        h = C.c_void_p()
        _check(lib().lisa_buffer_alloc(dev.h, nbytes, C.byref(h)))
        self.h, self.nbytes, self.dev = h, nbytes, dev

    @property
    def ptr(self) -> int:
        return lib().lisa_buffer_device_ptr(self.h)

    def write(self, arr: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(arr)
        _check(lib().lisa_buffer_write(self.h, offset, _ptr(a), a.nbytes))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(lib().lisa_buffer_read(self.h, offset, _ptr(out), out.nbytes))
        return out

    def free(self) -> None:
        if self.h:
            lib().lisa_buffer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Device:
    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        _check(lib().lisa_device_create(ordinal, C.byref(h)))
        self.h = h
        m = C.c_void_p()
        _check(lib().lisa_module_load_default(self.h, C.byref(m)))
        self.module = m
        self._fns: dict[str, C.c_void_p] = {}

    def name(self) -> str:
        buf = C.create_string_buffer(256)
        _check(lib().lisa_device_name(self.h, buf, 256))
        return buf.value.decode()

    def buffer(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        b = Buffer(self, max(a.nbytes, 4))
        b.write(a)
        return b

    def function(self, name: str):
        if name not in self._fns:
            f = C.c_void_p()
            _check(lib().lisa_function_get(self.module, name.encode(), C.byref(f)))
            self._fns[name] = f
        return self._fns[name]

    def synth_fill(self, buf: "Buffer", n: int, kind: int, key: int, key2: int = 0, dist: int = DIST_NORMAL,
                   a: float = 0.0, b: float = 1.0, capacity: int = 0, filled: int = 0) -> None:
        """lisa_synth_fill of n elements of `kind` into buf; refuses on the host
        any fill that would write past the buffer (the kernel has no size)."""
        if kind == FILL_KV:
            if not 0 < filled <= capacity or n != ATT_KVH * filled * ATT_HD:
                raise ValueError(f"KV fill: n={n} filled={filled} capacity={capacity}")
            need = ATT_KVH * capacity * ATT_HD * 2
        elif kind in (FILL_WORDS, FILL_F32, FILL_SB, FILL_BF16):
            need = n * (2 if kind == FILL_BF16 else 4)
        else:
            raise ValueError(f"unknown fill kind {kind}")
        if need > buf.nbytes:
            raise ValueError(f"fill of {need} bytes into a {buf.nbytes}-byte buffer")
        self.dispatch("lisa_synth_fill", SynthParams(buf.ptr, n, key, key2, kind, dist, a, b, capacity, filled),
                      (4096,), (256,))

    def dispatch(self, kernel: str, params: C.Structure, grid, block, wait: bool = True) -> None:
        """One dispatch of a kernel taking one argument block (lisa_kernels.h)."""
        enc = C.c_void_p()
        L = lib()
        _check(L.lisa_encoder_begin(self.h, C.byref(enc)))
        _check(L.lisa_encoder_set_function(enc, self.function(kernel)))
        _check(L.lisa_encoder_set_bytes(enc, 0, C.cast(C.pointer(params), C.c_void_p), C.sizeof(params)))
        gx, gy, gz = (tuple(grid) + (1, 1))[:3]
        tx, ty, tz = (tuple(block) + (1, 1))[:3]
        _check(L.lisa_encoder_dispatch_groups(enc, gx, gy, gz, tx, ty, tz))
        _check(L.lisa_encoder_end(enc, 1 if wait else 0))

    def synchronize(self) -> None:
        _check(lib().lisa_device_synchronize(self.h))

    def attention_decode(self, args: "AttnDecodeArgs", workspace: "Buffer | None" = None, wait: bool = True) -> None:
        """lisa_attention_decode: one decode layer's attention core (config 2)."""
        _check(lib().lisa_attention_decode(self.h, self.module, C.byref(args), workspace.h if workspace else None))
        if wait:
            self.synchronize()

    def attention_decode_noalloc(self, args: "AttnDecodeArgs", wait: bool = True) -> None:
        """lisa_attention_decode_noalloc: the same with the library's fixed scratch."""
        _check(lib().lisa_attention_decode_noalloc(self.h, self.module, C.byref(args)))
        if wait:
            self.synchronize()


# ---------------------------------------------------------------------------
# runner (src/model/runner.rs) and speculative loop (src/speculative/mod.rs)
# ---------------------------------------------------------------------------
@dataclass
class GreedyAcceptance:
    accepted_drafts: int
    emitted: list
    target_trim: int


def accept_greedy(drafts, target_tokens) -> GreedyAcceptance:
    """speculative/mod.rs:16-32."""
    if len(target_tokens) != len(drafts) + 1:
        raise ValueError("target_tokens must have one more entry than drafts")
    d = np.asarray(drafts, dtype=np.uint32)
    t = np.asarray(target_tokens, dtype=np.uint32)
    out = Acceptance()
    _check(lib().lisa_accept_greedy(_ptr(d), len(d), _ptr(t), C.byref(out)))
    return GreedyAcceptance(out.accepted_drafts, [int(x) for x in out.emitted[: out.emitted_count]],
                            out.target_trim)


def mtp_reconcile_plan(draft_count: int, round_appended: int, accepted: int):
    """speculative/mod.rs:49-65; replay entries are ("draft", i) or ("replacement",)."""
    p = ReconcilePlan()
    _check(lib().lisa_mtp_reconcile_plan(draft_count, round_appended, accepted, C.byref(p)))
    replay = [("draft", int(i)) if i >= 0 else ("replacement",) for i in p.replay[: p.replay_count]]
    return p.trim, replay


class WeightIndex:
    """WeightIndex (src/model/weights.rs) over safetensors shards, host-only."""

    def __init__(self, paths=None, snapshot=None):
        h = C.c_void_p()
        if snapshot is not None:
            _check(lib().lisa_weight_index_open_snapshot(str(snapshot).encode(), C.byref(h)))
        else:
            arr = (C.c_char_p * len(paths))(*[str(x).encode() for x in paths])
            _check(lib().lisa_weight_index_open(arr, len(paths), C.byref(h)))
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().lisa_weight_index_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return lib().lisa_weight_index_len(self.h)

    @property
    def shard_count(self) -> int:
        return lib().lisa_weight_index_shard_count(self.h)

    def slot(self, name: str) -> dict:
        s = WeightSlotStruct()
        _check(lib().lisa_weight_index_slot(self.h, name.encode(), C.byref(s)))
        return {"shard": s.shard, "dtype": DTYPES[s.dtype], "shape": [s.shape[i] for i in range(s.ndim)],
                "offset": s.offset, "data_start": s.data_start, "len": s.len}

    def validate(self, layers: int = 0, vocab: int = 0, mtp: bool = False) -> None:
        _check(lib().lisa_weight_index_validate(self.h, layers, vocab, 1 if mtp else 0))


class Runner:
    """QwenRunner + MtpRunner on one MI355X over synthetic q4 weights, or over
    a safetensors checkpoint (Runner.load)."""

    def __init__(self, layers: int = LAYERS, vocab: int = VOCAB, capacity: int = 4352, seed: int = 0x15A2026,
                 with_mtp: bool = False, use_graph: bool = True, device: int = 0, _handle=None):
        if _handle is None:
            cfg = RunnerConfig(layers, vocab, capacity, 1 if with_mtp else 0, seed, 1 if use_graph else 0, device)
            h = C.c_void_p()
            _check(lib().lisa_runner_create(C.byref(cfg), C.byref(h)))
        else:
            h = _handle
        self.h = h
        self.layers, self.vocab, self.capacity, self.seed = layers, vocab, capacity, seed

    @classmethod
    def load(cls, target_snapshot, mtp_snapshot=None, capacity: int = 4352, layers: int = LAYERS,
             vocab: int = VOCAB, use_graph: bool = True, device: int = 0) -> "Runner":
        """QwenRunner::load (+ MtpRunner::load) from snapshot directories."""
        cfg = RunnerConfig(layers, vocab, capacity, 0, 0, 1 if use_graph else 0, device)
        h = C.c_void_p()
        _check(lib().lisa_runner_load(str(target_snapshot).encode(),
                                      None if mtp_snapshot is None else str(mtp_snapshot).encode(),
                                      C.byref(cfg), C.byref(h)))
        return cls(layers, vocab, capacity, 0, mtp_snapshot is not None, use_graph, device, _handle=h)

    def load_mtp(self, mtp_snapshot, capacity: int) -> None:
        """MtpRunner::load(target, snapshot, capacity) into this runner."""
        _check(lib().lisa_mtp_load(self.h, str(mtp_snapshot).encode(), capacity))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().lisa_runner_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        return lib().lisa_runner_position(self.h)

    @property
    def weight_bytes(self) -> int:
        return lib().lisa_runner_weight_bytes(self.h)

    def reset_state(self) -> None:
        """QwenRunner::reset_state: the target's state only."""
        _check(lib().lisa_runner_reset_state(self.h))

    def fill_state(self, filled: int, seed: int) -> None:
        _check(lib().lisa_runner_fill_state(self.h, filled, seed))

    def forward_token_decode(self, token: int, want_hidden: bool = False):
        am = C.c_uint32()
        hidden = np.empty(HIDDEN, np.float32) if want_hidden else None
        _check(lib().lisa_runner_forward_token_decode(self.h, token, C.byref(am),
                                                      _ptr(hidden) if want_hidden else None))
        return (int(am.value), hidden) if want_hidden else int(am.value)

    def forward_token_with_hidden(self, token: int):
        am = C.c_uint32()
        hidden = np.empty(HIDDEN, np.float32)
        logits = np.empty(self.vocab, np.float32)
        _check(lib().lisa_runner_forward_token_with_hidden(self.h, token, C.byref(am), _ptr(hidden), _ptr(logits)))
        return int(am.value), hidden, logits

    def forward_prefill(self, tokens, chunk: int = 0, want_hidden: bool = False):
        """forward_prefill_with_progress (runner.rs:2129-2230): per-position
        argmax (and hidden f32[n][5120]) of the prompt; position += n."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        am = np.zeros(t.size, np.uint32)
        hidden = np.empty((t.size, HIDDEN), np.float32) if want_hidden else None
        _check(lib().lisa_runner_forward_prefill(self.h, _ptr(t), t.size, chunk, _ptr(am),
                                                 _ptr(hidden) if want_hidden else None))
        return (am, hidden) if want_hidden else am

    def decode_greedy(self, token: int, steps: int) -> np.ndarray:
        out = np.zeros(steps, np.uint32)
        _check(lib().lisa_runner_decode_greedy(self.h, token, steps, _ptr(out)))
        return out

    def profile_step(self, token: int, steps: int = 1) -> dict:
        """Eager M=1 steps with hipEvents around every launch: {kind: (total_ms, launches)}."""
        ms = np.zeros(len(KINDS), np.float32)
        cnt = np.zeros(len(KINDS), np.int32)
        _check(lib().lisa_runner_profile_step(self.h, token, steps, _ptr(ms), _ptr(cnt)))
        return {k: (float(ms[i]), int(cnt[i])) for i, k in enumerate(KINDS)}

    def profile_block3(self, tokens) -> dict:
        """One eager M=3 verify pass with hipEvents around every launch: {kind: (total_ms, launches)}."""
        t = np.asarray(tokens, dtype=np.uint32)
        ms = np.zeros(len(KINDS), np.float32)
        cnt = np.zeros(len(KINDS), np.int32)
        _check(lib().lisa_runner_profile_block3(self.h, _ptr(t), _ptr(ms), _ptr(cnt)))
        return {k: (float(ms[i]), int(cnt[i])) for i, k in enumerate(KINDS)}

    def verify_block3(self, tokens, want_hidden: bool = False, want_logits: bool = False):
        t = np.asarray(tokens, dtype=np.uint32)
        am = np.zeros(3, np.uint32)
        hidden = np.empty(3 * HIDDEN, np.float32) if want_hidden else None
        logits = np.empty(3 * self.vocab, np.float32) if want_logits else None
        _check(lib().lisa_runner_verify_block3(self.h, _ptr(t), _ptr(am),
                                               _ptr(hidden) if want_hidden else None,
                                               _ptr(logits) if want_logits else None))
        res = [am]
        if want_hidden:
            res.append(hidden.reshape(3, HIDDEN))
        if want_logits:
            res.append(logits.reshape(3, self.vocab))
        return res[0] if len(res) == 1 else tuple(res)

    def commit_verified_prefix(self, rows: int) -> None:
        _check(lib().lisa_runner_commit_verified_prefix(self.h, rows))

    def checkpoint_state(self):
        ck = C.c_void_p()
        _check(lib().lisa_runner_checkpoint_state(self.h, C.byref(ck)))
        return ck

    def restore_state(self, ck) -> None:
        _check(lib().lisa_runner_restore_state(self.h, ck))

    def free_checkpoint(self, ck) -> None:
        lib().lisa_checkpoint_free(ck)

    def upload_hidden(self, row: int, hidden: np.ndarray) -> None:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        _check(lib().lisa_runner_upload_hidden(self.h, row, _ptr(h)))

    def gdn_state(self, idx: int) -> np.ndarray:
        out = np.empty(GDN_STATE, np.float32)
        _check(lib().lisa_runner_read_gdn_state(self.h, idx, _ptr(out)))
        return out

    def conv_state(self, idx: int) -> np.ndarray:
        out = np.empty(3 * GDN_CONV_DIM, np.uint16)
        _check(lib().lisa_runner_read_conv_state(self.h, idx, _ptr(out)))
        return out

    # ---- drafter -------------------------------------------------------------
    def mtp_forward(self, token: int, cond_source: int, cond_row: int = 0) -> int:
        am = C.c_uint32()
        _check(lib().lisa_mtp_forward(self.h, token, cond_source, cond_row, C.byref(am)))
        return int(am.value)

    def mtp_upload_cond(self, hidden_bf16: np.ndarray) -> None:
        h = np.ascontiguousarray(hidden_bf16, dtype=np.uint16)
        _check(lib().lisa_mtp_upload_cond(self.h, _ptr(h)))

    def mtp_upload_normalized(self, hidden: np.ndarray) -> None:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        _check(lib().lisa_mtp_upload_normalized(self.h, _ptr(h)))

    def mtp_normalized(self) -> np.ndarray:
        out = np.empty(HIDDEN, np.uint16)
        _check(lib().lisa_mtp_read_normalized(self.h, _ptr(out)))
        return out

    @property
    def mtp_position(self) -> int:
        return lib().lisa_mtp_position(self.h)

    def mtp_trim_state(self, count: int) -> None:
        _check(lib().lisa_mtp_trim_state(self.h, count))

    def mtp_reset_state(self) -> None:
        """MtpRunner::reset_state: the drafter's K/V and position only."""
        _check(lib().lisa_mtp_reset_state(self.h))

    def mtp_forward_device(self, token: int, cond_is_target: bool, cond_off: int):
        """forward_position_decode_device addressed by (buffer, byte offset):
        returns (argmax, normalized_offset)."""
        am, off = C.c_uint32(), C.c_uint64()
        _check(lib().lisa_mtp_forward_device(self.h, token, 1 if cond_is_target else 0, cond_off, C.byref(am),
                                             C.byref(off)))
        return int(am.value), int(off.value)

    def mtp_forward_position_decode(self, token: int, hidden: np.ndarray):
        """forward_position_decode (runner.rs:2618-2680): (argmax, normalized f32[5120])."""
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        am = C.c_uint32()
        xn = np.empty(HIDDEN, np.float32)
        _check(lib().lisa_mtp_forward_position_decode(self.h, token, _ptr(h), C.byref(am), _ptr(xn)))
        return int(am.value), xn

    def mtp_forward_batch(self, tokens, hiddens, chunk: int = 0):
        """forward_position_batch_with_progress (runner.rs:3494-3581):
        (argmax[n], normalized f32[n][5120])."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        h = np.ascontiguousarray(hiddens, dtype=np.float32).reshape(t.size, HIDDEN)
        am = np.zeros(t.size, np.uint32)
        xn = np.empty((t.size, HIDDEN), np.float32)
        _check(lib().lisa_mtp_forward_batch(self.h, _ptr(t), _ptr(h), t.size, chunk, _ptr(am), _ptr(xn)))
        return am, xn

    def prefill_prompt(self, prompt, start: int = 0):
        """prefill_prompt_from (speculative/mod.rs:237-311): (bonus, target_hidden,
        (mtp_seed_token, mtp_seed_hidden))."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        bonus, seed = C.c_uint32(), C.c_uint32()
        th = np.empty(HIDDEN, np.float32)
        sh = np.empty(HIDDEN, np.float32)
        _check(lib().lisa_prefill_prompt(self.h, _ptr(p), p.size, start, C.byref(bonus), _ptr(th), C.byref(seed),
                                         _ptr(sh)))
        return int(bonus.value), th, (int(seed.value), sh)

    def mtp_checkpoint_state(self):
        """MtpRunner::checkpoint_state (runner.rs:2382-2398)."""
        ck = C.c_void_p()
        _check(lib().lisa_mtp_checkpoint_state(self.h, C.byref(ck)))
        return ck

    def mtp_restore_state(self, ck) -> None:
        """MtpRunner::restore_state (runner.rs:2400-2420)."""
        _check(lib().lisa_mtp_restore_state(self.h, ck))

    def free_mtp_checkpoint(self, ck) -> None:
        lib().lisa_mtp_checkpoint_free(ck)

    def generate_greedy_block3(self, bonus: int, target_hidden: np.ndarray, mtp_seed_token: int,
                               mtp_seed_hidden: np.ndarray, max_tokens: int, force_truth=None,
                               force_seed: int = 0, p_accept: float = 0.6):
        th = np.ascontiguousarray(target_hidden, dtype=np.float32)
        sh = np.ascontiguousarray(mtp_seed_hidden, dtype=np.float32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        stats = SpecStats()
        ft = None if force_truth is None else np.ascontiguousarray(force_truth, dtype=np.uint32)
        _check(lib().lisa_generate_greedy_block3(self.h, bonus, _ptr(th), mtp_seed_token, _ptr(sh), max_tokens,
                                                 _ptr(ft) if ft is not None else None,
                                                 0 if ft is None else len(ft), force_seed, p_accept, _ptr(out),
                                                 C.byref(stats)))
        return out[:max_tokens], {"rounds": stats.rounds, "accepted_drafts": stats.accepted_drafts,
                                  "drafted_tokens": stats.drafted_tokens, "target_forwards": stats.target_forwards}


def hidden_offset(row: int) -> int:
    """QwenRunner::hidden_offset (runner.rs:846-848) of the C ABI."""
    return int(lib().lisa_runner_hidden_offset(row))


def normalized_offset() -> int:
    """MtpRunner::normalized_offset (runner.rs:2689-2692) of the C ABI."""
    return int(lib().lisa_mtp_normalized_offset())


def resolve_cond(cond_is_target: bool, cond_off: int):
    """(cond_source, cond_row) of lisa_mtp_forward for a (buffer, offset) pair."""
    src, row = C.c_int32(), C.c_int32()
    _check(lib().lisa_mtp_resolve_cond(1 if cond_is_target else 0, cond_off, C.byref(src), C.byref(row)))
    return int(src.value), int(row.value)


def stream_key(seed: int, tensor_id: int) -> int:
    """lisa_synth.h lisa_stream_key, for tests that fill buffers directly."""
    M = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    return mix(seed ^ mix((tensor_id * 0x100000001B3 + 0xCBF29CE484222325) & M))


def tensor_id(scope: int, kind: int, part: int) -> int:
    return (scope << 12) | (kind << 2) | part
