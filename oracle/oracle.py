"""ctypes binding of the CPU oracle (oracle/_build/liblisa_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker — never by the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "liblisa_oracle.so"

_P = C.c_void_p
_SIGS = {
    "orc_q4_linear": (None, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, _P]),
    "orc_rms_norm": (None, [_P, _P, C.c_int, _P]),
    "orc_rms_norm_tiles": (None, [_P, _P, C.c_int, _P]),
    "orc_q4_gemm": (None, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P]),
    "orc_set_gemm_order": (None, [C.c_int]),
    "orc_model_prefill": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P]),
    "orc_residual": (None, [_P, _P, C.c_int, _P]),
    "orc_embed": (None, [_P, _P, _P, C.c_uint32, C.c_int, _P]),
    "orc_silu_mul": (None, [_P, _P, C.c_int, _P]),
    "orc_gdn_conv": (None, [_P, _P, _P, C.c_int, _P, _P]),
    "orc_gdn_recurrence": (None, [_P, _P, _P, _P, _P, _P, _P, _P, C.c_int, _P, _P, _P]),
    "orc_head_norm_rope": (None, [_P, _P, C.c_uint32, _P]),
    "orc_attention": (None, [_P, _P, _P, _P, _P, _P, _P, C.c_uint32, C.c_uint32, C.c_int, _P]),
    "orc_sdpa": (None, [_P, _P, _P, C.c_uint32, C.c_uint32, C.c_int, _P]),
    "orc_math": (None, [C.c_int, _P, C.c_size_t, _P]),
    "orc_argmax": (C.c_uint32, [_P, C.c_int]),
    "orc_model_create": (_P, [C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_int]),
    "orc_model_free": (None, [_P]),
    "orc_model_position": (C.c_uint32, [_P]),
    "orc_threads": (C.c_int, []),
    "orc_layer_is_attention": (C.c_int, [C.c_int]),
    "orc_model_fill_state": (None, [_P, C.c_uint32, C.c_uint64]),
    "orc_model_reset": (None, [_P]),
    "orc_model_forward": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P, _P]),
    "orc_model_commit": (C.c_int, [_P, C.c_int]),
    "orc_mtp_forward": (C.c_int, [_P, C.c_uint32, _P, _P, _P]),
    "orc_mtp_position": (C.c_uint32, [_P]),
    "orc_mtp_trim": (C.c_int, [_P, C.c_int]),
    "orc_mtp_prefill": (C.c_int, [_P, _P, _P, C.c_int, _P, _P]),
    "orc_model_tensor": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.POINTER(_P), C.POINTER(C.c_size_t)]),
    "orc_synth_bf16": (None, [C.c_uint64, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_size_t, _P]),
    "orc_synth_f32": (None, [C.c_uint64, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_size_t, _P]),
    "orc_synth_words": (None, [C.c_uint64, C.c_uint64, C.c_size_t, _P]),
}
_LIB = None

def _tensor_kinds():
    """LISA_T_* of include/lisa_model.h (the synthetic tensor catalogue), by name."""
    import re
    text = (ORACLE_DIR.parent / "include" / "lisa_model.h").read_text()
    body = re.search(r"enum \{\s*(LISA_T_INPUT_NORM = 1,.*?)\};", text, re.S).group(1)
    names = re.findall(r"(LISA_T_\w+)", body)
    kinds = {n[len("LISA_T_"):]: i + 1 for i, n in enumerate(names)}
    scope_mtp = int(re.search(r"#define LISA_SCOPE_MTP (\d+)", text).group(1))
    return kinds, scope_mtp


T, SCOPE_MTP = _tensor_kinds()

MATH = {"exp": 0, "exp2": 1, "log": 2, "sin": 3, "cos": 4, "rsqrt": 5, "bf16": 6, "silu_exp": 7,
        "softplus": 8, "sigmoid_exp": 9, "silu_exp2": 10, "sigmoid_exp2": 11}
DIST_UNIFORM, DIST_NORMAL = 1, 2


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def p(a):
    return None if a is None else np.ascontiguousarray(a).ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def q4_linear(x_bf16, w, scales, biases, n, k, m=1, ksplit=1):
    x = _c(x_bf16, np.uint16)
    w, s, b = _c(w, np.uint32), _c(scales, np.uint16), _c(biases, np.uint16)
    out = np.empty(m * n, np.float32)
    lib().orc_q4_linear(p(x), p(w), p(s), p(b), n, k, m, ksplit, p(out))
    return out.reshape(m, n)


def q4_gemm(a_bf16, w, scales, biases, n, k, m):
    """Prefill GEMM: f32 [m][n] of bf16 rows a[m][k] against bf16(fma(s, q, b)) weights."""
    out = np.empty(m * n, np.float32)
    lib().orc_q4_gemm(p(_c(a_bf16, np.uint16)), p(_c(w, np.uint32)), p(_c(scales, np.uint16)),
                      p(_c(biases, np.uint16)), n, k, m, p(out))
    return out.reshape(m, n)


def set_gemm_order(order):
    """0: the MFMA's order (f32 per 8 k, default); 1: double sum, one rounding."""
    lib().orc_set_gemm_order(order)


def residual(x_bf16, o_f32):
    x = _c(x_bf16, np.uint16)
    out = np.empty_like(x)
    lib().orc_residual(p(x), p(_c(o_f32, np.float32)), x.size, p(out))
    return out


def embed(w, scales, biases, token, hidden=5120):
    out = np.empty(hidden, np.uint16)
    lib().orc_embed(p(_c(w, np.uint32)), p(_c(scales, np.uint16)), p(_c(biases, np.uint16)), token, hidden, p(out))
    return out


def silu_mul(g_f32, u_f32):
    g = _c(g_f32, np.float32)
    out = np.empty(g.size, np.uint16)
    lib().orc_silu_mul(p(g), p(_c(u_f32, np.float32)), g.size, p(out))
    return out


def rms_norm(x_bf16, w_bf16):
    x = _c(x_bf16, np.uint16)
    out = np.empty_like(x)
    lib().orc_rms_norm(p(x), p(_c(w_bf16, np.uint16)), x.size, p(out))
    return out


def rms_norm_tiles(x_bf16, w_bf16):
    """RMSNorm with the statistic from 8-row tile partials (decode norms after a residual add)."""
    x = _c(x_bf16, np.uint16)
    out = np.empty_like(x)
    lib().orc_rms_norm_tiles(p(x), p(_c(w_bf16, np.uint16)), x.size, p(out))
    return out


def math(fn: str, x):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_math(MATH[fn], p(x), x.size, p(out))
    return out


def threads():
    return int(lib().orc_threads())


def layer_is_attention(i):
    return bool(lib().orc_layer_is_attention(i))


def argmax(v):
    v = _c(v, np.float32)
    return int(lib().orc_argmax(p(v), v.size))


def sdpa(query_bf16, key_cache, value_cache, capacity, base, m):
    out = np.empty(m * 24 * 256, np.float32)
    lib().orc_sdpa(p(_c(query_bf16, np.uint16)), p(_c(key_cache, np.uint16)), p(_c(value_cache, np.uint16)),
                   capacity, base, m, p(out))
    return out.reshape(m, 24, 256)


def gdn_conv(qkv, conv_w, conv_state, m, slots=False):
    cs = _c(conv_state, np.uint16).copy()
    out = np.empty(m * 10240, np.float32)
    sl = np.zeros(m * 3 * 10240, np.uint16) if slots else None
    lib().orc_gdn_conv(p(_c(qkv, np.float32)), p(_c(conv_w, np.uint16)), p(cs), m, p(out), p(sl))
    return out.reshape(m, 10240), cs, sl


def gdn_recurrence(conv_out, z, a, b, a_log, dt_bias, norm_w, state, m, slots=False):
    st = _c(state, np.float32).copy()
    gated = np.empty(m * 6144, np.uint16)
    y = np.empty(m * 6144, np.float32)
    sl = np.zeros(m * 48 * 128 * 128, np.float32) if slots else None
    lib().orc_gdn_recurrence(p(_c(conv_out, np.float32)), p(_c(z, np.float32)), p(_c(a, np.float32)),
                             p(_c(b, np.float32)), p(_c(a_log, np.uint16)), p(_c(dt_bias, np.uint16)),
                             p(_c(norm_w, np.uint16)), p(st), m, p(gated), p(sl), p(y))
    return gated.reshape(m, 6144), st, y.reshape(m, 6144), sl


def head_norm_rope(raw, w, position):
    out = np.empty(256, np.uint16)
    lib().orc_head_norm_rope(p(_c(raw, np.float32)), p(_c(w, np.uint16)), position, p(out))
    return out


def attention(q_proj, k_raw, v_raw, q_norm_w, k_norm_w, key_cache, value_cache, capacity, base, m):
    kc = _c(key_cache, np.uint16).copy()
    vc = _c(value_cache, np.uint16).copy()
    gated = np.empty(m * 6144, np.uint16)
    lib().orc_attention(p(_c(q_proj, np.float32)), p(_c(k_raw, np.float32)), p(_c(v_raw, np.float32)),
                        p(_c(q_norm_w, np.uint16)), p(_c(k_norm_w, np.uint16)), p(kc), p(vc), capacity, base, m,
                        p(gated))
    return gated.reshape(m, 6144), kc, vc


def synth_bf16(seed, tid, dist, a, b, n):
    out = np.empty(n, np.uint16)
    lib().orc_synth_bf16(seed, tid, dist, a, b, n, p(out))
    return out


def synth_f32(seed, tid, dist, a, b, n):
    out = np.empty(n, np.float32)
    lib().orc_synth_f32(seed, tid, dist, a, b, n, p(out))
    return out


def synth_words(seed, tid, n):
    out = np.empty(n, np.uint32)
    lib().orc_synth_words(seed, tid, n, p(out))
    return out


class Model:
    """CPU restatement of QwenRunner/MtpRunner over the same synthetic weights."""

    def __init__(self, layers, vocab, capacity, seed, with_mtp=False):
        self.h = lib().orc_model_create(layers, vocab, capacity, seed, 1 if with_mtp else 0)
        if not self.h:
            raise ValueError("bad oracle model configuration")
        self.vocab = vocab

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self):
        return lib().orc_model_position(self.h)

    def fill_state(self, filled, seed):
        lib().orc_model_fill_state(self.h, filled, seed)

    def reset(self):
        lib().orc_model_reset(self.h)

    def forward(self, tokens, capture=False, want_logits=False):
        t = _c(tokens, np.uint32)
        m = t.size
        am = np.zeros(m, np.uint32)
        hidden = np.empty(m * 5120, np.float32)
        logits = np.empty(m * self.vocab, np.float32) if want_logits else None
        rc = lib().orc_model_forward(self.h, p(t), m, 1 if capture else 0, p(am), p(hidden), p(logits))
        if rc:
            raise RuntimeError(f"oracle forward failed ({rc})")
        if want_logits:
            return am, hidden.reshape(m, 5120), logits.reshape(m, self.vocab)
        return am, hidden.reshape(m, 5120)

    def prefill(self, tokens, chunk=0, want_hidden=False):
        t = _c(tokens, np.uint32)
        am = np.zeros(t.size, np.uint32)
        hidden = np.empty((t.size, 5120), np.float32) if want_hidden else None
        rc = lib().orc_model_prefill(self.h, p(t), t.size, chunk, p(am), p(hidden))
        if rc:
            raise RuntimeError(f"oracle prefill failed ({rc})")
        return (am, hidden) if want_hidden else am

    def commit(self, rows):
        rc = lib().orc_model_commit(self.h, rows)
        if rc:
            raise RuntimeError(f"oracle commit failed ({rc})")

    def mtp_forward(self, token, cond_bf16):
        am = np.zeros(1, np.uint32)
        xn = np.empty(5120, np.uint16)
        rc = lib().orc_mtp_forward(self.h, token, p(_c(cond_bf16, np.uint16)), p(am), p(xn))
        if rc:
            raise RuntimeError(f"oracle mtp forward failed ({rc})")
        return int(am[0]), xn

    def mtp_prefill(self, tokens, hiddens):
        """MtpRunner::forward_position_batch: (argmax[n], normalized bf16[n][5120])."""
        t = _c(tokens, np.uint32)
        h = _c(hiddens, np.float32).reshape(t.size, 5120)
        am = np.zeros(t.size, np.uint32)
        xn = np.empty((t.size, 5120), np.uint16)
        rc = lib().orc_mtp_prefill(self.h, p(t), p(h), t.size, p(am), p(xn))
        if rc:
            raise RuntimeError(f"oracle mtp prefill failed ({rc})")
        return am, xn

    @property
    def mtp_position(self):
        return lib().orc_mtp_position(self.h)

    def mtp_trim(self, count):
        if lib().orc_mtp_trim(self.h, count):
            raise RuntimeError("bad trim")

    def tensor(self, scope, kind, part, dtype):
        """A writable numpy view of one model tensor (orc_model_tensor); the
        view is valid while the model lives."""
        ptr, nbytes = C.c_void_p(), C.c_size_t()
        rc = lib().orc_model_tensor(self.h, scope, kind, part, C.byref(ptr), C.byref(nbytes))
        if rc:
            raise KeyError(f"no tensor scope={scope} kind={kind} part={part} ({rc})")
        count = nbytes.value // np.dtype(dtype).itemsize
        buf = (C.c_char * nbytes.value).from_address(ptr.value)
        return np.frombuffer(buf, dtype=dtype, count=count)


# ---- host-side helpers shared by tests ----------------------------------------
def bf16_bits_to_f32(h):
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """Round to nearest even (NaN kept quiet), as lisa_f32_to_bf16."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def f32_to_bf16_trunc(x):
    """src/format/dtype.rs:42-47 (truncation)."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
