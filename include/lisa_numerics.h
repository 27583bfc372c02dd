/*
 * lisa_numerics.h — the scalar numerics contract of the decode path.
 *
 * Every rounding point and every transcendental used by the HIP kernels is
 * defined here once, in terms of IEEE-754 operations that are correctly
 * rounded on both the x86-64 host (SSE/FMA) and gfx950 (v_fma_f32, the
 * correctly-rounded f32 divide/sqrt sequences hipcc emits by default):
 * add, sub, mul, fma, div, sqrt, rint and bit manipulation. Built with
 * -ffp-contract=off on both sides, the same source therefore produces the same
 * bits on the CPU and on the GPU, which is what lets the GPU decode path be
 * compared bit-for-bit with a CPU evaluation of the same formulas.
 *
 * The reference compiles its Metal kernels with fast-math
 * (src/device/metal.rs:440-448), so its exp/log/rsqrt/sin/cos are only
 * ULP-accurate; the functions below are accurate to a few ULP (checked against
 * double-precision libm in tests/test_numerics.py) and follow textbook methods:
 * Cody-Waite additive range reduction followed by truncated Taylor series.
 */
#ifndef LISA_NUMERICS_H
#define LISA_NUMERICS_H

#include <stdint.h>

#if defined(__HIPCC__)
#define LISA_HD __host__ __device__ __forceinline__
#else
#define LISA_HD static inline
#endif

/* ---- bit casts and bf16 ------------------------------------------------- */

LISA_HD uint32_t lisa_f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
LISA_HD float lisa_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

/* bf16 bits -> f32 (exact). src/format/dtype.rs:36-40 */
LISA_HD float lisa_bf16_to_f32(uint16_t h) { return lisa_u2f((uint32_t)h << 16); }

/* f32 -> bf16 bits, round to nearest even; NaN stays NaN (quieted).
 * This is the in-kernel `bfloat(x)` conversion of the Metal shaders, which the
 * reference's own test models as RNE (tests/gdn_state.rs:7-11). */
#if defined(__HIP_DEVICE_COMPILE__)
/* gfx950 converts in hardware (v_cvt_pk_bf16_f32, round to nearest even). It
 * equals the bit arithmetic below for every non-NaN f32 and keeps NaN a NaN
 * (checked over all 2^32 inputs on an MI355X); only NaN payloads may differ. */
LISA_HD uint16_t lisa_f32_to_bf16(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
/* Two values packed lo | hi << 16 in one instruction. */
LISA_HD uint32_t lisa_f32x2_to_bf16x2(float lo, float hi) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}
#else
LISA_HD uint16_t lisa_f32_to_bf16(float x) {
  uint32_t u = lisa_f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
LISA_HD uint32_t lisa_f32x2_to_bf16x2(float lo, float hi) {
  return (uint32_t)lisa_f32_to_bf16(lo) | ((uint32_t)lisa_f32_to_bf16(hi) << 16);
}
#endif

/* float(bfloat(x)): round an f32 to the nearest bf16 value, kept as f32. */
LISA_HD float lisa_bf16r(float x) { return lisa_bf16_to_f32(lisa_f32_to_bf16(x)); }

/* Host-side truncating conversion (src/format/dtype.rs:42-47), used where the
 * reference uploads host f32 hiddens as bf16 (runner.rs:852-858). */
LISA_HD uint16_t lisa_f32_to_bf16_trunc(float x) { return (uint16_t)(lisa_f2u(x) >> 16); }

/* ---- basic correctly rounded helpers ------------------------------------ */

LISA_HD float lisa_fma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
LISA_HD float lisa_rint(float x) { return __builtin_rintf(x); }
LISA_HD float lisa_sqrt(float x) { return __builtin_sqrtf(x); }
/* rsqrt(v) evaluated as 1/sqrt(v): two correctly rounded operations. */
LISA_HD float lisa_rsqrt(float v) { return 1.0f / __builtin_sqrtf(v); }

/* 2^n as a float for integer n in [-126, 127]. */
LISA_HD float lisa_pow2i(int n) { return lisa_u2f((uint32_t)(n + 127) << 23); }

/* p * 2^n for n in [-151, 128] without overflow of the exponent field; one
 * rounding at most (only when the result is subnormal). */
LISA_HD float lisa_ldexp(float p, int n) {
  if (n > 127) return p * lisa_pow2i(127) * lisa_pow2i(n - 127);
  if (n < -126) return p * lisa_pow2i(n + 64) * lisa_pow2i(-64);
  return p * lisa_pow2i(n);
}

/* ---- exp / exp2 ---------------------------------------------------------
 * Cody-Waite: n = rint(x/ln2), r = x - n*ln2 (two-term ln2 with fma),
 * e^r by the degree-7 Taylor series on |r| <= 0.347, then scale by 2^n. */
LISA_HD float lisa_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return lisa_u2f(0x7f800000u);
  if (x < -103.97908782958984f) return 0.0f;
  const float n = lisa_rint(x * 1.44269502162933349609375f);
  float r = lisa_fma(-n, 0.693145751953125f, x);
  r = lisa_fma(-n, 1.428606765330187045037746429443359375e-06f, r);
  float p = 1.984126984126984e-04f;              /* 1/5040 */
  p = lisa_fma(p, r, 1.388888888888889e-03f);    /* 1/720 */
  p = lisa_fma(p, r, 8.333333333333333e-03f);    /* 1/120 */
  p = lisa_fma(p, r, 4.166666666666667e-02f);    /* 1/24 */
  p = lisa_fma(p, r, 1.666666666666667e-01f);    /* 1/6 */
  p = lisa_fma(p, r, 0.5f);
  p = lisa_fma(p, r, 1.0f);
  p = lisa_fma(p, r, 1.0f);
  return lisa_ldexp(p, (int)n);
}

/* 2^x: n = rint(x), f = x - n exact, 2^f = e^(f*ln2) by the same series. */
LISA_HD float lisa_exp2f(float x) {
  if (x != x) return x;
  if (x >= 128.0f) return lisa_u2f(0x7f800000u);
  if (x < -150.0f) return 0.0f;
  const float n = lisa_rint(x);
  const float f = x - n; /* exact: |f| <= 0.5 and x, n share an exponent range */
  /* r = f*ln2 with a two-term ln2 so that r carries ~36 bits */
  const float rh = f * 0.693145751953125f;        /* exact: ln2_hi has 12 bits */
  const float r = lisa_fma(f, 1.428606765330187045037746429443359375e-06f, rh);
  float p = 1.984126984126984e-04f;
  p = lisa_fma(p, r, 1.388888888888889e-03f);
  p = lisa_fma(p, r, 8.333333333333333e-03f);
  p = lisa_fma(p, r, 4.166666666666667e-02f);
  p = lisa_fma(p, r, 1.666666666666667e-01f);
  p = lisa_fma(p, r, 0.5f);
  p = lisa_fma(p, r, 1.0f);
  p = lisa_fma(p, r, 1.0f);
  return lisa_ldexp(p, (int)n);
}

/* ---- log ----------------------------------------------------------------
 * y = m * 2^e with m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s),
 * s = (m-1)/(m+1), by the odd series through s^11; log y = e*ln2 + log m.
 * Defined for finite y > 0 (the only use is softplus, y = 1 + e^x >= 1). */
LISA_HD float lisa_logf(float y) {
  if (!(y > 0.0f)) return (y == 0.0f) ? lisa_u2f(0xff800000u) : lisa_u2f(0x7fc00000u);
  if (y == lisa_u2f(0x7f800000u)) return y;
  uint32_t u = lisa_f2u(y);
  int e = 0;
  if (u < 0x00800000u) { /* subnormal: scale up by 2^32 */
    y = y * 4294967296.0f;
    u = lisa_f2u(y);
    e = -32;
  }
  e += (int)(u >> 23) - 127;
  float m = lisa_u2f((u & 0x007fffffu) | 0x3f800000u); /* [1,2) */
  if (m > 1.41421353816986083984375f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 9.0909090909090909e-02f;        /* 1/11 */
  p = lisa_fma(p, s2, 1.1111111111111111e-01f); /* 1/9 */
  p = lisa_fma(p, s2, 1.4285714285714285e-01f); /* 1/7 */
  p = lisa_fma(p, s2, 2.0000000298023224e-01f); /* 1/5 */
  p = lisa_fma(p, s2, 3.3333334326744080e-01f); /* 1/3 */
  p = p * s2;
  const float logm = lisa_fma(2.0f * s, p, 2.0f * s);
  const float ef = (float)e;
  return lisa_fma(ef, 0.693145751953125f,
                  lisa_fma(ef, 1.428606765330187045037746429443359375e-06f, logm));
}

/* ---- sin / cos ----------------------------------------------------------
 * k = rint(a*2/pi), r = a - k*pi/2 with a three-term pi/2 (Cody-Waite), then
 * Taylor series on |r| <= pi/4 and quadrant selection. Accurate for the
 * RoPE range |a| <= 2^20. */
LISA_HD void lisa_sincosf(float a, float* s_out, float* c_out) {
  const float k = lisa_rint(a * 0.636619746685028076171875f);
  float r = lisa_fma(-k, 1.57079637050628662109375f, a);
  r = lisa_fma(-k, -4.37113882867379730665497481822967529296875e-08f, r);
  r = lisa_fma(-k, -1.7151245100059375e-15f, r);
  const float r2 = r * r;
  float sp = 2.7557319223985893e-06f;            /* 1/9! */
  sp = lisa_fma(sp, r2, -1.9841269841269841e-04f);  /* -1/7! */
  sp = lisa_fma(sp, r2, 8.3333333333333332e-03f);   /* 1/5! */
  sp = lisa_fma(sp, r2, -1.6666666666666666e-01f);  /* -1/3! */
  const float sr = lisa_fma(sp * r2, r, r);
  float cp = -2.7557319223985888e-07f;           /* -1/10! */
  cp = lisa_fma(cp, r2, 2.4801587301587302e-05f);   /* 1/8! */
  cp = lisa_fma(cp, r2, -1.3888888888888889e-03f);  /* -1/6! */
  cp = lisa_fma(cp, r2, 4.1666666666666664e-02f);   /* 1/4! */
  cp = lisa_fma(cp, r2, -0.5f);
  const float cr = lisa_fma(cp, r2, 1.0f);
  const int q = ((int)k) & 3;
  float s, c;
  if (q == 0) { s = sr; c = cr; }
  else if (q == 1) { s = cr; c = -sr; }
  else if (q == 2) { s = -sr; c = -cr; }
  else { s = -cr; c = sr; }
  *s_out = s;
  *c_out = c;
}

/* ---- activation helpers, written exactly as the shaders write them ------ */

/* gdn.metal:16  silu(x) = x / (1 + exp(-x)) */
LISA_HD float lisa_silu_exp(float x) { return x / (1.0f + lisa_expf(-x)); }
/* gdn.metal:17-19  softplus(x) = x > 20 ? x : log(1 + exp(x)) */
LISA_HD float lisa_softplus(float x) { return (x > 20.0f) ? x : lisa_logf(1.0f + lisa_expf(x)); }
/* gdn.metal:200  sigmoid(x) = 1 / (1 + exp(-x)) */
LISA_HD float lisa_sigmoid_exp(float x) { return 1.0f / (1.0f + lisa_expf(-x)); }
/* mlp.metal:14  silu(g) = g / (1 + exp2(-log2(e) g)) */
LISA_HD float lisa_silu_exp2(float g) {
  return g / (1.0f + lisa_exp2f(-1.4426950408889634f * g));
}
/* attention.metal:528  sigmoid(g) = 1 / (1 + exp2(-log2(e) g)) */
LISA_HD float lisa_sigmoid_exp2(float g) {
  return 1.0f / (1.0f + lisa_exp2f(-1.4426950408889634f * g));
}

/* ---- RoPE inverse frequencies -------------------------------------------
 * inv_freq[j] = 1 / 1e7^(2j/64), j < 32 (attention.metal:147, theta 1e7,
 * rotary dims [0,64), NeoX pairs (j, j+32)); each entry is the f32 nearest to
 * the double-precision value, written out in hex so no libm pow is involved. */
#define LISA_ROPE_PAIRS 32
#define LISA_ROPE_INV_FREQ_TABLE                                             \
  { 0x1.000000p+0f, 0x1.356656p-1f, 0x1.75f034p-2f, 0x1.c3f06cp-3f,         \
    0x1.111aeep-3f, 0x1.4a12aep-4f, 0x1.8eec7ep-5f, 0x1.e222ecp-6f,         \
    0x1.235a72p-6f, 0x1.6020a4p-7f, 0x1.a99428p-8f, 0x1.012cfap-8f,         \
    0x1.36d21ap-9f, 0x1.77a7d8p-10f, 0x1.c603c4p-11f, 0x1.125c04p-11f,      \
    0x1.4b96bep-12f, 0x1.90c182p-13f, 0x1.e459c6p-14f, 0x1.24b0fep-14f,     \
    0x1.61bea2p-15f, 0x1.ab8884p-16f, 0x1.025b58p-16f, 0x1.383f88p-17f,     \
    0x1.796182p-18f, 0x1.c8198cp-19f, 0x1.139e96p-19f, 0x1.4d1c98p-20f,     \
    0x1.9298acp-21f, 0x1.e69338p-22f, 0x1.26091cp-22f, 0x1.635e88p-23f }

#endif /* LISA_NUMERICS_H */
