// oracle.cpp — CPU oracle of the lisa-rs decode path. TEST INFRASTRUCTURE:
// loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
//
// Every function restates the reference's Metal arithmetic (file:line cited)
// with the evaluation order fixed: which products are fused (fma), the order
// of every sum, and the reduction trees. The HIP kernels evaluate the same
// expressions in the same order, so agreement is bit-exact; agreement with
// the reference itself is pinned by the reference's own known-answer tests
// restated in tests/test_oracle.py (tolerance-based, as Metal uses fast-math).
//
// Reduction trees used throughout (names used in comments below):
//   tree64(v[64])  : xor butterfly over 64 lanes, masks 32,16,8,4,2,1,
//                    v'[i] = v[i] + v[i^m]; result v[0].
//   tree16(v[16])  : the same over 16 lanes, masks 8,4,2,1.
//   rows-of-256    : thread t (0..255) sums its elements t, t+256, ...
//                    sequentially (s = s + x*x), tree64 per 64-thread wave,
//                    then (W0 + W1) + (W2 + W3).
//   tree128        : lane l (0..63) holds v[l]^2 + v[l+64]^2, then tree64.
#include "oracle.h"

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../include/lisa_model.h"
#include "../include/lisa_numerics.h"
#include "../include/lisa_synth.h"

namespace {

inline float bf(uint16_t h) { return lisa_bf16_to_f32(h); }
inline uint16_t tobf(float x) { return lisa_f32_to_bf16(x); }
inline float bfr(float x) { return lisa_bf16r(x); }

float tree_xor(float* v, int n) {
  for (int m = n / 2; m >= 1; m >>= 1) {
    float t[64];
    for (int i = 0; i < n; ++i) t[i] = v[i] + v[i ^ m];
    std::memcpy(v, t, sizeof(float) * n);
  }
  return v[0];
}

// Ascending-distance butterfly: pairs at distance 1, then 2, 4, ..., n/2.
float tree_asc(float* v, int n) {
  for (int m = 1; m < n; m <<= 1) {
    float t[64];
    for (int i = 0; i < n; ++i) t[i] = v[i] + v[i ^ m];
    std::memcpy(v, t, sizeof(float) * n);
  }
  return v[0];
}

// Sum of squares of `cols` values (multiple of 8) as the q4 prologue of the
// HIP path computes it: thread t of 256 owns the 8-element chunks t, t+256, ...
// and sums their squares in element order; tree64 per wave of 64 threads;
// (W0 + W1) + (W2 + W3). Same statistic as norm.metal:10-47, different
// element-to-thread assignment.
float sumsq_chunks8(const float* x, int cols) {
  float lanes[256];
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int c = t; c < cols / 8; c += 256)
      for (int e = 0; e < 8; ++e) s = s + x[8 * c + e] * x[8 * c + e];
    lanes[t] = s;
  }
  float w[4];
  for (int q = 0; q < 4; ++q) w[q] = tree_xor(lanes + 64 * q, 64);
  return (w[0] + w[1]) + (w[2] + w[3]);
}

// Sum of squares of a 5120-wide residual row as the decode path computes it
// across two launches: the launch that adds the residual writes one partial per
// 8-row tile, ((r0^2 + r1^2) + (r2^2 + r3^2)) + ((r4^2 + r5^2) + (r6^2 + r7^2)),
// and the consuming launch's thread t of 256 sums partials t, t+256, t+512 in
// order, tree64 per wave, (W0 + W1) + (W2 + W3).
float sumsq_tiles8(const float* x, int cols) {
  const int tiles = cols / 8;
  std::vector<float> part(tiles);
  for (int b = 0; b < tiles; ++b) {
    const float* r = x + 8 * b;
    float s[4];
    for (int q = 0; q < 4; ++q) s[q] = r[2 * q] * r[2 * q] + r[2 * q + 1] * r[2 * q + 1];
    part[b] = (s[0] + s[1]) + (s[2] + s[3]);
  }
  float lanes[256];
  for (int t = 0; t < 256; ++t) {
    float acc = 0.0f;
    for (int b = t; b < tiles; b += 256) acc = acc + part[b];
    lanes[t] = acc;
  }
  float w[4];
  for (int q = 0; q < 4; ++q) w[q] = tree_xor(lanes + 64 * q, 64);
  return (w[0] + w[1]) + (w[2] + w[3]);
}

// Sum of squares of `cols` values (multiple of 256) with the rows-of-256 tree.
float sumsq_rows256(const float* x, int cols) {
  float lanes[256];
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int j = t; j < cols; j += 256) s = s + x[j] * x[j];
    lanes[t] = s;
  }
  float w[4];
  for (int q = 0; q < 4; ++q) w[q] = tree_xor(lanes + 64 * q, 64);
  return (w[0] + w[1]) + (w[2] + w[3]);
}

// tree128 sum of squares of 128 values.
float sumsq_tree128(const float* v) {
  float lanes[64];
  for (int l = 0; l < 64; ++l) lanes[l] = v[l] * v[l] + v[l + 64] * v[l + 64];
  return tree_xor(lanes, 64);
}

// RMSNorm of a row of f32 (bf16-valued) inputs; norm.metal:10-47:
// inv = rsqrt(sum/cols + eps), y = bf16(x * inv * w).
void rms_norm_f(const float* x, const uint16_t* w, int cols, uint16_t* out, bool tiles = false) {
  const float ss = tiles ? sumsq_tiles8(x, cols) : sumsq_chunks8(x, cols);
  const float inv = lisa_rsqrt(ss / (float)cols + LISA_EPS);
  for (int j = 0; j < cols; ++j) out[j] = tobf((x[j] * inv) * bf(w[j]));
}

// ---- q4 linear -------------------------------------------------------------
// qmv.metal:9-76. Per 64-wide group g of row n:
//   acc_lo = fma chain over the low nibbles  (x[k_even] * q)
//   acc_hi = fma chain over the high nibbles (x[k_odd]/16 * (byte & 0xf0)),
//            which is the reference's own odd-nibble trick (qmv.metal:30-36,49)
//   G = acc_lo + acc_hi / 16;  P_g = fma(scale, G, bias * X_g), X_g = the
//   ascending-distance tree64 of the group's 64 x values.
// Both chains are evaluated with the nibble factors scaled by 2^-24 (q * 2^-24
// and 16q * 2^-24, the values the HIP path reads as f16 subnormals) and the
// scale multiplied by 2^24; the scaling is exact, so outside subnormal ranges
// this is the unscaled arithmetic, and inside them it is still what the HIP
// path computes.
// The 16 lanes of a row-group accumulate P over g = 16i + lane (ascending i),
// then tree16 (the simd_sum of qmv.metal:71-75 with 16 lanes).
struct XPrep {
  std::vector<float> xs;  // x as f32
  std::vector<float> gsum;
};

constexpr float kNibScale = 0x1p-24f;
constexpr float kScaleUp = 0x1p24f;

void prep_x(const uint16_t* x, int k, XPrep& p) {
  p.xs.resize(k);
  p.gsum.resize(k / 64);
  for (int i = 0; i < k; ++i) p.xs[i] = bf(x[i]);
  for (int g = 0; g < k / 64; ++g) {
    float v[64];
    for (int i = 0; i < 64; ++i) v[i] = bf(x[64 * g + i]);
    p.gsum[g] = tree_asc(v, 64);
  }
}

inline float group_partial(const float* xs, const uint32_t* w8, float scale, float bias, float xsum) {
  float acc_lo = 0.0f, acc_hi = 0.0f;
  for (int j = 0; j < 8; ++j) {
    const uint32_t word = w8[j];
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (word >> (8 * b)) & 0xffu;
      acc_lo = lisa_fma(xs[8 * j + 2 * b], (float)(byte & 0x0fu) * kNibScale, acc_lo);
      acc_hi = lisa_fma(xs[8 * j + 2 * b + 1], (float)(byte & 0xf0u) * kNibScale, acc_hi);
    }
  }
  const float g = acc_lo + acc_hi * 0.0625f;
  return lisa_fma(scale * kScaleUp, g, bias * xsum);
}

// ksplit = 1: lane l sums its groups over all iterations, tree16.
// ksplit = 4: iterations split into four contiguous ranges
// [ITER*w/4, ITER*(w+1)/4); tree16 per range; (W0 + W1) + (W2 + W3).
float q4_row(const XPrep& xp, const uint32_t* wrow, const uint16_t* srow, const uint16_t* brow, int k,
             int ksplit) {
  const int groups = k / 64, iters = (groups + 15) / 16;
  float wsum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nsplit = (ksplit == 4) ? 4 : 1;
  for (int w = 0; w < nsplit; ++w) {
    const int i0 = (nsplit == 4) ? (iters * w) / 4 : 0, i1 = (nsplit == 4) ? (iters * (w + 1)) / 4 : iters;
    float lanes[16];
    for (int l = 0; l < 16; ++l) {
      float t = 0.0f;
      for (int i = i0; i < i1; ++i) {
        const int g = 16 * i + l;
        if (g >= groups) continue;
        t = t + group_partial(&xp.xs[64 * g], wrow + 8 * g, bf(srow[g]), bf(brow[g]), xp.gsum[g]);
      }
      lanes[l] = t;
    }
    wsum[w] = tree_xor(lanes, 16);
  }
  return (nsplit == 4) ? (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]) : wsum[0];
}

// AVX2 version of q4_row over 8 rows at once; identical operations per lane.
void q4_rows8(const XPrep& xp, const uint32_t* w, const uint16_t* s, const uint16_t* b, int k,
              int row0, int ksplit, float* out /*8*/) {
  const int groups = k / 64, wpr = k / 8, iters = groups / 16;
  const int nsplit = (ksplit == 4) ? 4 : 1;
  __m256 wsum[4];
  for (int sp = 0; sp < nsplit; ++sp) {
    const int i0 = (nsplit == 4) ? (iters * sp) / 4 : 0, i1 = (nsplit == 4) ? (iters * (sp + 1)) / 4 : iters;
    __m256 lanes[16];
    for (int l = 0; l < 16; ++l) {
      __m256 t = _mm256_setzero_ps();
      for (int it = i0; it < i1; ++it) {
        const int g = 16 * it + l;
        __m256 lo = _mm256_setzero_ps(), hi = _mm256_setzero_ps();
        alignas(32) float sc[8], bi[8];
        for (int r = 0; r < 8; ++r) {
          sc[r] = bf(s[(size_t)(row0 + r) * groups + g]) * kScaleUp;
          bi[r] = bf(b[(size_t)(row0 + r) * groups + g]);
        }
        const float* xs = &xp.xs[64 * g];
        for (int j = 0; j < 8; ++j) {
          alignas(32) uint32_t wd[8];
          for (int r = 0; r < 8; ++r) wd[r] = w[(size_t)(row0 + r) * wpr + 8 * g + j];
          const __m256i wv = _mm256_load_si256((const __m256i*)wd);
          for (int bb = 0; bb < 4; ++bb) {
            const __m256i byte = _mm256_and_si256(_mm256_srli_epi32(wv, 8 * bb), _mm256_set1_epi32(0xff));
            const __m256 qlo = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_and_si256(byte, _mm256_set1_epi32(0x0f))),
                                             _mm256_set1_ps(kNibScale));
            const __m256 qhi = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_and_si256(byte, _mm256_set1_epi32(0xf0))),
                                             _mm256_set1_ps(kNibScale));
            lo = _mm256_fmadd_ps(_mm256_set1_ps(xs[8 * j + 2 * bb]), qlo, lo);
            hi = _mm256_fmadd_ps(_mm256_set1_ps(xs[8 * j + 2 * bb + 1]), qhi, hi);
          }
        }
        const __m256 gv = _mm256_add_ps(lo, _mm256_mul_ps(hi, _mm256_set1_ps(0.0625f)));
        const __m256 pp = _mm256_fmadd_ps(_mm256_load_ps(sc), gv,
                                          _mm256_mul_ps(_mm256_load_ps(bi), _mm256_set1_ps(xp.gsum[g])));
        t = _mm256_add_ps(t, pp);
      }
      lanes[l] = t;
    }
    for (int m = 8; m >= 1; m >>= 1) {
      __m256 tmp[16];
      for (int i = 0; i < 16; ++i) tmp[i] = _mm256_add_ps(lanes[i], lanes[i ^ m]);
      for (int i = 0; i < 16; ++i) lanes[i] = tmp[i];
    }
    wsum[sp] = lanes[0];
  }
  const __m256 res = (nsplit == 4) ? _mm256_add_ps(_mm256_add_ps(wsum[0], wsum[1]), _mm256_add_ps(wsum[2], wsum[3]))
                                   : wsum[0];
  _mm256_storeu_ps(out, res);
}

void q4_linear_prepped(const XPrep* xp, int m_rows, const uint32_t* w, const uint16_t* s,
                       const uint16_t* b, int n, int k, int ksplit, float* out) {
  const int groups = k / 64, wpr = k / 8;
  const int n8 = (k % 1024 == 0) ? (n & ~7) : 0;
#pragma omp parallel for schedule(static)
  for (int r0 = 0; r0 < n8; r0 += 8) {
    for (int m = 0; m < m_rows; ++m) {
      float o[8];
      q4_rows8(xp[m], w, s, b, k, r0, ksplit, o);
      for (int r = 0; r < 8; ++r) out[(size_t)m * n + r0 + r] = o[r];
    }
  }
  for (int r = n8; r < n; ++r)
    for (int m = 0; m < m_rows; ++m)
      out[(size_t)m * n + r] =
          q4_row(xp[m], w + (size_t)r * wpr, s + (size_t)r * groups, b + (size_t)r * groups, k, ksplit);
}

// ---- synthetic tensors -------------------------------------------------------
struct Q4 {
  std::vector<uint32_t> w;
  std::vector<uint16_t> s, b;
  int n = 0, k = 0;
};

void synth_words(uint64_t seed, uint64_t id, size_t n, uint32_t* out) {
  const uint64_t key = lisa_stream_key(seed, id);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = lisa_synth_word(key, i);
}
void synth_bf16(uint64_t seed, uint64_t id, int dist, float a, float b, size_t n, uint16_t* out) {
  const uint64_t key = lisa_stream_key(seed, id);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = tobf(lisa_synth_value(key, i, dist, a, b));
}
void synth_f32(uint64_t seed, uint64_t id, int dist, float a, float b, size_t n, float* out) {
  const uint64_t key = lisa_stream_key(seed, id);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = lisa_synth_value(key, i, dist, a, b);
}

Q4 make_q4(uint64_t seed, int scope, int kind, int n, int k) {
  Q4 q;
  q.n = n;
  q.k = k;
  q.w.resize((size_t)n * k / 8);
  q.s.resize((size_t)n * k / 64);
  q.b.resize((size_t)n * k / 64);
  synth_words(seed, lisa_tensor_id(scope, kind, 0), q.w.size(), q.w.data());
  synth_bf16(seed, lisa_tensor_id(scope, kind, 1), LISA_DIST_UNIFORM, LISA_SCALE_LO, LISA_SCALE_HI,
             q.s.size(), q.s.data());
  // zero-mean groups: b = bf16(s * (u - 7.5)), u ~ U(-1, 1) from the bias stream
  std::vector<float> u(q.b.size());
  synth_f32(seed, lisa_tensor_id(scope, kind, 2), LISA_DIST_UNIFORM, -LISA_MODEL_BIAS_SPREAD, LISA_MODEL_BIAS_SPREAD,
            u.size(), u.data());
  for (size_t i = 0; i < u.size(); ++i) q.b[i] = tobf(bf(q.s[i]) * (u[i] - LISA_MODEL_BIAS_CENTER));
  return q;
}

std::vector<uint16_t> make_vec(uint64_t seed, int scope, int kind, int n, float lo, float hi) {
  std::vector<uint16_t> v(n);
  synth_bf16(seed, lisa_tensor_id(scope, kind, 0), LISA_DIST_UNIFORM, lo, hi, n, v.data());
  return v;
}

std::vector<uint16_t> make_norm(uint64_t seed, int scope, int kind, int n) {
  return make_vec(seed, scope, kind, n, 0.9f, 1.1f);
}

// The HIP launch splits the group iterations of a tile across the four waves
// of a workgroup for every K except the 5120-wide inputs.
int ksplit_for(int k) { return k == LISA_HIDDEN ? 1 : 4; }

void q4_apply(const Q4& q, const std::vector<XPrep>& xp, int m_rows, float* out) {
  q4_linear_prepped(xp.data(), m_rows, q.w.data(), q.s.data(), q.b.data(), q.n, q.k, ksplit_for(q.k), out);
}

}  // namespace

// =============================================================================
// kernel-level C API
// =============================================================================
extern "C" {

void orc_q4_linear(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, int n_rows, int k, int m_rows, int ksplit, float* out) {
  std::vector<XPrep> xp(m_rows);
  for (int m = 0; m < m_rows; ++m) prep_x(x + (size_t)m * k, k, xp[m]);
  q4_linear_prepped(xp.data(), m_rows, w, scales, biases, n_rows, k, ksplit, out);
}

// Prefill q4 GEMM (gemm.metal:238-266): each weight dequantized to
// bf16(fma(scale, q, bias)); C[m][n] accumulated in f32 in the order the
// gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16, K ascending in blocks of 16)
// accumulates: once per 8 consecutive k, acc = f32(acc + sum of the 8 exact
// products). Measured on the MI355X this reproduces ~99.2 % of the kernel's
// outputs bit for bit on model-like data (the rest within a few ulps, the
// hardware's own internal rounding), against ~21 % for one rounding at the
// end, so the GPU prefill is compared within a tolerance. A product of two
// bf16 values is exact in double and so is a sum of eight of them here.
static int g_gemm_order = 0;  // 0: f32 per 8 k (the MFMA's order); 1: double sum, one rounding

void orc_set_gemm_order(int order) { g_gemm_order = order ? 1 : 0; }

void orc_q4_gemm(const uint16_t* a, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int n_rows,
                 int k, int m_rows, float* out) {
  const int wpr = k / 8, groups = k / 64;
  const bool blocked = g_gemm_order == 0;
  std::vector<float> af((size_t)m_rows * k);
  for (size_t i = 0; i < af.size(); ++i) af[i] = bf(a[i]);
  const int nblocks = (n_rows + 3) / 4;
#pragma omp parallel
  {
    // dequantized weights of 4 rows, interleaved: wt[4 kk + j] = row j, column kk
    std::vector<double> wt((size_t)4 * k);
#pragma omp for schedule(dynamic, 4)
    for (int nb = 0; nb < nblocks; ++nb) {
      const int n0 = 4 * nb, nn = std::min(4, n_rows - n0);
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + std::min(j, nn - 1);
        for (int g = 0; g < groups; ++g) {
          const float sc = bf(scales[(size_t)n * groups + g]), bi = bf(biases[(size_t)n * groups + g]);
          for (int e = 0; e < 64; ++e) {
            const int kk = 64 * g + e;
            const uint32_t q = (w[(size_t)n * wpr + kk / 8] >> (4 * (kk % 8))) & 0xfu;
            wt[(size_t)4 * kk + j] = (double)bfr(lisa_fma(sc, (float)q, bi));
          }
        }
      }
      int m = 0;
      for (; m + 3 <= m_rows; m += 3) {
        const float* a0 = &af[(size_t)m * k];
        const float* a1 = a0 + k;
        const float* a2 = a1 + k;
        __m256d c0 = _mm256_setzero_pd(), c1 = _mm256_setzero_pd(), c2 = _mm256_setzero_pd();
        for (int k0 = 0; k0 < k; k0 += 8) {
          __m256d s0 = _mm256_setzero_pd(), s1 = _mm256_setzero_pd(), s2 = _mm256_setzero_pd();
          for (int kk = k0; kk < k0 + 8; ++kk) {
            const __m256d wv = _mm256_loadu_pd(&wt[(size_t)4 * kk]);
            s0 = _mm256_fmadd_pd(_mm256_set1_pd((double)a0[kk]), wv, s0);
            s1 = _mm256_fmadd_pd(_mm256_set1_pd((double)a1[kk]), wv, s1);
            s2 = _mm256_fmadd_pd(_mm256_set1_pd((double)a2[kk]), wv, s2);
          }
          // acc = f32(acc + block): the sum in double, one rounding to f32
          c0 = _mm256_add_pd(c0, s0);
          c1 = _mm256_add_pd(c1, s1);
          c2 = _mm256_add_pd(c2, s2);
          if (blocked) {
            c0 = _mm256_cvtps_pd(_mm256_cvtpd_ps(c0));
            c1 = _mm256_cvtps_pd(_mm256_cvtpd_ps(c1));
            c2 = _mm256_cvtps_pd(_mm256_cvtpd_ps(c2));
          }
        }
        alignas(32) double r0[4], r1[4], r2[4];
        _mm256_store_pd(r0, c0);
        _mm256_store_pd(r1, c1);
        _mm256_store_pd(r2, c2);
        for (int j = 0; j < nn; ++j) {
          out[(size_t)m * n_rows + n0 + j] = (float)r0[j];
          out[(size_t)(m + 1) * n_rows + n0 + j] = (float)r1[j];
          out[(size_t)(m + 2) * n_rows + n0 + j] = (float)r2[j];
        }
      }
      for (; m < m_rows; ++m) {
        const float* a0 = &af[(size_t)m * k];
        __m256d c0 = _mm256_setzero_pd();
        for (int k0 = 0; k0 < k; k0 += 8) {
          __m256d s0 = _mm256_setzero_pd();
          for (int kk = k0; kk < k0 + 8; ++kk)
            s0 = _mm256_fmadd_pd(_mm256_set1_pd((double)a0[kk]), _mm256_loadu_pd(&wt[(size_t)4 * kk]), s0);
          c0 = _mm256_add_pd(c0, s0);
          if (blocked) c0 = _mm256_cvtps_pd(_mm256_cvtpd_ps(c0));
        }
        alignas(32) double r0[4];
        _mm256_store_pd(r0, c0);
        for (int j = 0; j < nn; ++j) out[(size_t)m * n_rows + n0 + j] = (float)r0[j];
      }
    }
  }
}

void orc_rms_norm(const uint16_t* x, const uint16_t* w, int cols, uint16_t* out) {
  std::vector<float> xf(cols);
  for (int j = 0; j < cols; ++j) xf[j] = bf(x[j]);
  rms_norm_f(xf.data(), w, cols, out);
}

// RMSNorm with the tile-partial statistic (residual-add launch + consumer).
void orc_rms_norm_tiles(const uint16_t* x, const uint16_t* w, int cols, uint16_t* out) {
  std::vector<float> xf(cols);
  for (int j = 0; j < cols; ++j) xf[j] = bf(x[j]);
  rms_norm_f(xf.data(), w, cols, out, true);
}

void orc_residual(const uint16_t* x, const float* o, int n, uint16_t* y) {
  for (int i = 0; i < n; ++i) y[i] = tobf(bf(x[i]) + bfr(o[i]));
}

// embed.metal:6-28: value = float(q)*scale + bias, stored bf16.
void orc_embed(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t token,
               int hidden, uint16_t* out) {
  const size_t wpr = hidden / 8, gpr = hidden / 64;
  for (int c = 0; c < hidden; ++c) {
    const uint32_t word = w[(size_t)token * wpr + c / 8];
    const uint32_t q = (word >> ((c & 7) * 4)) & 0xfu;
    const float v = (float)q * bf(scales[(size_t)token * gpr + c / 64]) + bf(biases[(size_t)token * gpr + c / 64]);
    out[c] = tobf(v);
  }
}

// mlp.metal:6-17
void orc_silu_mul(const float* g, const float* u, int n, uint16_t* act) {
  for (int i = 0; i < n; ++i) act[i] = tobf(lisa_silu_exp2(bfr(g[i])) * bfr(u[i]));
}

// gdn.metal:125-207 (conv part) and 212-240 (history update).
void orc_gdn_conv(const float* qkv, const uint16_t* conv_w, uint16_t* conv_state, int m_rows,
                  float* conv_out, uint16_t* slots) {
  const int C = LISA_GDN_CONV_DIM;
  if (m_rows < 1) return;
#pragma omp parallel for schedule(static)
  for (int c = 0; c < C; ++c) {
    std::vector<float> hist(3 + m_rows);
    for (int i = 0; i < 3; ++i) hist[i] = bf(conv_state[(size_t)i * C + c]);
    for (int t = 0; t < m_rows; ++t) hist[3 + t] = bfr(qkv[(size_t)t * C + c]);
    for (int t = 0; t < m_rows; ++t) {
      float acc = 0.0f;
      for (int tap = 0; tap < 4; ++tap) acc = acc + hist[t + tap] * bf(conv_w[(size_t)c * 4 + tap]);
      const float conv = bfr(acc);
      conv_out[(size_t)t * C + c] = bfr(lisa_silu_exp(conv));
      if (slots)
        for (int i = 0; i < 3; ++i) slots[((size_t)t * 3 + i) * C + c] = tobf(hist[t + 1 + i]);
    }
    for (int i = 0; i < 3; ++i) conv_state[(size_t)i * C + c] = tobf(hist[m_rows + i]);
  }
}

// gdn.metal:125-207 (norms and gates), 245-328 (recurrence), 367-391 (gate).
void orc_gdn_recurrence(const float* conv_out, const float* z, const float* a, const float* b,
                        const uint16_t* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float* state, int m_rows, uint16_t* gated, float* slots, float* y_out) {
  const int C = LISA_GDN_CONV_DIM, HD = LISA_GDN_HD, VH = LISA_GDN_VH;
  const float inv = 1.0f / lisa_sqrt((float)HD);  // runner.rs:1317 scales
  const float q_scale = inv * inv, k_scale = inv;
#pragma omp parallel for schedule(static)
  for (int h = 0; h < VH; ++h) {
    const int kh = h / (VH / LISA_GDN_KH);
    float* S = state + (size_t)h * HD * HD;
    for (int t = 0; t < m_rows; ++t) {
      const float* co = conv_out + (size_t)t * C;
      float cq[128], ck[128], qn[128], kn[128];
      for (int i = 0; i < HD; ++i) {
        cq[i] = co[kh * HD + i];
        ck[i] = co[LISA_GDN_KEY_DIM + kh * HD + i];
      }
      const float q_inv = lisa_rsqrt(sumsq_tree128(cq) / (float)HD + 1.0e-6f) * q_scale;
      const float k_inv = lisa_rsqrt(sumsq_tree128(ck) / (float)HD + 1.0e-6f) * k_scale;
      for (int i = 0; i < HD; ++i) {
        qn[i] = bfr(cq[i] * q_inv);
        kn[i] = bfr(ck[i] * k_inv);
      }
      const float beta = bfr(lisa_sigmoid_exp(bfr(b[(size_t)t * VH + h])));
      const float dt_arg = bfr(bfr(a[(size_t)t * VH + h]) + bf(dt_bias[h]));
      const float dt = bfr(lisa_softplus(dt_arg));
      const float decay = lisa_expf(-lisa_expf(bf(a_log[h])) * dt);
      float y[128];
      for (int v = 0; v < HD; ++v) {
        float* row = S + (size_t)v * HD;
        for (int k = 0; k < HD; ++k) row[k] = row[k] * decay;
        // row . vector over 128: quarters of 32, each the sum (r0 + r1) + (r2 + r3)
        // of four ascending fma runs of 8; quarters combined (q0 + q1) + (q2 + q3)
        auto dot128 = [&](const float* vec) {
          float pqr[4];
          for (int q = 0; q < 4; ++q) {
            float r[4];
            for (int j = 0; j < 4; ++j) {
              const int k0 = 32 * q + 8 * j;
              float p = row[k0] * vec[k0];
              for (int k = k0 + 1; k < k0 + 8; ++k) p = lisa_fma(row[k], vec[k], p);
              r[j] = p;
            }
            pqr[q] = (r[0] + r[1]) + (r[2] + r[3]);
          }
          return (pqr[0] + pqr[1]) + (pqr[2] + pqr[3]);
        };
        const float kv = dot128(kn);
        const float vval = co[2 * LISA_GDN_KEY_DIM + h * HD + v];
        const float delta = (vval - kv) * beta;
        for (int k = 0; k < HD; ++k) row[k] = lisa_fma(delta, kn[k], row[k]);
        y[v] = bfr(dot128(qn));
      }
      if (y_out)
        for (int v = 0; v < HD; ++v) y_out[(size_t)t * LISA_GDN_VALUE_DIM + h * HD + v] = y[v];
      const float ginv = lisa_rsqrt(sumsq_tree128(y) / 128.0f + LISA_EPS);
      for (int v = 0; v < HD; ++v) {
        const float n = bfr((y[v] * ginv) * bf(norm_w[v]));
        const float zz = bfr(z[(size_t)t * LISA_GDN_VALUE_DIM + h * HD + v]);
        gated[(size_t)t * LISA_GDN_VALUE_DIM + h * HD + v] = tobf(n * lisa_silu_exp(zz));
      }
      if (slots)
        std::memcpy(slots + (size_t)t * LISA_GDN_STATE + (size_t)h * HD * HD, S,
                    sizeof(float) * HD * HD);
    }
  }
}

// attention.metal:118-155 / 158-197: RMSNorm with learned gain then partial
// NeoX RoPE on dims [0,64) with pairs (j, j+32); sum of squares by
// rows-of-256 (one element per thread).
void orc_head_norm_rope(const float* raw, const uint16_t* w, uint32_t position, uint16_t* out) {
  static const float inv_freq[LISA_ROPE_PAIRS] = LISA_ROPE_INV_FREQ_TABLE;
  float v[256], n[256];
  for (int j = 0; j < 256; ++j) v[j] = bfr(raw[j]);
  const float inv = lisa_rsqrt(sumsq_rows256(v, 256) / 256.0f + LISA_EPS);
  for (int j = 0; j < 256; ++j) n[j] = (v[j] * inv) * bf(w[j]);
  for (int j = 0; j < 32; ++j) {
    const float angle = (float)position * inv_freq[j];
    float s, c;
    lisa_sincosf(angle, &s, &c);
    out[j] = tobf(n[j] * c - n[j + 32] * s);
    out[j + 32] = tobf(n[j + 32] * c + n[j] * s);
  }
  for (int j = 64; j < 256; ++j) out[j] = tobf(n[j]);
}

// attention.metal:158-197 (store), 550-604 (slice partials), 611-641 (merge),
// 520-531 (output gate). Slice s covers tokens [64s, 64s+64) of the row's own
// context, so a row's result does not depend on the other rows of the batch.
void orc_attention(const float* q_proj, const float* k_raw, const float* v_raw,
                   const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* key_cache,
                   uint16_t* value_cache, uint32_t capacity, uint32_t base, int m_rows,
                   uint16_t* gated) {
  const int HD = LISA_ATT_HD;
  for (int t = 0; t < m_rows; ++t) {
    const uint32_t pos = base + t;
    for (int kvh = 0; kvh < LISA_ATT_KVH; ++kvh) {
      uint16_t kr[256];
      orc_head_norm_rope(k_raw + (size_t)t * LISA_ATT_KV_OUT + kvh * HD, k_norm_w, pos, kr);
      const size_t off = ((size_t)kvh * capacity + pos) * HD;
      std::memcpy(key_cache + off, kr, sizeof(kr));
      for (int j = 0; j < HD; ++j) value_cache[off + j] = tobf(v_raw[(size_t)t * LISA_ATT_KV_OUT + kvh * HD + j]);
    }
  }
  std::vector<uint16_t> query((size_t)m_rows * LISA_ATT_OUT);
  for (int t = 0; t < m_rows; ++t)
    for (int h = 0; h < LISA_ATT_QH; ++h)
      orc_head_norm_rope(q_proj + (size_t)t * LISA_ATT_Q_OUT + h * 512, q_norm_w, base + t,
                         &query[(size_t)t * LISA_ATT_OUT + h * HD]);
  std::vector<float> o((size_t)m_rows * LISA_ATT_OUT);
  orc_sdpa(query.data(), key_cache, value_cache, capacity, base, m_rows, o.data());
  for (int t = 0; t < m_rows; ++t)
    for (int h = 0; h < LISA_ATT_QH; ++h)
      for (int d = 0; d < HD; ++d) {
        const float g = bfr(q_proj[(size_t)t * LISA_ATT_Q_OUT + h * 512 + 256 + d]);
        gated[(size_t)t * LISA_ATT_OUT + h * HD + d] =
            tobf(o[(size_t)t * LISA_ATT_OUT + h * HD + d] * lisa_sigmoid_exp2(g));
      }
}

// attention.metal:550-604 and 611-641: per slice s of 64 tokens of the row's
// own context, scores (4 accumulators over d mod 4, then (a0+a1)+(a2+a3)),
// slice max, p = exp2(log2e*(score-max)), denominator by tree64 over the 64
// token lanes, P.V accumulated over tokens in order; then the flash merge in
// ascending slice order with fma. query bf16[m][24][256]; out f32[m][24][256].
void orc_sdpa(const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache, uint32_t capacity,
              uint32_t base, int m_rows, float* out) {
  const int HD = LISA_ATT_HD;
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < m_rows; ++t) {
    for (int h = 0; h < LISA_ATT_QH; ++h) {
      const uint32_t pos = base + t, ctx = pos + 1;
      const int kvh = h / (LISA_ATT_QH / LISA_ATT_KVH);
      float q[256];
      for (int d = 0; d < HD; ++d) q[d] = bf(query[(size_t)t * LISA_ATT_OUT + h * HD + d]);
      const int used = (int)((ctx + LISA_ATT_SLICE - 1) / LISA_ATT_SLICE);
      std::vector<float> ms(used), dens(used), acc((size_t)used * HD);
      for (int s = 0; s < used; ++s) {
        const uint32_t t0 = s * LISA_ATT_SLICE, t1 = std::min<uint32_t>(t0 + LISA_ATT_SLICE, ctx);
        float score[64], p[64];
        float mx = -INFINITY;
        for (uint32_t tok = t0; tok < t1; ++tok) {
          const uint16_t* kr = key_cache + ((size_t)kvh * capacity + tok) * HD;
          float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          for (int d = 0; d < HD; ++d) a4[d & 3] = lisa_fma(q[d], bf(kr[d]), a4[d & 3]);
          score[tok - t0] = ((a4[0] + a4[1]) + (a4[2] + a4[3])) * 0.0625f;
          mx = std::max(mx, score[tok - t0]);
        }
        for (int i = 0; i < 64; ++i)
          p[i] = (i < (int)(t1 - t0)) ? lisa_exp2f(1.4426950408889634f * (score[i] - mx)) : 0.0f;
        float den_l[64];
        std::memcpy(den_l, p, sizeof(p));
        dens[s] = tree_xor(den_l, 64);
        ms[s] = mx;
        for (int d = 0; d < HD; ++d) {
          float a = 0.0f;
          for (uint32_t tok = t0; tok < t1; ++tok)
            a = lisa_fma(p[tok - t0], bf(value_cache[((size_t)kvh * capacity + tok) * HD + d]), a);
          acc[(size_t)s * HD + d] = a;
        }
      }
      float gmax = -INFINITY;
      for (int s = 0; s < used; ++s) gmax = std::max(gmax, ms[s]);
      std::vector<float> wts(used);
      float tot = 0.0f;
      for (int s = 0; s < used; ++s) {
        wts[s] = lisa_exp2f(1.4426950408889634f * (ms[s] - gmax));
        tot = lisa_fma(wts[s], dens[s], tot);
      }
      for (int d = 0; d < HD; ++d) {
        float res = 0.0f;
        for (int s = 0; s < used; ++s) res = lisa_fma(wts[s], acc[(size_t)s * HD + d], res);
        out[(size_t)t * LISA_ATT_OUT + h * HD + d] = res / tot;
      }
    }
  }
}

uint32_t orc_argmax(const float* v, int n) {
  uint32_t best = 0;
  float bv = -INFINITY;
  bool any = false;
  for (int i = 0; i < n; ++i) {
    if (!any) {
      if (v[i] == v[i]) { bv = v[i]; best = i; any = true; }
    } else if (v[i] > bv) {
      bv = v[i];
      best = i;
    }
  }
  return best;
}

void orc_synth_bf16(uint64_t seed, uint64_t tensor_id, int dist, float a, float b, size_t n,
                    uint16_t* out) {
  synth_bf16(seed, tensor_id, dist, a, b, n, out);
}

// Element-wise evaluation of the shared numerics (lisa_numerics.h) for tests:
// fn 0 exp, 1 exp2, 2 log, 3 sin, 4 cos, 5 rsqrt, 6 bf16 round, 7 silu(exp),
// 8 softplus, 9 sigmoid(exp), 10 silu(exp2), 11 sigmoid(exp2).
void orc_math(int fn, const float* x, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) {
    const float v = x[i];
    float s, c;
    switch (fn) {
      case 0: out[i] = lisa_expf(v); break;
      case 1: out[i] = lisa_exp2f(v); break;
      case 2: out[i] = lisa_logf(v); break;
      case 3: lisa_sincosf(v, &s, &c); out[i] = s; break;
      case 4: lisa_sincosf(v, &s, &c); out[i] = c; break;
      case 5: out[i] = lisa_rsqrt(v); break;
      case 6: out[i] = lisa_bf16r(v); break;
      case 7: out[i] = lisa_silu_exp(v); break;
      case 8: out[i] = lisa_softplus(v); break;
      case 9: out[i] = lisa_sigmoid_exp(v); break;
      case 10: out[i] = lisa_silu_exp2(v); break;
      default: out[i] = lisa_sigmoid_exp2(v); break;
    }
  }
}
void orc_synth_f32(uint64_t seed, uint64_t tensor_id, int dist, float a, float b, size_t n,
                   float* out) {
  synth_f32(seed, tensor_id, dist, a, b, n, out);
}
void orc_synth_words(uint64_t seed, uint64_t tensor_id, size_t n, uint32_t* out) {
  synth_words(seed, tensor_id, n, out);
}

}  // extern "C"

// =============================================================================
// model-level restatement
// =============================================================================
struct OrcLayer {
  bool attention = false;
  std::vector<uint16_t> input_norm, post_norm;
  Q4 gate, up, down;
  // GDN
  Q4 qkv, z, a, b, out;
  std::vector<uint16_t> conv_w, a_log, dt_bias, gnorm;
  int state_index = -1;
  // attention
  Q4 q, k, v, o;
  std::vector<uint16_t> q_norm, k_norm;
  int cache_index = -1;
};

struct OrcMtp {
  std::vector<uint16_t> pre_fc_emb, pre_fc_hid, input_norm, post_norm, final_norm, q_norm, k_norm;
  Q4 fc, q, k, v, o, gate, up, down;
  std::vector<uint16_t> key_cache, value_cache;
  uint32_t position = 0;
};

struct OrcModel {
  int layers = 0, vocab = 0, gdn_layers = 0, attn_layers = 0;
  uint32_t capacity = 0;
  uint64_t seed = 0;
  std::vector<OrcLayer> L;
  Q4 embed, head;
  std::vector<uint16_t> final_norm;
  std::vector<float> gdn_state;       // [gdn][48*128*128]
  std::vector<uint16_t> conv_state;   // [gdn][3][10240]
  std::vector<float> gdn_slots;       // [3][gdn][state]
  std::vector<uint16_t> conv_slots;   // [3][gdn][3][10240]
  std::vector<uint16_t> key_cache, value_cache;  // [attn][4][cap][256]
  uint32_t position = 0;
  int64_t verify_base = -1;
  bool has_mtp = false;
  OrcMtp mtp;
};

static void embed_rows(const OrcModel* M, const uint32_t* tokens, int m, std::vector<float>& h) {
  h.assign((size_t)m * LISA_HIDDEN, 0.0f);
  std::vector<uint16_t> row(LISA_HIDDEN);
  for (int t = 0; t < m; ++t) {
    orc_embed(M->embed.w.data(), M->embed.s.data(), M->embed.b.data(), tokens[t], LISA_HIDDEN, row.data());
    for (int c = 0; c < LISA_HIDDEN; ++c) h[(size_t)t * LISA_HIDDEN + c] = bf(row[c]);
  }
}

// tiles: the statistic is summed from per-8-row tile partials of the residual
// rows (every decode-path norm except the one after the embedding).
static void norm_rows(const std::vector<float>& h, int m, const std::vector<uint16_t>& w,
                      std::vector<XPrep>& xp, std::vector<uint16_t>* keep = nullptr, bool tiles = false) {
  xp.resize(m);
  std::vector<uint16_t> x(LISA_HIDDEN);
  if (keep) keep->resize((size_t)m * LISA_HIDDEN);
  for (int t = 0; t < m; ++t) {
    rms_norm_f(&h[(size_t)t * LISA_HIDDEN], w.data(), LISA_HIDDEN, x.data(), tiles);
    prep_x(x.data(), LISA_HIDDEN, xp[t]);
    if (keep) std::memcpy(keep->data() + (size_t)t * LISA_HIDDEN, x.data(), LISA_HIDDEN * 2);
  }
}

static void prep_rows(const std::vector<uint16_t>& x, int m, int k, std::vector<XPrep>& xp) {
  xp.resize(m);
  for (int t = 0; t < m; ++t) prep_x(&x[(size_t)t * k], k, xp[t]);
}

static void residual_rows(const std::vector<float>& h, const std::vector<float>& o, int m,
                          std::vector<float>& r) {
  r.resize((size_t)m * LISA_HIDDEN);
  for (size_t i = 0; i < (size_t)m * LISA_HIDDEN; ++i) r[i] = bfr(h[i] + bfr(o[i]));
}

static void mlp_block(const Q4& gate, const Q4& up, const Q4& down, const std::vector<XPrep>& xp,
                      int m, std::vector<float>& branch) {
  std::vector<float> g((size_t)m * LISA_INTER), u((size_t)m * LISA_INTER);
  q4_apply(gate, xp, m, g.data());
  q4_apply(up, xp, m, u.data());
  std::vector<uint16_t> act((size_t)m * LISA_INTER);
  orc_silu_mul(g.data(), u.data(), m * LISA_INTER, act.data());
  std::vector<XPrep> ap;
  prep_rows(act, m, LISA_INTER, ap);
  branch.resize((size_t)m * LISA_HIDDEN);
  q4_apply(down, ap, m, branch.data());
}

static void attention_block(const Q4& q, const Q4& k, const Q4& v, const Q4& o,
                            const std::vector<uint16_t>& qn, const std::vector<uint16_t>& kn,
                            uint16_t* kc, uint16_t* vc, uint32_t capacity, uint32_t base,
                            const std::vector<XPrep>& xp, int m, std::vector<float>& branch) {
  std::vector<float> qp((size_t)m * LISA_ATT_Q_OUT), kr((size_t)m * LISA_ATT_KV_OUT),
      vr((size_t)m * LISA_ATT_KV_OUT);
  q4_apply(q, xp, m, qp.data());
  q4_apply(k, xp, m, kr.data());
  q4_apply(v, xp, m, vr.data());
  std::vector<uint16_t> gated((size_t)m * LISA_ATT_OUT);
  orc_attention(qp.data(), kr.data(), vr.data(), qn.data(), kn.data(), kc, vc, capacity, base, m,
                gated.data());
  std::vector<XPrep> gp;
  prep_rows(gated, m, LISA_ATT_OUT, gp);
  branch.resize((size_t)m * LISA_HIDDEN);
  q4_apply(o, gp, m, branch.data());
}

extern "C" {

OrcModel* orc_model_create(int layers, int vocab, int capacity, uint64_t seed, int with_mtp) {
  if (layers <= 0 || layers % 4 != 0 || vocab <= 0 || capacity <= 0) return nullptr;
  OrcModel* M = new OrcModel();
  M->layers = layers;
  M->vocab = vocab;
  M->capacity = capacity;
  M->seed = seed;
  M->L.resize(layers);
  for (int i = 0; i < layers; ++i) {
    OrcLayer& l = M->L[i];
    const int sc = i + 1;
    l.attention = lisa_layer_is_attention(i);
    l.input_norm = make_norm(seed, sc, LISA_T_INPUT_NORM, LISA_HIDDEN);
    l.post_norm = make_norm(seed, sc, LISA_T_POST_NORM, LISA_HIDDEN);
    l.gate = make_q4(seed, sc, LISA_T_MLP_GATE, LISA_INTER, LISA_HIDDEN);
    l.up = make_q4(seed, sc, LISA_T_MLP_UP, LISA_INTER, LISA_HIDDEN);
    l.down = make_q4(seed, sc, LISA_T_MLP_DOWN, LISA_HIDDEN, LISA_INTER);
    if (l.attention) {
      l.q = make_q4(seed, sc, LISA_T_ATT_Q, LISA_ATT_Q_OUT, LISA_HIDDEN);
      l.k = make_q4(seed, sc, LISA_T_ATT_K, LISA_ATT_KV_OUT, LISA_HIDDEN);
      l.v = make_q4(seed, sc, LISA_T_ATT_V, LISA_ATT_KV_OUT, LISA_HIDDEN);
      l.o = make_q4(seed, sc, LISA_T_ATT_O, LISA_HIDDEN, LISA_ATT_OUT);
      l.q_norm = make_norm(seed, sc, LISA_T_ATT_Q_NORM, LISA_ATT_HD);
      l.k_norm = make_norm(seed, sc, LISA_T_ATT_K_NORM, LISA_ATT_HD);
      l.cache_index = M->attn_layers++;
    } else {
      l.qkv = make_q4(seed, sc, LISA_T_GDN_QKV, LISA_GDN_CONV_DIM, LISA_HIDDEN);
      l.z = make_q4(seed, sc, LISA_T_GDN_Z, LISA_GDN_VALUE_DIM, LISA_HIDDEN);
      l.a = make_q4(seed, sc, LISA_T_GDN_A, LISA_GDN_VH, LISA_HIDDEN);
      l.b = make_q4(seed, sc, LISA_T_GDN_B, LISA_GDN_VH, LISA_HIDDEN);
      l.out = make_q4(seed, sc, LISA_T_GDN_OUT, LISA_HIDDEN, LISA_GDN_VALUE_DIM);
      l.conv_w = make_vec(seed, sc, LISA_T_GDN_CONV_W, LISA_GDN_CONV_DIM * 4, -0.5f, 0.5f);
      l.a_log = make_vec(seed, sc, LISA_T_GDN_A_LOG, LISA_GDN_VH, -2.0f, 0.0f);
      l.dt_bias = make_vec(seed, sc, LISA_T_GDN_DT_BIAS, LISA_GDN_VH, -1.0f, 1.0f);
      l.gnorm = make_norm(seed, sc, LISA_T_GDN_NORM, LISA_GDN_HD);
      l.state_index = M->gdn_layers++;
    }
  }
  M->embed = make_q4(seed, 0, LISA_T_EMBED, vocab, LISA_HIDDEN);
  M->head = make_q4(seed, 0, LISA_T_LM_HEAD, vocab, LISA_HIDDEN);
  M->final_norm = make_norm(seed, 0, LISA_T_FINAL_NORM, LISA_HIDDEN);
  M->gdn_state.assign((size_t)M->gdn_layers * LISA_GDN_STATE, 0.0f);
  M->conv_state.assign((size_t)M->gdn_layers * 3 * LISA_GDN_CONV_DIM, 0);
  M->gdn_slots.assign((size_t)3 * M->gdn_layers * LISA_GDN_STATE, 0.0f);
  M->conv_slots.assign((size_t)3 * M->gdn_layers * 3 * LISA_GDN_CONV_DIM, 0);
  const size_t cache = (size_t)M->attn_layers * LISA_ATT_KVH * capacity * LISA_ATT_HD;
  M->key_cache.assign(cache, 0);
  M->value_cache.assign(cache, 0);
  if (with_mtp) {
    const int sc = LISA_SCOPE_MTP;
    OrcMtp& t = M->mtp;
    M->has_mtp = true;
    t.pre_fc_emb = make_norm(seed, sc, LISA_T_MTP_PRE_FC_EMB, LISA_HIDDEN);
    t.pre_fc_hid = make_norm(seed, sc, LISA_T_MTP_PRE_FC_HID, LISA_HIDDEN);
    t.fc = make_q4(seed, sc, LISA_T_MTP_FC, LISA_HIDDEN, 2 * LISA_HIDDEN);
    t.input_norm = make_norm(seed, sc, LISA_T_INPUT_NORM, LISA_HIDDEN);
    t.post_norm = make_norm(seed, sc, LISA_T_POST_NORM, LISA_HIDDEN);
    t.final_norm = make_norm(seed, sc, LISA_T_FINAL_NORM, LISA_HIDDEN);
    t.q = make_q4(seed, sc, LISA_T_ATT_Q, LISA_ATT_Q_OUT, LISA_HIDDEN);
    t.k = make_q4(seed, sc, LISA_T_ATT_K, LISA_ATT_KV_OUT, LISA_HIDDEN);
    t.v = make_q4(seed, sc, LISA_T_ATT_V, LISA_ATT_KV_OUT, LISA_HIDDEN);
    t.o = make_q4(seed, sc, LISA_T_ATT_O, LISA_HIDDEN, LISA_ATT_OUT);
    t.q_norm = make_norm(seed, sc, LISA_T_ATT_Q_NORM, LISA_ATT_HD);
    t.k_norm = make_norm(seed, sc, LISA_T_ATT_K_NORM, LISA_ATT_HD);
    t.gate = make_q4(seed, sc, LISA_T_MLP_GATE, LISA_INTER, LISA_HIDDEN);
    t.up = make_q4(seed, sc, LISA_T_MLP_UP, LISA_INTER, LISA_HIDDEN);
    t.down = make_q4(seed, sc, LISA_T_MLP_DOWN, LISA_HIDDEN, LISA_INTER);
    t.key_cache.assign((size_t)LISA_ATT_KVH * capacity * LISA_ATT_HD, 0);
    t.value_cache.assign((size_t)LISA_ATT_KVH * capacity * LISA_ATT_HD, 0);
  }
  return M;
}

void orc_model_free(OrcModel* m) { delete m; }
uint32_t orc_model_position(const OrcModel* m) { return m->position; }
int orc_threads(void) { return omp_get_max_threads(); }
int orc_layer_is_attention(int layer) { return lisa_layer_is_attention(layer); }
uint32_t orc_mtp_position(const OrcModel* m) { return m->mtp.position; }

void orc_model_reset(OrcModel* M) {
  std::fill(M->gdn_state.begin(), M->gdn_state.end(), 0.0f);
  std::fill(M->conv_state.begin(), M->conv_state.end(), 0);
  std::fill(M->key_cache.begin(), M->key_cache.end(), 0);
  std::fill(M->value_cache.begin(), M->value_cache.end(), 0);
  if (M->has_mtp) {
    std::fill(M->mtp.key_cache.begin(), M->mtp.key_cache.end(), 0);
    std::fill(M->mtp.value_cache.begin(), M->mtp.value_cache.end(), 0);
    M->mtp.position = 0;
  }
  M->position = 0;
  M->verify_base = -1;
}

// Synthetic start state: GDN state N(0,0.01), conv history and KV rows N(0,1).
// Element indices are independent of capacity: KV element (kvh, pos, d) is
// number (kvh * 2^20 + pos) * 256 + d of its stream.
static void fill_kv(uint64_t seed, int scope, uint16_t* kc, uint16_t* vc, uint32_t capacity,
                    uint32_t filled) {
  const uint64_t kk = lisa_stream_key(seed, lisa_tensor_id(scope, LISA_T_KEY_CACHE, 0));
  const uint64_t vk = lisa_stream_key(seed, lisa_tensor_id(scope, LISA_T_VALUE_CACHE, 0));
#pragma omp parallel for collapse(2) schedule(static)
  for (int kvh = 0; kvh < LISA_ATT_KVH; ++kvh)
    for (uint32_t p = 0; p < filled; ++p)
      for (int d = 0; d < LISA_ATT_HD; ++d) {
        const uint64_t e = (((uint64_t)kvh << 20) + p) * LISA_ATT_HD + d;
        const size_t off = ((size_t)kvh * capacity + p) * LISA_ATT_HD + d;
        kc[off] = tobf(lisa_synth_value(kk, e, LISA_DIST_NORMAL, 0.0f, 1.0f));
        vc[off] = tobf(lisa_synth_value(vk, e, LISA_DIST_NORMAL, 0.0f, 1.0f));
      }
}

void orc_model_fill_state(OrcModel* M, uint32_t filled, uint64_t seed) {
  orc_model_reset(M);
  for (int i = 0; i < M->layers; ++i) {
    const OrcLayer& l = M->L[i];
    const int sc = i + 1;
    if (!l.attention) {
      synth_f32(seed, lisa_tensor_id(sc, LISA_T_GDN_STATE, 0), LISA_DIST_NORMAL, 0.0f, 0.01f,
                LISA_GDN_STATE, &M->gdn_state[(size_t)l.state_index * LISA_GDN_STATE]);
      synth_bf16(seed, lisa_tensor_id(sc, LISA_T_CONV_STATE, 0), LISA_DIST_NORMAL, 0.0f, 1.0f,
                 3 * LISA_GDN_CONV_DIM, &M->conv_state[(size_t)l.state_index * 3 * LISA_GDN_CONV_DIM]);
    } else {
      const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * M->capacity * LISA_ATT_HD;
      fill_kv(seed, sc, &M->key_cache[off], &M->value_cache[off], M->capacity, filled);
    }
  }
  if (M->has_mtp) {
    fill_kv(seed, LISA_SCOPE_MTP, M->mtp.key_cache.data(), M->mtp.value_cache.data(), M->capacity, filled);
    M->mtp.position = filled;
  }
  M->position = filled;
}

int orc_model_forward(OrcModel* M, const uint32_t* tokens, int m, int capture, uint32_t* argmax_out,
                      float* hidden_out, float* logits_out) {
  if (m < 1 || m > 3) return -1;
  for (int t = 0; t < m; ++t)
    if ((int)tokens[t] >= M->vocab) return -2;
  if (M->position + m > M->capacity) return -3;
  const uint32_t base = M->position;
  std::vector<float> H, R, B;
  embed_rows(M, tokens, m, H);
  std::vector<XPrep> xp;
  for (int i = 0; i < M->layers; ++i) {
    OrcLayer& l = M->L[i];
    norm_rows(H, m, l.input_norm, xp, nullptr, i > 0);
    if (!l.attention) {
      const int si = l.state_index;
      std::vector<float> qkv((size_t)m * LISA_GDN_CONV_DIM), z((size_t)m * LISA_GDN_VALUE_DIM),
          a((size_t)m * LISA_GDN_VH), b((size_t)m * LISA_GDN_VH);
      q4_apply(l.qkv, xp, m, qkv.data());
      q4_apply(l.z, xp, m, z.data());
      q4_apply(l.a, xp, m, a.data());
      q4_apply(l.b, xp, m, b.data());
      std::vector<float> conv_out((size_t)m * LISA_GDN_CONV_DIM);
      std::vector<uint16_t> cslots;
      if (capture) cslots.resize((size_t)m * 3 * LISA_GDN_CONV_DIM);
      uint16_t* cs = &M->conv_state[(size_t)si * 3 * LISA_GDN_CONV_DIM];
      orc_gdn_conv(qkv.data(), l.conv_w.data(), cs, m, conv_out.data(), capture ? cslots.data() : nullptr);
      std::vector<float> gslots;
      if (capture) gslots.resize((size_t)m * LISA_GDN_STATE);
      std::vector<uint16_t> gated((size_t)m * LISA_GDN_VALUE_DIM);
      float* st = &M->gdn_state[(size_t)si * LISA_GDN_STATE];
      orc_gdn_recurrence(conv_out.data(), z.data(), a.data(), b.data(), l.a_log.data(),
                         l.dt_bias.data(), l.gnorm.data(), st, m, gated.data(),
                         capture ? gslots.data() : nullptr, nullptr);
      if (capture) {
        for (int t = 0; t < m; ++t) {
          std::memcpy(&M->gdn_slots[((size_t)t * M->gdn_layers + si) * LISA_GDN_STATE],
                      &gslots[(size_t)t * LISA_GDN_STATE], sizeof(float) * LISA_GDN_STATE);
          std::memcpy(&M->conv_slots[((size_t)t * M->gdn_layers + si) * 3 * LISA_GDN_CONV_DIM],
                      &cslots[(size_t)t * 3 * LISA_GDN_CONV_DIM], 2 * 3 * LISA_GDN_CONV_DIM);
        }
      }
      std::vector<XPrep> gp;
      prep_rows(gated, m, LISA_GDN_VALUE_DIM, gp);
      B.resize((size_t)m * LISA_HIDDEN);
      q4_apply(l.out, gp, m, B.data());
    } else {
      const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * M->capacity * LISA_ATT_HD;
      attention_block(l.q, l.k, l.v, l.o, l.q_norm, l.k_norm, &M->key_cache[off],
                      &M->value_cache[off], M->capacity, base, xp, m, B);
    }
    residual_rows(H, B, m, R);
    norm_rows(R, m, l.post_norm, xp, nullptr, true);
    mlp_block(l.gate, l.up, l.down, xp, m, B);
    residual_rows(R, B, m, H);
  }
  norm_rows(H, m, M->final_norm, xp, nullptr, true);
  std::vector<float> logits((size_t)m * M->vocab);
  q4_apply(M->head, xp, m, logits.data());
  for (int t = 0; t < m; ++t) {
    if (argmax_out) argmax_out[t] = orc_argmax(&logits[(size_t)t * M->vocab], M->vocab);
  }
  if (hidden_out) std::memcpy(hidden_out, H.data(), sizeof(float) * H.size());
  if (logits_out) std::memcpy(logits_out, logits.data(), sizeof(float) * logits.size());
  M->position += m;
  M->verify_base = capture ? (int64_t)base : -1;
  return 0;
}

static void gemm_q4(const std::vector<uint16_t>& a, int m, const Q4& w, std::vector<float>& c) {
  c.resize((size_t)m * w.n);
  orc_q4_gemm(a.data(), w.w.data(), w.s.data(), w.b.data(), w.n, w.k, m, c.data());
}

static void norm_rows_bf16(const std::vector<float>& h, int m, const std::vector<uint16_t>& w,
                           std::vector<uint16_t>& x) {
  x.resize((size_t)m * LISA_HIDDEN);
  for (int t = 0; t < m; ++t) rms_norm_f(&h[(size_t)t * LISA_HIDDEN], w.data(), LISA_HIDDEN, &x[(size_t)t * LISA_HIDDEN]);
}

// forward_prefill_with_progress (runner.rs:2129-2230): chunks of `chunk` rows;
// GEMM projections, conv/recurrence over the chunk's rows, attention rows as in
// decode, residual + norms per row.
int orc_model_prefill(OrcModel* M, const uint32_t* tokens, int n, int chunk, uint32_t* argmax_out,
                      float* hidden_out) {
  if (n < 0) return -1;
  for (int t = 0; t < n; ++t)
    if ((int)tokens[t] >= M->vocab) return -2;
  if (M->position + n > M->capacity) return -3;
  if (chunk <= 0 || chunk > 512) chunk = 512;
  for (int b0 = 0; b0 < n; b0 += chunk) {
    const int m = std::min(chunk, n - b0);
    const uint32_t base = M->position;
    std::vector<float> H, B;
    std::vector<uint16_t> X;
    embed_rows(M, tokens + b0, m, H);
    for (int i = 0; i < M->layers; ++i) {
      OrcLayer& l = M->L[i];
      if (i > 0) residual_rows(H, B, m, H);
      norm_rows_bf16(H, m, l.input_norm, X);
      if (!l.attention) {
        const int si = l.state_index;
        std::vector<float> qkv, z, a, b;
        gemm_q4(X, m, l.qkv, qkv);
        gemm_q4(X, m, l.z, z);
        gemm_q4(X, m, l.a, a);
        gemm_q4(X, m, l.b, b);
        std::vector<float> conv_out((size_t)m * LISA_GDN_CONV_DIM);
        orc_gdn_conv(qkv.data(), l.conv_w.data(), &M->conv_state[(size_t)si * 3 * LISA_GDN_CONV_DIM], m,
                     conv_out.data(), nullptr);
        std::vector<uint16_t> gated((size_t)m * LISA_GDN_VALUE_DIM);
        orc_gdn_recurrence(conv_out.data(), z.data(), a.data(), b.data(), l.a_log.data(), l.dt_bias.data(),
                           l.gnorm.data(), &M->gdn_state[(size_t)si * LISA_GDN_STATE], m, gated.data(), nullptr,
                           nullptr);
        gemm_q4(gated, m, l.out, B);
      } else {
        std::vector<float> qp, kr, vr;
        gemm_q4(X, m, l.q, qp);
        gemm_q4(X, m, l.k, kr);
        gemm_q4(X, m, l.v, vr);
        const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * M->capacity * LISA_ATT_HD;
        std::vector<uint16_t> gated((size_t)m * LISA_ATT_OUT);
        orc_attention(qp.data(), kr.data(), vr.data(), l.q_norm.data(), l.k_norm.data(), &M->key_cache[off],
                      &M->value_cache[off], M->capacity, base, m, gated.data());
        gemm_q4(gated, m, l.o, B);
      }
      residual_rows(H, B, m, H);
      norm_rows_bf16(H, m, l.post_norm, X);
      std::vector<float> g, u;
      gemm_q4(X, m, l.gate, g);
      gemm_q4(X, m, l.up, u);
      std::vector<uint16_t> act((size_t)m * LISA_INTER);
      orc_silu_mul(g.data(), u.data(), m * LISA_INTER, act.data());
      gemm_q4(act, m, l.down, B);
    }
    residual_rows(H, B, m, H);
    norm_rows_bf16(H, m, M->final_norm, X);
    std::vector<float> logits;
    gemm_q4(X, m, M->head, logits);
    for (int t = 0; t < m; ++t)
      if (argmax_out) argmax_out[b0 + t] = orc_argmax(&logits[(size_t)t * M->vocab], M->vocab);
    if (hidden_out) std::memcpy(hidden_out + (size_t)b0 * LISA_HIDDEN, H.data(), sizeof(float) * H.size());
    M->position += m;
  }
  M->verify_base = -1;
  return 0;
}

// MtpRunner::forward_position_batch_with_progress (runner.rs:3494-3581): the
// drafter over n positions (token t, target hidden t) in chunks of 512 rows,
// on the prefill kernels' arithmetic: the host hidden is uploaded with the
// truncating f32 -> bf16 conversion (dtype.rs:42-47), each half of the fc
// input is an RMSNorm row (rms_norm_rows_stride, norm.metal:142-181), every
// projection is a q4 GEMM with bf16-rounded dequantized weights, attention is
// the causal rows form at the drafter's position, and the last norm's rows are
// the returned hidden. argmax_out[n], normalized_out bf16[n][5120] (nullable).
int orc_mtp_prefill(OrcModel* M, const uint32_t* tokens, const float* hiddens, int n, uint32_t* argmax_out,
                    uint16_t* normalized_out) {
  if (!M->has_mtp) return -1;
  if (n < 0) return -2;
  for (int t = 0; t < n; ++t)
    if ((int)tokens[t] >= M->vocab) return -3;
  OrcMtp& T = M->mtp;
  if (T.position + (uint32_t)n > M->capacity) return -4;
  const int chunk = 512;
  for (int b0 = 0; b0 < n; b0 += chunk) {
    const int m = std::min(chunk, n - b0);
    const uint32_t base = T.position;
    std::vector<float> E, Hh, R, B;
    embed_rows(M, tokens + b0, m, E);
    std::vector<uint16_t> fc_in((size_t)m * 2 * LISA_HIDDEN), cond(LISA_HIDDEN);
    for (int t = 0; t < m; ++t) {
      rms_norm_f(&E[(size_t)t * LISA_HIDDEN], T.pre_fc_emb.data(), LISA_HIDDEN, &fc_in[(size_t)t * 2 * LISA_HIDDEN]);
      const float* h = hiddens + (size_t)(b0 + t) * LISA_HIDDEN;
      std::vector<float> hb(LISA_HIDDEN);
      for (int c = 0; c < LISA_HIDDEN; ++c) hb[c] = bf(lisa_f32_to_bf16_trunc(h[c]));
      rms_norm_f(hb.data(), T.pre_fc_hid.data(), LISA_HIDDEN, &fc_in[(size_t)t * 2 * LISA_HIDDEN + LISA_HIDDEN]);
    }
    std::vector<float> fc;
    gemm_q4(fc_in, m, T.fc, fc);
    Hh.resize(fc.size());
    for (size_t i = 0; i < fc.size(); ++i) Hh[i] = bfr(fc[i]);  // f32_to_bf16 (norm.metal:132-137)
    std::vector<uint16_t> X;
    norm_rows_bf16(Hh, m, T.input_norm, X);
    std::vector<float> qp, kr, vr;
    gemm_q4(X, m, T.q, qp);
    gemm_q4(X, m, T.k, kr);
    gemm_q4(X, m, T.v, vr);
    std::vector<uint16_t> gated((size_t)m * LISA_ATT_OUT);
    orc_attention(qp.data(), kr.data(), vr.data(), T.q_norm.data(), T.k_norm.data(), T.key_cache.data(),
                  T.value_cache.data(), M->capacity, base, m, gated.data());
    gemm_q4(gated, m, T.o, B);
    residual_rows(Hh, B, m, R);
    norm_rows_bf16(R, m, T.post_norm, X);
    std::vector<float> g, u;
    gemm_q4(X, m, T.gate, g);
    gemm_q4(X, m, T.up, u);
    std::vector<uint16_t> act((size_t)m * LISA_INTER);
    orc_silu_mul(g.data(), u.data(), m * LISA_INTER, act.data());
    gemm_q4(act, m, T.down, B);
    residual_rows(R, B, m, Hh);
    norm_rows_bf16(Hh, m, T.final_norm, X);
    std::vector<float> logits;
    gemm_q4(X, m, M->head, logits);
    for (int t = 0; t < m; ++t)
      if (argmax_out) argmax_out[b0 + t] = orc_argmax(&logits[(size_t)t * M->vocab], M->vocab);
    if (normalized_out) std::memcpy(normalized_out + (size_t)b0 * LISA_HIDDEN, X.data(), 2 * X.size());
    T.position += m;
  }
  return 0;
}

int orc_model_commit(OrcModel* M, int rows) {
  if (M->verify_base < 0) return -1;
  if (rows < 1 || rows > 3) return -2;
  const uint32_t base = (uint32_t)M->verify_base;
  M->verify_base = -1;
  if (rows < 3) {
    const size_t gs = (size_t)M->gdn_layers * LISA_GDN_STATE;
    const size_t cs = (size_t)M->gdn_layers * 3 * LISA_GDN_CONV_DIM;
    std::memcpy(M->gdn_state.data(), &M->gdn_slots[(size_t)(rows - 1) * gs], sizeof(float) * gs);
    std::memcpy(M->conv_state.data(), &M->conv_slots[(size_t)(rows - 1) * cs], 2 * cs);
  }
  M->position = base + rows;
  return 0;
}

int orc_mtp_forward(OrcModel* M, uint32_t token, const uint16_t* cond, uint32_t* argmax_out,
                    uint16_t* normalized_out) {
  if (!M->has_mtp) return -1;
  if ((int)token >= M->vocab) return -2;
  OrcMtp& t = M->mtp;
  if (t.position >= M->capacity) return -3;
  std::vector<uint16_t> e(LISA_HIDDEN), x((size_t)2 * LISA_HIDDEN);
  orc_embed(M->embed.w.data(), M->embed.s.data(), M->embed.b.data(), token, LISA_HIDDEN, e.data());
  orc_rms_norm(e.data(), t.pre_fc_emb.data(), LISA_HIDDEN, x.data());
  orc_rms_norm(cond, t.pre_fc_hid.data(), LISA_HIDDEN, x.data() + LISA_HIDDEN);
  std::vector<XPrep> xp(1);
  prep_x(x.data(), 2 * LISA_HIDDEN, xp[0]);
  std::vector<float> fc(LISA_HIDDEN);
  q4_apply(t.fc, xp, 1, fc.data());
  std::vector<float> H(LISA_HIDDEN), R, B;
  for (int c = 0; c < LISA_HIDDEN; ++c) H[c] = bfr(fc[c]);  // f32_to_bf16 (norm.metal:132-137)
  norm_rows(H, 1, t.input_norm, xp);
  attention_block(t.q, t.k, t.v, t.o, t.q_norm, t.k_norm, t.key_cache.data(), t.value_cache.data(),
                  M->capacity, t.position, xp, 1, B);
  residual_rows(H, B, 1, R);
  norm_rows(R, 1, t.post_norm, xp, nullptr, true);
  mlp_block(t.gate, t.up, t.down, xp, 1, B);
  residual_rows(R, B, 1, H);
  std::vector<uint16_t> xn;
  norm_rows(H, 1, t.final_norm, xp, &xn, true);
  std::vector<float> logits(M->vocab);
  q4_apply(M->head, xp, 1, logits.data());
  if (argmax_out) *argmax_out = orc_argmax(logits.data(), M->vocab);
  if (normalized_out) std::memcpy(normalized_out, xn.data(), 2 * LISA_HIDDEN);
  t.position += 1;
  return 0;
}

int orc_mtp_trim(OrcModel* M, int count) {
  if (count < 0 || (uint32_t)count > M->mtp.position) return -1;
  M->mtp.position -= count;
  return 0;
}

// Test hook: the storage of one model tensor, addressed like the synthetic
// catalogue (scope = layer + 1, 0 for globals, LISA_SCOPE_MTP for the drafter;
// part 0 = packed words or plain vector, 1 = scales, 2 = biases; the drafter's
// KV caches under LISA_T_KEY_CACHE / LISA_T_VALUE_CACHE). Tests overwrite
// weights through it to pin the wiring of the model functions.
int orc_model_tensor(OrcModel* M, int scope, int kind, int part, void** ptr, size_t* bytes) {
  auto q4 = [&](Q4& q) -> int {
    if (part == 0) { *ptr = q.w.data(); *bytes = q.w.size() * 4; return 0; }
    if (part == 1) { *ptr = q.s.data(); *bytes = q.s.size() * 2; return 0; }
    if (part == 2) { *ptr = q.b.data(); *bytes = q.b.size() * 2; return 0; }
    return -1;
  };
  auto vec = [&](std::vector<uint16_t>& v) -> int {
    if (part != 0) return -1;
    *ptr = v.data();
    *bytes = v.size() * 2;
    return 0;
  };
  if (scope == LISA_SCOPE_MTP) {
    if (!M->has_mtp) return -2;
    OrcMtp& t = M->mtp;
    switch (kind) {
      case LISA_T_MTP_PRE_FC_EMB: return vec(t.pre_fc_emb);
      case LISA_T_MTP_PRE_FC_HID: return vec(t.pre_fc_hid);
      case LISA_T_INPUT_NORM: return vec(t.input_norm);
      case LISA_T_POST_NORM: return vec(t.post_norm);
      case LISA_T_FINAL_NORM: return vec(t.final_norm);
      case LISA_T_ATT_Q_NORM: return vec(t.q_norm);
      case LISA_T_ATT_K_NORM: return vec(t.k_norm);
      case LISA_T_MTP_FC: return q4(t.fc);
      case LISA_T_ATT_Q: return q4(t.q);
      case LISA_T_ATT_K: return q4(t.k);
      case LISA_T_ATT_V: return q4(t.v);
      case LISA_T_ATT_O: return q4(t.o);
      case LISA_T_MLP_GATE: return q4(t.gate);
      case LISA_T_MLP_UP: return q4(t.up);
      case LISA_T_MLP_DOWN: return q4(t.down);
      case LISA_T_KEY_CACHE: return vec(t.key_cache);
      case LISA_T_VALUE_CACHE: return vec(t.value_cache);
      default: return -3;
    }
  }
  if (scope == 0) {
    switch (kind) {
      case LISA_T_EMBED: return q4(M->embed);
      case LISA_T_LM_HEAD: return q4(M->head);
      case LISA_T_FINAL_NORM: return vec(M->final_norm);
      default: return -3;
    }
  }
  if (scope < 1 || scope > M->layers) return -4;
  OrcLayer& l = M->L[scope - 1];
  // a layer's slice of the recurrent state and of the K/V caches
  auto span = [&](void* base, size_t nbytes) -> int {
    if (part != 0) return -1;
    *ptr = base;
    *bytes = nbytes;
    return 0;
  };
  if (!l.attention && kind == LISA_T_GDN_STATE)
    return span(&M->gdn_state[(size_t)l.state_index * LISA_GDN_STATE], sizeof(float) * LISA_GDN_STATE);
  if (!l.attention && kind == LISA_T_CONV_STATE)
    return span(&M->conv_state[(size_t)l.state_index * 3 * LISA_GDN_CONV_DIM], 2 * 3 * LISA_GDN_CONV_DIM);
  if (l.attention && (kind == LISA_T_KEY_CACHE || kind == LISA_T_VALUE_CACHE)) {
    const size_t n = (size_t)LISA_ATT_KVH * M->capacity * LISA_ATT_HD;
    std::vector<uint16_t>& c = kind == LISA_T_KEY_CACHE ? M->key_cache : M->value_cache;
    return span(&c[(size_t)l.cache_index * n], 2 * n);
  }
  switch (kind) {
    case LISA_T_INPUT_NORM: return vec(l.input_norm);
    case LISA_T_POST_NORM: return vec(l.post_norm);
    case LISA_T_MLP_GATE: return q4(l.gate);
    case LISA_T_MLP_UP: return q4(l.up);
    case LISA_T_MLP_DOWN: return q4(l.down);
    default: break;
  }
  if (l.attention) {
    switch (kind) {
      case LISA_T_ATT_Q: return q4(l.q);
      case LISA_T_ATT_K: return q4(l.k);
      case LISA_T_ATT_V: return q4(l.v);
      case LISA_T_ATT_O: return q4(l.o);
      case LISA_T_ATT_Q_NORM: return vec(l.q_norm);
      case LISA_T_ATT_K_NORM: return vec(l.k_norm);
      default: return -3;
    }
  }
  switch (kind) {
    case LISA_T_GDN_QKV: return q4(l.qkv);
    case LISA_T_GDN_Z: return q4(l.z);
    case LISA_T_GDN_A: return q4(l.a);
    case LISA_T_GDN_B: return q4(l.b);
    case LISA_T_GDN_OUT: return q4(l.out);
    case LISA_T_GDN_CONV_W: return vec(l.conv_w);
    case LISA_T_GDN_A_LOG: return vec(l.a_log);
    case LISA_T_GDN_DT_BIAS: return vec(l.dt_bias);
    case LISA_T_GDN_NORM: return vec(l.gnorm);
    default: return -3;
  }
}

}  // extern "C"
