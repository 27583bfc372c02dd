// kernels.hip — gfx950 kernels of the decode path, built into
// lisa_kernels.hsaco and loaded with hipModuleLoad by the runtime bridge.
//
// Families (reference shader families in brackets):
//   lisa_qmv_k*_m*        q4 linear with fused prologue/epilogue
//                         [F1/F2 QMV, F4 embed, F6 RMSNorm, F7 residual,
//                          F8 SwiGLU, F9/F10 GDN conv + history, F5 argmax]
//   lisa_gdn_recurrence_* gated-delta recurrence + gated RMSNorm [F9 gates, F11, F12]
//   lisa_attn_partial_*   q/k norm + RoPE, KV append, split-K slice partials [F13, F14]
//   lisa_attn_merge_*     flash merge of the slices + output gate [F14]
//   lisa_step_finalize    argmax finish + device-side token/position feedback [F5]
//   lisa_synth_fill       seeded synthetic tensors
//
// Numerics: every expression below is written in the evaluation order the CPU
// oracle (oracle/oracle.cpp) restates, with the helpers of lisa_numerics.h;
// the file is compiled with -ffp-contract=off so only explicit fmas fuse.
// Reductions use fixed xor-butterfly trees (ds_swizzle within 32 lanes,
// ds_bpermute across the two halves of a wave).
#include <hip/hip_runtime.h>

#include "lisa_kernels.h"
#include "lisa_model.h"
#include "lisa_numerics.h"
#include "lisa_synth.h"

#define DEV __device__ __forceinline__

__constant__ float kRopeInvFreq[LISA_ROPE_PAIRS] = LISA_ROPE_INV_FREQ_TABLE;

// ---------------------------------------------------------------------------
// cross-lane helpers
// ---------------------------------------------------------------------------
template <int MASK>
DEV float xor_lane(float v) {
  if constexpr (MASK >= 32) {
    return __shfl_xor(v, MASK, 64);
  } else {
    // ds_swizzle bitmask mode: and_mask = 0x1f, or_mask = 0, xor_mask = MASK.
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (MASK << 10) | 0x1f));
  }
}

DEV float tree64(float v) {
  v = v + xor_lane<32>(v);
  v = v + xor_lane<16>(v);
  v = v + xor_lane<8>(v);
  v = v + xor_lane<4>(v);
  v = v + xor_lane<2>(v);
  v = v + xor_lane<1>(v);
  return v;
}

DEV float tree16(float v) {
  v = v + xor_lane<8>(v);
  v = v + xor_lane<4>(v);
  v = v + xor_lane<2>(v);
  v = v + xor_lane<1>(v);
  return v;
}

DEV float max64(float v) {
  v = fmaxf(v, xor_lane<32>(v));
  v = fmaxf(v, xor_lane<16>(v));
  v = fmaxf(v, xor_lane<8>(v));
  v = fmaxf(v, xor_lane<4>(v));
  v = fmaxf(v, xor_lane<2>(v));
  v = fmaxf(v, xor_lane<1>(v));
  return v;
}

DEV float bf2f(uint16_t h) { return lisa_bf16_to_f32(h); }
DEV float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
DEV float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// ===========================================================================
// q4 linear
// ===========================================================================
// Work split: 256 threads = 4 waves; a wave owns an 8-row tile; the 16 lanes
// of row-group rp (lane/16) own rows (2rp, 2rp+1) of the tile (for GATEUP the
// gate and up rows of one output), and lane li = lane%16 walks the 64-wide
// groups g = li, li+16, ... of K. Per group and row the partial is
//   acc_lo = fma chain x[k_even] * lo_nibble,  acc_hi = fma chain (x[k_odd]/16) * (byte & 0xf0)
//   P = fma(scale, acc_lo + acc_hi, bias * X_g)
// (qmv.metal:26-55 with 64-wide groups), accumulated per lane in ascending g,
// then tree16 across the row-group (qmv.metal:71-75).
//
// x lives in LDS, one copy per input row, odd positions pre-divided by 16
// (exact), 16-byte chunks rotated by the group index so that the 16 lanes of
// a row-group hit distinct banks. X_g (sum of the group's 64 x values in
// ascending order) sits after it.

template <int K, int M, bool XF32>
struct QmvLds {
  static constexpr int G = K / 64;
  /* prologues that normalize a 5120-wide row need a staging row in LDS */
  static constexpr bool NORM = (K == LISA_HIDDEN || K == 2 * LISA_HIDDEN);
  static constexpr int XBYTES = M * K * (XF32 ? 4 : 2);
  static constexpr int GBYTES = M * G * 4 + (64 + 32 * M) * 4;
  static constexpr int TBYTES = NORM ? LISA_HIDDEN * 4 : 0;
  static constexpr int BYTES = XBYTES + GBYTES + TBYTES;
};

template <bool XF32>
DEV void lds_put_x(unsigned char* lds, int K, int m, int k, float v) {
  const int g = k >> 6;
  const float vs = (k & 1) ? v / 16.0f : v;
  if (XF32) {
    const int c = (k >> 2) & 15;
    float* xs = reinterpret_cast<float*>(lds) + (size_t)m * K;
    xs[g * 64 + 4 * ((c + g) & 15) + (k & 3)] = vs;
  } else {
    const int c = (k >> 3) & 7;
    uint16_t* xb = reinterpret_cast<uint16_t*>(lds) + (size_t)m * K;
    xb[g * 64 + 8 * ((c + g) & 7) + (k & 7)] = lisa_f32_to_bf16(vs);
  }
}

template <bool XF32>
DEV float lds_get_x(const unsigned char* lds, int K, int m, int k) {
  const int g = k >> 6;
  float vs;
  if (XF32) {
    const int c = (k >> 2) & 15;
    const float* xs = reinterpret_cast<const float*>(lds) + (size_t)m * K;
    vs = xs[g * 64 + 4 * ((c + g) & 15) + (k & 3)];
  } else {
    const int c = (k >> 3) & 7;
    const uint16_t* xb = reinterpret_cast<const uint16_t*>(lds) + (size_t)m * K;
    vs = bf2f(xb[g * 64 + 8 * ((c + g) & 7) + (k & 7)]);
  }
  return (k & 1) ? vs * 16.0f : vs;
}

// RMSNorm statistic of one 5120-wide row given each thread's partial sum of
// squares over its elements j = tid + 256 i: rows-of-256 tree (norm.metal:10-47).
DEV float rms_inv_5120(float s, float* red, int tid) {
  s = tree64(s);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  return lisa_rsqrt(tot / (float)LISA_HIDDEN + LISA_EPS);
}

DEV float embed_value(const uint32_t* ew, const uint32_t* esb, uint32_t tok, int j) {
  const uint32_t word = ew[(size_t)tok * (LISA_HIDDEN / 8) + (j >> 3)];
  const uint32_t q = (word >> ((j & 7) * 4)) & 0xfu;
  const uint32_t sb = esb[(size_t)tok * (LISA_HIDDEN / 64) + (j >> 6)];
  // embed.metal:24-26: float(q) * scale + bias, stored bf16
  return lisa_bf16r((float)q * lo_bf(sb) + hi_bf(sb));
}

// Fill LDS with x (and X_g) for all M rows according to the prologue mode.
template <int K, int M, bool XF32>
DEV void qmv_prologue(const LisaQmvParams& p, unsigned char* lds) {
  constexpr int G = K / 64;
  const int tid = threadIdx.x;
  float* gsum = reinterpret_cast<float*>(lds + QmvLds<K, M, XF32>::XBYTES);
  float* red = gsum + M * G;
  const bool writer = blockIdx.x == 0;
  if (p.pro_mode == LISA_PRO_LOADX) {
    for (int m = 0; m < M; ++m)
      for (int k8 = tid; k8 < K / 8; k8 += 256) {
        const uint4 v = *reinterpret_cast<const uint4*>(p.x_in + (size_t)m * K + 8 * k8);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lds_put_x<XF32>(lds, K, m, 8 * k8 + 2 * e, lo_bf(w[e]));
          lds_put_x<XF32>(lds, K, m, 8 * k8 + 2 * e + 1, hi_bf(w[e]));
        }
      }
  } else if constexpr (QmvLds<K, M, XF32>::NORM) {
    float* tmp = reinterpret_cast<float*>(lds + QmvLds<K, M, XF32>::XBYTES + QmvLds<K, M, XF32>::GBYTES);
    const int halves = (p.pro_mode == LISA_PRO_MTPFC) ? 2 : 1;
    for (int m = 0; m < M; ++m) {
      for (int hf = 0; hf < halves; ++hf) {
        float ss = 0.0f;
#pragma unroll 4
        for (int i = 0; i < LISA_HIDDEN / 256; ++i) {
          const int j = tid + 256 * i;
          const size_t off = (size_t)m * LISA_HIDDEN + j;
          float v;
          switch (p.pro_mode) {
            case LISA_PRO_RESNORM: v = lisa_bf16r(bf2f(p.h_in[off]) + lisa_bf16r(p.o_in[off])); break;
            case LISA_PRO_EMBED: v = embed_value(p.emb_w, p.emb_sb, p.tokens[m], j); break;
            case LISA_PRO_CAST: v = lisa_bf16r(p.o_in[off]); break;
            case LISA_PRO_NORM: v = bf2f(p.h_in[off]); break;
            default: /* MTPFC */
              v = (hf == 0) ? embed_value(p.emb_w, p.emb_sb, p.tokens[0], j) : bf2f(p.x_in[j]);
              break;
          }
          tmp[j] = v;
          ss = ss + v * v;
        }
        const float inv = rms_inv_5120(ss, red, tid);
        const uint16_t* nw = (hf == 0) ? p.norm_w : p.norm_w2;
#pragma unroll 4
        for (int i = 0; i < LISA_HIDDEN / 256; ++i) {
          const int j = tid + 256 * i;
          const float r = tmp[j];
          const float x = lisa_bf16r((r * inv) * bf2f(nw[j]));
          lds_put_x<XF32>(lds, K, m, hf * LISA_HIDDEN + j, x);
          if (writer) {
            if (p.r_out && p.pro_mode != LISA_PRO_MTPFC)
              p.r_out[(size_t)m * LISA_HIDDEN + j] = lisa_f32_to_bf16(r);
            if (p.x_out) p.x_out[(size_t)m * K + hf * LISA_HIDDEN + j] = lisa_f32_to_bf16(x);
          }
        }
        __syncthreads();
      }
    }
  }
  __syncthreads();
  for (int m = 0; m < M; ++m)
    for (int g = tid; g < G; g += 256) {
      float s = 0.0f;
      for (int k = 0; k < 64; ++k) s = s + lds_get_x<XF32>(lds, K, m, 64 * g + k);
      gsum[m * G + g] = s;
    }
  __syncthreads();
}

// One group's dot for the two weight rows of a lane and M input rows. The
// x values of a 4-element chunk are loaded once and used by both rows.
template <int K, int M, bool XF32>
DEV void group_dot2(const unsigned char* lds, int g, const uint32_t (&w0)[8], const uint32_t (&w1)[8],
                    uint32_t sb0, uint32_t sb1, const float* gsum, float* T0, float* T1) {
  constexpr int G = K / 64;
  float lo0[M], hi0[M], lo1[M], hi1[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { lo0[m] = 0.0f; hi0[m] = 0.0f; lo1[m] = 0.0f; hi1[m] = 0.0f; }
  if constexpr (XF32) {
    const float* xs = reinterpret_cast<const float*>(lds) + g * 64;
#pragma unroll 4
    for (int c = 0; c < 16; ++c) {
      const int sh = 16 * (c & 1);
      const uint32_t ml0 = w0[c >> 1] & 0x0f0f0f0fu, mh0 = w0[c >> 1] & 0xf0f0f0f0u;
      const uint32_t ml1 = w1[c >> 1] & 0x0f0f0f0fu, mh1 = w1[c >> 1] & 0xf0f0f0f0u;
      const float a0 = (float)((ml0 >> sh) & 0xffu), b0 = (float)((mh0 >> sh) & 0xffu);
      const float a1 = (float)((ml0 >> (sh + 8)) & 0xffu), b1 = (float)((mh0 >> (sh + 8)) & 0xffu);
      const float c0 = (float)((ml1 >> sh) & 0xffu), d0 = (float)((mh1 >> sh) & 0xffu);
      const float c1 = (float)((ml1 >> (sh + 8)) & 0xffu), d1 = (float)((mh1 >> (sh + 8)) & 0xffu);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float4 x4 = *reinterpret_cast<const float4*>(xs + (size_t)m * K + 4 * ((c + g) & 15));
        lo0[m] = lisa_fma(x4.x, a0, lo0[m]);
        hi0[m] = lisa_fma(x4.y, b0, hi0[m]);
        lo0[m] = lisa_fma(x4.z, a1, lo0[m]);
        hi0[m] = lisa_fma(x4.w, b1, hi0[m]);
        lo1[m] = lisa_fma(x4.x, c0, lo1[m]);
        hi1[m] = lisa_fma(x4.y, d0, hi1[m]);
        lo1[m] = lisa_fma(x4.z, c1, lo1[m]);
        hi1[m] = lisa_fma(x4.w, d1, hi1[m]);
      }
    }
  } else {
    const uint16_t* xb = reinterpret_cast<const uint16_t*>(lds) + g * 64;
#pragma unroll 2
    for (int c = 0; c < 8; ++c) {
      const uint32_t ml0 = w0[c] & 0x0f0f0f0fu, mh0 = w0[c] & 0xf0f0f0f0u;
      const uint32_t ml1 = w1[c] & 0x0f0f0f0fu, mh1 = w1[c] & 0xf0f0f0f0u;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4 xv = *reinterpret_cast<const uint4*>(xb + (size_t)m * K + 8 * ((c + g) & 7));
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float xe = lo_bf(xw[b]), xo = hi_bf(xw[b]);
          lo0[m] = lisa_fma(xe, (float)((ml0 >> (8 * b)) & 0xffu), lo0[m]);
          hi0[m] = lisa_fma(xo, (float)((mh0 >> (8 * b)) & 0xffu), hi0[m]);
          lo1[m] = lisa_fma(xe, (float)((ml1 >> (8 * b)) & 0xffu), lo1[m]);
          hi1[m] = lisa_fma(xo, (float)((mh1 >> (8 * b)) & 0xffu), hi1[m]);
        }
      }
    }
  }
  const float s0 = lo_bf(sb0), bb0 = hi_bf(sb0), s1 = lo_bf(sb1), bb1 = hi_bf(sb1);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float xg = gsum[m * G + g];
    T0[m] = T0[m] + lisa_fma(s0, lo0[m] + hi0[m], bb0 * xg);
    T1[m] = T1[m] + lisa_fma(s1, lo1[m] + hi1[m], bb1 * xg);
  }
}

template <int M>
DEV void conv_epilogue(const LisaQmvParams& p, float* out, int c, const float* pr) {
  const int C = LISA_GDN_CONV_DIM;
  float hist[3 + M];
#pragma unroll
  for (int i = 0; i < 3; ++i) hist[i] = bf2f(p.conv_state[(size_t)i * C + c]);
#pragma unroll
  for (int t = 0; t < M; ++t) hist[3 + t] = lisa_bf16r(pr[t]);
  float w[4];
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) w[tap] = bf2f(p.conv_w[(size_t)c * 4 + tap]);
#pragma unroll
  for (int t = 0; t < M; ++t) {
    // gdn.metal:163-170: acc += x * w over the 4 taps, conv = bf16(acc), out = bf16(silu(conv))
    float acc = 0.0f;
#pragma unroll
    for (int tap = 0; tap < 4; ++tap) acc = acc + hist[t + tap] * w[tap];
    out[(size_t)t * C + c] = lisa_bf16r(lisa_silu_exp(lisa_bf16r(acc)));
    if (p.capture && p.conv_slots && t + 1 < M) {
      uint16_t* sl = p.conv_slots + (size_t)t * p.conv_slot_stride;
#pragma unroll
      for (int i = 0; i < 3; ++i) sl[(size_t)i * C + c] = lisa_f32_to_bf16(hist[t + 1 + i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) p.conv_state[(size_t)i * C + c] = lisa_f32_to_bf16(hist[M + i]);
}

DEV bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return (v > bv) || (v == bv && i < bi);
}

template <int K, int M, bool XF32>
DEV void qmv_body(const LisaQmvParams& p, unsigned char* lds) {
  constexpr int G = K / 64;
  constexpr int ITER = G / 16;
  static_assert(G % 16 == 0, "K must be a multiple of 1024");
  qmv_prologue<K, M, XF32>(p, lds);
  const float* gsum = reinterpret_cast<const float*>(lds + QmvLds<K, M, XF32>::XBYTES);
  float* red = const_cast<float*>(gsum) + M * G;

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, rp = lane >> 4;
  const uint32_t tiles = p.tile_start[p.n_mats];
  float best_v[M];
  uint32_t best_i[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { best_v[m] = -INFINITY; best_i[m] = 0xffffffffu; }

  // ksplit == 1: each wave owns its own 8-row tile over the whole of K.
  // ksplit == 4: the four waves share one 8-row tile; wave w walks the group
  // iterations [ITER*w/4, ITER*(w+1)/4) and the wave results are combined as
  // (W0 + W1) + (W2 + W3) by wave 0.
  const bool split = p.ksplit == 4;
  const uint32_t tstep = split ? gridDim.x : gridDim.x * 4;
  const int it0 = split ? (ITER * wv) / 4 : 0, it1 = split ? (ITER * (wv + 1)) / 4 : ITER;
  float* kred = red + 64;  // [4 waves][8 rows][M]
  for (uint32_t tile = split ? blockIdx.x : blockIdx.x * 4 + wv; tile < tiles; tile += tstep) {
    int e = 0;
    while (e + 1 < (int)p.n_mats && tile >= p.tile_start[e + 1]) ++e;
    const LisaQ4Mat mt = p.mats[e];
    const uint32_t lt = tile - p.tile_start[e];
    uint32_t r0, r1;
    const uint32_t *w0, *w1, *s0, *s1;
    if (mt.kind == LISA_EPI_GATEUP) {
      r0 = r1 = lt * 4 + rp;
      w0 = mt.w; s0 = mt.sb; w1 = mt.w2; s1 = mt.sb2;
    } else {
      r0 = lt * 8 + 2 * rp;
      r1 = r0 + 1;
      w0 = w1 = mt.w; s0 = s1 = mt.sb;
    }
    const bool v0 = r0 < mt.rows, v1 = r1 < mt.rows;
    const uint32_t c0 = v0 ? r0 : mt.rows - 1, c1 = v1 ? r1 : mt.rows - 1;
    const uint4* wp0 = reinterpret_cast<const uint4*>(w0 + (size_t)c0 * (K / 8));
    const uint4* wp1 = reinterpret_cast<const uint4*>(w1 + (size_t)c1 * (K / 8));
    const uint32_t* sp0 = s0 + (size_t)c0 * G;
    const uint32_t* sp1 = s1 + (size_t)c1 * G;

    float T0[M], T1[M];
#pragma unroll
    for (int m = 0; m < M; ++m) { T0[m] = 0.0f; T1[m] = 0.0f; }

    if (it0 < it1) {
      const int gf = 16 * it0 + li;
      uint4 na0 = wp0[2 * gf], nb0 = wp0[2 * gf + 1], na1 = wp1[2 * gf], nb1 = wp1[2 * gf + 1];
      uint32_t ns0 = sp0[gf], ns1 = sp1[gf];
      for (int it = it0; it < it1; ++it) {
        const int g = 16 * it + li;
        const uint32_t cw0[8] = {na0.x, na0.y, na0.z, na0.w, nb0.x, nb0.y, nb0.z, nb0.w};
        const uint32_t cw1[8] = {na1.x, na1.y, na1.z, na1.w, nb1.x, nb1.y, nb1.z, nb1.w};
        const uint32_t q0 = ns0, q1 = ns1;
        if (it + 1 < it1) {
          const int gn = g + 16;
          na0 = wp0[2 * gn]; nb0 = wp0[2 * gn + 1];
          na1 = wp1[2 * gn]; nb1 = wp1[2 * gn + 1];
          ns0 = sp0[gn]; ns1 = sp1[gn];
        }
        group_dot2<K, M, XF32>(lds, g, cw0, cw1, q0, q1, gsum, T0, T1);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) { T0[m] = tree16(T0[m]); T1[m] = tree16(T1[m]); }
    if (split) {
      if (li == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          kred[(wv * 8 + 2 * rp) * M + m] = T0[m];
          kred[(wv * 8 + 2 * rp + 1) * M + m] = T1[m];
        }
      }
      __syncthreads();
      if (wv == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const int a = 2 * rp, b = 2 * rp + 1;
          T0[m] = (kred[(0 * 8 + a) * M + m] + kred[(1 * 8 + a) * M + m]) +
                  (kred[(2 * 8 + a) * M + m] + kred[(3 * 8 + a) * M + m]);
          T1[m] = (kred[(0 * 8 + b) * M + m] + kred[(1 * 8 + b) * M + m]) +
                  (kred[(2 * 8 + b) * M + m] + kred[(3 * 8 + b) * M + m]);
        }
      }
      __syncthreads();
      if (wv != 0) continue;
    }

    switch (mt.kind) {
      case LISA_EPI_STORE: {
        float* out = static_cast<float*>(mt.out);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          if (li == 2 * m && v0) out[(size_t)m * mt.rows + r0] = T0[m];
          if (li == 2 * m + 1 && v1) out[(size_t)m * mt.rows + r1] = T1[m];
        }
        break;
      }
      case LISA_EPI_GATEUP: {
        uint16_t* out = static_cast<uint16_t*>(mt.out);
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (li == m && v0) {
            // mlp.metal:11-16
            const float gte = lisa_bf16r(T0[m]), up = lisa_bf16r(T1[m]);
            out[(size_t)m * mt.rows + r0] = lisa_f32_to_bf16(lisa_silu_exp2(gte) * up);
          }
        break;
      }
      case LISA_EPI_CONV: {
        if (li == 0 && v0) conv_epilogue<M>(p, static_cast<float*>(mt.out), (int)r0, T0);
        if (li == 1 && v1) conv_epilogue<M>(p, static_cast<float*>(mt.out), (int)r1, T1);
        break;
      }
      default: { /* ARGMAX */
        float* out = static_cast<float*>(mt.out);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          if (li == 2 * m && v0) {
            out[(size_t)m * mt.rows + r0] = T0[m];
            if (better(T0[m], r0, best_v[m], best_i[m])) { best_v[m] = T0[m]; best_i[m] = r0; }
          }
          if (li == 2 * m + 1 && v1) {
            out[(size_t)m * mt.rows + r1] = T1[m];
            if (better(T1[m], r1, best_v[m], best_i[m])) { best_v[m] = T1[m]; best_i[m] = r1; }
          }
        }
        break;
      }
    }
  }

  if (p.am_val) {
    // workgroup-level (max, lowest index) per input row
    __syncthreads();
    float* cv = red;  // reuse: [M][256] would not fit; reduce per m sequentially
    uint32_t* ci = reinterpret_cast<uint32_t*>(red + 32);
    for (int m = 0; m < M; ++m) {
      float v = best_v[m];
      uint32_t i = best_i[m];
      // wave reduction
#pragma unroll
      for (int msk = 1; msk < 64; msk <<= 1) {
        const float ov = __shfl_xor(v, msk, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)i, msk, 64);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
      }
      if (lane == 0) { cv[wv] = v; ci[wv] = i; }
      __syncthreads();
      if (threadIdx.x == 0) {
        float bv = cv[0];
        uint32_t bi = ci[0];
        for (int q = 1; q < 4; ++q)
          if (better(cv[q], ci[q], bv, bi)) { bv = cv[q]; bi = ci[q]; }
        p.am_val[(size_t)m * gridDim.x + blockIdx.x] = bv;
        p.am_idx[(size_t)m * gridDim.x + blockIdx.x] = bi;
      }
      __syncthreads();
    }
  }
}

#define QMV_KERNEL(K, M, XF32)                                                           \
  extern "C" __global__ __launch_bounds__(256) void lisa_qmv_k##K##_m##M(LisaQmvParams p) { \
    __shared__ __attribute__((aligned(16))) unsigned char lds[QmvLds<K, M, XF32>::BYTES];  \
    qmv_body<K, M, XF32>(p, lds);                                                        \
  }

QMV_KERNEL(5120, 1, true)
QMV_KERNEL(5120, 3, true)
QMV_KERNEL(6144, 1, true)
QMV_KERNEL(6144, 3, true)
QMV_KERNEL(10240, 1, true)
QMV_KERNEL(17408, 1, true)
QMV_KERNEL(17408, 3, false)
QMV_KERNEL(1024, 1, true)
QMV_KERNEL(1024, 3, true)

// ===========================================================================
// GDN recurrence (gdn.metal:245-328) + gates (gdn.metal:170-205) + gated
// RMSNorm (gdn.metal:367-391). One workgroup per value head, 512 threads:
// thread (v, q) = (tid/4, tid%4) owns state row v, columns [32q, 32q+32).
// ===========================================================================
template <int M>
DEV void gdn_body(const LisaGdnParams& p) {
  const int h = blockIdx.x, kh = h / (LISA_GDN_VH / LISA_GDN_KH);
  const int tid = threadIdx.x, v = tid >> 2, q = tid & 3, lane = tid & 63, wave = tid >> 6;
  __shared__ float qn[128], kn[128], ybuf[128], sc[4];
  float* srow = p.state + (size_t)h * 128 * 128 + (size_t)v * 128 + 32 * q;
  float S[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 f = reinterpret_cast<const float4*>(srow)[i];
    S[4 * i] = f.x; S[4 * i + 1] = f.y; S[4 * i + 2] = f.z; S[4 * i + 3] = f.w;
  }
  for (int t = 0; t < M; ++t) {
    const float* co = p.conv_out + (size_t)t * LISA_GDN_CONV_DIM;
    if (wave < 2) {
      // q (wave 0) / k (wave 1) RMS with tree128, scaled 1/128 and 1/sqrt(128)
      const float* src = co + (wave == 0 ? 0 : LISA_GDN_KEY_DIM) + kh * 128;
      const float c0 = src[lane], c1 = src[lane + 64];
      const float tot = tree64(c0 * c0 + c1 * c1);
      const float inv = lisa_rsqrt(tot / 128.0f + 1.0e-6f) * (wave == 0 ? p.q_scale : p.k_scale);
      float* dst = wave == 0 ? qn : kn;
      dst[lane] = lisa_bf16r(c0 * inv);
      dst[lane + 64] = lisa_bf16r(c1 * inv);
    } else if (tid == 128) {
      const float beta = lisa_bf16r(lisa_sigmoid_exp(lisa_bf16r(p.b[(size_t)t * LISA_GDN_VH + h])));
      const float dt_arg = lisa_bf16r(lisa_bf16r(p.a[(size_t)t * LISA_GDN_VH + h]) + bf2f(p.dt_bias[h]));
      const float dt = lisa_bf16r(lisa_softplus(dt_arg));
      sc[0] = beta;
      sc[1] = lisa_expf(-lisa_expf(bf2f(p.a_log[h])) * dt);
    }
    __syncthreads();
    const float beta = sc[0], decay = sc[1];
#pragma unroll
    for (int k = 0; k < 32; ++k) S[k] = S[k] * decay;
    float pk = S[0] * kn[32 * q];
#pragma unroll
    for (int k = 1; k < 32; ++k) pk = lisa_fma(S[k], kn[32 * q + k], pk);
    pk = pk + xor_lane<1>(pk);
    pk = pk + xor_lane<2>(pk);
    const float vval = co[2 * LISA_GDN_KEY_DIM + h * 128 + v];
    const float delta = (vval - pk) * beta;
#pragma unroll
    for (int k = 0; k < 32; ++k) S[k] = lisa_fma(delta, kn[32 * q + k], S[k]);
    float py = S[0] * qn[32 * q];
#pragma unroll
    for (int k = 1; k < 32; ++k) py = lisa_fma(S[k], qn[32 * q + k], py);
    py = py + xor_lane<1>(py);
    py = py + xor_lane<2>(py);
    if (q == 0) ybuf[v] = lisa_bf16r(py);
    if (p.capture && p.slots && t + 1 < M) {
      float4* dst = reinterpret_cast<float4*>(p.slots + (size_t)t * p.slot_stride + (size_t)h * 128 * 128 +
                                              (size_t)v * 128 + 32 * q);
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = make_float4(S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]);
    }
    __syncthreads();
    if (wave == 0) {
      const float y0 = ybuf[lane], y1 = ybuf[lane + 64];
      const float tot = tree64(y0 * y0 + y1 * y1);
      if (lane == 0) sc[2] = lisa_rsqrt(tot / 128.0f + LISA_EPS);
    }
    __syncthreads();
    if (tid < 128) {
      const float y = ybuf[tid];
      const float n = lisa_bf16r((y * sc[2]) * bf2f(p.norm_w[tid]));
      const size_t o = (size_t)t * LISA_GDN_VALUE_DIM + h * 128 + tid;
      const float z = lisa_bf16r(p.z[o]);
      p.gated[o] = lisa_f32_to_bf16(n * lisa_silu_exp(z));
      if (p.y_out) p.y_out[o] = y;
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    reinterpret_cast<float4*>(srow)[i] = make_float4(S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]);
}

extern "C" __global__ __launch_bounds__(512) void lisa_gdn_recurrence_m1(LisaGdnParams p) { gdn_body<1>(p); }
extern "C" __global__ __launch_bounds__(512) void lisa_gdn_recurrence_m3(LisaGdnParams p) { gdn_body<3>(p); }

// ===========================================================================
// split-K decode attention
// ===========================================================================
// Norm + partial RoPE of one 256-wide head by one wave: lane l holds elements
// l, l+64, l+128, l+192; the sum of squares is tree64 of each element column
// then (W0+W1)+(W2+W3) — the rows-of-256 tree with one element per thread
// (attention.metal:99-114, 118-155).
DEV void head_norm_rope_wave(const float* raw, const uint16_t* w, uint32_t pos, int lane, float out[4]) {
  float v[4], wsum[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = lisa_bf16r(raw[lane + 64 * j]);
    wsum[j] = tree64(v[j] * v[j]);
  }
  const float tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  const float inv = lisa_rsqrt(tot / 256.0f + LISA_EPS);
  float n[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) n[j] = (v[j] * inv) * bf2f(w[lane + 64 * j]);
  const float other = xor_lane<32>(n[0]);  // n[l+32] for l<32, n[l-32] for l>=32
  const float angle = (float)pos * kRopeInvFreq[lane & 31];
  float s, c;
  lisa_sincosf(angle, &s, &c);
  if (lane < 32)
    out[0] = lisa_bf16r(n[0] * c - other * s);
  else
    out[0] = lisa_bf16r(n[0] * c + other * s);
#pragma unroll
  for (int j = 1; j < 4; ++j) out[j] = lisa_bf16r(n[j]);
}

template <int M>
DEV void attn_partial_body(const LisaAttnParams& p) {
  constexpr int T = LISA_ATT_SLICE, HD = LISA_ATT_HD, KP = HD + 8;
  const uint32_t base = *p.pos;
  const int s = blockIdx.x, kvh = blockIdx.y;
  const uint32_t t0 = (uint32_t)s * T;
  if (t0 >= base + M) return;
  __shared__ __attribute__((aligned(16))) uint16_t Kt[T * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[T * HD];
  __shared__ __attribute__((aligned(16))) float qv[M * 6 * HD];
  __shared__ float pb[M * 6 * T];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t cache_base = (size_t)kvh * p.capacity * HD;

  // 1. rows of the slice already in the cache (positions < base)
  const int nold = (base > t0) ? (int)min((uint32_t)T, base - t0) : 0;
  for (int c = tid; c < nold * (HD / 8); c += 256) {
    const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
    const size_t off = cache_base + (size_t)(t0 + row) * HD + col;
    *reinterpret_cast<uint4*>(&Kt[row * KP + col]) = *reinterpret_cast<const uint4*>(p.key_cache + off);
    *reinterpret_cast<uint4*>(&Vt[row * HD + col]) = *reinterpret_cast<const uint4*>(p.value_cache + off);
  }
  // 2. rows appended by this step that fall into the slice (kv_cache_store_decode)
  if (wave < M) {
    const uint32_t pos = base + wave;
    if (pos >= t0 && pos < t0 + T && pos < p.capacity) {
      float kr[4];
      head_norm_rope_wave(p.k_raw + (size_t)wave * LISA_ATT_KV_OUT + kvh * HD, p.k_norm_w, pos, lane, kr);
      const int row = (int)(pos - t0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        const uint16_t kb = lisa_f32_to_bf16(kr[j]);
        const uint16_t vb = lisa_f32_to_bf16(p.v_raw[(size_t)wave * LISA_ATT_KV_OUT + kvh * HD + d]);
        Kt[row * KP + d] = kb;
        Vt[row * HD + d] = vb;
        p.key_cache[cache_base + (size_t)pos * HD + d] = kb;
        p.value_cache[cache_base + (size_t)pos * HD + d] = vb;
      }
    }
  }
  // 3. normalized, rotated queries of the 6 heads sharing this KV head
  for (int pr = wave; pr < 6 * M; pr += 4) {
    const int t = pr / 6, i = pr % 6, h = kvh * 6 + i;
    float qo[4];
    head_norm_rope_wave(p.q_proj + (size_t)t * LISA_ATT_Q_OUT + h * 512, p.q_norm_w, base + t, lane, qo);
#pragma unroll
    for (int j = 0; j < 4; ++j) qv[(t * 6 + i) * HD + lane + 64 * j] = qo[j];
  }
  __syncthreads();
  // 4. scores and slice softmax statistics: lane = token of the slice
  for (int pr = wave; pr < 6 * M; pr += 4) {
    const int t = pr / 6, i = pr % 6, h = kvh * 6 + i;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    float score = -INFINITY;
    if (lane < n) {
      const float* qh = qv + (t * 6 + i) * HD;
      const uint16_t* kr = Kt + lane * KP;
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 4
      for (int d = 0; d < HD; d += 8) {
        const uint4 kk = *reinterpret_cast<const uint4*>(kr + d);
        const float4 qa = *reinterpret_cast<const float4*>(qh + d);
        const float4 qb = *reinterpret_cast<const float4*>(qh + d + 4);
        a0 = lisa_fma(qa.x, lo_bf(kk.x), a0);
        a1 = lisa_fma(qa.y, hi_bf(kk.x), a1);
        a2 = lisa_fma(qa.z, lo_bf(kk.y), a2);
        a3 = lisa_fma(qa.w, hi_bf(kk.y), a3);
        a0 = lisa_fma(qb.x, lo_bf(kk.z), a0);
        a1 = lisa_fma(qb.y, hi_bf(kk.z), a1);
        a2 = lisa_fma(qb.z, lo_bf(kk.w), a2);
        a3 = lisa_fma(qb.w, hi_bf(kk.w), a3);
      }
      score = ((a0 + a1) + (a2 + a3)) * 0.0625f;
    }
    const float mx = max64(score);
    const float pv = (lane < n) ? lisa_exp2f(1.4426950408889634f * (score - mx)) : 0.0f;
    const float den = tree64(pv);
    pb[(t * 6 + i) * T + lane] = pv;
    if (lane == 0) {
      float* ml = p.part_ml + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * 2;
      ml[0] = mx;
      ml[1] = den;
    }
  }
  __syncthreads();
  // 5. P.V: thread = output dimension
  for (int t = 0; t < M; ++t) {
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    float acc[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) acc[i] = 0.0f;
    for (int tok = 0; tok < n; ++tok) {
      const float vv = bf2f(Vt[tok * HD + tid]);
#pragma unroll
      for (int i = 0; i < 6; ++i) acc[i] = lisa_fma(pb[(t * 6 + i) * T + tok], vv, acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int h = kvh * 6 + i;
      p.part_o[(((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * HD + tid] = acc[i];
    }
  }
}

#define ATT_MAX_SLICES 1024
template <int M>
DEV void attn_merge_body(const LisaAttnParams& p) {
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const uint32_t ctx = *p.pos + t + 1;
  const int used = (int)((ctx + LISA_ATT_SLICE - 1) / LISA_ATT_SLICE);
  __shared__ float ws[ATT_MAX_SLICES], dn[ATT_MAX_SLICES], red[4];
  const float* ml = p.part_ml + ((size_t)t * LISA_ATT_QH + h) * p.s_max * 2;
  float mx = -INFINITY;
  for (int s = tid; s < used; s += 256) mx = fmaxf(mx, ml[2 * s]);
  mx = max64(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float gmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  for (int s = tid; s < used; s += 256) {
    ws[s] = lisa_exp2f(1.4426950408889634f * (ml[2 * s] - gmax));
    dn[s] = ml[2 * s + 1];
  }
  __syncthreads();
  const float* po = p.part_o + ((size_t)t * LISA_ATT_QH + h) * p.s_max * LISA_ATT_HD + tid;
  float res = 0.0f, tot = 0.0f;
  for (int s = 0; s < used; ++s) {
    res = lisa_fma(ws[s], po[(size_t)s * LISA_ATT_HD], res);
    tot = lisa_fma(ws[s], dn[s], tot);
  }
  const float o = res / tot;
  const float g = lisa_bf16r(p.q_proj[(size_t)t * LISA_ATT_Q_OUT + h * 512 + 256 + tid]);
  p.gated[(size_t)t * LISA_ATT_OUT + h * LISA_ATT_HD + tid] = lisa_f32_to_bf16(o * lisa_sigmoid_exp2(g));
}

extern "C" __global__ __launch_bounds__(256) void lisa_attn_partial_m1(LisaAttnParams p) { attn_partial_body<1>(p); }
extern "C" __global__ __launch_bounds__(256) void lisa_attn_partial_m3(LisaAttnParams p) { attn_partial_body<3>(p); }
extern "C" __global__ __launch_bounds__(256) void lisa_attn_merge_m1(LisaAttnParams p) { attn_merge_body<1>(p); }
extern "C" __global__ __launch_bounds__(256) void lisa_attn_merge_m3(LisaAttnParams p) { attn_merge_body<3>(p); }

// ===========================================================================
// argmax finish (runner.rs:1077-1095 on the device) + step bookkeeping
// ===========================================================================
extern "C" __global__ __launch_bounds__(256) void lisa_step_finalize(LisaFinalizeParams p) {
  __shared__ float cv[4];
  __shared__ uint32_t ci[4];
  __shared__ uint32_t res[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (uint32_t m = 0; m < p.m_rows; ++m) {
    float v = -INFINITY;
    uint32_t i = 0xffffffffu;
    for (uint32_t j = tid; j < p.n_part; j += 256) {
      const float ov = p.am_val[(size_t)m * p.n_part + j];
      const uint32_t oi = p.am_idx[(size_t)m * p.n_part + j];
      if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    for (int msk = 1; msk < 64; msk <<= 1) {
      const float ov = __shfl_xor(v, msk, 64);
      const uint32_t oi = (uint32_t)__shfl_xor((int)i, msk, 64);
      if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    if (lane == 0) { cv[wave] = v; ci[wave] = i; }
    __syncthreads();
    if (tid == 0) {
      float bv = cv[0];
      uint32_t bi = ci[0];
      for (int q = 1; q < 4; ++q)
        if (better(cv[q], ci[q], bv, bi)) { bv = cv[q]; bi = ci[q]; }
      if (bi == 0xffffffffu) bi = 0;
      res[m & 3] = bi;
      p.argmax_out[m] = bi;
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (p.next_token) p.next_token[0] = res[(p.m_rows - 1) & 3];
    if (p.history && p.step) {
      const uint32_t st = *p.step;
      if (st < p.history_cap) p.history[st] = res[0];
      *p.step = st + 1;
    }
    if (p.pos) *p.pos = *p.pos + p.pos_advance;
  }
}

// ===========================================================================
// synthetic fills (lisa_synth.h)
// ===========================================================================
extern "C" __global__ __launch_bounds__(256) void lisa_synth_fill(LisaSynthParams p) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.n; i += stride) {
    switch (p.kind) {
      case LISA_FILL_WORDS:
        static_cast<uint32_t*>(p.out)[i] = lisa_synth_word(p.key, i);
        break;
      case LISA_FILL_BF16:
        static_cast<uint16_t*>(p.out)[i] = lisa_f32_to_bf16(lisa_synth_value(p.key, i, (int)p.dist, p.a, p.b));
        break;
      case LISA_FILL_F32:
        static_cast<float*>(p.out)[i] = lisa_synth_value(p.key, i, (int)p.dist, p.a, p.b);
        break;
      case LISA_FILL_SB: {
        const uint16_t s = lisa_f32_to_bf16(lisa_synth_value(p.key, i, LISA_DIST_UNIFORM, LISA_SCALE_LO, LISA_SCALE_HI));
        const uint16_t b = lisa_f32_to_bf16(lisa_synth_value(p.key2, i, LISA_DIST_UNIFORM, LISA_BIAS_LO, LISA_BIAS_HI));
        static_cast<uint32_t*>(p.out)[i] = (uint32_t)s | ((uint32_t)b << 16);
        break;
      }
      default: { /* KV rows: i runs over [4][filled][256] */
        const uint64_t d = i % LISA_ATT_HD, row = i / LISA_ATT_HD;
        const uint64_t pos = row % p.filled, kvh = row / p.filled;
        const uint64_t e = ((kvh << 20) + pos) * LISA_ATT_HD + d;
        static_cast<uint16_t*>(p.out)[(kvh * p.capacity + pos) * LISA_ATT_HD + d] =
            lisa_f32_to_bf16(lisa_synth_value(p.key, e, LISA_DIST_NORMAL, 0.0f, 1.0f));
        break;
      }
    }
  }
}
