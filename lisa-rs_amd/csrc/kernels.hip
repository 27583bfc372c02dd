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
//   lisa_copy_bytes       device-to-device copy
//   lisa_q4_gemm, lisa_rows, lisa_gdn_conv_rows, lisa_gdn_{prep,scan,out}_rows,
//   lisa_attn_{store,partial,merge}_rows   batched prefill [F1 GEMM, F4-F14 rows forms]
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
// v of lane l ^ MASK. Masks 1 and 2 are DPP quad permutes and 8 is a DPP
// rotate by 8 within each row of 16 ((l + 8) mod 16 = l ^ 8), so those steps
// fold into the consuming VALU op; 4 and 16 use ds_swizzle, 32 ds_bpermute.
template <int MASK>
DEV float xor_lane(float v) {
  if constexpr (MASK == 1 || MASK == 2 || MASK == 8) {
    constexpr int ctrl = MASK == 1 ? 0xb1 /* quad_perm [1,0,3,2] */
                         : MASK == 2 ? 0x4e /* quad_perm [2,3,0,1] */
                                     : 0x128 /* row_ror:8 */;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
  } else if constexpr (MASK >= 32) {
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

// A device word every lane needs (the decode position) as a vector load: the
// index is an opaque zero, so the load is not turned into a scalar load, which
// would wait behind the argument-block loads and other scalar loads (several
// dependent round trips). Issue it first; read it with readfirstlane.
DEV uint32_t vload_u32(const uint32_t* ptr) {
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  return ptr[zero];
}
DEV float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
DEV float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// ===========================================================================
// q4 linear
// ===========================================================================
// Arithmetic (the reference's qmv.metal:9-76 with 64-wide groups). Per
// 64-group g of a row with nibbles q_k, scale s and bias b:
//   acc_lo = fma chain over even k ascending of x_k * q_k
//   acc_hi = fma chain over odd k ascending of x_k * (16 q_k)     [the odd-nibble trick, qmv.metal:30-36]
//   P_g    = fma(s, acc_lo + acc_hi / 16, b * X_g),  X_g = sum of the group's 64 x
// The hardware evaluates the same chains in a power-of-two scaled form: a
// nibble field of a packed word, masked in place, read as an f16 bit pattern
// is the subnormal q * 2^-24 (low nibble of a half) or 16q * 2^-24 (high
// nibble), which v_fma_mix_f32 consumes directly. Scaling by 2^-24 commutes
// with rounding in the normal range, so the chains are the oracle's chains
// times 2^-24 exactly, and fma(s * 2^24, lo' + hi' / 16, b * X_g) equals P_g.
// The oracle computes the same scaled form.
//
// Work split: a wave owns an 8-row tile; the 16 lanes of row-group rp = lane/16
// own two rows (rows 2rp, 2rp+1 of the tile, or the gate and up rows of one
// output), lane li = lane%16 walks groups g = 16i + li and sums P_g in
// ascending i, then tree16 across the row-group (qmv.metal:71-75).
// K = 5120: each wave owns one tile over the whole of K (4 tiles per
// workgroup). Other K: the four waves share one tile, wave w takes group
// iterations [ITER*w/4, ITER*(w+1)/4), and the results are combined as
// (W0 + W1) + (W2 + W3).
//
// One tile per wave, no persistent loop: every wave issues its weight stream
// right behind the prologue loads (so the prologue never waits for weights;
// under a normalizing prologue only the first iteration goes ahead of it, to
// keep the register count low enough for the whole grid to be resident), and
// the dispatcher balances the tail.
//
// x lives in LDS as f32 in 64-element groups padded to 272 bytes: the 16 lanes
// of a row-group read 16 consecutive groups at the same offset, and the
// padding puts them on disjoint banks, so every read address is a per-lane
// base plus an immediate. X_g follows it. Launches with a workgroup prologue
// (K = 5120, the MTP fc) stage every input row whole, once per workgroup;
// split-K plain-x launches stage x per wave and per group iteration instead
// (WaveSlot below).

template <int K, int M>
struct QmvCfg {
  static constexpr int G = K / 64;
  static constexpr int ITER = G / 16;
  static constexpr bool SPLIT = (K != LISA_HIDDEN);
  static constexpr int IMAX = SPLIT ? (ITER + 3) / 4 : ITER;
  static constexpr int NCH = K / 8;                 // 8-element chunks of x
  static constexpr int RX = (NCH + 255) / 256;      // chunk rounds per thread (plain x)
  static constexpr bool NORMK = (K == LISA_HIDDEN || K == 2 * LISA_HIDDEN);
  static constexpr int RR = (NORMK && RX < 3) ? 3 : RX;
  static constexpr int GSTRIDE = 272;               // bytes per padded 64-group
  static constexpr int ROWBYTES = G * GSTRIDE;
  static constexpr int XBYTES = M * ROWBYTES;
  static constexpr int GBYTES = M * G * 4;
  static constexpr int RBYTES = 64 * 4;
  static constexpr int KBYTES = 4 * 8 * M * 4;
  static_assert(G % 16 == 0, "K must be a multiple of 1024");
};

// Split-K plain-x launches: each wave converts, for one group iteration at a
// time, the 1024 x values [1024 ii, 1024 ii + 1024) of every input row to f32
// in its own LDS slot (16 padded groups per row, then the 16 X_g per row);
// lane l converts values [16 l, 16 l + 16), a quarter of group l / 4. The
// bf16 unpack then happens once per wave rather than once per row-group, and
// a wave reads only LDS it wrote, so no workgroup barrier is involved.
template <int M>
struct WaveSlot {
  static constexpr int ROWB = 16 * 272;
  static constexpr int XB = M * ROWB;
  static constexpr int BYTES = XB + M * 16 * 4;
};

template <int K, int M, int MODE>
DEV constexpr bool qmv_wave_staged() {
  return QmvCfg<K, M>::SPLIT && MODE == LISA_PRO_LOADX;
}

template <int K, int M, int MODE>
DEV constexpr int qmv_lds_bytes() {
  using C = QmvCfg<K, M>;
  return (qmv_wave_staged<K, M, MODE>() ? 4 * WaveSlot<M>::BYTES : C::XBYTES + C::GBYTES) + C::RBYTES +
         C::KBYTES;
}

// The 5120-wide segments a normalizing prologue reads: 640 chunks of 8, thread
// t owns chunks t, t + 256, t + 512 (< 640).
constexpr int kSegChunks = LISA_HIDDEN / 8;

template <int R>
struct ProRaw {
  uint4 a[R], b[R], c[R], w[R];
};

DEV float h16(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// acc + x * (f16 bit pattern), one v_fma_mix_f32
DEV float fmix_lo(float x, uint32_t p, float acc) { return __builtin_fmaf(x, h16(p & 0xffffu), acc); }
DEV float fmix_hi(float x, uint32_t p, float acc) { return __builtin_fmaf(x, h16(p >> 16), acc); }

// Eight bf16-valued floats packed as bf16 pairs (exact: the values are bf16 already).
DEV uint4 pack_bf8(const float (&v)[8]) {
  return make_uint4(lisa_f32x2_to_bf16x2(v[0], v[1]), lisa_f32x2_to_bf16x2(v[2], v[3]),
                    lisa_f32x2_to_bf16x2(v[4], v[5]), lisa_f32x2_to_bf16x2(v[6], v[7]));
}

DEV void unpack_bf8(const uint4& u, float (&v)[8]) {
  v[0] = lo_bf(u.x); v[1] = hi_bf(u.x); v[2] = lo_bf(u.y); v[3] = hi_bf(u.y);
  v[4] = lo_bf(u.z); v[5] = hi_bf(u.z); v[6] = lo_bf(u.w); v[7] = hi_bf(u.w);
}

template <int K, int M>
DEV void put_chunk(unsigned char* lds, int m, int k0, const float (&x)[8]) {
  using C = QmvCfg<K, M>;
  const int g = k0 >> 6, j = (k0 >> 3) & 7;
  unsigned char* base = lds + m * C::ROWBYTES + g * C::GSTRIDE;
  *reinterpret_cast<float4*>(base + 32 * j) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4*>(base + 32 * j + 16) = make_float4(x[4], x[5], x[6], x[7]);
}

// Sum of eight values, pairs first: the distance-1, 2, 4 levels of the X_g tree.
DEV float sum8(const float (&x)[8]) {
  return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}

// X_g of the chunk's group: ascending-distance tree over the 64 values
// (distances 1, 2, 4 inside the chunk, 8, 16, 32 across the 8 lanes that hold
// the group's chunks). Every lane calls it; lane c%8 == 0 stores.
template <int K, int M>
DEV void put_gsum(float* gsum, int m, int k0, bool valid, const float (&x)[8]) {
  float s = sum8(x);
  s = s + xor_lane<1>(s);
  s = s + xor_lane<2>(s);
  s = s + xor_lane<4>(s);
  if (valid && ((k0 >> 3) & 7) == 0) gsum[m * QmvCfg<K, M>::G + (k0 >> 6)] = s;
}


// RMSNorm statistic of one 5120-wide segment from each thread's partial sum of
// squares: tree64 per wave, then (W0 + W1) + (W2 + W3).
// One lane forms the factor and the workgroup reads it back, so the IEEE
// divide and square root run once per workgroup rather than once per lane.
DEV float seg_rms_inv(float s, float* red, int tid) {
  s = tree64(s);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    red[4] = lisa_rsqrt(tot / (float)LISA_HIDDEN + LISA_EPS);
  }
  __syncthreads();
  return red[4];
}

// Eight values rounded to bf16 (returned as floats) and the packed bf16 pairs.
DEV void round_bf8(const float (&f)[8], float (&x)[8], uint4& packed) {
  const uint32_t u0 = lisa_f32x2_to_bf16x2(f[0], f[1]), u1 = lisa_f32x2_to_bf16x2(f[2], f[3]);
  const uint32_t u2 = lisa_f32x2_to_bf16x2(f[4], f[5]), u3 = lisa_f32x2_to_bf16x2(f[6], f[7]);
  packed = make_uint4(u0, u1, u2, u3);
  unpack_bf8(packed, x);
}

// Sources of a normalized segment (pro_mode, or the two halves of MTPFC).
enum SegSrc { SEG_RESNORM, SEG_EMBED, SEG_CAST, SEG_NORM, SEG_PRENORM };

template <int MODE>
DEV constexpr int seg_source(int seg) {
  return MODE == LISA_PRO_RESNORM ? SEG_RESNORM
         : MODE == LISA_PRO_EMBED ? SEG_EMBED
         : MODE == LISA_PRO_CAST  ? SEG_CAST
         : MODE == LISA_PRO_NORM  ? SEG_NORM
         : MODE == LISA_PRO_PRENORM ? SEG_PRENORM
         : (seg == 0 ? SEG_EMBED : SEG_NORM); /* MTPFC */
}

// Raw loads of segment `seg` of input row m.
template <int MODE, int SEG, int R>
DEV void seg_load(const LisaQmvParams& p, int m, ProRaw<R>& raw) {
  const int tid = threadIdx.x;
  constexpr int src = seg_source<MODE>(SEG);
  const uint16_t* nw = SEG == 0 ? p.norm_w : p.norm_w2;
  const uint16_t* hsrc = (MODE == LISA_PRO_MTPFC) ? p.x_in : p.h_in + (size_t)m * LISA_HIDDEN;
  const float* osrc = p.o_in + (size_t)m * LISA_HIDDEN;
  uint32_t tok = 0;
  if constexpr (src == SEG_EMBED) tok = p.tokens[MODE == LISA_PRO_MTPFC ? 0 : m];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int c = min(tid + 256 * i, kSegChunks - 1);
    raw.w[i] = reinterpret_cast<const uint4*>(nw)[c];
    if constexpr (src == SEG_RESNORM || src == SEG_NORM || src == SEG_PRENORM)
      raw.a[i] = reinterpret_cast<const uint4*>(hsrc)[c];
    if constexpr (src == SEG_RESNORM || src == SEG_CAST) {
      raw.b[i] = reinterpret_cast<const uint4*>(osrc)[2 * c];
      raw.c[i] = reinterpret_cast<const uint4*>(osrc)[2 * c + 1];
    }
    if constexpr (src == SEG_EMBED) {
      raw.a[i].x = p.emb_w[(size_t)tok * (LISA_HIDDEN / 8) + c];
      raw.a[i].y = p.emb_sb[(size_t)tok * (LISA_HIDDEN / 64) + (c >> 3)];
    }
  }
}

// Decode, normalize and stage one 5120-wide segment (norm.metal:10-47; the
// residual add of the residual encoders; embed.metal:24-26).
template <int K, int M, int MODE, int SEG, int R>
DEV void seg_process(const LisaQmvParams& p, unsigned char* lds, int m, const ProRaw<R>& raw) {
  using C = QmvCfg<K, M>;
  const int tid = threadIdx.x;
  float* gsum = reinterpret_cast<float*>(lds + C::XBYTES);
  float* red = gsum + M * C::G;
  constexpr int src = seg_source<MODE>(SEG);
  // chunk 2 (c = tid + 512 < 640) exists on waves 0 and 1 only: a wave-uniform skip
  const bool has2 = __builtin_amdgcn_readfirstlane(tid >> 6) < 2;
  float v[3][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (i == 2 && !has2) break;
    const bool valid = tid + 256 * i < kSegChunks;
    float hv[8] = {}, ov[8] = {};
    if constexpr (src == SEG_RESNORM || src == SEG_NORM || src == SEG_PRENORM) unpack_bf8(raw.a[i], hv);
    if constexpr (src == SEG_RESNORM || src == SEG_CAST) {
      ov[0] = __uint_as_float(raw.b[i].x); ov[1] = __uint_as_float(raw.b[i].y);
      ov[2] = __uint_as_float(raw.b[i].z); ov[3] = __uint_as_float(raw.b[i].w);
      ov[4] = __uint_as_float(raw.c[i].x); ov[5] = __uint_as_float(raw.c[i].y);
      ov[6] = __uint_as_float(raw.c[i].z); ov[7] = __uint_as_float(raw.c[i].w);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r;
      if constexpr (src == SEG_RESNORM) r = lisa_bf16r(hv[e] + lisa_bf16r(ov[e]));
      else if constexpr (src == SEG_CAST) r = lisa_bf16r(ov[e]);
      else if constexpr (src == SEG_NORM || src == SEG_PRENORM) r = hv[e];
      else r = lisa_bf16r((float)((raw.a[i].x >> (4 * e)) & 0xfu) * lo_bf(raw.a[i].y) + hi_bf(raw.a[i].y));
      v[i][e] = r;
      if constexpr (src != SEG_PRENORM)
        if (valid) ss = ss + r * r;
    }
    if constexpr (src == SEG_PRENORM) {
      // the 8-row tile sum of squares of the residual rows,
      // ((r0^2 + r1^2) + (r2^2 + r3^2)) + ((r4^2 + r5^2) + (r6^2 + r7^2)),
      // formed from the chunk's residual values this prologue already holds
      const float part = ((hv[0] * hv[0] + hv[1] * hv[1]) + (hv[2] * hv[2] + hv[3] * hv[3])) +
                         ((hv[4] * hv[4] + hv[5] * hv[5]) + (hv[6] * hv[6] + hv[7] * hv[7]));
      if (valid) ss = ss + part;
    }
  }
  const float inv = seg_rms_inv(ss, red, tid);
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (i == 2 && !has2) break;
    const int c = tid + 256 * i;
    const bool valid = c < kSegChunks;
    float wv[8], f[8], x[8];
    uint4 xb;
    unpack_bf8(raw.w[i], wv);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (v[i][e] * inv) * wv[e];
    round_bf8(f, x, xb);
    const int k0 = SEG * LISA_HIDDEN + 8 * c;
    if (valid) put_chunk<K, M>(lds, m, k0, x);
    put_gsum<K, M>(gsum, m, k0, valid, x);
    if (valid && writer) {
      if (MODE != LISA_PRO_MTPFC && p.r_out) {
        reinterpret_cast<uint4*>(p.r_out + (size_t)m * LISA_HIDDEN)[c] = pack_bf8(v[i]);
      }
      if (p.x_out) reinterpret_cast<uint4*>(p.x_out + (size_t)m * K + SEG * LISA_HIDDEN)[c] = xb;
    }
  }
}

// Plain x (LOADX): raw loads and staging of input row m.
template <int K, int M, int R>
DEV void x_load(const LisaQmvParams& p, int m, ProRaw<R>& raw) {
  using C = QmvCfg<K, M>;
  const uint4* src = reinterpret_cast<const uint4*>(p.x_in + (size_t)m * K);
#pragma unroll
  for (int i = 0; i < C::RX; ++i) raw.a[i] = src[min((int)threadIdx.x + 256 * i, C::NCH - 1)];
}

template <int K, int M, int R>
DEV void x_process(unsigned char* lds, int m, const ProRaw<R>& raw) {
  using C = QmvCfg<K, M>;
  float* gsum = reinterpret_cast<float*>(lds + C::XBYTES);
#pragma unroll
  for (int i = 0; i < C::RX; ++i) {
    const int c = threadIdx.x + 256 * i;
    const bool valid = c < C::NCH;
    float x[8];
    unpack_bf8(raw.a[i], x);
    if (valid) put_chunk<K, M>(lds, m, 8 * c, x);
    put_gsum<K, M>(gsum, m, 8 * c, valid, x);
  }
}

// Raw x of a split-K plain-x launch for the wave's group iterations: for
// iteration i (clamped into the wave's range like its weights) and row m, lane
// l loads the 16 bf16 values [1024 ii + 16 l, 1024 ii + 16 l + 16).
template <int K, int M>
DEV void wx_load(const LisaQmvParams& p, int it0, int it1, int lane, uint4 (&xr)[QmvCfg<K, M>::IMAX][M][2],
                 int i0 = 0, int i1 = QmvCfg<K, M>::IMAX) {
#pragma unroll
  for (int i = i0; i < i1; ++i) {
    const int ii = max(min(it0 + i, it1 - 1), 0);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* src = reinterpret_cast<const uint4*>(p.x_in + (size_t)m * K) + 128 * ii + 2 * lane;
      xr[i][m][0] = src[0];
      xr[i][m][1] = src[1];
    }
  }
}

// One iteration's x into the wave's slot: f32 values, and X_g as the
// ascending-distance tree (distances 1, 2, 4 inside each 8-value chunk by sum8,
// 8 inside the lane, 16 and 32 across the group's four lanes).
template <int M>
DEV void wx_stage(unsigned char* slot, int lane, const uint4 (&xr)[M][2]) {
  const int gl = lane >> 2, q = lane & 3;
  float* gs = reinterpret_cast<float*>(slot + WaveSlot<M>::XB);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float a[8], b[8];
    unpack_bf8(xr[m][0], a);
    unpack_bf8(xr[m][1], b);
    unsigned char* dst = slot + m * WaveSlot<M>::ROWB + gl * 272 + q * 64;
    *reinterpret_cast<float4*>(dst) = make_float4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<float4*>(dst + 16) = make_float4(a[4], a[5], a[6], a[7]);
    *reinterpret_cast<float4*>(dst + 32) = make_float4(b[0], b[1], b[2], b[3]);
    *reinterpret_cast<float4*>(dst + 48) = make_float4(b[4], b[5], b[6], b[7]);
    float s = sum8(a) + sum8(b);
    s = s + xor_lane<1>(s);
    s = s + xor_lane<2>(s);
    if (q == 0) gs[m * 16 + gl] = s;
  }
}

// Orders the wave's own LDS writes and reads around a slot hand-over (LDS
// operations of one wave complete in issue order; this keeps the compiler from
// moving them across).
DEV void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

// PRENORM of several input rows: every row's residual chunks and the shared
// norm gains, loaded in one batch before the weight stream.
template <int M>
struct PreRaw {
  uint4 a[M][3], w[3];
};

template <int M>
DEV void prenorm_rows_load(const LisaQmvParams& p, PreRaw<M>& raw) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int c = min(tid + 256 * i, kSegChunks - 1);
    raw.w[i] = reinterpret_cast<const uint4*>(p.norm_w)[c];
#pragma unroll
    for (int m = 0; m < M; ++m) raw.a[m][i] = reinterpret_cast<const uint4*>(p.h_in + (size_t)m * LISA_HIDDEN)[c];
  }
}

// Normalize and stage M rows (norm.metal:10-47): per row the chunk map, the
// sums of squares, the reduction order and the staged values of the one-row
// path (seg_process), with the rows' statistics formed in one round of
// barriers (lane m of wave 0 forms row m's factor) rather than one per row.
template <int K, int M>
DEV void prenorm_rows(const LisaQmvParams& p, unsigned char* lds, const PreRaw<M>& raw) {
  using C = QmvCfg<K, M>;
  static_assert(K == LISA_HIDDEN && 5 * M <= C::RBYTES / 4, "PRENORM rows of the wrong width");
  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* gsum = reinterpret_cast<float*>(lds + C::XBYTES);
  float* red = gsum + M * C::G;
  const bool has2 = wv < 2;  // chunk tid + 512 < 640: waves 0 and 1
  float ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    ss[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i == 2 && !has2) break;
      const bool valid = tid + 256 * i < kSegChunks;
      float hv[8];
      unpack_bf8(raw.a[m][i], hv);
      const float part = ((hv[0] * hv[0] + hv[1] * hv[1]) + (hv[2] * hv[2] + hv[3] * hv[3])) +
                         ((hv[4] * hv[4] + hv[5] * hv[5]) + (hv[6] * hv[6] + hv[7] * hv[7]));
      if (valid) ss[m] = ss[m] + part;
    }
    ss[m] = tree64(ss[m]);
  }
  __syncthreads();
  if ((tid & 63) == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) red[4 * m + wv] = ss[m];
  }
  __syncthreads();
  if (tid < M) {
    const float* rm = red + 4 * tid;
    red[4 * M + tid] = lisa_rsqrt(((rm[0] + rm[1]) + (rm[2] + rm[3])) / (float)LISA_HIDDEN + LISA_EPS);
  }
  __syncthreads();
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float inv = red[4 * M + m];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i == 2 && !has2) break;
      const int c = tid + 256 * i;
      const bool valid = c < kSegChunks;
      float hv[8], wf[8], f[8], x[8];
      uint4 xb;
      unpack_bf8(raw.a[m][i], hv);
      unpack_bf8(raw.w[i], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (hv[e] * inv) * wf[e];
      round_bf8(f, x, xb);
      if (valid) put_chunk<K, M>(lds, m, 8 * c, x);
      put_gsum<K, M>(gsum, m, 8 * c, valid, x);
      if (valid && writer) {
        if (p.r_out) reinterpret_cast<uint4*>(p.r_out + (size_t)m * LISA_HIDDEN)[c] = raw.a[m][i];
        if (p.x_out) reinterpret_cast<uint4*>(p.x_out + (size_t)m * K)[c] = xb;
      }
    }
  }
  __syncthreads();
}

template <int K, int M, int MODE, int R>
DEV void pro_load(const LisaQmvParams& p, int m, ProRaw<R>& raw) {
  if constexpr (MODE == LISA_PRO_LOADX) x_load<K, M, R>(p, m, raw);
  else seg_load<MODE, 0, R>(p, m, raw);
}

// Stage x and X_g of all M rows. Row 0's first segment was loaded by the
// caller (before the weight stream); the rest is loaded here.
template <int K, int M, int MODE, int R>
DEV void qmv_prologue(const LisaQmvParams& p, unsigned char* lds, ProRaw<R>& raw) {
  if constexpr (MODE != LISA_PRO_LOADX) {
    static_assert(K == LISA_HIDDEN * (MODE == LISA_PRO_MTPFC ? 2 : 1), "normalizing prologue of the wrong width");
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m > 0) seg_load<MODE, 0, R>(p, m, raw);
      seg_process<K, M, MODE, 0, R>(p, lds, m, raw);
      if constexpr (MODE == LISA_PRO_MTPFC) {
        seg_load<MODE, 1, R>(p, m, raw);
        seg_process<K, M, MODE, 1, R>(p, lds, m, raw);
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m > 0) x_load<K, M, R>(p, m, raw);
      x_process<K, M, R>(lds, m, raw);
    }
  }
  __syncthreads();
}

template <int M>
DEV void conv_epilogue(const LisaQmvParams& p, float* out, int c, const float* pr, const uint32_t (&cs)[3],
                       uint2 cw) {
  const int C = LISA_GDN_CONV_DIM;
  float hist[3 + M];
#pragma unroll
  for (int i = 0; i < 3; ++i) hist[i] = lo_bf(cs[i]);
#pragma unroll
  for (int t = 0; t < M; ++t) hist[3 + t] = lisa_bf16r(pr[t]);
  const float w[4] = {lo_bf(cw.x), hi_bf(cw.x), lo_bf(cw.y), hi_bf(cw.y)};
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

// The weights of a wave's group iterations for the two rows of a lane.
template <int IMAX>
struct Unit {
  uint4 a0[IMAX], b0[IMAX], a1[IMAX], b1[IMAX];
  uint32_t s0[IMAX], s1[IMAX];
};

struct TileRef {
  uint32_t r0, r1;
  bool v0, v1;
  const uint4 *wp0, *wp1;
  const uint32_t *sp0, *sp1;
  void* out;
  uint32_t rows, kind;
  // the same rows as wave-uniform matrix bases and per-lane (clamped) row
  // indices, for loads that add a 32-bit byte offset to a scalar base
  const uint32_t *wb0, *wb1, *sb0, *sb1;
  uint32_t c0, c1;
};

// Tile count of a launch, tile_start[n_mats], selected from the entries
// rather than indexed (an indexed read would wait for n_mats first).
DEV uint32_t qmv_tiles(const LisaQmvParams& p) {
  uint32_t t = p.tile_start[0];
#pragma unroll
  for (int i = 1; i <= LISA_QMV_MAX_MATS; ++i) t = (uint32_t)i == p.n_mats ? p.tile_start[i] : t;
  return t;
}

// The matrix of a tile comes from independent comparisons against the
// tile_start entries below n_mats, and its fields are selected from all
// matrices' fields, so the kernel-argument reads form one round trip instead
// of a chain of dependent ones ahead of the first weight load.
template <int K>
DEV TileRef tile_ref(const LisaQmvParams& p, uint32_t tile, int rp) {
  constexpr int G = K / 64;
  constexpr int NM = LISA_QMV_MAX_MATS;
  uint32_t ts[NM];
  const uint32_t* mw[NM];
  const uint32_t* msb[NM];
  const uint32_t* mw2[NM];
  const uint32_t* msb2[NM];
  void* mout[NM];
  uint32_t mrows[NM], mkind[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    ts[i] = p.tile_start[i];
    mw[i] = p.mats[i].w; msb[i] = p.mats[i].sb; mw2[i] = p.mats[i].w2; msb2[i] = p.mats[i].sb2;
    mout[i] = p.mats[i].out; mrows[i] = p.mats[i].rows; mkind[i] = p.mats[i].kind;
    // keeps the compiler from deferring the up-projection reads into a branch
    asm volatile("" : : "s"(mw2[i]), "s"(msb2[i]), "s"(mout[i]));
  }
  int e = 0;
#pragma unroll
  for (int i = 1; i < NM; ++i) e += ((uint32_t)i < p.n_mats && tile >= ts[i]) ? 1 : 0;
  uint32_t t0 = ts[0];
  const uint32_t *w = mw[0], *sb = msb[0], *w2 = mw2[0], *sb2 = msb2[0];
  void* out = mout[0];
  uint32_t rows = mrows[0], kind = mkind[0];
#pragma unroll
  for (int i = 1; i < NM; ++i) {
    const bool is = e == i;
    t0 = is ? ts[i] : t0;
    w = is ? mw[i] : w; sb = is ? msb[i] : sb; w2 = is ? mw2[i] : w2; sb2 = is ? msb2[i] : sb2;
    out = is ? mout[i] : out; rows = is ? mrows[i] : rows; kind = is ? mkind[i] : kind;
  }
  TileRef t;
  t.out = out;
  t.rows = rows;
  t.kind = kind;
  const uint32_t lt = tile - t0;
  const bool pair = kind == LISA_EPI_GATEUP;
  t.r0 = pair ? lt * 4 + rp : lt * 8 + 2 * rp;
  t.r1 = pair ? t.r0 : t.r0 + 1;
  const uint32_t *w0 = w, *s0 = sb;
  const uint32_t *w1 = pair ? w2 : w, *s1 = pair ? sb2 : sb;
  t.v0 = t.r0 < rows;
  t.v1 = t.r1 < rows;
  const uint32_t c0 = t.v0 ? t.r0 : rows - 1, c1 = t.v1 ? t.r1 : rows - 1;
  t.wp0 = reinterpret_cast<const uint4*>(w0 + (size_t)c0 * (K / 8));
  t.wp1 = reinterpret_cast<const uint4*>(w1 + (size_t)c1 * (K / 8));
  t.sp0 = s0 + (size_t)c0 * G;
  t.sp1 = s1 + (size_t)c1 * G;
  t.wb0 = w0; t.wb1 = w1; t.sb0 = s0; t.sb1 = s1;
  t.c0 = c0; t.c1 = c1;
  return t;
}

// load_unit with each address a scalar matrix base plus a 32-bit per-lane
// byte offset (one register per address instead of a 64-bit pointer); the
// row offsets stay below 2^32 bytes for every matrix of the model.
template <int K, int IMAX>
DEV void load_unit_off(Unit<IMAX>& u, const TileRef& t, int it0, int it1, int li, int i0, int i1) {
  auto w16 = [](const uint32_t* base, uint32_t off) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + off);
  };
  auto w4 = [](const uint32_t* base, uint32_t off) {
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(base) + off);
  };
#pragma unroll
  for (int i = i0; i < i1; ++i) {
    const int ii = max(min(it0 + i, it1 - 1), 0);
    const uint32_t g = 16 * ii + li;
    const uint32_t o0 = t.c0 * (uint32_t)(K / 2) + 32 * g, o1 = t.c1 * (uint32_t)(K / 2) + 32 * g;
    u.a0[i] = w16(t.wb0, o0);
    u.b0[i] = w16(t.wb0, o0 + 16);
    u.a1[i] = w16(t.wb1, o1);
    u.b1[i] = w16(t.wb1, o1 + 16);
    u.s0[i] = w4(t.sb0, t.c0 * (uint32_t)(K / 16) + 4 * g);
    u.s1[i] = w4(t.sb1, t.c1 * (uint32_t)(K / 16) + 4 * g);
  }
}

// Every load is unconditional (iterations past the wave's range re-read its
// last one) so the loads of a wave form one straight run.
template <int K, int IMAX>
DEV void load_unit(Unit<IMAX>& u, const TileRef& t, int it0, int it1, int li, int i0, int i1) {
#pragma unroll
  for (int i = i0; i < i1; ++i) {
    const int ii = max(min(it0 + i, it1 - 1), 0);
    const int g = 16 * ii + li;
    u.a0[i] = t.wp0[2 * g];
    u.b0[i] = t.wp0[2 * g + 1];
    u.a1[i] = t.wp1[2 * g];
    u.b1[i] = t.wp1[2 * g + 1];
    u.s0[i] = t.sp0[g];
    u.s1[i] = t.sp1[g];
  }
}

// One group of the lane's two rows against the M staged x rows: x of row m,
// group g at xs + m * ROWB + 272 g, its X_g at gsum[m * GROW + g].
template <int ROWB, int GROW, int M>
DEV void group_dot2(const unsigned char* xs, int g, const uint4& a0, const uint4& b0, const uint4& a1,
                    const uint4& b1, uint32_t sb0, uint32_t sb1, const float* gsum, float (&T0)[M],
                    float (&T1)[M]) {
  const uint32_t w0[8] = {a0.x, a0.y, a0.z, a0.w, b0.x, b0.y, b0.z, b0.w};
  const uint32_t w1[8] = {a1.x, a1.y, a1.z, a1.w, b1.x, b1.y, b1.z, b1.w};
  float lo0[M], hi0[M], lo1[M], hi1[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { lo0[m] = 0.0f; hi0[m] = 0.0f; lo1[m] = 0.0f; hi1[m] = 0.0f; }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // nibble fields in place: e0|e4, e1|e5 (x16), e2|e6, e3|e7 (x16)
    const uint32_t p0 = w0[j] & 0x000f000fu, p1 = w0[j] & 0x00f000f0u, t0 = w0[j] >> 8;
    const uint32_t p2 = t0 & 0x000f000fu, p3 = t0 & 0x00f000f0u;
    const uint32_t q0 = w1[j] & 0x000f000fu, q1 = w1[j] & 0x00f000f0u, t1 = w1[j] >> 8;
    const uint32_t q2 = t1 & 0x000f000fu, q3 = t1 & 0x00f000f0u;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[8];
      const unsigned char* base = xs + m * ROWB + g * 272;
      const float4 xa = *reinterpret_cast<const float4*>(base + 32 * j);
      const float4 xb = *reinterpret_cast<const float4*>(base + 32 * j + 16);
      x[0] = xa.x; x[1] = xa.y; x[2] = xa.z; x[3] = xa.w;
      x[4] = xb.x; x[5] = xb.y; x[6] = xb.z; x[7] = xb.w;
      lo0[m] = fmix_lo(x[0], p0, lo0[m]);
      lo0[m] = fmix_lo(x[2], p2, lo0[m]);
      lo0[m] = fmix_hi(x[4], p0, lo0[m]);
      lo0[m] = fmix_hi(x[6], p2, lo0[m]);
      hi0[m] = fmix_lo(x[1], p1, hi0[m]);
      hi0[m] = fmix_lo(x[3], p3, hi0[m]);
      hi0[m] = fmix_hi(x[5], p1, hi0[m]);
      hi0[m] = fmix_hi(x[7], p3, hi0[m]);
      lo1[m] = fmix_lo(x[0], q0, lo1[m]);
      lo1[m] = fmix_lo(x[2], q2, lo1[m]);
      lo1[m] = fmix_hi(x[4], q0, lo1[m]);
      lo1[m] = fmix_hi(x[6], q2, lo1[m]);
      hi1[m] = fmix_lo(x[1], q1, hi1[m]);
      hi1[m] = fmix_lo(x[3], q3, hi1[m]);
      hi1[m] = fmix_hi(x[5], q1, hi1[m]);
      hi1[m] = fmix_hi(x[7], q3, hi1[m]);
    }
  }
  const float s0 = lo_bf(sb0) * 16777216.0f, bb0 = hi_bf(sb0);
  const float s1 = lo_bf(sb1) * 16777216.0f, bb1 = hi_bf(sb1);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float xg = gsum[m * GROW + g];
    T0[m] = T0[m] + lisa_fma(s0, lo0[m] + hi0[m] * 0.0625f, bb0 * xg);
    T1[m] = T1[m] + lisa_fma(s1, lo1[m] + hi1[m] * 0.0625f, bb1 * xg);
  }
}

// Global inputs of a tile's epilogue, read at the start of the launch so the
// epilogue does not begin with a memory round trip: the residual pair h[r0],
// h[r1] (RESID) or the channel's three conv-state values and four taps (CONV).
template <int M>
struct EpiPre {
  uint32_t h[M];
  uint32_t cs[3];
  uint2 cw;
};

template <int M, int EPI>
DEV void epi_preload(const LisaQmvParams& p, const TileRef& tr, int li, EpiPre<M>& e) {
  const uint32_t kind = EPI >= 0 ? (uint32_t)EPI : tr.kind;
  if (kind == LISA_EPI_RESID) {
    const uint32_t r = tr.v1 ? tr.r0 : 0;
#pragma unroll
    for (int m = 0; m < M; ++m) e.h[m] = *reinterpret_cast<const uint32_t*>(p.h_in + (size_t)m * LISA_HIDDEN + r);
  } else if (kind == LISA_EPI_CONV) {
    const uint32_t c = (li & 1) ? (tr.v1 ? tr.r1 : 0) : (tr.v0 ? tr.r0 : 0);
#pragma unroll
    for (int i = 0; i < 3; ++i) e.cs[i] = p.conv_state[(size_t)i * LISA_GDN_CONV_DIM + c];
    e.cw = *reinterpret_cast<const uint2*>(p.conv_w + (size_t)c * 4);
  }
}

// The epilogue of a tile's finished sums T0/T1 (EPI, or the tile's matrix
// kind when EPI < 0); argmax candidates update best_v/best_i.
template <int M, int EPI>
DEV void qmv_epilogue(const LisaQmvParams& p, const TileRef& tr, int li, EpiPre<M>& pre, const float (&T0)[M],
                      const float (&T1)[M], float (&best_v)[M], uint32_t (&best_i)[M]) {
  // the preloaded epilogue inputs are first used here: without this, their
  // conversions are hoisted to the loads and the wave waits for its whole
  // weight stream right after issuing it
  if (EPI < 0 || EPI == LISA_EPI_RESID || EPI == LISA_EPI_CONV) {
#pragma unroll
    for (int m = 0; m < M; ++m) asm volatile("" : "+v"(pre.h[m]));
#pragma unroll
    for (int i = 0; i < 3; ++i) asm volatile("" : "+v"(pre.cs[i]));
    asm volatile("" : "+v"(pre.cw.x), "+v"(pre.cw.y));
  }
  const struct { void* out; uint32_t rows, kind; } mt{tr.out, tr.rows, tr.kind};
  const uint32_t r0 = tr.r0, r1 = tr.r1;
  const bool v0 = tr.v0, v1 = tr.v1;
  switch (EPI >= 0 ? (uint32_t)EPI : mt.kind) {
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
      if (li == 0 && v0) conv_epilogue<M>(p, static_cast<float*>(mt.out), (int)r0, T0, pre.cs, pre.cw);
      if (li == 1 && v1) conv_epilogue<M>(p, static_cast<float*>(mt.out), (int)r1, T1, pre.cs, pre.cw);
      break;
    }
    case LISA_EPI_RESID: {
      // r = bf16(h + bf16(y)) in place
      uint16_t* hres = const_cast<uint16_t*>(p.h_in);  // read-write for this epilogue
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (li == 0 && v0 && v1) {
          const float ra = lisa_bf16r(lo_bf(pre.h[m]) + lisa_bf16r(T0[m]));
          const float rb = lisa_bf16r(hi_bf(pre.h[m]) + lisa_bf16r(T1[m]));
          hres[(size_t)m * LISA_HIDDEN + r0] = lisa_f32_to_bf16(ra);
          hres[(size_t)m * LISA_HIDDEN + r1] = lisa_f32_to_bf16(rb);
        }
      }
      break;
    }
    default: { /* ARGMAX */
      float* out = static_cast<float*>(mt.out);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (li == 2 * m && v0) out[(size_t)m * mt.rows + r0] = T0[m];
        if (li == 2 * m + 1 && v1) out[(size_t)m * mt.rows + r1] = T1[m];
        if (li == 0) {
          if (v0 && better(T0[m], r0, best_v[m], best_i[m])) { best_v[m] = T0[m]; best_i[m] = r0; }
          if (v1 && better(T1[m], r1, best_v[m], best_i[m])) { best_v[m] = T1[m]; best_i[m] = r1; }
        }
      }
      break;
    }
  }
}

// EPI: the epilogue of every matrix of the launch, or -1 to read it per tile.
template <int K, int M, int MODE, int EPI>
DEV void qmv_body(const LisaQmvParams& p, unsigned char* lds) {
  using C = QmvCfg<K, M>;
  // split-K plain-x launches stage x per wave and per group iteration (WaveSlot)
  constexpr bool WAVEX = qmv_wave_staged<K, M, MODE>();
  const float* gsum = reinterpret_cast<const float*>(lds + C::XBYTES);
  float* red = reinterpret_cast<float*>(lds + (WAVEX ? 4 * WaveSlot<M>::BYTES : C::XBYTES + C::GBYTES));
  float* kred = red + 64;  // [4 waves][8 rows][M]

  // wv is wave-uniform: keeping it scalar keeps the matrix lookup on scalar loads
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, rp = lane >> 4;
  // One word of every 64-byte line of the kernel arguments, read in one batch
  // and consumed: the lookups below read further words of these lines in a
  // chain of dependent scalar loads, and the first touch of a line misses the
  // scalar cache, so without this every link of the chain waits for memory.
  {
    const uint32_t* kw = reinterpret_cast<const uint32_t*>(&p);
    static_assert(sizeof(LisaQmvParams) > 384 && sizeof(LisaQmvParams) <= 448, "seven argument lines");
    asm volatile("" : : "s"(kw[0]), "s"(kw[16]), "s"(kw[32]), "s"(kw[48]), "s"(kw[64]), "s"(kw[80]), "s"(kw[96]));
  }
  const uint32_t tiles = qmv_tiles(p);
  const uint32_t tile = C::SPLIT ? blockIdx.x : blockIdx.x * 4 + wv;
  const bool tile_ok = tile < tiles;
  const int it0 = C::SPLIT ? (C::ITER * wv) / 4 : 0;
  const int it1 = C::SPLIT ? (C::ITER * (wv + 1)) / 4 : C::ITER;
  // several rows under PRENORM: all rows' loads up front, one statistic round
  constexpr bool PRE_ROWS = MODE == LISA_PRO_PRENORM && M > 1;
  ProRaw<WAVEX || PRE_ROWS ? 1 : C::RR> raw;
  PreRaw<PRE_ROWS ? M : 1> pre_rows;
  uint4 xr[WAVEX ? C::IMAX : 1][M][2];
  // issue order: prologue loads, then the weight stream (the fences keep the
  // scheduler from interleaving them, so the prologue waits only for its own).
  // The weights are software-pipelined two group iterations deep: the loads of
  // iteration i + 2 are issued as soon as iteration i has been consumed. A
  // wave that issued its whole stream up front would stall at issue (the
  // memory pipeline backs up) and could not start its dot products until the
  // last load had gone out, so its arithmetic would pile up at the end of the
  // launch; two iterations in flight per wave keep the pipeline full. A
  // normalizing prologue holds many registers while it works, so only the
  // first iteration is in flight across it, which keeps the register count low
  // enough for every workgroup of the launch to be resident in one round.
  // Non-split plain-x launches (small and rare) issue their whole stream first.
  // Several input rows: each iteration's x is loaded with its weights (all of
  // it up front held 120 registers at three rows, two waves per SIMD).
  constexpr bool LAZYX = WAVEX && M > 1;
  constexpr int XDEPTH = C::IMAX < 2 ? C::IMAX : 2;
  if constexpr (WAVEX) wx_load<K, M>(p, it0, it1, lane, xr, 0, LAZYX ? XDEPTH : C::IMAX);
  else if constexpr (PRE_ROWS) prenorm_rows_load<M>(p, pre_rows);
  else pro_load<K, M, MODE, WAVEX ? 1 : C::RR>(p, 0, raw);
  __builtin_amdgcn_sched_barrier(0);
  const TileRef tr = tile_ref<K>(p, tile_ok ? tile : tiles - 1, rp);
  Unit<C::IMAX> u;
  constexpr int DEPTH = MODE == LISA_PRO_LOADX && !WAVEX ? C::IMAX : (C::IMAX < 2 ? C::IMAX : 2);
  constexpr int EARLY = MODE == LISA_PRO_LOADX ? DEPTH : 1;
  load_unit<K, C::IMAX>(u, tr, it0, it1, li, 0, EARLY);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PRE_ROWS) prenorm_rows<K, M>(p, lds, pre_rows);
  else if constexpr (!WAVEX) qmv_prologue<K, M, MODE, WAVEX || PRE_ROWS ? 1 : C::RR>(p, lds, raw);
  __builtin_amdgcn_sched_barrier(0);
  load_unit<K, C::IMAX>(u, tr, it0, it1, li, EARLY, DEPTH);
  // epilogue inputs (residual pair, GDN conv state and taps): read here,
  // behind the first weights, so the epilogue does not start with a memory
  // round trip
  EpiPre<M> pre;
  if (!C::SPLIT || wv == 0) epi_preload<M, EPI>(p, tr, li, pre);

  float T0[M], T1[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { T0[m] = 0.0f; T1[m] = 0.0f; }
  unsigned char* slot = lds + wv * WaveSlot<M>::BYTES;
#pragma unroll
  for (int i = 0; i < C::IMAX; ++i) {
    if (it0 + i < it1) {
      if constexpr (WAVEX) {
        wx_stage<M>(slot, lane, xr[i]);
        wave_lds_fence();
        group_dot2<WaveSlot<M>::ROWB, 16, M>(slot, li, u.a0[i], u.b0[i], u.a1[i], u.b1[i], u.s0[i], u.s1[i],
                                              reinterpret_cast<const float*>(slot + WaveSlot<M>::XB), T0, T1);
        wave_lds_fence();
      } else {
        group_dot2<C::ROWBYTES, C::G, M>(lds, 16 * (it0 + i) + li, u.a0[i], u.b0[i], u.a1[i], u.b1[i], u.s0[i],
                                         u.s1[i], gsum, T0, T1);
      }
    }
    if (i + DEPTH < C::IMAX) {
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (LAZYX) wx_load<K, M>(p, it0, it1, lane, xr, i + DEPTH, i + DEPTH + 1);
      load_unit<K, C::IMAX>(u, tr, it0, it1, li, i + DEPTH, i + DEPTH + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) { T0[m] = tree16(T0[m]); T1[m] = tree16(T1[m]); }

  bool active = tile_ok;
  if constexpr (C::SPLIT) {
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
    active = active && wv == 0;
  }

  float best_v[M];
  uint32_t best_i[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { best_v[m] = -INFINITY; best_i[m] = 0xffffffffu; }

  if (active) qmv_epilogue<M, EPI>(p, tr, li, pre, T0, T1, best_v, best_i);

  if (p.am_val) {
    // workgroup (max, lowest index) per input row
    __syncthreads();
    float* cv = red;
    uint32_t* ci = reinterpret_cast<uint32_t*>(red + 32);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = best_v[m];
      uint32_t i = best_i[m];
#pragma unroll
      for (int msk = 1; msk < 64; msk <<= 1) {
        const float ov = __shfl_xor(v, msk, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)i, msk, 64);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
      }
      if (lane == 0) { cv[wv] = v; ci[wv] = i; }
      __syncthreads();
      if (tid == 0) {
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
  if constexpr (K == LISA_HIDDEN && !C::SPLIT && !WAVEX && MODE != LISA_PRO_LOADX) {
    // GDN in-projection: workgroup w < 48 forms the per-group contributions of
    // rows w of the a and b matrices against the staged x (thread g < 80 forms
    // group g as a q4 tile's lane forms each of its groups, from a running sum
    // of 0), last, when the tile's registers are free. The launch then carries
    // no a/b tiles: their 12 tiles would make 515 workgroups, three past two
    // per CU.
    if (p.gate_ab != nullptr && blockIdx.x < LISA_GDN_VH && tid < C::G) {
      const uint32_t hh = blockIdx.x;
      const uint4* aw = reinterpret_cast<const uint4*>(p.gate_a_w + (size_t)hh * (K / 8));
      const uint4* bw = reinterpret_cast<const uint4*>(p.gate_b_w + (size_t)hh * (K / 8));
      const uint4 a0 = aw[2 * tid], b0 = aw[2 * tid + 1], a1 = bw[2 * tid], b1 = bw[2 * tid + 1];
      const uint32_t s0 = p.gate_a_sb[(size_t)hh * C::G + tid], s1 = p.gate_b_sb[(size_t)hh * C::G + tid];
      float G0[M], G1[M];
#pragma unroll
      for (int m = 0; m < M; ++m) { G0[m] = 0.0f; G1[m] = 0.0f; }
      group_dot2<C::ROWBYTES, C::G, M>(lds, tid, a0, b0, a1, b1, s0, s1, gsum, G0, G1);
      // lane (tid & 15)'s slot: a's five groups, then b's
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float* dst = p.gate_ab + ((size_t)m * LISA_GDN_VH + hh) * LISA_GDN_GATE_FLOATS + 12 * (tid & 15) + (tid >> 4);
        dst[0] = G0[m];
        dst[5] = G1[m];
      }
    }
  }
}

// One kernel per (K, M, prologue): lisa_qmv_k<K>_m<M>_<x|resnorm|embed|cast|norm|mtpfc|prenorm>,
// plus variants whose epilogue is fixed at compile time:
// lisa_qmv_k5120_m<M>_<resnorm|prenorm>_<gateup|argmax> (MLP gate/up, lm_head).
#define QMV_KERNEL(K, M, MODE, NAME)                                                             \
  extern "C" __global__ __launch_bounds__(256) void lisa_qmv_k##K##_m##M##_##NAME(LisaQmvParams p) { \
    __shared__ __attribute__((aligned(16))) unsigned char lds[qmv_lds_bytes<K, M, MODE>()];        \
    qmv_body<K, M, MODE, -1>(p, lds);                                                            \
  }
#define QMV_KERNEL_EPI(K, M, MODE, NAME, EPI, ENAME)                                             \
  extern "C" __global__ __launch_bounds__(256) void lisa_qmv_k##K##_m##M##_##NAME##_##ENAME(       \
      LisaQmvParams p) {                                                                         \
    __shared__ __attribute__((aligned(16))) unsigned char lds[qmv_lds_bytes<K, M, MODE>()];        \
    qmv_body<K, M, MODE, EPI>(p, lds);                                                           \
  }

QMV_KERNEL(5120, 1, LISA_PRO_LOADX, x)
QMV_KERNEL(5120, 1, LISA_PRO_RESNORM, resnorm)
QMV_KERNEL(5120, 1, LISA_PRO_EMBED, embed)
QMV_KERNEL(5120, 1, LISA_PRO_CAST, cast)
QMV_KERNEL(5120, 1, LISA_PRO_NORM, norm)
QMV_KERNEL(5120, 3, LISA_PRO_LOADX, x)
QMV_KERNEL(5120, 3, LISA_PRO_RESNORM, resnorm)
QMV_KERNEL(5120, 3, LISA_PRO_EMBED, embed)
QMV_KERNEL(5120, 3, LISA_PRO_NORM, norm)
QMV_KERNEL(5120, 1, LISA_PRO_PRENORM, prenorm)
QMV_KERNEL(5120, 3, LISA_PRO_PRENORM, prenorm)
QMV_KERNEL(6144, 1, LISA_PRO_LOADX, x)
QMV_KERNEL(6144, 3, LISA_PRO_LOADX, x)
QMV_KERNEL(10240, 1, LISA_PRO_LOADX, x)
QMV_KERNEL(10240, 1, LISA_PRO_MTPFC, mtpfc)
QMV_KERNEL(17408, 1, LISA_PRO_LOADX, x)
QMV_KERNEL(17408, 3, LISA_PRO_LOADX, x)
QMV_KERNEL(1024, 1, LISA_PRO_LOADX, x)
QMV_KERNEL(1024, 3, LISA_PRO_LOADX, x)
QMV_KERNEL_EPI(5120, 1, LISA_PRO_RESNORM, resnorm, LISA_EPI_GATEUP, gateup)
QMV_KERNEL_EPI(5120, 3, LISA_PRO_RESNORM, resnorm, LISA_EPI_GATEUP, gateup)
QMV_KERNEL_EPI(5120, 1, LISA_PRO_RESNORM, resnorm, LISA_EPI_ARGMAX, argmax)
QMV_KERNEL_EPI(5120, 3, LISA_PRO_RESNORM, resnorm, LISA_EPI_ARGMAX, argmax)
QMV_KERNEL_EPI(5120, 1, LISA_PRO_PRENORM, prenorm, LISA_EPI_GATEUP, gateup)
QMV_KERNEL_EPI(5120, 3, LISA_PRO_PRENORM, prenorm, LISA_EPI_GATEUP, gateup)
QMV_KERNEL_EPI(5120, 1, LISA_PRO_PRENORM, prenorm, LISA_EPI_ARGMAX, argmax)
QMV_KERNEL_EPI(5120, 3, LISA_PRO_PRENORM, prenorm, LISA_EPI_ARGMAX, argmax)

// ---------------------------------------------------------------------------
// K = 5120 PRENORM launches on one workgroup per CU.
//
// Four-wave workgroups own four 8-row tiles each and run the normalizing
// prologue once per workgroup. With M rows staged the x buffer is M times the
// one-row one (65 KB at three rows), so they fit two per CU: the MLP
// gate/up's 1088 workgroups then run in three rounds, repeating the prologue
// in each. qmv_wide gives a CU one workgroup of NW waves owning NW + XT
// consecutive tiles and runs the prologue once over its 64 NW threads:
// * the MLP gate/up (LISA_QMV_WIDE_TILES = 17 tiles, 4352 = 256 x 17): 16
//   waves run one tile each exactly as the four-wave kernel does, and the five
//   group iterations of the 17th tile (XT = 1) run one each on waves 0..4,
//   which store the per-group terms; after a barrier wave 15 adds them in
//   iteration order from 0 and finishes that tile. A tile's running sum is
//   the sum of its per-group terms in iteration order from 0 either way;
// * the GDN and attention in-projections (2048 = 256 x 8 and 1792 = 256 x 7
//   tiles): 8 or 7 waves, one tile each (XT = 0), each tile's own epilogue
//   (STORE or CONV), and the GDN gate contributions from workgroups 0..47.
// Every output is the bits of the four-wave kernel (and of the one-row step).
// ---------------------------------------------------------------------------

template <int M>
struct WideCfg {
  using C = QmvCfg<LISA_HIDDEN, M>;
  static constexpr int XB = C::XBYTES + C::GBYTES;      // staged rows, then X_g
  static constexpr int RED = XB;                        // statistics: [M][4] partials, [M] factors
  static constexpr int SCR = RED + 64 * 4;              // chunk sums [M][640] / extra-tile terms
  static constexpr int SCR_BYTES = (M * kSegChunks > C::IMAX * 64 * 2 * M ? M * kSegChunks : C::IMAX * 64 * 2 * M) * 4;
  static constexpr int BYTES = SCR + SCR_BYTES;
  static_assert(5 * M <= 64, "statistics slots");
};

// Chunks per thread of a prologue over NT threads.
template <int NT>
constexpr int kWideChunks = (kSegChunks + NT - 1) / NT;

// PRENORM of M rows over NT >= 256 threads: thread t holds chunks t, t + NT,
// .. (< 640) of every row. The per-thread sums of squares of the 256-thread
// prologue (chunks t, t + 256, t + 512, added in that order) are formed by
// threads 0..255 from the chunk sums the owners put in LDS, then tree64 and
// (W0 + W1) + (W2 + W3) as there: the statistic, the staged x and X_g are the
// bits of prenorm_rows.
template <int M, int NT>
DEV void prenorm_wide(const LisaQmvParams& p, unsigned char* lds, const uint4 (&ha)[kWideChunks<NT>][M],
                      const uint4 (&hw)[kWideChunks<NT>]) {
  using W = WideCfg<M>;
  using C = QmvCfg<LISA_HIDDEN, M>;
  constexpr int CH = kWideChunks<NT>;
  static_assert(NT >= 256 && NT % 64 == 0, "prologue threads");
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* gsum = reinterpret_cast<float*>(lds + C::XBYTES);
  float* red = reinterpret_cast<float*>(lds + W::RED);
  float* parts = reinterpret_cast<float*>(lds + W::SCR);
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + NT * i;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float hv[8];
      unpack_bf8(ha[i][m], hv);
      const float part = ((hv[0] * hv[0] + hv[1] * hv[1]) + (hv[2] * hv[2] + hv[3] * hv[3])) +
                         ((hv[4] * hv[4] + hv[5] * hv[5]) + (hv[6] * hv[6] + hv[7] * hv[7]));
      if (c < kSegChunks) parts[m * kSegChunks + c] = part;
    }
  }
  __syncthreads();
  if (wv < 4) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float* pm = parts + m * kSegChunks;
      float ss = pm[tid];
      ss = ss + pm[tid + 256];
      if (wv < 2) ss = ss + pm[tid + 512];
      ss = tree64(ss);
      if (lane == 0) red[4 * m + wv] = ss;
    }
  }
  __syncthreads();
  if (tid < M) {
    const float* rm = red + 4 * tid;
    red[4 * M + tid] = lisa_rsqrt(((rm[0] + rm[1]) + (rm[2] + rm[3])) / (float)LISA_HIDDEN + LISA_EPS);
  }
  __syncthreads();
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + NT * i;
    const bool valid = c < kSegChunks;
    float wf[8];
    unpack_bf8(hw[i], wf);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float inv = red[4 * M + m];
      float hv[8], f[8], x[8];
      uint4 xb;
      unpack_bf8(ha[i][m], hv);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (hv[e] * inv) * wf[e];
      round_bf8(f, x, xb);
      if (valid) put_chunk<LISA_HIDDEN, M>(lds, m, 8 * c, x);
      put_gsum<LISA_HIDDEN, M>(gsum, m, 8 * c, valid, x);
      if (valid && writer) {
        if (p.r_out) reinterpret_cast<uint4*>(p.r_out + (size_t)m * LISA_HIDDEN)[c] = ha[i][m];
        if (p.x_out) reinterpret_cast<uint4*>(p.x_out + (size_t)m * LISA_HIDDEN)[c] = xb;
      }
    }
  }
  __syncthreads();
}

// M rows, NW waves each owning one tile, XT (0 or 1) extra tile spread over
// waves 0..4, epilogue EPI (-1: per tile kind; no ARGMAX). EARLY of a tile's
// group iterations are issued before the prologue, DEPTH are in flight during
// the loop. Launch 64 NW threads per workgroup and tiles / (NW + XT)
// workgroups.
// x of a LOADX launch over NT threads: thread t stages chunks t, t + NT, ..
// (< 640) of every row, each chunk and its group's X_g as the 256-thread
// prologue forms them (x_process), so the staged rows are the same bits.
template <int M, int NT>
DEV void loadx_wide(unsigned char* lds, const uint4 (&xa)[kWideChunks<NT>][M]) {
  using C = QmvCfg<LISA_HIDDEN, M>;
  float* gsum = reinterpret_cast<float*>(lds + C::XBYTES);
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kWideChunks<NT>; ++i) {
    const int c = tid + NT * i;
    const bool valid = c < kSegChunks;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[8];
      unpack_bf8(xa[i][m], x);
      if (valid) put_chunk<LISA_HIDDEN, M>(lds, m, 8 * c, x);
      put_gsum<LISA_HIDDEN, M>(gsum, m, 8 * c, valid, x);
    }
  }
  __syncthreads();
}

template <int M, int NW, int XT, int EPI, int EARLY, int DEPTH, int PRO = LISA_PRO_PRENORM>
DEV void qmv_wide(const LisaQmvParams& p, unsigned char* lds) {
  static_assert(PRO == LISA_PRO_PRENORM || PRO == LISA_PRO_LOADX, "wide prologues");
  constexpr int K = LISA_HIDDEN, NT = 64 * NW, TPW = NW + XT, CH = kWideChunks<NT>;
  using C = QmvCfg<K, M>;
  using W = WideCfg<M>;
  static_assert(XT == 0 || (XT == 1 && NW == 16 && EPI == LISA_EPI_GATEUP && C::IMAX <= NW - 1), "extra-tile layout");
  static_assert(EPI != LISA_EPI_ARGMAX, "no argmax partials");
  static_assert(0 <= EARLY && EARLY <= DEPTH && DEPTH <= C::IMAX, "pipeline depths");
  const float* gsum = reinterpret_cast<const float*>(lds + C::XBYTES);
  float* xterm = reinterpret_cast<float*>(lds + W::SCR);  // [IMAX][64 lanes][2M]

  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, rp = lane >> 4;
  {
    const uint32_t* kw = reinterpret_cast<const uint32_t*>(&p);
    asm volatile("" : : "s"(kw[0]), "s"(kw[16]), "s"(kw[32]), "s"(kw[48]), "s"(kw[64]), "s"(kw[80]), "s"(kw[96]));
  }
  const uint32_t tiles = qmv_tiles(p);
  const uint32_t base = blockIdx.x * TPW;
  const uint32_t tile = base + wv, xtile = base + NW;
  const bool tile_ok = tile < tiles;
  const bool xwave = XT > 0 && wv < C::IMAX;  // runs iteration wv of the extra tile

  // PRENORM: residual rows and norm weights; LOADX: the x rows (in ha)
  uint4 ha[CH][M], hw[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = min(tid + NT * i, kSegChunks - 1);
    if constexpr (PRO == LISA_PRO_PRENORM) hw[i] = reinterpret_cast<const uint4*>(p.norm_w)[c];
#pragma unroll
    for (int m = 0; m < M; ++m)
      ha[i][m] = reinterpret_cast<const uint4*>((PRO == LISA_PRO_PRENORM ? p.h_in : p.x_in) + (size_t)m * LISA_HIDDEN)[c];
  }
  __builtin_amdgcn_sched_barrier(0);
  const TileRef tr = tile_ref<K>(p, tile_ok ? tile : tiles - 1, rp);
  Unit<C::IMAX> u;
  Unit<1> xu;
  load_unit_off<K, C::IMAX>(u, tr, 0, C::ITER, li, 0, EARLY);
  if (xwave) {
    const TileRef xr = tile_ref<K>(p, xtile < tiles ? xtile : tiles - 1, rp);
    load_unit_off<K, 1>(xu, xr, wv, wv + 1, li, 0, 1);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PRO == LISA_PRO_PRENORM) prenorm_wide<M, NT>(p, lds, ha, hw);
  else loadx_wide<M, NT>(lds, ha);
  __builtin_amdgcn_sched_barrier(0);
  // waves 0..4 first run the extra tile's iteration wv (its weights were
  // issued with the prologue's loads) and issue the tile's further iterations
  // after it, so the extra weights never sit beside two of the tile's
  if constexpr (XT > 0) {
    if (xwave) {
      float X0[M], X1[M];
#pragma unroll
      for (int m = 0; m < M; ++m) { X0[m] = 0.0f; X1[m] = 0.0f; }
      group_dot2<C::ROWBYTES, C::G, M>(lds, 16 * wv + li, xu.a0[0], xu.b0[0], xu.a1[0], xu.b1[0], xu.s0[0],
                                       xu.s1[0], gsum, X0, X1);
      float* dst = xterm + (wv * 64 + lane) * 2 * M;
#pragma unroll
      for (int m = 0; m < M; ++m) { dst[m] = X0[m]; dst[M + m] = X1[m]; }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  load_unit_off<K, C::IMAX>(u, tr, 0, C::ITER, li, EARLY, DEPTH);
  __builtin_amdgcn_sched_barrier(0);
  // the epilogue's global inputs (GDN conv state and taps), behind the weights
  EpiPre<M> pre;
  if constexpr (EPI != LISA_EPI_GATEUP) epi_preload<M, EPI>(p, tr, li, pre);

  float T0[M], T1[M];
#pragma unroll
  for (int m = 0; m < M; ++m) { T0[m] = 0.0f; T1[m] = 0.0f; }
#pragma unroll
  for (int i = 0; i < C::IMAX; ++i) {
    group_dot2<C::ROWBYTES, C::G, M>(lds, 16 * i + li, u.a0[i], u.b0[i], u.a1[i], u.b1[i], u.s0[i], u.s1[i], gsum,
                                     T0, T1);
    if (i + DEPTH < C::IMAX) {
      __builtin_amdgcn_sched_barrier(0);
      load_unit_off<K, C::IMAX>(u, tr, 0, C::ITER, li, i + DEPTH, i + DEPTH + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // mlp.metal:11-16
  auto gateup_store = [&](const TileRef& t, const float (&A)[M], const float (&B)[M], int sl) {
    uint16_t* out = static_cast<uint16_t*>(t.out);
    // the row is opaque here, so its store addresses are formed now rather
    // than before the loop and carried across it
    uint32_t r = t.r0;
    asm volatile("" : "+v"(r));
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (sl == m && t.v0) {
        const float gte = lisa_bf16r(A[m]), up = lisa_bf16r(B[m]);
        out[(size_t)m * t.rows + r] = lisa_f32_to_bf16(lisa_silu_exp2(gte) * up);
      }
  };
#pragma unroll
  for (int m = 0; m < M; ++m) { T0[m] = tree16(T0[m]); T1[m] = tree16(T1[m]); }
  if (tile_ok) {
    if constexpr (EPI == LISA_EPI_GATEUP) {
      gateup_store(tr, T0, T1, li);
    } else {
      float best_v[M];
      uint32_t best_i[M];
#pragma unroll
      for (int m = 0; m < M; ++m) { best_v[m] = -INFINITY; best_i[m] = 0xffffffffu; }
      qmv_epilogue<M, EPI>(p, tr, li, pre, T0, T1, best_v, best_i);
    }
  }
  if constexpr (XT > 0) {
    __syncthreads();
    if (wv == NW - 1 && xtile < tiles) {
      // lane indices formed again here, not carried across the loop
      int fl = (int)threadIdx.x;
      asm volatile("" : "+v"(fl));
      fl &= 63;
      const TileRef xr = tile_ref<K>(p, xtile, fl >> 4);
      float A[M], B[M];
#pragma unroll
      for (int m = 0; m < M; ++m) { A[m] = 0.0f; B[m] = 0.0f; }
#pragma unroll
      for (int i = 0; i < C::IMAX; ++i) {
        const float* src = xterm + (i * 64 + fl) * 2 * M;
#pragma unroll
        for (int m = 0; m < M; ++m) { A[m] = A[m] + src[m]; B[m] = B[m] + src[M + m]; }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) { A[m] = tree16(A[m]); B[m] = tree16(B[m]); }
      gateup_store(xr, A, B, fl & 15);
    }
  }
  // GDN in-projection: workgroup w < 48 forms the per-group contributions of
  // rows w of the a and b matrices against the staged x, as the four-wave
  // kernel does
  if constexpr (EPI != LISA_EPI_GATEUP) {
    if (p.gate_ab != nullptr && blockIdx.x < LISA_GDN_VH && tid < C::G) {
      const uint32_t hh = blockIdx.x;
      const uint4* aw = reinterpret_cast<const uint4*>(p.gate_a_w + (size_t)hh * (K / 8));
      const uint4* bw = reinterpret_cast<const uint4*>(p.gate_b_w + (size_t)hh * (K / 8));
      const uint4 a0 = aw[2 * tid], b0 = aw[2 * tid + 1], a1 = bw[2 * tid], b1 = bw[2 * tid + 1];
      const uint32_t s0 = p.gate_a_sb[(size_t)hh * C::G + tid], s1 = p.gate_b_sb[(size_t)hh * C::G + tid];
      float G0[M], G1[M];
#pragma unroll
      for (int m = 0; m < M; ++m) { G0[m] = 0.0f; G1[m] = 0.0f; }
      group_dot2<C::ROWBYTES, C::G, M>(lds, tid, a0, b0, a1, b1, s0, s1, gsum, G0, G1);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float* dst = p.gate_ab + ((size_t)m * LISA_GDN_VH + hh) * LISA_GDN_GATE_FLOATS + 12 * (tid & 15) + (tid >> 4);
        dst[0] = G0[m];
        dst[5] = G1[m];
      }
    }
  }
}

// The MLP gate/up. Three rows are VALU-bound: no weights ahead of the
// prologue, so its residual loads are not queued behind the weight stream and
// the dot products start earlier (35.2 -> 31.0 us); one row is memory-bound
// and keeps a one-iteration head start (without it 20.7 -> 22.1 us).
extern "C" __global__ __launch_bounds__(LISA_QMV_WIDE_THREADS) void lisa_qmv_k5120_m3_prenorm_gateup_wide(
    LisaQmvParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[WideCfg<3>::BYTES];
  qmv_wide<3, 16, 1, LISA_EPI_GATEUP, 0, 2>(p, lds);
}
extern "C" __global__ __launch_bounds__(LISA_QMV_WIDE_THREADS) void lisa_qmv_k5120_m1_prenorm_gateup_wide(
    LisaQmvParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[WideCfg<1>::BYTES];
  qmv_wide<1, 16, 1, LISA_EPI_GATEUP, 1, 2>(p, lds);
}

// The GDN and attention in-projections (STORE and CONV matrices, GDN gate
// contributions): NW = 8 or 7 waves, one tile each, with a one-iteration
// weight head start. Three rows: 20.9 -> 19.4 us (GDN) and 17.3 -> 15.9 us
// (attention) against the four-wave kernel; one row: level (10.8 -> 10.7,
// 9.4 -> 9.2 us). Without the head start three rows gain less (20.5, 17.5 us)
// and one row loses (11.8, 10.4 us).
#define LISA_QMV_INPROJ_WIDE(M, NW)                                                                            \
  extern "C" __global__ __launch_bounds__(64 * NW) void lisa_qmv_k5120_m##M##_prenorm_wide##NW(LisaQmvParams p) { \
    __shared__ __attribute__((aligned(16))) unsigned char lds[WideCfg<M>::BYTES];                                \
    qmv_wide<M, NW, 0, -1, 1, 2>(p, lds);                                                                          \
  }
LISA_QMV_INPROJ_WIDE(1, 7)
LISA_QMV_INPROJ_WIDE(1, 8)
LISA_QMV_INPROJ_WIDE(3, 7)
LISA_QMV_INPROJ_WIDE(3, 8)
#undef LISA_QMV_INPROJ_WIDE

// A one-row LOADX launch of STORE matrices of 2049..2304 tiles (the 17408-row
// projection of the config-0 GEMV: 2176 tiles): one workgroup of nine waves per
// CU, one tile per wave, x staged once per CU; both pipelined iterations go
// ahead of the staging, which only converts x.
extern "C" __global__ __launch_bounds__(576) void lisa_qmv_k5120_m1_x_wide9(LisaQmvParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[WideCfg<1>::BYTES];
  qmv_wide<1, 9, 0, LISA_EPI_STORE, 2, 2, LISA_PRO_LOADX>(p, lds);
}

// ===========================================================================
// GDN recurrence (gdn.metal:245-328) + gates (gdn.metal:170-205) + gated
// RMSNorm (gdn.metal:367-391). One workgroup per value head, 512 threads:
// thread (v, q) = (tid/4, tid%4) owns the runs q, q+4, q+8, q+12 of 8 of state
// row v (gdn_row_step_il).
// ===========================================================================
// q or k of one key head (gdn.metal q/k norm): RMS over 128 values as tree64 of
// c0^2 + c1^2 (lane l holds c[l], c[l+64]), scaled, rounded to bf16.
DEV void gdn_qk_norm(float c0, float c1, float scale, float& n0, float& n1) {
  const float tot = tree64(c0 * c0 + c1 * c1);
  const float inv = lisa_rsqrt(tot / 128.0f + 1.0e-6f) * scale;
  n0 = lisa_bf16r(c0 * inv);
  n1 = lisa_bf16r(c1 * inv);
}

// beta = sigmoid(b), decay = exp(-exp(a_log) softplus(a + dt_bias)) of one value head.
DEV void gdn_gates(float braw, float araw, uint16_t dt_bias, uint16_t a_log, float& beta, float& decay) {
  beta = lisa_bf16r(lisa_sigmoid_exp(lisa_bf16r(braw)));
  const float dt_arg = lisa_bf16r(lisa_bf16r(araw) + bf2f(dt_bias));
  const float dt = lisa_bf16r(lisa_softplus(dt_arg));
  decay = lisa_expf(-lisa_expf(bf2f(a_log)) * dt);
}

// Row dot products of the delta rule (k.S and q.S over a state row of 128, the
// oracle's order): sixteen ascending fma runs of 8 (r_i over elements 8i..8i+7,
// the first term a product), quarters Q_j = (r_4j + r_4j+1) + (r_4j+2 + r_4j+3),
// row = (Q0 + Q1) + (Q2 + Q3). A time step of a state row: S *= decay,
// delta = (v - k.S) beta, S += delta k, readout q.S.
// Decode step with the row's sixteen runs interleaved over its four lanes:
// lane q owns runs q, q+4, q+8, q+12, S[8j + e] = element 8(q + 4j) + e, so in
// each 16-byte load or store the four lanes of a row touch one 128-byte line
// (with quarters of 32 contiguous per lane they would touch four). kq and qq
// point at element 8q. Quarter j (runs 4j..4j+3, one on each lane) is formed
// by xor 1, 2, and every lane then adds (Q0 + Q1) + (Q2 + Q3).
DEV float gdn_dot_il(const float (&S)[32], const float* vec) {
  float Q[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float r = S[8 * j] * vec[32 * j];
#pragma unroll
    for (int e = 1; e < 8; ++e) r = lisa_fma(S[8 * j + e], vec[32 * j + e], r);
    r = r + xor_lane<1>(r);
    Q[j] = r + xor_lane<2>(r);
  }
  return (Q[0] + Q[1]) + (Q[2] + Q[3]);
}

DEV float gdn_row_step_il(float (&S)[32], const float* kq, const float* qq, float vval, float beta, float decay) {
#pragma unroll
  for (int k = 0; k < 32; ++k) S[k] = S[k] * decay;
  const float pk = gdn_dot_il(S, kq);
  const float delta = (vval - pk) * beta;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) S[8 * j + e] = lisa_fma(delta, kq[32 * j + e], S[8 * j + e]);
  return gdn_dot_il(S, qq);
}

// Element offset of the lane's 16-byte chunk i (0..7) of its state row.
DEV int gdn_il_chunk(int q, int i) { return 8 * q + 32 * (i >> 1) + 4 * (i & 1); }

// Gated RMSNorm output of one element: bf16(bf16(y rinv w) silu(bf16 z)).
DEV uint16_t gdn_gated(float y, float rinv, float nw, float zraw) {
  const float n = lisa_bf16r((y * rinv) * nw);
  const float z = lisa_bf16r(zraw);
  return lisa_f32_to_bf16(n * lisa_silu_exp(z));
}

// Workgroups past the heads: the next q4 launch's 8-row tiles into the L2 of
// the XCD that launch's workgroup t runs on (workgroups go to the 8 XCDs
// round-robin by id, and the recurrence leaves the memory system mostly idle).
// Every load is issued before any is used; a tile is its pf_k / 4 W chunks
// and pf_k / 32 SB chunks of 16 bytes, at most 4 x 512.
typedef uint32_t lisa_u32x4 __attribute__((ext_vector_type(4)));
DEV void gdn_l2_prefetch(const LisaGdnParams& p) {
  constexpr int MAXT = 4;
  const uint32_t j = blockIdx.x - LISA_GDN_VH, x = j & 7, k = j >> 3, per = (gridDim.x - LISA_GDN_VH) >> 3;
  const uint32_t wq = p.pf_k / 4, sq = p.pf_k / 32;
  const uint4* w = reinterpret_cast<const uint4*>(p.pf_w);
  const uint4* sb = reinterpret_cast<const uint4*>(p.pf_sb);
  for (uint32_t i = 0; i < min(p.pf_delay, 64u); ++i) __builtin_amdgcn_s_sleep(8);
  lisa_u32x4 v[MAXT][4];
#pragma unroll
  for (int n = 0; n < MAXT; ++n) {
    const uint32_t t = x + 8 * (k + n * per);
    const bool ok = t < p.pf_tiles;
    const uint32_t ts = ok ? t : 0;  // tiles past the matrix address tile 0 (and load nothing)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t i = min(threadIdx.x + 512u * r, wq + sq - 1);
      const uint4* src = i < wq ? w + (size_t)ts * wq + i : sb + (size_t)ts * sq + (i - wq);
      v[n][r] = ok ? *reinterpret_cast<const lisa_u32x4*>(src) : lisa_u32x4{0, 0, 0, 0};
    }
  }
  uint32_t acc = 0;
#pragma unroll
  for (int n = 0; n < MAXT; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc ^= v[n][r].x ^ v[n][r].y ^ v[n][r].z ^ v[n][r].w;
  if (acc == 0x2545f491u) p.pf_sink[0] = acc;
}

// GSRC: a and b come from the in-projection's group contributions (gate_ab).
template <int M, bool GSRC>
DEV void gdn_body(const LisaGdnParams& p) {
  const int rows = M;
  const int h = blockIdx.x, kh = h / (LISA_GDN_VH / LISA_GDN_KH);
  const int tid = threadIdx.x, v = tid >> 2, q = tid & 3, lane = tid & 63, wave = tid >> 6;
  __shared__ float qn[128], kn[128], ybuf[128], sc[4];
  // Loads return in issue order within a wave: every row's small inputs go
  // first (q on wave 0 / k on wave 1 of the key head, the state row's v value,
  // z and the norm weight; the gate inputs are uniform, scalar loads), then
  // the 128 B of state this thread owns, so the norms and gates are formed
  // while the state arrives. None of these loads sits behind a branch: where
  // a branch merges loaded registers, the compiler waits for the loads, which
  // put a whole memory round trip in front of the state loads. Threads that
  // do not use a value load an in-bounds copy of it instead.
  float c0[M], c1[M], vval[M], zraw[M], braw[M], araw[M];
  float gav[M][5], gbv[M][5];
#pragma unroll
  for (int t = 0; t < M; ++t) {
    const float* co = p.conv_out + (size_t)t * LISA_GDN_CONV_DIM;
    const float* src = co + ((wave & 1) ? LISA_GDN_KEY_DIM : 0) + kh * 128;
    c0[t] = src[lane];
    c1[t] = src[lane + 64];
    vval[t] = co[2 * LISA_GDN_KEY_DIM + h * 128 + v];
    zraw[t] = p.z[(size_t)t * LISA_GDN_VALUE_DIM + h * 128 + (tid & 127)];
    braw[t] = 0.0f;
    araw[t] = 0.0f;
    if constexpr (!GSRC) {
      braw[t] = p.b[(size_t)t * LISA_GDN_VH + h];
      araw[t] = p.a[(size_t)t * LISA_GDN_VH + h];
    } else {
      // the in-projection's group contributions for lane li's groups
      // li, 16 + li, .., 64 + li (summed below by wave 2, once the state loads
      // are out)
      const float4* ga = reinterpret_cast<const float4*>(
          p.gate_ab + ((size_t)t * LISA_GDN_VH + h) * LISA_GDN_GATE_FLOATS + 12 * (lane & 15));
      const float4 g0 = ga[0], g1 = ga[1], g2 = ga[2];
      gav[t][0] = g0.x; gav[t][1] = g0.y; gav[t][2] = g0.z; gav[t][3] = g0.w; gav[t][4] = g1.x;
      gbv[t][0] = g1.y; gbv[t][1] = g1.z; gbv[t][2] = g1.w; gbv[t][3] = g2.x; gbv[t][4] = g2.y;
    }
  }
  const float nwt = bf2f(p.norm_w[tid & 127]);
  __builtin_amdgcn_sched_barrier(0);
  float* srow = p.state + (size_t)h * 128 * 128 + (size_t)v * 128;
  float S[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 f = *reinterpret_cast<const float4*>(srow + gdn_il_chunk(q, i));
    S[4 * i] = f.x; S[4 * i + 1] = f.y; S[4 * i + 2] = f.z; S[4 * i + 3] = f.w;
  }
  __builtin_amdgcn_sched_barrier(0);
  if (GSRC && wave == 2) {
    // a and b as a q4 launch forms a row: lane li adds its five group
    // contributions to a running sum from 0 in order, then tree16 (thread 128,
    // lane 0 of wave 2, forms the gates from them)
#pragma unroll
    for (int t = 0; t < M; ++t) {
      float ta = 0.0f, tb = 0.0f;
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        ta = ta + gav[t][i];
        tb = tb + gbv[t][i];
      }
      araw[t] = tree16(ta);
      braw[t] = tree16(tb);
    }
  }
#pragma unroll
  for (int t = 0; t < rows; ++t) {
    const size_t o = (size_t)t * LISA_GDN_VALUE_DIM + h * 128 + tid;
    if (wave < 2) {
      // q (wave 0) / k (wave 1) RMS with tree128, scaled 1/128 and 1/sqrt(128)
      float n0, n1;
      gdn_qk_norm(c0[t], c1[t], wave == 0 ? p.q_scale : p.k_scale, n0, n1);
      float* dst = wave == 0 ? qn : kn;
      dst[lane] = n0;
      dst[lane + 64] = n1;
    } else if (tid == 128) {
      gdn_gates(braw[t], araw[t], p.dt_bias[h], p.a_log[h], sc[0], sc[1]);
    }
    __syncthreads();
    const float py = gdn_row_step_il(S, kn + 8 * q, qn + 8 * q, vval[t], sc[0], sc[1]);
    if (q == 0) ybuf[v] = lisa_bf16r(py);
    if (p.capture && p.slots && t + 1 < rows) {
      float* dst = p.slots + (size_t)t * p.slot_stride + (size_t)h * 128 * 128 + (size_t)v * 128;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<float4*>(dst + gdn_il_chunk(q, i)) = make_float4(S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]);
    }
    // the state is final after the last row: its 64 KB per workgroup go out
    // now and drain while the gated norm runs
    if (t + 1 == rows) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<float4*>(srow + gdn_il_chunk(q, i)) = make_float4(S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]);
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
      p.gated[o] = gdn_gated(y, sc[2], nwt, zraw[t]);
      if (p.y_out) p.y_out[o] = y;
    }
    if (t + 1 < rows) __syncthreads();
  }
}

// Prefill over rows, in three launches with the arithmetic of gdn_body:
// lisa_gdn_prep_rows (grid (m, 9) x 256): normalized q and k of every row and
//   key head into qk [m][2][2048], beta and decay into gates [m][48][2];
// lisa_gdn_scan_rows (grid (48, 8) x 256, 16 state rows per workgroup,
//   sixteen lanes per state row with one run of 8 elements each): the
//   sequential delta-rule scan, with no barrier in the time loop (each state
//   row only needs the precomputed inputs), each time step's inputs loaded
//   eight steps ahead and staged eight steps at a time. A step is a chain of
//   dependent VALU work per state row, so the rows are spread over every CU
//   and each lane carries one run;
//   readout y (bf16 values) into y_out [m][6144];
// lisa_gdn_out_rows (grid (m, 48) x 128): gated RMSNorm of y into gated.
extern "C" __global__ __launch_bounds__(256) void lisa_gdn_prep_rows(LisaGdnParams p) {
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* co = p.conv_out + (size_t)t * LISA_GDN_CONV_DIM;
  if (blockIdx.y < 8) {
    const int pi = blockIdx.y * 4 + wave, which = pi / LISA_GDN_KH, kh = pi % LISA_GDN_KH;
    const float* src = co + which * LISA_GDN_KEY_DIM + kh * 128;
    float n0, n1;
    gdn_qk_norm(src[lane], src[lane + 64], which == 0 ? p.q_scale : p.k_scale, n0, n1);
    float* dst = p.qk + ((size_t)t * 2 + which) * LISA_GDN_KEY_DIM + kh * 128;
    dst[lane] = n0;
    dst[lane + 64] = n1;
  } else if (tid < LISA_GDN_VH) {
    float beta, decay;
    gdn_gates(p.b[(size_t)t * LISA_GDN_VH + tid], p.a[(size_t)t * LISA_GDN_VH + tid], p.dt_bias[tid], p.a_log[tid],
              beta, decay);
    reinterpret_cast<float2*>(p.gates)[(size_t)t * LISA_GDN_VH + tid] = make_float2(beta, decay);
  }
}

// Per-row inputs of the scan as one lane sees them: its 16 B of the row's k
// (lanes 0-31) or q (lanes 32-63) of the key head, the head's (beta, decay) and
// the v values of the lane's R state rows (v0 + 16 r).
// (native vector types: HIP's float4 struct copies lower to memcpy, which keeps
// an array of these out of registers)
typedef float lisa_f32x4 __attribute__((ext_vector_type(4)));
typedef float lisa_f32x2 __attribute__((ext_vector_type(2)));
template <int R>
struct GdnRowIn {
  lisa_f32x4 kq;
  lisa_f32x2 g;
  float v[R];
};

// state rows v0 + 16 r, r < R
template <int R>
DEV void gdn_row_load(const LisaGdnParams& p, int t, int h, int kh, int v0, int lane, GdnRowIn<R>& in) {
  const int which = lane < 32 ? 1 : 0;  // k, then q
  in.kq = reinterpret_cast<const lisa_f32x4*>(p.qk + ((size_t)t * 2 + which) * LISA_GDN_KEY_DIM + kh * 128)[lane & 31];
  in.g = reinterpret_cast<const lisa_f32x2*>(p.gates)[(size_t)t * LISA_GDN_VH + h];
  const float* vr = p.conv_out + (size_t)t * LISA_GDN_CONV_DIM + 2 * LISA_GDN_KEY_DIM + h * 128 + v0;
#pragma unroll
  for (int r = 0; r < R; ++r) in.v[r] = vr[16 * r];
}

// N row dots of the scan, each over a lane's 8 elements (run o of its row;
// lane o = 0..15 of the row): xor 1 adds the run pairs (r_4j + r_4j+1), xor 2
// forms quarter j, then (Q0 + Q1) / (Q2 + Q3) and the row. Each level leaves
// its groups of 2, 4 and 8 lanes holding one value, so the last two levels
// take the half-row mirror (lane i <- 7 - i within 8) and the row mirror (lane
// i <- 15 - i), DPP moves that bring each lane the other group's value as
// xor 4 and xor 8 do. The N chains are interleaved statement by statement: a
// wave issues in order, so each chain's dependent-latency gaps hold the
// others' instructions; each result is the same bits as alone.
template <int N>
DEV void gdn_dot8_n(const float (&X)[N][8], const float (&V)[N][8], float (&res)[N]) {
  float a[N];
#pragma unroll
  for (int n = 0; n < N; ++n) a[n] = X[n][0] * V[n][0];
#pragma unroll
  for (int e = 1; e < 8; ++e)
#pragma unroll
    for (int n = 0; n < N; ++n) a[n] = lisa_fma(X[n][e], V[n][e], a[n]);
#pragma unroll
  for (int n = 0; n < N; ++n) a[n] = a[n] + xor_lane<1>(a[n]);
#pragma unroll
  for (int n = 0; n < N; ++n) a[n] = a[n] + xor_lane<2>(a[n]);
#pragma unroll
  for (int n = 0; n < N; ++n)
    a[n] = a[n] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[n]), 0x141 /* row_half_mirror */,
                                                             0xf, 0xf, false));
#pragma unroll
  for (int n = 0; n < N; ++n)
    res[n] = a[n] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[n]), 0x140 /* row_mirror */, 0xf,
                                                               0xf, false));
}

// Grid (48 value heads, 8) x 256 threads: sixteen lanes per state row of the
// head (lane o owning run o, elements 8o .. 8o + 7), four rows per wave, 1536
// waves. (R rows per lane, v and v + 16, with grid (48, 8 / R) runs each
// row's arithmetic unchanged; two per lane, one wave per SIMD, measured
// slower than two one-row waves sharing a SIMD.)
extern "C" __global__ __launch_bounds__(256) void lisa_gdn_scan_rows(LisaGdnParams p) {
  constexpr int R = 1, D = 8;
  const int rows = (int)p.m_rows;
  const int h = blockIdx.x, kh = h / (LISA_GDN_VH / LISA_GDN_KH);
  const int tid = threadIdx.x, o = tid & 15, lane = tid & 63, wave = tid >> 6;
  const int v0 = blockIdx.y * 16 * R + (tid >> 4);
  // each wave stages D rows' k and q at a time in its own LDS ring (a wave
  // reads only what it wrote, so no workgroup barrier is needed)
  __shared__ lisa_f32x4 kqs[4][D][64];
  float* srow[R];
  float S[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    srow[r] = p.state + (size_t)h * 128 * 128 + (size_t)(v0 + 16 * r) * 128 + 8 * o;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float4 f = reinterpret_cast<const float4*>(srow[r])[i];
      S[r][4 * i] = f.x; S[r][4 * i + 1] = f.y; S[r][4 * i + 2] = f.z; S[r][4 * i + 3] = f.w;
    }
  }
  auto rd = [&](int j, int off, float (&dst)[8]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const lisa_f32x4 f = kqs[wave][j][off + 2 * o + i];
      dst[4 * i] = f.x; dst[4 * i + 1] = f.y; dst[4 * i + 2] = f.z; dst[4 * i + 3] = f.w;
    }
  };
  // one time step of the lane's rows: the state update and the readout y = q . S
  auto step = [&](int j, lisa_f32x2 g, const float (&vin)[R], float (&yo)[R]) {
    float kv[8], qv[8];
    rd(j, 0, kv);
    rd(j, 32, qv);
    float K[R][8], Q[R][8], pk[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        S[r][k] = S[r][k] * g.y;
        K[r][k] = kv[k];
        Q[r][k] = qv[k];
      }
    gdn_dot8_n<R>(S, K, pk);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float delta = (vin[r] - pk[r]) * g.x;
#pragma unroll
      for (int k = 0; k < 8; ++k) S[r][k] = lisa_fma(delta, kv[k], S[r][k]);
    }
    gdn_dot8_n<R>(S, Q, yo);
#pragma unroll
    for (int r = 0; r < R; ++r) yo[r] = lisa_bf16r(yo[r]);
  };
  GdnRowIn<R> in[D];
#pragma unroll
  for (int j = 0; j < D; ++j) gdn_row_load<R>(p, min(j, rows - 1), h, kh, v0, lane, in[j]);
  // a block's readouts are stored at the start of the next block, ahead of
  // its wait for the inputs, so that wait does not include the stores (loads
  // and stores share the wave's counter, in issue order); lane o stores time
  // step o % 8's readout of state row v0 + 16 ((o / 8) % R) (at R = 1 lanes o
  // and o + 8 store the same value)
  const int sj = o & 7, sr = (o >> 3) % R;
  float yo = 0.0f;
  int ny = 0, ty = 0;
  float* ycol = p.y_out + h * 128 + v0 + 16 * sr;
  for (int t0 = 0; t0 < rows; t0 += D) {
    // the previous block (whole: only the last block can be short, and it is
    // stored after the loop): one store per lane on every path, so the wait
    // below can count it; the first block has no predecessor and writes into
    // the lane's own state element, which the final state store overwrites
    {
      float* dst = ny == D ? ycol + (size_t)(ty + sj) * LISA_GDN_VALUE_DIM : srow[0];
      *dst = ny == D ? yo : S[0][0];
    }
    lisa_f32x2 g[D];
    float vin[D][R];
#pragma unroll
    for (int j = 0; j < D; ++j) {
      kqs[wave][j][lane] = in[j].kq;
      g[j] = in[j].g;
#pragma unroll
      for (int r = 0; r < R; ++r) vin[j][r] = in[j].v[r];
    }
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < D; ++j) gdn_row_load<R>(p, min(t0 + D + j, rows - 1), h, kh, v0, lane, in[j]);
    const int n = min(D, rows - t0);
    float y[D][R];
    if (n == D) {
      // step() software-pipelined: time step j's k . S chains run beside time
      // step j - 1's readouts (both read only the state after step j - 1),
      // and step j + 1's k and step j's q come from LDS while step j computes
      float kc[8], kn[8], qc[8], qp[8];
      rd(0, 0, kc);
#pragma unroll
      for (int j = 0; j < D; ++j) {
        if (j + 1 < D) rd(j + 1, 0, kn);
        rd(j, 32, qc);
        float X[2 * R][8], V[2 * R][8], res[2 * R];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            X[R + r][k] = S[r][k];  // the state after step j - 1, for its readout
            S[r][k] = S[r][k] * g[j].y;
            X[r][k] = S[r][k];
            V[r][k] = kc[k];
            V[R + r][k] = qp[k];
          }
        if (j == 0) {
          float pk[R];
          float XK[R][8], VK[R][8];
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < 8; ++k) { XK[r][k] = X[r][k]; VK[r][k] = V[r][k]; }
          gdn_dot8_n<R>(XK, VK, pk);
#pragma unroll
          for (int r = 0; r < R; ++r) res[r] = pk[r];
        } else {
          gdn_dot8_n<2 * R>(X, V, res);
#pragma unroll
          for (int r = 0; r < R; ++r) y[j - 1][r] = lisa_bf16r(res[R + r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float delta = (vin[j][r] - res[r]) * g[j].x;
#pragma unroll
          for (int k = 0; k < 8; ++k) S[r][k] = lisa_fma(delta, kc[k], S[r][k]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          qp[k] = qc[k];
          if (j + 1 < D) kc[k] = kn[k];
        }
      }
      float Q[R][8], yl[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int k = 0; k < 8; ++k) Q[r][k] = qp[k];
      gdn_dot8_n<R>(S, Q, yl);
#pragma unroll
      for (int r = 0; r < R; ++r) y[D - 1][r] = lisa_bf16r(yl[r]);
    } else {
#pragma unroll
      for (int j = 0; j < D; ++j)
        if (j < n) step(j, g[j], vin[j], y[j]);
    }
    wave_lds_fence();
    yo = y[0][0];
#pragma unroll
    for (int j = 0; j < D; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r) yo = (sj == j && sr == r) ? y[j][r] : yo;
    ny = n;
    ty = t0;
  }
  if (sj < ny) ycol[(size_t)(ty + sj) * LISA_GDN_VALUE_DIM] = yo;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 2; ++i)
      reinterpret_cast<float4*>(srow[r])[i] = make_float4(S[r][4 * i], S[r][4 * i + 1], S[r][4 * i + 2], S[r][4 * i + 3]);
}

extern "C" __global__ __launch_bounds__(128) void lisa_gdn_out_rows(LisaGdnParams p) {
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  __shared__ float rinv;
  const size_t o = (size_t)t * LISA_GDN_VALUE_DIM + h * 128;
  const float y = p.y_out[o + tid];
  const float zraw = p.z[o + tid], nwt = bf2f(p.norm_w[tid]);
  if (tid < 64) {
    const float y0 = y, y1 = p.y_out[o + lane + 64];
    const float tot = tree64(y0 * y0 + y1 * y1);
    if (lane == 0) rinv = lisa_rsqrt(tot / 128.0f + LISA_EPS);
  }
  __syncthreads();
  p.gated[o + tid] = gdn_gated(y, rinv, nwt, zraw);
}

// Workgroups 0..47: one value head each; past them, L2 prefetch of the next
// launch's weights.
template <int M>
DEV void gdn_entry(const LisaGdnParams& p) {
  if (blockIdx.x >= LISA_GDN_VH) {
    if (p.pf_w) gdn_l2_prefetch(p);
    return;
  }
  if (p.gate_ab) gdn_body<M, true>(p);
  else gdn_body<M, false>(p);
}
extern "C" __global__ __launch_bounds__(512) void lisa_gdn_recurrence_m1(LisaGdnParams p) { gdn_entry<1>(p); }
extern "C" __global__ __launch_bounds__(512) void lisa_gdn_recurrence_m3(LisaGdnParams p) { gdn_entry<3>(p); }

// ===========================================================================
// split-K decode attention
// ===========================================================================
// Norm + partial RoPE of one 256-wide head by one wave: lane l holds elements
// l, l+64, l+128, l+192; the sum of squares is tree64 of each element column
// then (W0+W1)+(W2+W3) — the rows-of-256 tree with one element per thread
// (attention.metal:99-114, 118-155).
// The pieces of head_norm_rope_wave, so a wave can issue the loads of all of
// its heads before the first one is processed and share the rotation of a
// position across heads.
DEV void hnr_load(const float* raw, const uint16_t* w, int lane, float (&v)[4], float (&wv)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = raw[lane + 64 * j];
    wv[j] = bf2f(w[lane + 64 * j]);
  }
}

DEV void rope_sincos(uint32_t pos, int lane, float& s, float& c) {
  const float angle = (float)pos * kRopeInvFreq[lane & 31];
  lisa_sincosf(angle, &s, &c);
}

// The same rotation with the lane's inverse frequency kRopeInvFreq[lane % 32]
// already loaded.
DEV void rope_sincos_f(uint32_t pos, float inv_freq, float& s, float& c) {
  lisa_sincosf((float)pos * inv_freq, &s, &c);
}

DEV void hnr_finish(const float (&raw)[4], const float (&wv)[4], float s, float c, int lane, float out[4]) {
  float v[4], wsum[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = lisa_bf16r(raw[j]);
    wsum[j] = tree64(v[j] * v[j]);
  }
  const float tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  const float inv = lisa_rsqrt(tot / 256.0f + LISA_EPS);
  float n[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) n[j] = (v[j] * inv) * wv[j];
  const float other = xor_lane<32>(n[0]);  // n[l+32] for l<32, n[l-32] for l>=32
  if (lane < 32)
    out[0] = lisa_bf16r(n[0] * c - other * s);
  else
    out[0] = lisa_bf16r(n[0] * c + other * s);
#pragma unroll
  for (int j = 1; j < 4; ++j) out[j] = lisa_bf16r(n[j]);
}

DEV void head_norm_rope_wave(const float* raw, const uint16_t* w, uint32_t pos, int lane, float out[4]) {
  float v[4], wv[4], s, c;
  hnr_load(raw, w, lane, v, wv);
  rope_sincos(pos, lane, s, c);
  hnr_finish(v, wv, s, c, lane, out);
}

// Scores of one row for two heads a, b of the same KV head over a slice of n
// cached tokens by one wave (lane = token; attention.metal:550-604): per head
// q.k with four accumulators over d mod 4, each an ascending fma chain,
// ((a0 + a1) + (a2 + a3)) / 16, slice max, p = exp2(log2e (score - max)),
// denominator tree64. Each K chunk is read and widened once for both heads.
DEV void slice_scores2(const float* qa, const float* qb, const uint16_t* Kt, int kp, int n, int lane,
                       float* pba, float* pbb, float* mla, float* mlb) {
  float sa = -INFINITY, sb = -INFINITY;
  if (lane < n) {
    const uint16_t* kr = Kt + lane * kp;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f, b3 = 0.0f;
#pragma unroll 2
    for (int d = 0; d < LISA_ATT_HD; d += 8) {
      const uint4 kk = *reinterpret_cast<const uint4*>(kr + d);
      const float4 xa = *reinterpret_cast<const float4*>(qa + d);
      const float4 ya = *reinterpret_cast<const float4*>(qa + d + 4);
      const float4 xb = *reinterpret_cast<const float4*>(qb + d);
      const float4 yb = *reinterpret_cast<const float4*>(qb + d + 4);
      const float k0 = lo_bf(kk.x), k1 = hi_bf(kk.x), k2 = lo_bf(kk.y), k3 = hi_bf(kk.y);
      const float k4 = lo_bf(kk.z), k5 = hi_bf(kk.z), k6 = lo_bf(kk.w), k7 = hi_bf(kk.w);
      a0 = lisa_fma(xa.x, k0, a0); a1 = lisa_fma(xa.y, k1, a1); a2 = lisa_fma(xa.z, k2, a2); a3 = lisa_fma(xa.w, k3, a3);
      b0 = lisa_fma(xb.x, k0, b0); b1 = lisa_fma(xb.y, k1, b1); b2 = lisa_fma(xb.z, k2, b2); b3 = lisa_fma(xb.w, k3, b3);
      a0 = lisa_fma(ya.x, k4, a0); a1 = lisa_fma(ya.y, k5, a1); a2 = lisa_fma(ya.z, k6, a2); a3 = lisa_fma(ya.w, k7, a3);
      b0 = lisa_fma(yb.x, k4, b0); b1 = lisa_fma(yb.y, k5, b1); b2 = lisa_fma(yb.z, k6, b2); b3 = lisa_fma(yb.w, k7, b3);
    }
    sa = ((a0 + a1) + (a2 + a3)) * 0.0625f;
    sb = ((b0 + b1) + (b2 + b3)) * 0.0625f;
  }
  const float ma = max64(sa), mb = max64(sb);
  const float pa = (lane < n) ? lisa_exp2f(1.4426950408889634f * (sa - ma)) : 0.0f;
  const float pbv = (lane < n) ? lisa_exp2f(1.4426950408889634f * (sb - mb)) : 0.0f;
  const float da = tree64(pa), db = tree64(pbv);
  pba[lane] = pa;
  pbb[lane] = pbv;
  if (lane == 0) {
    mla[0] = ma;
    mla[1] = da;
    mlb[0] = mb;
    mlb[1] = db;
  }
}

// P.V of one row over the slice for three heads (rows of pb3 T apart) and the
// two output dimensions 2dp, 2dp+1: six chains acc = fma(p_tok, v_tok, acc)
// over the tokens in order; one 32-bit V read per token serves all six.
DEV void slice_pv3(const float* pb3, const uint16_t* Vt, int n, int dp, float (&acc)[3][2]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) acc[i][0] = acc[i][1] = 0.0f;
#pragma unroll 4
  for (int tok = 0; tok < n; ++tok) {
    const uint32_t vw = *reinterpret_cast<const uint32_t*>(Vt + tok * LISA_ATT_HD + 2 * dp);
    const float v0 = lo_bf(vw), v1 = hi_bf(vw);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const float pv = pb3[i * LISA_ATT_SLICE + tok];
      acc[i][0] = lisa_fma(pv, v0, acc[i][0]);
      acc[i][1] = lisa_fma(pv, v1, acc[i][1]);
    }
  }
}

// Loads return in issue order within a wave, so the partial issues them
// smallest and most urgent first: the decode position (a vector load, see
// vload_u32), the raw query heads, the lane's RoPE frequency (constant-index
// scalar loads: a vector table load is sunk to its first use), the appended
// rows' raw key and value, and then every K and V row of the slice, clamped
// below the capacity, before the position is known. The queries are normalized
// and rotated, and the appended rows written, while the slice is in flight.
// The slice's q.k runs on 12 M items (row, head pair, class d mod 4), one per
// wave: each is one of the four accumulators of attention.metal:550-604's dot
// (an ascending fma chain over d = r, r + 4, ..), read from K and q stored
// class-major in LDS (element d of a row at (d & 3) 64 + (d >> 2), rows padded
// to 264 entries); after a barrier, one wave per (row, head pair) forms
// ((a0 + a1) + (a2 + a3)) / 16 and the slice softmax statistics. P.V: thread
// (d, item) owns dimension d of three heads, chains over the tokens in order.
// One row: spreading q.k over twelve waves instead of three, 59.2 -> 55.4 us
// at ctx 32768 and 16.1 -> 15.9 us at ctx 4096 (partial + merge). Three rows
// keep attn_partial_pairs below (one wave per row and head pair, all four
// accumulators; 387 against 408 us per verify).
typedef uint32_t lisa_u32x4 __attribute__((ext_vector_type(4)));
template <int M, int NT>
DEV void attn_partial_body(const LisaAttnParams& p) {
  constexpr int T = LISA_ATT_SLICE, HD = LISA_ATT_HD, KP = HD + 8, NW = NT / 64;
  const int s = blockIdx.x, kvh = blockIdx.y;
  const uint32_t t0 = (uint32_t)s * T;
  __shared__ __attribute__((aligned(16))) uint16_t Kc[T * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[T * HD];
  __shared__ __attribute__((aligned(16))) float qc[M * 6 * HD];
  __shared__ __attribute__((aligned(16))) float pb[M * 6 * T];
  __shared__ __attribute__((aligned(16))) float sc[M * 6 * 4 * T];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t cache_base = (size_t)kvh * p.capacity * HD;
  const uint32_t pos_v = vload_u32(p.pos);
  constexpr int QP = (6 * M + NW - 1) / NW;
  float qraw[QP][4], qw[QP][4];
#pragma unroll
  for (int j = 0; j < QP; ++j) {
    const int pr = min(wave + NW * j, 6 * M - 1), t = pr / 6, i = pr % 6;
    hnr_load(p.q_proj + (size_t)t * LISA_ATT_Q_OUT + (kvh * 6 + i) * 512, p.q_norm_w, lane, qraw[j], qw[j]);
  }
  float inv_freq = 0.0f;
#pragma unroll
  for (int j = 0; j < LISA_ROPE_PAIRS; ++j) inv_freq = (lane & 31) == j ? kRopeInvFreq[j] : inv_freq;
  const int wr = min(wave, M - 1);
  float nkraw[4], nkw[4], nvraw[4];
  hnr_load(p.k_raw + (size_t)wr * LISA_ATT_KV_OUT + kvh * HD, p.k_norm_w, lane, nkraw, nkw);
#pragma unroll
  for (int j = 0; j < 4; ++j) nvraw[j] = p.v_raw[(size_t)wr * LISA_ATT_KV_OUT + kvh * HD + lane + 64 * j];
  __builtin_amdgcn_sched_barrier(0);
  constexpr int R = T * (HD / 8) / NT;
  lisa_u32x4 kr[R], vr[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int c = tid + NT * i, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
    const size_t off = cache_base + (size_t)min(t0 + row, p.capacity - 1) * HD + col;
    kr[i] = *reinterpret_cast<const lisa_u32x4*>(p.key_cache + off);
    vr[i] = *reinterpret_cast<const lisa_u32x4*>(p.value_cache + off);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t base = __builtin_amdgcn_readfirstlane(pos_v);
  if (t0 >= base + M) return;
  float rs[M], rc[M];
#pragma unroll
  for (int t = 0; t < M; ++t) rope_sincos_f(base + t, inv_freq, rs[t], rc[t]);
  // queries, class-major: element d of head (t, i) at qc[(t 6 + i) 256 + (d & 3) 64 + (d >> 2)]
#pragma unroll
  for (int j = 0; j < QP; ++j) {
    const int pr = wave + NW * j;
    if (pr >= 6 * M) break;
    const int t = pr / 6, i = pr % 6;
    float qo[4];
    hnr_finish(qraw[j], qw[j], rs[t], rc[t], lane, qo);
#pragma unroll
    for (int e = 0; e < 4; ++e) qc[(t * 6 + i) * HD + (lane & 3) * 64 + (lane >> 2) + 16 * e] = qo[e];
  }
  if (wave < M) {
    const uint32_t pos = base + wave;
    if (pos >= t0 && pos < t0 + T && pos < p.capacity) {
      float kn[4];
      hnr_finish(nkraw, nkw, rs[wave], rc[wave], lane, kn);
      const int row = (int)(pos - t0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        const uint16_t kb = lisa_f32_to_bf16(kn[j]);
        const uint16_t vb = lisa_f32_to_bf16(nvraw[j]);
        Kc[row * KP + (lane & 3) * 64 + (lane >> 2) + 16 * j] = kb;
        Vt[row * HD + d] = vb;
        p.key_cache[cache_base + (size_t)pos * HD + d] = kb;
        p.value_cache[cache_base + (size_t)pos * HD + d] = vb;
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // K class-major: the chunk's elements col + e and col + e + 4 (class e) are
  // entries 2 (c % 32), 2 (c % 32) + 1 of class e of the row
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int c = tid + NT * i, row = c / (HD / 8), cc = c % (HD / 8), col = cc * 8;
    if (t0 + row < base) {
      const lisa_u32x4 k = kr[i];
      uint32_t* kd = reinterpret_cast<uint32_t*>(&Kc[row * KP + 2 * cc]);
      kd[0] = (k.x & 0xffffu) | (k.z << 16);
      kd[32] = (k.x >> 16) | (k.z & 0xffff0000u);
      kd[64] = (k.y & 0xffffu) | (k.w << 16);
      kd[96] = (k.y >> 16) | (k.w & 0xffff0000u);
      *reinterpret_cast<lisa_u32x4*>(&Vt[row * HD + col]) = vr[i];
    }
  }
  __syncthreads();
  // 5a. item (row t, head pair, class r): lane = token, the class-r accumulator
  // of heads 2 pair and 2 pair + 1 (an ascending fma chain over d = r, r + 4, ..)
  for (int it = wave; it < 12 * M; it += NW) {
    const int t = it / 12, pr = (it % 12) >> 2, r = it & 3, i = 2 * pr;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    if (lane < n) {
      const uint16_t* kk = Kc + lane * KP + r * 64;
      const float* qa = qc + (t * 6 + i) * HD + r * 64;
      const float* qb = qa + HD;
      float a = 0.0f, b = 0.0f;
#pragma unroll 2
      for (int j = 0; j < 64; j += 8) {
        const uint4 k8 = *reinterpret_cast<const uint4*>(kk + j);
        const float4 xa = *reinterpret_cast<const float4*>(qa + j), ya = *reinterpret_cast<const float4*>(qa + j + 4);
        const float4 xb = *reinterpret_cast<const float4*>(qb + j), yb = *reinterpret_cast<const float4*>(qb + j + 4);
        const float k0 = lo_bf(k8.x), k1 = hi_bf(k8.x), k2 = lo_bf(k8.y), k3 = hi_bf(k8.y);
        const float k4 = lo_bf(k8.z), k5 = hi_bf(k8.z), k6 = lo_bf(k8.w), k7 = hi_bf(k8.w);
        a = lisa_fma(xa.x, k0, a); b = lisa_fma(xb.x, k0, b);
        a = lisa_fma(xa.y, k1, a); b = lisa_fma(xb.y, k1, b);
        a = lisa_fma(xa.z, k2, a); b = lisa_fma(xb.z, k2, b);
        a = lisa_fma(xa.w, k3, a); b = lisa_fma(xb.w, k3, b);
        a = lisa_fma(ya.x, k4, a); b = lisa_fma(yb.x, k4, b);
        a = lisa_fma(ya.y, k5, a); b = lisa_fma(yb.y, k5, b);
        a = lisa_fma(ya.z, k6, a); b = lisa_fma(yb.z, k6, b);
        a = lisa_fma(ya.w, k7, a); b = lisa_fma(yb.w, k7, b);
      }
      sc[((t * 6 + i) * 4 + r) * T + lane] = a;
      sc[((t * 6 + i + 1) * 4 + r) * T + lane] = b;
    }
  }
  __syncthreads();
  // 5b. item (row t, head pair): scores ((a0 + a1) + (a2 + a3)) / 16 and the
  // slice softmax statistics, as slice_scores2
  for (int it = wave; it < 3 * M; it += NW) {
    const int t = it / 3, i = 2 * (it % 3), h = kvh * 6 + i;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    float sa = -INFINITY, sb = -INFINITY;
    if (lane < n) {
      const float* ca = sc + (t * 6 + i) * 4 * T + lane;
      const float* cb = ca + 4 * T;
      sa = ((ca[0] + ca[T]) + (ca[2 * T] + ca[3 * T])) * 0.0625f;
      sb = ((cb[0] + cb[T]) + (cb[2 * T] + cb[3 * T])) * 0.0625f;
    }
    const float ma = max64(sa), mb = max64(sb);
    const float pa = (lane < n) ? lisa_exp2f(1.4426950408889634f * (sa - ma)) : 0.0f;
    const float pbv = (lane < n) ? lisa_exp2f(1.4426950408889634f * (sb - mb)) : 0.0f;
    const float da = tree64(pa), db = tree64(pbv);
    pb[(t * 6 + i) * T + lane] = pa;
    pb[(t * 6 + i + 1) * T + lane] = pbv;
    if (lane == 0) {
      float* ml = p.part_ml + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * 2;
      ml[0] = ma;
      ml[1] = da;
      ml[(size_t)p.s_max * 2] = mb;
      ml[(size_t)p.s_max * 2 + 1] = db;
    }
  }
  __syncthreads();
  // 6. P.V: thread (d, item) = (tid % 256, tid / 256): dimension d of heads
  // 3 hg .. 3 hg + 2 of row t (item = 2 t + hg), chains over the tokens in order
  const int d = tid & 255;
  for (int item = tid >> 8; item < 2 * M; item += NT / 256) {
    const int t = item >> 1, hg = item & 1;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    const float* p3 = pb + (t * 6 + 3 * hg) * T;
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f;
#pragma unroll 4
    for (int tok = 0; tok < n; ++tok) {
      const float v = bf2f(Vt[tok * HD + d]);
      acc0 = lisa_fma(p3[tok], v, acc0);
      acc1 = lisa_fma(p3[T + tok], v, acc1);
      acc2 = lisa_fma(p3[2 * T + tok], v, acc2);
    }
    float* po = p.part_o + (((size_t)t * LISA_ATT_QH + kvh * 6 + 3 * hg) * p.s_max + s) * HD + d;
    po[0] = acc0;
    po[(size_t)p.s_max * HD] = acc1;
    po[(size_t)2 * p.s_max * HD] = acc2;
  }
}

// Three rows: the same stages with q.k as one item per (row, head pair), lane =
// token, all four accumulators in one lane (slice_scores2), and P.V thread
// (dp, hg) = (tid % 128, tid / 128) owning dimensions 2dp, 2dp+1 of heads
// 3hg..3hg+2 (slice_pv3); K and q row-major in LDS.
template <int M, int NT>
DEV void attn_partial_pairs(const LisaAttnParams& p) {
  constexpr int T = LISA_ATT_SLICE, HD = LISA_ATT_HD, KP = HD + 8, NW = NT / 64;
  const int s = blockIdx.x, kvh = blockIdx.y;
  const uint32_t t0 = (uint32_t)s * T;
  __shared__ __attribute__((aligned(16))) uint16_t Kt[T * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[T * HD];
  __shared__ __attribute__((aligned(16))) float qv[M * 6 * HD];
  __shared__ __attribute__((aligned(16))) float pb[M * 6 * T];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t cache_base = (size_t)kvh * p.capacity * HD;
  const uint32_t pos_v = vload_u32(p.pos);

  // 0. the raw query heads of this wave (pairs pr = wave + NW j of row t = pr / 6,
  // head i = pr % 6), the RoPE frequency, and wave t < M: row t's raw key, its
  // norm weights and raw value
  constexpr int QP = (6 * M + NW - 1) / NW;
  float qraw[QP][4], qw[QP][4];
#pragma unroll
  for (int j = 0; j < QP; ++j) {
    const int pr = min(wave + NW * j, 6 * M - 1), t = pr / 6, i = pr % 6;
    hnr_load(p.q_proj + (size_t)t * LISA_ATT_Q_OUT + (kvh * 6 + i) * 512, p.q_norm_w, lane, qraw[j], qw[j]);
  }
  float inv_freq = 0.0f;
#pragma unroll
  for (int j = 0; j < LISA_ROPE_PAIRS; ++j) inv_freq = (lane & 31) == j ? kRopeInvFreq[j] : inv_freq;
  const int wr = min(wave, M - 1);
  float nkraw[4], nkw[4], nvraw[4];
  hnr_load(p.k_raw + (size_t)wr * LISA_ATT_KV_OUT + kvh * HD, p.k_norm_w, lane, nkraw, nkw);
#pragma unroll
  for (int j = 0; j < 4; ++j) nvraw[j] = p.v_raw[(size_t)wr * LISA_ATT_KV_OUT + kvh * HD + lane + 64 * j];
  __builtin_amdgcn_sched_barrier(0);
  // 1. every row of the slice (chunk c = tid + NT i: row c / 32, columns
  // 8 (c % 32) ..), clamped below the capacity (native vector types: HIP's
  // uint4 struct copies lower to memcpy, which keeps an array of them out of
  // registers)
  constexpr int R = T * (HD / 8) / NT;
  lisa_u32x4 kr[R], vr[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int c = tid + NT * i, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
    const size_t off = cache_base + (size_t)min(t0 + row, p.capacity - 1) * HD + col;
    kr[i] = *reinterpret_cast<const lisa_u32x4*>(p.key_cache + off);
    vr[i] = *reinterpret_cast<const lisa_u32x4*>(p.value_cache + off);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t base = __builtin_amdgcn_readfirstlane(pos_v);
  if (t0 >= base + M) return;
  // 2. normalized, rotated queries of the 6 heads sharing this KV head (one
  // rotation per row position)
  float rs[M], rc[M];
#pragma unroll
  for (int t = 0; t < M; ++t) rope_sincos_f(base + t, inv_freq, rs[t], rc[t]);
#pragma unroll
  for (int j = 0; j < QP; ++j) {
    const int pr = wave + NW * j;
    if (pr >= 6 * M) break;
    const int t = pr / 6, i = pr % 6;
    float qo[4];
    hnr_finish(qraw[j], qw[j], rs[t], rc[t], lane, qo);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[(t * 6 + i) * HD + lane + 64 * e] = qo[e];
  }
  // 3. rows appended by this step that fall into the slice (kv_cache_store_decode)
  if (wave < M) {
    const uint32_t pos = base + wave;
    if (pos >= t0 && pos < t0 + T && pos < p.capacity) {
      float kn[4];
      hnr_finish(nkraw, nkw, rs[wave], rc[wave], lane, kn);
      const int row = (int)(pos - t0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        const uint16_t kb = lisa_f32_to_bf16(kn[j]);
        const uint16_t vb = lisa_f32_to_bf16(nvraw[j]);
        Kt[row * KP + d] = kb;
        Vt[row * HD + d] = vb;
        p.key_cache[cache_base + (size_t)pos * HD + d] = kb;
        p.value_cache[cache_base + (size_t)pos * HD + d] = vb;
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 4. rows already in the cache (positions < base) go to LDS; later rows lie
  // past every row's context
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int c = tid + NT * i, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
    if (t0 + row < base) {
      *reinterpret_cast<lisa_u32x4*>(&Kt[row * KP + col]) = kr[i];
      *reinterpret_cast<lisa_u32x4*>(&Vt[row * HD + col]) = vr[i];
    }
  }
  __syncthreads();
  // 5. scores and slice softmax statistics: item (row t, head pair k) per wave,
  // lane = token of the slice
  for (int it = wave; it < 3 * M; it += NW) {
    const int t = it / 3, i = 2 * (it % 3), h = kvh * 6 + i;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    const float* qa = qv + (t * 6 + i) * HD;
    float* ml = p.part_ml + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * 2;
    slice_scores2(qa, qa + HD, Kt, KP, n, lane, pb + (t * 6 + i) * T, pb + (t * 6 + i + 1) * T, ml,
                  ml + (size_t)p.s_max * 2);
  }
  __syncthreads();
  // 6. P.V: thread group g = tid / 128 takes the (row, head group) items
  // g, g + NT / 128, .. of the 2 M items (row t = item / 2, heads 3 (item % 2) ..)
  const int dp = tid & 127;
  for (int item = tid >> 7; item < 2 * M; item += NT / 128) {
    const int t = item >> 1, hg = item & 1;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    float acc[3][2];
    slice_pv3(pb + (t * 6 + 3 * hg) * T, Vt, n, dp, acc);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int h = kvh * 6 + 3 * hg + i;
      *reinterpret_cast<float2*>(p.part_o + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * HD + 2 * dp) =
          make_float2(acc[i][0], acc[i][1]);
    }
  }
}

#define ATT_MAX_SLICES 1024
// Flash merge of the slice partials of one (head, row) in ascending slice order
// (attention.metal:611-641): weights w_s = exp2(log2e (m_s - max m)), output
// (sum w_s o_s) / (sum w_s den_s), both as fma chains; then the output gate.
// The output gate's input and the statistics of the first 256 slices (index
// clamped to the allocated s_max slices) are loaded before the position is
// known, so the statistics do not wait for it.
template <int M>
DEV void attn_merge_body(const LisaAttnParams& p) {
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const uint32_t pos_v = vload_u32(p.pos);
  const float graw = p.q_proj[(size_t)t * LISA_ATT_Q_OUT + h * 512 + 256 + tid];
  __shared__ float ws[ATT_MAX_SLICES], dn[ATT_MAX_SLICES], red[4];
  const float* ml = p.part_ml + ((size_t)t * LISA_ATT_QH + h) * p.s_max * 2;
  const int s0 = min(tid, (int)p.s_max - 1);
  const float m0 = ml[2 * s0], d0 = ml[2 * s0 + 1];
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t ctx = __builtin_amdgcn_readfirstlane(pos_v) + t + 1;
  // slices past the allocated s_max (a caller whose position outruns the grid
  // it launched) are never read
  const int used = min((int)((ctx + LISA_ATT_SLICE - 1) / LISA_ATT_SLICE), (int)p.s_max);
  float mx = tid < used ? m0 : -INFINITY;
  for (int s = tid + 256; s < used; s += 256) mx = fmaxf(mx, ml[2 * s]);
  mx = max64(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float gmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (tid < used) {
    ws[tid] = lisa_exp2f(1.4426950408889634f * (m0 - gmax));
    dn[tid] = d0;
  }
  for (int s = tid + 256; s < used; s += 256) {
    ws[s] = lisa_exp2f(1.4426950408889634f * (ml[2 * s] - gmax));
    dn[s] = ml[2 * s + 1];
  }
  __syncthreads();
  const float* po = p.part_o + ((size_t)t * LISA_ATT_QH + h) * p.s_max * LISA_ATT_HD + tid;
  float res = 0.0f, tot = 0.0f;
#pragma unroll 32
  for (int s = 0; s < used; ++s) {
    res = lisa_fma(ws[s], po[(size_t)s * LISA_ATT_HD], res);
    tot = lisa_fma(ws[s], dn[s], tot);
  }
  const float o = res / tot;
  const float g = lisa_bf16r(graw);
  p.gated[(size_t)t * LISA_ATT_OUT + h * LISA_ATT_HD + tid] = lisa_f32_to_bf16(o * lisa_sigmoid_exp2(g));
}

extern "C" __global__ __launch_bounds__(LISA_ATT_PARTIAL_THREADS(1)) void lisa_attn_partial_m1(LisaAttnParams p) {
  attn_partial_body<1, LISA_ATT_PARTIAL_THREADS(1)>(p);
}
extern "C" __global__ __launch_bounds__(LISA_ATT_PARTIAL_THREADS(3)) void lisa_attn_partial_m3(LisaAttnParams p) {
  attn_partial_pairs<3, LISA_ATT_PARTIAL_THREADS(3)>(p);
}
extern "C" __global__ __launch_bounds__(256) void lisa_attn_merge_m1(LisaAttnParams p) { attn_merge_body<1>(p); }
extern "C" __global__ __launch_bounds__(256) void lisa_attn_merge_m3(LisaAttnParams p) { attn_merge_body<3>(p); }

// ===========================================================================
// batched prefill (runner.rs:2129-2230)
// ===========================================================================
// q4 GEMM (gemm.metal:152-341 semantics): C[m][n] = sum_k A[m][k] * Wd[n][k],
// Wd = bf16(fma(scale, q, bias)), bf16 MFMA 32x32x16 with f32 accumulation.
// Output tile 256 x BN per workgroup (lisa_q4_gemm: BN = 128, 4 waves;
// lisa_q4_gemm_wide: BN = 256, 8 waves), one 64-wide K step per q4 group. The
// waves split the tile 2 x 2 or 2 x 4; each owns a 128 x 64 block as 4 x 2 MFMA
// blocks (accumulators in AGPRs). LDS holds two stages of the A rows and the dequantized W rows (rows
// padded to 72 bf16, so the 8 lanes of each 128-byte LDS pass read distinct
// banks); global loads run two K steps ahead in two register sets, and the
// A copy and W dequant of step s+1 are interleaved with step s's MFMAs (the
// MFMAs run in the matrix core while the VALU works), so each K step needs
// one barrier. The launcher picks the tile per shape (fewer, longer tiles
// against the last round on 256 CUs).
typedef __bf16 lisa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lisa_f32x16 __attribute__((ext_vector_type(16)));
// Native 4 x u32 vectors for the staging registers (HIP's uint4 struct copies
// lower to memcpy, which keeps loop-carried arrays of them out of registers).
typedef uint32_t lisa_u32x4 __attribute__((ext_vector_type(4)));

constexpr int GEMM_BM = LISA_GEMM_TILE_M, GEMM_PAD = 72;

// NT threads (4 or 8 waves): waves split the BM x BN tile 2 x WN; each wave
// owns a BM/2 x BN/WN block as AB x NB MFMA blocks.
template <int BN, int NT, int BM = GEMM_BM>
struct GemmCfg {
  static constexpr int WAVES = NT / 64;
  static constexpr int WN = WAVES / 2;                 // waves along N (2 or 4)
  static constexpr int AB = BM / 64;                   // 32-row A blocks per wave
  static constexpr int RA = BM * 8 / NT;               // A chunks per thread and K step
  static constexpr int RW = BN * 2 / NT;               // W 16 B chunks per thread and K step
  static constexpr int NB = BN / WN / 32;              // 32-wide N blocks per wave
  static_assert(RA % 4 == 0 && RW >= 1 && NB >= 1 && AB >= 1 && (32 * RW) % (AB * NB) == 0, "tile");
};

template <int BN, int NT, int BM>
DEV void gemm_lstore(uint16_t* as, uint16_t* ws, int tid, const lisa_u32x4* a, const lisa_u32x4* w, uint32_t sb) {
  using G = GemmCfg<BN, NT, BM>;
#pragma unroll
  for (int i = 0; i < G::RA; ++i) {
    const int u = tid + NT * i;
    *reinterpret_cast<lisa_u32x4*>(&as[(u >> 3) * GEMM_PAD + (u & 7) * 8]) = a[i];
  }
  const float sc = lo_bf(sb), bi = hi_bf(sb);
#pragma unroll
  for (int r = 0; r < G::RW; ++r) {
    const int u = G::RW * tid + r;
    uint16_t* dst = &ws[(u >> 1) * GEMM_PAD + (u & 1) * 32];
    const uint32_t wd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = lisa_fma(sc, (float)((wd[j] >> (4 * e)) & 0xfu), bi);
      *reinterpret_cast<uint4*>(dst + 8 * j) =
          make_uint4(lisa_f32x2_to_bf16x2(v[0], v[1]), lisa_f32x2_to_bf16x2(v[2], v[3]),
                     lisa_f32x2_to_bf16x2(v[4], v[5]), lisa_f32x2_to_bf16x2(v[6], v[7]));
    }
  }
}

template <int BN, int NT, int BM>
DEV void gemm_frags(const uint16_t* as, const uint16_t* ws, int wm, int wn, int lane, int ks,
                    lisa_bf16x8 (&af)[GemmCfg<BN, NT, BM>::AB], lisa_bf16x8 (&bf)[GemmCfg<BN, NT, BM>::NB]) {
  using G = GemmCfg<BN, NT, BM>;
#pragma unroll
  for (int i = 0; i < G::AB; ++i)
    af[i] = *reinterpret_cast<const lisa_bf16x8*>(
        &as[(wm * (BM / 2) + i * 32 + (lane & 31)) * GEMM_PAD + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
  for (int j = 0; j < G::NB; ++j)
    bf[j] = *reinterpret_cast<const lisa_bf16x8*>(
        &ws[(wn * (BN / G::WN) + j * 32 + (lane & 31)) * GEMM_PAD + ks * 16 + 8 * (lane >> 5)]);
}

template <int BN, int NT, int BM>
DEV void gemm_step(const uint16_t* as_r, const uint16_t* ws_r, uint16_t* as_w, uint16_t* ws_w, int tid, int wm, int wn,
                   int lane, const lisa_u32x4* a, const lisa_u32x4* w, uint32_t sb,
                   lisa_f32x16 (&acc)[GemmCfg<BN, NT, BM>::AB][GemmCfg<BN, NT, BM>::NB]) {
  using G = GemmCfg<BN, NT, BM>;
  lisa_bf16x8 af[2][G::AB], bf[2][G::NB];
  gemm_frags<BN, NT, BM>(as_r, ws_r, wm, wn, lane, 0, af[0], bf[0]);
  const float sc = lo_bf(sb), bi = hi_bf(sb);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c = ks & 1;
    if (ks + 1 < 4) gemm_frags<BN, NT, BM>(as_r, ws_r, wm, wn, lane, ks + 1, af[c ^ 1], bf[c ^ 1]);
#pragma unroll
    for (int i = 0; i < G::AB; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < G::RW; ++r) {
      const uint32_t word = ks == 0 ? w[r].x : ks == 1 ? w[r].y : ks == 2 ? w[r].z : w[r].w;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = lisa_fma(sc, (float)((word >> (4 * e)) & 0xfu), bi);
      const int u = G::RW * tid + r;
      *reinterpret_cast<uint4*>(&ws_w[(u >> 1) * GEMM_PAD + (u & 1) * 32 + 8 * ks]) =
          make_uint4(lisa_f32x2_to_bf16x2(v[0], v[1]), lisa_f32x2_to_bf16x2(v[2], v[3]),
                     lisa_f32x2_to_bf16x2(v[4], v[5]), lisa_f32x2_to_bf16x2(v[6], v[7]));
    }
#pragma unroll
    for (int i = ks * (G::RA / 4); i < (ks + 1) * (G::RA / 4); ++i) {
      const int u = tid + NT * i;
      *reinterpret_cast<lisa_u32x4*>(&as_w[(u >> 3) * GEMM_PAD + (u & 7) * 8]) = a[i];
    }
    if (ks + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x100, G::AB + G::NB, 0);
#pragma unroll
    for (int q = 0; q < G::AB * G::NB; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 32 * G::RW / (G::AB * G::NB) + 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x200, G::RA / 4 + G::RW, 0);
  }
}

// SWIGLU: the tile's W rows are the gate and up rows of BN / 2 output
// columns, laid out so that MFMA block j of wave wn holds matrix j (0 gate,
// 1 up) of columns n0 + wn * 32 + (0..31); the epilogue then finds the gate
// and up sums of an output in the same lane and writes bf16(silu(bf16 g) *
// bf16 u) (mlp.metal:11-16) instead of the two f32 outputs.
template <int BN, int NT, bool SWIGLU = false, int BM = GEMM_BM>
DEV void q4_gemm_body(const LisaGemmParams& p, uint16_t (*As)[BM * GEMM_PAD], uint16_t (*Ws)[BN * GEMM_PAD]) {
  using G = GemmCfg<BN, NT, BM>;
  static_assert(!SWIGLU || G::NB == 2, "the gate/up tile pairs two 32-wide blocks per wave");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WN, wn = wave % G::WN;
  const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * (SWIGLU ? BN / 2 : BN);
  const uint32_t K = p.k, nk = K / 64;

  const lisa_u32x4* asrc[G::RA];
#pragma unroll
  for (int i = 0; i < G::RA; ++i) {
    const int u = tid + NT * i;
    const uint32_t row = min(m0 + (uint32_t)(u >> 3), p.m - 1);
    asrc[i] = reinterpret_cast<const lisa_u32x4*>(p.a + (size_t)row * K) + (u & 7);
  }
  // the W row this thread stages: LDS row l = (RW tid) / 2 (RW = 1 on the
  // SWIGLU tile), of matrix (l / 32) % 2 and column n0 + (l / 64) 32 + l % 32
  // there
  const uint32_t lrow = (uint32_t)((G::RW * tid) >> 1);
  const bool upm = SWIGLU && ((lrow >> 5) & 1);
  const uint32_t wrow = min(SWIGLU ? n0 + (lrow >> 6) * 32 + (lrow & 31) : n0 + lrow, p.n - 1);
  const uint32_t* wmat = upm ? p.w2 : p.w;
  const uint32_t* sbmat = upm ? p.sb2 : p.sb;
  const lisa_u32x4* wsrc = reinterpret_cast<const lisa_u32x4*>(wmat + (size_t)wrow * (K / 8)) + ((G::RW * tid) & 1);
  const uint32_t* sbsrc = sbmat + (size_t)wrow * (K / 64);

  lisa_f32x16 acc[G::AB][G::NB];
#pragma unroll
  for (int i = 0; i < G::AB; ++i)
#pragma unroll
    for (int j = 0; j < G::NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#define GEMM_GLOAD(A, W, SB, STEP)                                                        \
  {                                                                                       \
    const uint32_t st_ = min((uint32_t)(STEP), nk - 1);                                   \
    _Pragma("unroll") for (int i = 0; i < G::RA; ++i) A[i] = asrc[i][st_ * 8];            \
    _Pragma("unroll") for (int r = 0; r < G::RW; ++r) W[r] = wsrc[st_ * 2 + r];           \
    SB = sbsrc[st_] & ((uint32_t)(STEP) < nk ? 0xffffffffu : 0u);                         \
  }
  lisa_u32x4 a0[G::RA], a1[G::RA], w0[G::RW], w1[G::RW];
  uint32_t sb0, sb1;
  GEMM_GLOAD(a0, w0, sb0, 0);
  GEMM_GLOAD(a1, w1, sb1, 1);
  gemm_lstore<BN, NT, BM>(As[0], Ws[0], tid, a0, w0, sb0);
  __syncthreads();
  // Pairs of K steps. With an odd number of steps the second half of the
  // last pair is a phantom step past K whose scale and bias words are zero, so
  // its dequantized W rows are zero and it adds nothing; an exit inside the
  // pair, or a separate tail step, would keep the accumulators out of the
  // matrix registers (the eight-wave tile then spills).
  for (uint32_t step = 0; step < nk; step += 2) {
    GEMM_GLOAD(a0, w0, sb0, step + 2);
    gemm_step<BN, NT, BM>(As[0], Ws[0], As[1], Ws[1], tid, wm, wn, lane, a1, w1, sb1, acc);
    __syncthreads();
    GEMM_GLOAD(a1, w1, sb1, step + 3);
    gemm_step<BN, NT, BM>(As[1], Ws[1], As[0], Ws[0], tid, wm, wn, lane, a0, w0, sb0, acc);
    __syncthreads();
  }
#undef GEMM_GLOAD
  if constexpr (SWIGLU) {
    const uint32_t col = n0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < G::AB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m && col < p.n) {
          const float a = lisa_bf16r(lisa_silu_exp2(lisa_bf16r(acc[i][0][r])) * lisa_bf16r(acc[i][1][r]));
          p.act[(size_t)row * p.ldc + col] = lisa_f32_to_bf16(a);
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < G::AB; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) {
        const uint32_t col = n0 + wn * (BN / G::WN) + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row < p.m && col < p.n) p.c[(size_t)row * p.ldc + col] = acc[i][j][r];
        }
      }
  }
}

// lisa_q4_gemm: one 4-wave workgroup per CU (the LDS stages take 108 KB), so the
// whole register file is available to its waves. lisa_q4_gemm_wide: eight
// waves, two per SIMD (252 registers each), so one wave's MFMAs run while the
// other waits on a barrier, an LDS read or its dequant.
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void lisa_q4_gemm(
    LisaGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][GEMM_BM * GEMM_PAD];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][LISA_GEMM_TILE_N * GEMM_PAD];
  q4_gemm_body<LISA_GEMM_TILE_N, 256>(p, As, Ws);
}
// Small projections (few tiles against the CUs): the 128 x 128 tile on four
// waves, each a 64 x 64 block of 2 x 2 MFMA blocks; two workgroups fit per CU.
// Every output takes the same MFMA sequence as in the 256 x 128 tile.
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void lisa_q4_gemm_m128(
    LisaGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][LISA_GEMM_TILE_M_SMALL * GEMM_PAD];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][LISA_GEMM_TILE_N * GEMM_PAD];
  q4_gemm_body<LISA_GEMM_TILE_N, 256, false, LISA_GEMM_TILE_M_SMALL>(p, As, Ws);
}
extern "C" __global__ __launch_bounds__(LISA_GEMM_THREADS_WIDE) __attribute__((amdgpu_waves_per_eu(2, 2))) void lisa_q4_gemm_wide(
    LisaGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][GEMM_BM * GEMM_PAD];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][LISA_GEMM_TILE_N_WIDE * GEMM_PAD];
  q4_gemm_body<LISA_GEMM_TILE_N_WIDE, LISA_GEMM_THREADS_WIDE>(p, As, Ws);
}
// The MLP's gate/up pair with the SwiGLU epilogue: 256 rows x 128 outputs per
// workgroup (the eight-wave tile over 128 gate and 128 up rows).
extern "C" __global__ __launch_bounds__(LISA_GEMM_THREADS_WIDE) __attribute__((amdgpu_waves_per_eu(2, 2))) void lisa_q4_gemm_swiglu(
    LisaGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][GEMM_BM * GEMM_PAD];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][LISA_GEMM_TILE_N_WIDE * GEMM_PAD];
  q4_gemm_body<LISA_GEMM_TILE_N_WIDE, LISA_GEMM_THREADS_WIDE, true>(p, As, Ws);
}

// Per-row kernels. NORM/RESNORM follow the q4 prologue's arithmetic exactly
// (chunks of 8 per thread, same statistic), so a prefill row normalizes as a
// decode step does.
extern "C" __global__ __launch_bounds__(256) void lisa_rows(LisaRowsParams p) {
  __shared__ float red[64];
  const int tid = threadIdx.x, t = blockIdx.y;
  switch (p.mode) {
    case LISA_ROWS_EMBED: {
      const uint32_t tok = p.tokens[t];
      for (int c = tid; c < kSegChunks; c += 256) {
        const uint32_t word = p.emb_w[(size_t)tok * (LISA_HIDDEN / 8) + c];
        const uint32_t sb = p.emb_sb[(size_t)tok * (LISA_HIDDEN / 64) + (c >> 3)];
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = lisa_bf16r((float)((word >> (4 * e)) & 0xfu) * lo_bf(sb) + hi_bf(sb));
        reinterpret_cast<uint4*>(p.r_out + (size_t)t * LISA_HIDDEN)[c] = pack_bf8(v);
      }
      break;
    }
    case LISA_ROWS_NORM:
    case LISA_ROWS_RESNORM: {
      // RESNORM without h_in: r = bf16(o) (the MTP fc output cast, norm.metal:132-137)
      const bool has_h = p.h_in != nullptr;
      const uint4* hs = reinterpret_cast<const uint4*>((has_h ? p.h_in : p.norm_w) + (has_h ? (size_t)t * LISA_HIDDEN : 0));
      const uint4* os = reinterpret_cast<const uint4*>(p.o_in + (size_t)t * LISA_HIDDEN);
      const uint4* ws = reinterpret_cast<const uint4*>(p.norm_w);
      float v[3][8];
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int c = min(tid + 256 * i, kSegChunks - 1);
        const bool valid = tid + 256 * i < kSegChunks;
        float hv[8];
        unpack_bf8(hs[c], hv);
        if (!has_h)
#pragma unroll
          for (int e = 0; e < 8; ++e) hv[e] = 0.0f;
        if (p.mode == LISA_ROWS_RESNORM) {
          const uint4 o0 = os[2 * c], o1 = os[2 * c + 1];
          const float ov[8] = {__uint_as_float(o0.x), __uint_as_float(o0.y), __uint_as_float(o0.z),
                               __uint_as_float(o0.w), __uint_as_float(o1.x), __uint_as_float(o1.y),
                               __uint_as_float(o1.z), __uint_as_float(o1.w)};
#pragma unroll
          for (int e = 0; e < 8; ++e) v[i][e] = lisa_bf16r(hv[e] + lisa_bf16r(ov[e]));
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[i][e] = hv[e];
        }
        if (valid)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = ss + v[i][e] * v[i][e];
      }
      const float inv = seg_rms_inv(ss, red, tid);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int c = tid + 256 * i;
        if (c >= kSegChunks) continue;
        float wv[8], x[8];
        unpack_bf8(ws[c], wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = lisa_bf16r((v[i][e] * inv) * wv[e]);
        reinterpret_cast<uint4*>(p.x_out + (size_t)t * (p.x_stride ? p.x_stride : LISA_HIDDEN))[c] = pack_bf8(x);
        if (p.mode == LISA_ROWS_RESNORM)
          reinterpret_cast<uint4*>(p.r_out + (size_t)t * LISA_HIDDEN)[c] = pack_bf8(v[i]);
      }
      break;
    }
    case LISA_ROWS_SILU: {
      // mlp.metal:11-16; blockIdx.x walks the row in 2048-wide pieces
      const uint32_t j = blockIdx.x * 2048u + (uint32_t)tid * 8u;
      if (j >= p.width) break;
      const float* g = p.g_in + (size_t)t * p.width + j;
      const float* u = p.u_in + (size_t)t * p.width + j;
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = lisa_bf16r(lisa_silu_exp2(lisa_bf16r(g[e])) * lisa_bf16r(u[e]));
      *reinterpret_cast<uint4*>(p.act_out + (size_t)t * p.width + j) = pack_bf8(a);
      break;
    }
    default: { /* ARGMAX: embed.metal:78-118, ties to the lowest index */
      const float* lg = p.logits + (size_t)t * p.width;
      float bv = -INFINITY;
      uint32_t bi = 0xffffffffu;
      for (uint32_t j = tid; j < p.width; j += 256)
        if (better(lg[j], j, bv, bi)) { bv = lg[j]; bi = j; }
      for (int msk = 1; msk < 64; msk <<= 1) {
        const float ov = __shfl_xor(bv, msk, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, msk, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      uint32_t* ri = reinterpret_cast<uint32_t*>(red + 32);
      if ((tid & 63) == 0) { red[tid >> 6] = bv; ri[tid >> 6] = bi; }
      __syncthreads();
      if (tid == 0) {
        for (int q = 1; q < 4; ++q)
          if (better(red[q], ri[q], red[0], ri[0])) { red[0] = red[q]; ri[0] = ri[q]; }
        p.argmax_out[t] = ri[0] == 0xffffffffu ? 0u : ri[0];
      }
      break;
    }
  }
}

// GDN causal conv + SiLU over m rows (gdn.metal:125-170 prefill form, 212-240
// history update): thread = channel, rows in order, the arithmetic of the
// decode conv epilogue.
// Causal conv over rows, parallel in time: grid (40, ceil(m / 64)) x 256; thread
// (channel c, row block b) forms rows 64b .. 64b+63 from x[64b-3 .. 64b+63]
// (rows before 0 come from the carried conv state). Block 0 is the only reader
// of the old state and, after reading it, the only writer of the new one.
extern "C" __global__ __launch_bounds__(256) void lisa_gdn_conv_rows(LisaConvRowsParams p) {
  const int C = LISA_GDN_CONV_DIM;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int m = (int)p.m_rows, t0 = blockIdx.y * 64;
  if (t0 >= m) return;
  float w[4];
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) w[tap] = bf2f(p.conv_w[(size_t)c * 4 + tap]);
  // history h(t) for t in [t0-3, t0+63]: x rows, or the old state before row 0
  float x[67];
#pragma unroll
  for (int j = 0; j < 67; ++j) {
    const int t = t0 - 3 + j;
    const int tc = min(max(t, 0), m - 1);
    const float raw = p.qkv[(size_t)tc * C + c];
    x[j] = lisa_bf16r(raw);
  }
  if (t0 == 0) {
    float s[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) s[i] = bf2f(p.conv_state[(size_t)i * C + c]);
#pragma unroll
    for (int i = 0; i < 3; ++i) x[i] = s[i];
    // new state: h(m-3), h(m-2), h(m-1) of the sequence [old state, x rows]
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int t = m - 3 + i;
      const float hv = t >= 0 ? lisa_bf16r(p.qkv[(size_t)t * C + c]) : s[3 + t];
      p.conv_state[(size_t)i * C + c] = lisa_f32_to_bf16(hv);
    }
  }
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    if (t0 + j >= m) break;
    float acc = 0.0f;
    acc = acc + x[j] * w[0];
    acc = acc + x[j + 1] * w[1];
    acc = acc + x[j + 2] * w[2];
    acc = acc + x[j + 3] * w[3];
    p.conv_out[(size_t)(t0 + j) * C + c] = lisa_bf16r(lisa_silu_exp(lisa_bf16r(acc)));
  }
}

// Prefill attention (attention.metal:364-480 semantics) in the decode path's
// split-K form, so every row equals what a decode step at its position gives.
// 1. K/V rows appended and queries normalized + rotated: grid (m, 7); y = 0
//    handles the 4 KV heads, y = 1..6 four query heads each, one wave per head.
extern "C" __global__ __launch_bounds__(256) void lisa_attn_store_rows(LisaAttnParams p) {
  const int t = blockIdx.x, grp = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t pos = *p.pos + t;
  constexpr int HD = LISA_ATT_HD;
  float o[4];
  if (grp == 0) {
    const int kvh = wave;
    head_norm_rope_wave(p.k_raw + (size_t)t * LISA_ATT_KV_OUT + kvh * HD, p.k_norm_w, pos, lane, o);
    const size_t off = ((size_t)kvh * p.capacity + pos) * HD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = lane + 64 * j;
      p.key_cache[off + d] = lisa_f32_to_bf16(o[j]);
      p.value_cache[off + d] = lisa_f32_to_bf16(p.v_raw[(size_t)t * LISA_ATT_KV_OUT + kvh * HD + d]);
    }
  } else {
    const int h = (grp - 1) * 4 + wave;
    head_norm_rope_wave(p.q_proj + (size_t)t * LISA_ATT_Q_OUT + h * 512, p.q_norm_w, pos, lane, o);
#pragma unroll
    for (int j = 0; j < 4; ++j) p.query[((size_t)t * LISA_ATT_QH + h) * HD + lane + 64 * j] = lisa_bf16r(o[j]);
  }
}

// 2. slice partials: grid (s_max, 4, ceil(m / ATT_RB)); a workgroup of sixteen
//    waves takes one 64-token slice of one KV head for ATT_RB rows (its LDS
//    allows one workgroup per CU, so the waves that interleave the score and
//    P.V loops are all in it).
//
// The score items take their query values (the same for every lane, lane =
// token) as scalar operands of the fmas rather than as broadcast LDS reads,
// which bounded the loop: the query rows are read through the constant
// address space, whose wave-uniform loads the compiler issues as scalar loads
// (and waits for itself). The rows are written by the previous launch and not
// written here.
typedef __attribute__((address_space(4))) const float* lisa_cfloat_ptr;

// The slice scores of all six query heads of a KV head for one row, query
// values read by scalar loads from q (the six heads' rows, contiguous): each
// head's four accumulators, chains and softmax statistics are slice_scores2's;
// one conversion of a K element serves the six heads. pb: [6][T]; the
// statistics of head i at ml + i * mls.
DEV void slice_scores6_sq(lisa_cfloat_ptr q, const uint16_t* Kt, int kp, int n, int lane, float* pb, float* ml,
                          size_t mls) {
  constexpr int HD = LISA_ATT_HD;
  const uint16_t* kr = Kt + lane * kp;
  float a[6][4];
#pragma unroll
  for (int i = 0; i < 6; ++i) a[i][0] = a[i][1] = a[i][2] = a[i][3] = 0.0f;
#pragma unroll 2
  for (int d = 0; d < HD; d += 8) {
    const uint4 kk = *reinterpret_cast<const uint4*>(kr + d);
    const float k[8] = {lo_bf(kk.x), hi_bf(kk.x), lo_bf(kk.y), hi_bf(kk.y),
                        lo_bf(kk.z), hi_bf(kk.z), lo_bf(kk.w), hi_bf(kk.w)};
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 6; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) a[i][e] = lisa_fma(q[i * HD + d + 4 * half + e], k[4 * half + e], a[i][e]);
  }
  float sc[6], mx[6], pv[6], den[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) sc[i] = lane < n ? ((a[i][0] + a[i][1]) + (a[i][2] + a[i][3])) * 0.0625f : -INFINITY;
#pragma unroll
  for (int i = 0; i < 6; ++i) mx[i] = max64(sc[i]);
#pragma unroll
  for (int i = 0; i < 6; ++i) pv[i] = lane < n ? lisa_exp2f(1.4426950408889634f * (sc[i] - mx[i])) : 0.0f;
#pragma unroll
  for (int i = 0; i < 6; ++i) den[i] = tree64(pv[i]);
#pragma unroll
  for (int i = 0; i < 6; ++i) pb[i * LISA_ATT_SLICE + lane] = pv[i];
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      ml[i * mls] = mx[i];
      ml[i * mls + 1] = den[i];
    }
  }
}

// slice_pv3 over the six heads of a KV head: thread dp owns dimensions 2dp,
// 2dp + 1 of each head, every chain over the tokens in order as there.
DEV void slice_pv6(const float* pb6, const uint16_t* Vt, int n, int dp, float (&acc)[6][2]) {
#pragma unroll
  for (int i = 0; i < 6; ++i) acc[i][0] = acc[i][1] = 0.0f;
#pragma unroll 4
  for (int tok = 0; tok < n; ++tok) {
    const uint32_t vw = *reinterpret_cast<const uint32_t*>(Vt + tok * LISA_ATT_HD + 2 * dp);
    const float v0 = lo_bf(vw), v1 = hi_bf(vw);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const float pv = pb6[i * LISA_ATT_SLICE + tok];
      acc[i][0] = lisa_fma(pv, v0, acc[i][0]);
      acc[i][1] = lisa_fma(pv, v1, acc[i][1]);
    }
  }
}

constexpr int ATT_RB = LISA_ATT_ROWS_PER_WG;
extern "C" __global__ __launch_bounds__(LISA_ATT_ROWS_THREADS) void lisa_attn_partial_rows(LisaAttnParams p) {
  constexpr int T = LISA_ATT_SLICE, HD = LISA_ATT_HD, KP = HD + 8, NT = LISA_ATT_ROWS_THREADS, NW = NT / 64;
  const uint32_t base = *p.pos;
  const int s = blockIdx.x, kvh = blockIdx.y, r0 = blockIdx.z * ATT_RB;
  const int nr = min(ATT_RB, (int)p.m_rows - r0);
  const uint32_t t0 = (uint32_t)s * T;
  if (nr <= 0 || t0 >= base + (uint32_t)(r0 + nr)) return;
  __shared__ __attribute__((aligned(16))) uint16_t Kt[T * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[T * HD];
  __shared__ float pb[ATT_RB * 6 * T];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t cache_base = (size_t)kvh * p.capacity * HD;
  const int nrows = (int)min((uint32_t)T, base + (uint32_t)(r0 + nr) - t0);
  for (int c = tid; c < nrows * (HD / 8); c += NT) {
    const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
    const size_t off = cache_base + (size_t)(t0 + row) * HD + col;
    *reinterpret_cast<uint4*>(&Kt[row * KP + col]) = *reinterpret_cast<const uint4*>(p.key_cache + off);
    *reinterpret_cast<uint4*>(&Vt[row * HD + col]) = *reinterpret_cast<const uint4*>(p.value_cache + off);
  }
  __syncthreads();
  // scores: item (row tt, all six heads of the KV head) per wave
  for (int tt = wave; tt < nr; tt += NW) {
    const int t = r0 + tt, h = kvh * 6;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    const lisa_cfloat_ptr q = (lisa_cfloat_ptr)(p.query + ((size_t)t * LISA_ATT_QH + h) * HD);
    float* ml = p.part_ml + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * 2;
    slice_scores6_sq(q, Kt, KP, n, lane, pb + tt * 6 * T, ml, (size_t)p.s_max * 2);
  }
  __syncthreads();
  // P.V: thread (dp, rr) owns dimensions 2dp, 2dp+1 of the six heads of rows
  // rr, rr + NT / 128, ..
  const int dp = tid & 127;
  for (int tt = tid >> 7; tt < nr; tt += NT / 128) {
    const int t = r0 + tt;
    const uint32_t ctx = base + t + 1;
    if (ctx <= t0) continue;
    const int n = (int)min((uint32_t)T, ctx - t0);
    float acc[6][2];
    slice_pv6(pb + tt * 6 * T, Vt, n, dp, acc);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int h = kvh * 6 + i;
      *reinterpret_cast<float2*>(p.part_o + (((size_t)t * LISA_ATT_QH + h) * p.s_max + s) * HD + 2 * dp) =
          make_float2(acc[i][0], acc[i][1]);
    }
  }
}

// 3. merge + output gate per (head, row): the decode merge, grid (24, m).
extern "C" __global__ __launch_bounds__(256) void lisa_attn_merge_rows(LisaAttnParams p) { attn_merge_body<0>(p); }

// ===========================================================================
// argmax finish (runner.rs:1077-1095 on the device) + step bookkeeping
// ===========================================================================
// 1024 threads; every thread keeps eight independent partial loads in flight
// per pass. (max, lowest index) is a total order on non-NaN values, so the
// result does not depend on the reduction order.
extern "C" __global__ __launch_bounds__(1024) void lisa_step_finalize(LisaFinalizeParams p) {
  __shared__ float cv[16];
  __shared__ uint32_t ci[16];
  __shared__ uint32_t res[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t n = p.n_part;
  for (uint32_t m = 0; m < p.m_rows; ++m) {
    const float* av = p.am_val + (size_t)m * n;
    const uint32_t* ai = p.am_idx + (size_t)m * n;
    float v = -INFINITY;
    uint32_t i = 0xffffffffu;
    for (uint32_t j0 = 0; j0 < n; j0 += 8 * 1024) {
      float ov[8];
      uint32_t oi[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t j = min(j0 + (uint32_t)(u * 1024 + tid), n - 1);
        ov[u] = av[j];
        oi[u] = ai[j];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (j0 + (uint32_t)(u * 1024 + tid) < n && better(ov[u], oi[u], v, i)) { v = ov[u]; i = oi[u]; }
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
      for (int q = 1; q < 16; ++q)
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
// device copy
// ===========================================================================
extern "C" __global__ __launch_bounds__(256) void lisa_copy_bytes(LisaCopyParams p) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint4* src = static_cast<const uint4*>(p.src);
  uint4* dst = static_cast<uint4*>(p.dst);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.n16; i += stride) dst[i] = src[i];
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
        const float u = lisa_synth_value(p.key2, i, LISA_DIST_UNIFORM, -LISA_MODEL_BIAS_SPREAD, LISA_MODEL_BIAS_SPREAD);
        const uint16_t b = lisa_f32_to_bf16(lisa_bf16_to_f32(s) * (u - LISA_MODEL_BIAS_CENTER));
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
