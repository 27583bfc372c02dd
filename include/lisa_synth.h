/*
 * lisa_synth.h — seeded synthetic checkpoint values (host and device).
 *
 * The reference loads MLX-affine 4-bit checkpoints from safetensors shards
 * (src/model/runner.rs:337-417, src/model/weights.rs:22-42). There is no
 * network and no checkpoint here, so the decode path runs on random-init
 * weights of exactly the reference's tensor shapes and dtypes
 * (runner.rs:3769-3955). Every value is a pure function of
 * (seed, tensor id, element index): a counter-based generator (the SplitMix64
 * output function applied to key + (i+1)*golden-gamma), so the GPU can fill
 * 15 GB of weights in milliseconds and the CPU can regenerate any element
 * bit-identically. Normal variates use Box-Muller with the shared numerics
 * (lisa_logf, lisa_sincosf, correctly rounded sqrt), so they also agree bit
 * for bit between host and device.
 */
#ifndef LISA_SYNTH_H
#define LISA_SYNTH_H

#include "lisa_numerics.h"

/* Distribution kinds of a synthetic tensor. */
enum {
  LISA_DIST_BITS = 0,    /* raw 32-bit words: uniform nibbles for packed q4 */
  LISA_DIST_UNIFORM = 1, /* U(lo, hi) */
  LISA_DIST_NORMAL = 2,  /* N(mean=lo, std=hi) */
};

LISA_HD uint64_t lisa_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Random 64-bit word number i of the stream `key`. */
LISA_HD uint64_t lisa_rand64(uint64_t key, uint64_t i) {
  return lisa_mix64(key + (i + 1ull) * 0x9E3779B97F4A7C15ull);
}

/* Uniform in [0,1) with 24 random bits. */
LISA_HD float lisa_rand_unit(uint64_t r) { return (float)(uint32_t)(r >> 40) * (1.0f / 16777216.0f); }

/* Key of a tensor stream: FNV-1a of its id mixed with the global seed. */
LISA_HD uint64_t lisa_stream_key(uint64_t seed, uint64_t tensor_id) {
  return lisa_mix64(seed ^ lisa_mix64(tensor_id * 0x100000001B3ull + 0xCBF29CE484222325ull));
}

/* Element i of a synthetic f32 stream. */
LISA_HD float lisa_synth_value(uint64_t key, uint64_t i, int dist, float a, float b) {
  const uint64_t r = lisa_rand64(key, i);
  if (dist == LISA_DIST_UNIFORM) {
    const float u = lisa_rand_unit(r);
    return lisa_fma(u, b - a, a);
  }
  /* Box-Muller on two 24-bit uniforms; u1 in (0,1]. */
  const float u1 = (float)((uint32_t)(r >> 40) + 1u) * (1.0f / 16777216.0f);
  const float u2 = (float)((uint32_t)(r >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
  const float rad = lisa_sqrt(-2.0f * lisa_logf(u1));
  float s, c;
  lisa_sincosf(6.28318548202514648438f * u2, &s, &c);
  return lisa_fma(rad * c, b, a);
}

/* Packed q4 word i (8 uniform nibbles). */
LISA_HD uint32_t lisa_synth_word(uint64_t key, uint64_t i) { return (uint32_t)lisa_rand64(key, i); }

#endif /* LISA_SYNTH_H */
