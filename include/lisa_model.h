/*
 * lisa_model.h — geometry, layer schedule and synthetic-tensor catalogue of
 * the 27B-shaped hybrid GDN/attention decoder.
 *
 * Geometry is hard-coded exactly as the reference hard-codes it
 * (src/model/mod.rs:6-22, src/model/runner.rs:16-51); only the number of
 * layers, the vocabulary size and the KV capacity are run-time values so that
 * tests can run reduced models with the real per-layer shapes.
 */
#ifndef LISA_MODEL_H
#define LISA_MODEL_H

#include <stdint.h>

#define LISA_HIDDEN 5120
#define LISA_INTER 17408
#define LISA_VOCAB 248320
#define LISA_LAYERS 64
#define LISA_GROUP 64 /* MLX affine q4 group size along K */

#define LISA_GDN_KH 16
#define LISA_GDN_VH 48
#define LISA_GDN_HD 128
#define LISA_GDN_KEY_DIM (LISA_GDN_KH * LISA_GDN_HD)                   /* 2048 */
#define LISA_GDN_VALUE_DIM (LISA_GDN_VH * LISA_GDN_HD)                 /* 6144 */
#define LISA_GDN_CONV_DIM (2 * LISA_GDN_KEY_DIM + LISA_GDN_VALUE_DIM)  /* 10240 */
#define LISA_GDN_STATE (LISA_GDN_VH * LISA_GDN_HD * LISA_GDN_HD)       /* floats/layer */
#define LISA_GDN_CONV_K 4

#define LISA_ATT_QH 24
#define LISA_ATT_KVH 4
#define LISA_ATT_HD 256
#define LISA_ATT_Q_OUT (LISA_ATT_QH * 2 * LISA_ATT_HD) /* 12288: [query 256 | gate 256] per head */
#define LISA_ATT_KV_OUT (LISA_ATT_KVH * LISA_ATT_HD)   /* 1024 */
#define LISA_ATT_OUT (LISA_ATT_QH * LISA_ATT_HD)       /* 6144 */
#define LISA_ATT_SLICE 64 /* KV tokens per split-K slice (attention.metal:26) */

#define LISA_EPS 1e-6f

/* Layer i is full attention iff (i+1) % 4 == 0 (src/model/mod.rs:16-22). */
static inline int lisa_layer_is_attention(int i) { return ((i + 1) % 4) == 0; }

/* ---- synthetic tensor catalogue ----------------------------------------
 * Tensor id = (scope << 12) | (kind << 2) | part, scope = layer + 1 for
 * per-layer tensors, 0 for globals, LISA_SCOPE_MTP for the drafter;
 * part 0 = packed weight / plain tensor, 1 = scales, 2 = biases. */
#define LISA_SCOPE_MTP 4000
enum {
  LISA_T_INPUT_NORM = 1,
  LISA_T_POST_NORM,
  LISA_T_MLP_GATE,
  LISA_T_MLP_UP,
  LISA_T_MLP_DOWN,
  LISA_T_GDN_QKV,
  LISA_T_GDN_Z,
  LISA_T_GDN_A,
  LISA_T_GDN_B,
  LISA_T_GDN_OUT,
  LISA_T_GDN_CONV_W,
  LISA_T_GDN_A_LOG,
  LISA_T_GDN_DT_BIAS,
  LISA_T_GDN_NORM,
  LISA_T_ATT_Q,
  LISA_T_ATT_K,
  LISA_T_ATT_V,
  LISA_T_ATT_O,
  LISA_T_ATT_Q_NORM,
  LISA_T_ATT_K_NORM,
  LISA_T_EMBED,
  LISA_T_FINAL_NORM,
  LISA_T_LM_HEAD,
  LISA_T_MTP_PRE_FC_EMB,
  LISA_T_MTP_PRE_FC_HID,
  LISA_T_MTP_FC,
  /* activations / state streams */
  LISA_T_GDN_STATE,
  LISA_T_CONV_STATE,
  LISA_T_KEY_CACHE,
  LISA_T_VALUE_CACHE,
  LISA_T_ACTIVATION,
  LISA_T_COUNT
};

static inline uint64_t lisa_tensor_id(int scope, int kind, int part) {
  return ((uint64_t)(uint32_t)scope << 12) | ((uint64_t)kind << 2) | (uint64_t)part;
}

/* Builder-chosen distributions (BASELINE configs 0-2 fix the q4 ones):
 * q4 scales ~U(0.005,0.02), nibbles uniform, biases zero-mean (below); RMSNorm
 * gains 1+U(-0.1,0.1); conv1d weights U(-0.5,0.5); A_log U(-2,0);
 * dt_bias U(-1,1); GDN state N(0,0.01); conv history, KV cache and
 * activations N(0,1). */
#define LISA_SCALE_LO 0.005f
#define LISA_SCALE_HI 0.02f
#define LISA_BIAS_LO -0.1f
#define LISA_BIAS_HI 0.1f

/* Bias of a synthetic model group: zero-mean groups like an MLX-quantized
 * checkpoint, b = bf16(s * (u - 7.5)) with s the group's bf16 scale and
 * u ~ U(-1, 1) from the bias stream, so q*s + b spans [s(u-7.5), s(u+7.5)].
 * (BASELINE config 0's biases U(-0.1, 0.1) give every weight a mean of about
 * +0.09 and a logit vector dominated by one common-mode direction; the
 * single-kernel tests keep those.) */
#define LISA_MODEL_BIAS_CENTER 7.5f
#define LISA_MODEL_BIAS_SPREAD 1.0f

#endif /* LISA_MODEL_H */
