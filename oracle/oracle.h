/*
 * oracle.h — CPU oracle of the lisa-rs decode path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it.
 * It restates the reference's Metal shader arithmetic
 * (the .metal files under src/kernels/shaders/) and runner dispatch order
 * (src/model/runner.rs) on the CPU, with every rounding point and every
 * reduction order written out, so that the HIP path can be compared with it
 * bit for bit. Each function cites the reference lines it follows.
 *
 * Conventions: bf16 values are passed as uint16_t bit patterns; q4 linears use
 * the MLX layout of the reference (W u32[N][K/8] low nibble first,
 * scales/biases bf16[N][K/64]).
 */
#ifndef LISA_ORACLE_H
#define LISA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernel-level restatements ---------------------------------------- */

/* K1/K3 q4 linear (qmv.metal:9-76, 159-234): out[m][n] f32 for M input rows;
 * ksplit (1 or 4) selects the summation order of the HIP launch shape. */
void orc_q4_linear(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, int n_rows, int k, int m_rows, int ksplit, float* out);

/* Accumulation order of orc_q4_gemm: 0 (default) the MFMA's, f32 once per 8
 * consecutive k; 1 the double-precision sum rounded once. Both are valid
 * orders of the reference's sum; tests use 1 to measure how far a change of
 * summation order alone moves a deep model. */
void orc_set_gemm_order(int order);

/* K5 RMSNorm of one 5120-wide (or any multiple of 256) bf16 row
 * (norm.metal:10-47): out = bf16(x*inv*w). */
void orc_rms_norm(const uint16_t* x, const uint16_t* w, int cols, uint16_t* out);

/* K6 residual (norm.metal:50-57): y = bf16(x + bf16(o)). */
void orc_residual(const uint16_t* x, const float* o, int n, uint16_t* y);

/* K4 embedding lookup (embed.metal:6-28). */
void orc_embed(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t token,
               int hidden, uint16_t* out);

/* K7 SwiGLU (mlp.metal:6-17): act = bf16(silu(bf16 g) * bf16 u). */
void orc_silu_mul(const float* g, const float* u, int n, uint16_t* act);

/* K8/K9 conv for one GDN layer over m_rows tokens (gdn.metal:125-207,
 * 212-240). qkv f32[m][10240] raw projections; conv_w bf16[10240][4];
 * conv_state bf16[3][10240] updated in place; conv_out f32[m][10240];
 * slots (nullable) bf16[m][3][10240] written after each token. */
void orc_gdn_conv(const float* qkv, const uint16_t* conv_w, uint16_t* conv_state, int m_rows,
                  float* conv_out, uint16_t* slots);

/* K10/K11 gated-delta recurrence + gated RMSNorm for one GDN layer
 * (gdn.metal:125-207 gates, 245-328, 367-391). state f32[48][128][128]
 * updated in place; gated bf16[m][6144]; slots (nullable) f32[m][48*128*128];
 * y_out (nullable) f32[m][6144] pre-norm readout. */
void orc_gdn_recurrence(const float* conv_out, const float* z, const float* a, const float* b,
                        const uint16_t* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float* state, int m_rows, uint16_t* gated, float* slots, float* y_out);

/* K12/K13 q/k norm + partial RoPE of one 256-wide head
 * (attention.metal:118-155, 158-197): out bf16[256]. */
void orc_head_norm_rope(const float* raw, const uint16_t* w, uint32_t position, uint16_t* out);

/* K14/K15/K16 split-K decode attention for m_rows query rows at positions
 * base+t over a [4][capacity][256] bf16 cache (attention.metal:550-641,
 * 520-531). q_proj f32[m][12288] raw; k_raw/v_raw f32[m][1024] (stored into
 * the caches at base+t first, kv_cache_store_decode); gated bf16[m][6144]. */
void orc_attention(const float* q_proj, const float* k_raw, const float* v_raw,
                   const uint16_t* q_norm_w, const uint16_t* k_norm_w, uint16_t* key_cache,
                   uint16_t* value_cache, uint32_t capacity, uint32_t base, int m_rows,
                   uint16_t* gated);

/* K14/K15 core: split-K SDPA of roped bf16 queries [m][24][256] against the
 * caches, rows at positions base+t; out f32[m][24][256] (before the gate). */
void orc_sdpa(const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache, uint32_t capacity,
              uint32_t base, int m_rows, float* out);

/* RMSNorm whose statistic is summed from per-8-row tile partials (the decode
 * path's norms after a residual-add launch). */
void orc_rms_norm_tiles(const uint16_t* x, const uint16_t* w, int cols, uint16_t* out);

/* K20 prefill q4 GEMM: bf16(fma(s, q, b)) dequant, double accumulation, f32 out [m][n]. */
void orc_q4_gemm(const uint16_t* a, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int n_rows,
                 int k, int m_rows, float* out);

/* Shared numerics element-wise (see oracle.cpp orc_math for fn codes). */
void orc_math(int fn, const float* x, size_t n, float* out);

/* K17 argmax, ties to the lowest index (embed.metal:33-71, runner.rs:1077-1095). */
uint32_t orc_argmax(const float* v, int n);

/* ---- model-level restatement (runner.rs) ------------------------------ */

typedef struct OrcModel OrcModel;

/* Create a synthetic model: `layers` (multiple of 4, schedule (i+1)%4==0 is
 * attention), vocabulary `vocab`, KV capacity, seed; with_mtp adds the
 * 1-layer drafter. Weights are generated with lisa_synth.h so that the HIP
 * runner generating the same seed sees identical values. */
OrcModel* orc_model_create(int layers, int vocab, int capacity, uint64_t seed, int with_mtp);
void orc_model_free(OrcModel* m);
uint32_t orc_model_position(const OrcModel* m);
/* OpenMP threads the oracle runs on. */
int orc_threads(void);

/* Layer schedule of the hybrid stack (src/model/mod.rs:16-22). */
int orc_layer_is_attention(int layer);
/* Fill recurrent state, conv history and the first `filled` KV positions with
 * synthetic values and set position = filled (the bench's 4k-context start). */
void orc_model_fill_state(OrcModel* m, uint32_t filled, uint64_t seed);
void orc_model_reset(OrcModel* m);

/* One target forward of m_rows (1 or 3) tokens at positions position..+m-1
 * (runner.rs:505-591, 734-909). capture=1 records per-row GDN/conv slots for
 * commit. Outputs (nullable): argmax[m], hidden f32[m][5120] (last decoder
 * state before the final norm), logits f32[m][vocab]. position += m. */
int orc_model_forward(OrcModel* m, const uint32_t* tokens, int m_rows, int capture,
                      uint32_t* argmax, float* hidden, float* logits);
/* commit_verified_prefix (runner.rs:911-944). Returns 0 or -1 on error. */
/* H11 forward_prefill_with_progress over `n` tokens in chunks (<= 512). */
int orc_model_prefill(OrcModel* m, const uint32_t* tokens, int n, int chunk, uint32_t* argmax_out, float* hidden_out);
int orc_model_commit(OrcModel* m, int rows);

/* MTP drafter step (runner.rs:2711-2765): cond is the bf16 conditioning
 * hidden [5120]; outputs argmax and the drafter's normalized hidden (bf16). */
int orc_mtp_forward(OrcModel* m, uint32_t token, const uint16_t* cond, uint32_t* argmax,
                    uint16_t* normalized);
uint32_t orc_mtp_position(const OrcModel* m);
int orc_mtp_trim(OrcModel* m, int count);

/* MtpRunner::forward_position_batch (runner.rs:3486-3581): the drafter over n
 * (token, target hidden f32[5120]) positions with the prefill kernels'
 * arithmetic; argmax_out[n], normalized_out bf16[n][5120] (nullable). */
int orc_mtp_prefill(OrcModel* m, const uint32_t* tokens, const float* hiddens, int n, uint32_t* argmax_out,
                    uint16_t* normalized_out);

/* Test hook: pointer to and size of one model tensor (scope = layer + 1, 0 for
 * globals, LISA_SCOPE_MTP; kind = LISA_T_*; part 0 words/vector, 1 scales,
 * 2 biases); 0 on success. Tests overwrite weights through it. */
int orc_model_tensor(OrcModel* m, int scope, int kind, int part, void** ptr, size_t* bytes);

/* Copy of a synthetic tensor as generated (for tests). */
void orc_synth_bf16(uint64_t seed, uint64_t tensor_id, int dist, float a, float b, size_t n,
                    uint16_t* out);
void orc_synth_f32(uint64_t seed, uint64_t tensor_id, int dist, float a, float b, size_t n,
                   float* out);
void orc_synth_words(uint64_t seed, uint64_t tensor_id, size_t n, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* LISA_ORACLE_H */
