/*
 * lisa_kernels.h — argument blocks of the gfx950 kernels in lisa_kernels.hsaco.
 *
 * Every kernel takes exactly one by-value argument block, so a dispatch is
 * `lisa_encoder_set_bytes(enc, 0, &params, sizeof params)` followed by
 * `lisa_encoder_dispatch_groups` — the same set_bytes/dispatch_thread_groups
 * pattern the reference's encoders use (src/device/metal.rs:342-376). Device
 * addresses are plain 64-bit pointers (lisa_buffer_device_ptr + byte offset).
 *
 * Kernel names (hipModuleGetFunction) are listed next to each block.
 */
#ifndef LISA_KERNELS_H
#define LISA_KERNELS_H

#include <stdint.h>

/* ---- q4 linear with fused prologue/epilogue -----------------------------
 * Kernels: lisa_qmv_k{5120,6144,10240,17408}_m{1,3}
 * Weights use the resident layout: W u32[N][K/8] (MLX, low nibble first) and
 * SB u32[N][K/64] with SB = scale_bf16 | bias_bf16 << 16 (one load per group).
 * One launch covers up to 4 matrices that share the input x; the virtual row
 * space is split into 8-row tiles, each matrix owning a contiguous tile range
 * [tile_start[e], tile_start[e+1]), tile_start[n_mats] the total.
 * ksplit is 4 for K != 5120 (the kernels lisa_qmv_k{6144,10240,17408}_*: one
 * tile per workgroup, its group iterations split over the 4 waves; these are
 * the projections back to the 5120-row residual) and 1 for K = 5120 (one tile
 * per wave): a fixed rule, so the summation order of every output is a
 * function of K. */
#define LISA_QMV_MAX_MATS 4

/* lisa_qmv_k5120_m3_prenorm_gateup_wide: the three-row MLP gate/up (one
 * GATEUP matrix pair, PRENORM prologue) on workgroups of LISA_QMV_WIDE_THREADS
 * threads, each owning LISA_QMV_WIDE_TILES consecutive 8-row tiles; grid
 * ceil(tiles / LISA_QMV_WIDE_TILES). Outputs are the bits of the four-wave
 * lisa_qmv_k5120_m3_prenorm_gateup. */
#define LISA_QMV_WIDE_THREADS 1024
#define LISA_QMV_WIDE_TILES 17

/* lisa_qmv_k5120_m{1,3}_prenorm_wide{7,8}: a PRENORM launch of STORE and CONV
 * matrices (optionally with the GDN gate contributions) on workgroups of
 * 64 NW threads, NW = 7 or 8, one 8-row tile per wave; grid ceil(tiles / NW).
 * The runner takes them when tiles = LISA_QMV_WIDE_GROUPS x NW (the GDN and
 * attention in-projections: one workgroup per CU). Outputs are the bits of
 * the four-wave lisa_qmv_k5120_m{1,3}_prenorm. */
#define LISA_QMV_WIDE_GROUPS 256

/* lisa_qmv_k5120_m1_x_wide9: a one-row LOADX launch of STORE matrices of
 * (8 x 256, 9 x 256] tiles (the config-0 GEMV: 2176 tiles) on workgroups of
 * 64 x LISA_QMV_X_WIDE_WAVES threads, one tile per wave; grid ceil(tiles / 9).
 * Outputs are the bits of the four-wave lisa_qmv_k5120_m1_x. */
#define LISA_QMV_X_WIDE_WAVES 9

enum {
  LISA_PRO_LOADX = 0,   /* x = bf16 x_in[M][K] */
  LISA_PRO_RESNORM = 1, /* r = bf16(h_in + bf16(o_in)); x = RMSNorm(r, norm_w) */
  LISA_PRO_EMBED = 2,   /* r = q4 embedding row of tokens[m]; x = RMSNorm(r) */
  LISA_PRO_CAST = 3,    /* r = bf16(o_in); x = RMSNorm(r) */
  LISA_PRO_NORM = 4,    /* r = h_in; x = RMSNorm(r) */
  LISA_PRO_MTPFC = 5,   /* x = [RMSNorm(embed(tok), norm_w) | RMSNorm(x_in, norm_w2)] */
  LISA_PRO_PRENORM = 6  /* x = RMSNorm(h_in) of residual rows an EPI_RESID launch produced;
                           the statistic sums per-8-row tile partials
                           ((r0^2+r1^2)+(r2^2+r3^2))+((r4^2+r5^2)+(r6^2+r7^2)) */
};

enum {
  LISA_EPI_STORE = 0,  /* out f32[M][rows] */
  LISA_EPI_GATEUP = 1, /* rows j of (w, w2) -> out bf16[M][rows] = bf16(silu(g)*u) */
  LISA_EPI_CONV = 2,   /* GDN qkv: causal conv + SiLU -> out f32[M][rows], conv state update */
  LISA_EPI_ARGMAX = 3, /* out f32 logits[M][rows] + per-workgroup (max, idx) partials */
  LISA_EPI_RESID = 4   /* rows of the 5120-wide residual: h_in[m][j] <- bf16(h_in[m][j] +
                          bf16(y)) in place (normalized by a PRENORM consumer) */
};

typedef struct LisaQ4Mat {
  const uint32_t* w;
  const uint32_t* sb;
  const uint32_t* w2; /* GATEUP: up projection */
  const uint32_t* sb2;
  void* out;
  uint32_t rows;
  uint32_t kind;
} LisaQ4Mat;

/* floats per (row, value head) of the in-projection's gate contributions */
#define LISA_GDN_GATE_FLOATS 192

typedef struct LisaQmvParams {
  /* prologue */
  const uint16_t* x_in;
  const uint16_t* h_in; /* residual rows bf16 [M][5120]; EPI_RESID updates them in place */
  const float* o_in;
  const uint32_t* tokens;
  const uint32_t* emb_w;
  const uint32_t* emb_sb;
  const uint16_t* norm_w;
  const uint16_t* norm_w2;
  uint16_t* r_out; /* written by workgroup 0: r rows bf16[M][5120] */
  uint16_t* x_out; /* written by workgroup 0: normalized x bf16[M][K] */
  /* CONV epilogue */
  const uint16_t* conv_w;  /* bf16[10240][4] */
  uint16_t* conv_state;    /* bf16[3][10240] of this layer */
  uint16_t* conv_slots;    /* slot 0 of this layer, bf16[3][10240]; nullable */
  uint64_t conv_slot_stride; /* elements between slot t and t+1 */
  /* ARGMAX epilogue */
  float* am_val; /* [M][gridDim.x] */
  uint32_t* am_idx;
  /* matrices */
  LisaQ4Mat mats[LISA_QMV_MAX_MATS];
  uint32_t tile_start[LISA_QMV_MAX_MATS + 1];
  uint32_t n_mats;
  uint32_t pro_mode;
  uint32_t capture;
  uint32_t ksplit; /* 1 or 4: waves of a workgroup split K of one tile */
  /* GDN in-projection (K = 5120, normalizing prologue): when gate_ab is set,
   * workgroup w < 48 also forms the 80 per-group contributions of rows w of the
   * q4 a and b matrices [48][5120] against its staged x, stored f32
   * gate_ab[m][w][LISA_GDN_GATE_FLOATS]: for lane li < 16 of a q4 tile, 12
   * floats at 12 li holding a's groups li, 16 + li, .., 64 + li, then b's, then
   * two unused; the recurrence adds them in a q4 launch's order. */
  const uint32_t* gate_a_w;
  const uint32_t* gate_a_sb;
  const uint32_t* gate_b_w;
  const uint32_t* gate_b_sb;
  float* gate_ab;
} LisaQmvParams;

/* ---- GDN recurrence + gated RMSNorm --------------------------------------
 * Kernels: lisa_gdn_recurrence_m{1,3}; grid 48 workgroups x 512 threads, or
 * 48 + 8 n with the L2 prefetch workgroups (pf_* below).
 * Prefill over m rows: lisa_gdn_prep_rows grid (m, 9) x 256, then
 * lisa_gdn_scan_rows grid (48, 8) x 256 (y_out required), then lisa_gdn_out_rows
 * grid (m, 48) x 128; together they equal the decode kernel applied row by row. */
typedef struct LisaGdnParams {
  const float* conv_out; /* [M][10240] */
  const float* z;        /* [M][6144] raw */
  const float* a;        /* [M][48] raw */
  const float* b;        /* [M][48] raw */
  const uint16_t* a_log;
  const uint16_t* dt_bias;
  const uint16_t* norm_w;
  float* state;    /* this layer [48][128][128] */
  float* slots;    /* slot 0 of this layer; nullable */
  uint64_t slot_stride; /* floats between slot t and t+1 */
  uint16_t* gated; /* [M][6144] bf16 */
  float* y_out;    /* nullable: pre-norm readout [M][6144] */
  float q_scale, k_scale;
  uint32_t capture;
  uint32_t m_rows; /* prefill kernels: number of rows (time steps) */
  float* qk;       /* prefill: normalized q, k per row [m][2][2048] */
  float* gates;    /* prefill: (beta, decay) per row and value head [m][48][2] */
  /* Decode: when set, a and b of head h come from the in-projection's group
   * contributions gate_ab[m][h][LISA_GDN_GATE_FLOATS] (see LisaQmvParams.gate_ab)
   * and the a, b fields are unused. */
  const float* gate_ab;
  /* Decode: workgroups past the 48 heads (a grid of 48 + 8 n, n >= 1) only
   * load the 8-row q4 tiles of the next launch's matrix (W u32[rows][pf_k/8],
   * SB u32[rows][pf_k/64]; pf_tiles tiles, at most 32 n; pf_k a multiple of 64,
   * at most 7168), tile t by a workgroup on XCD t mod 8, the XCD whose L2 serves
   * that launch's workgroup t. pf_sink (4 bytes) receives a checksum of the
   * loaded words only if it equals a fixed value. The prefetch workgroups
   * first sleep pf_delay x 512 cycles (at most 64), so that the heads' state
   * loads go out first. */
  const uint32_t* pf_w;
  const uint32_t* pf_sb;
  uint32_t* pf_sink;
  uint32_t pf_tiles;
  uint32_t pf_k;
  uint32_t pf_delay;
  uint32_t pad0;
} LisaGdnParams;

/* ---- split-K decode attention --------------------------------------------
 * Kernels: lisa_attn_partial_m{1,3} grid (s_max, 4) x LISA_ATT_PARTIAL_THREADS(M),
 *          lisa_attn_merge_m{1,3}   grid (24, M) x 256. */
/* threads of lisa_attn_partial_m<M>: sixteen waves for one row and for three */
#define LISA_ATT_PARTIAL_THREADS(M) ((M) == 3 ? 1024 : 1024)
typedef struct LisaAttnParams {
  const float* q_proj; /* [M][12288] raw */
  const float* k_raw;  /* [M][1024] */
  const float* v_raw;  /* [M][1024] */
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  uint16_t* key_cache;   /* this layer [4][capacity][256] */
  uint16_t* value_cache;
  float* part_o;  /* [M][24][s_max][256] */
  float* part_ml; /* [M][24][s_max][2] = (max, denominator) */
  const uint32_t* pos; /* device position of row 0 */
  uint16_t* gated;     /* [M][6144] bf16 */
  uint32_t capacity;
  uint32_t s_max;
  /* *_rows (prefill) kernels: normalized rotated queries [m][24][256], the
   * bf16-rounded values as f32, written by lisa_attn_store_rows, and the row
   * count */
  float* query;
  uint32_t m_rows;
  uint32_t pad0;
} LisaAttnParams;

/* ---- argmax finish + device-side step bookkeeping ------------------------
 * Kernel: lisa_step_finalize, grid 1 x 256. */
typedef struct LisaFinalizeParams {
  const float* am_val;
  const uint32_t* am_idx;
  uint32_t* argmax_out;  /* [M] */
  uint32_t* next_token;  /* nullable: receives argmax[M-1] */
  uint32_t* history;     /* nullable: history[*step] = argmax[0] */
  uint32_t* step;        /* nullable */
  uint32_t* pos;         /* nullable: *pos += pos_advance */
  uint32_t n_part;
  uint32_t m_rows;
  uint32_t pos_advance;
  uint32_t history_cap;
} LisaFinalizeParams;

/* ---- synthetic fills -------------------------------------------------------
 * Kernel: lisa_synth_fill, grid-stride. */
enum {
  LISA_FILL_WORDS = 0, /* u32 words */
  LISA_FILL_BF16 = 1,  /* bf16 of lisa_synth_value(key, i, dist, a, b) */
  LISA_FILL_F32 = 2,
  LISA_FILL_SB = 3,    /* packed q4 scale/bias pairs from key (scales) and key2 (biases) */
  LISA_FILL_KV = 4     /* bf16 [4][capacity][256] rows < filled, index (kvh<<20 + pos)*256 + d */
};

typedef struct LisaSynthParams {
  void* out;
  uint64_t n;
  uint64_t key;
  uint64_t key2;
  uint32_t kind;
  uint32_t dist;
  float a, b;
  uint32_t capacity;
  uint32_t filled;
} LisaSynthParams;

/* ---- batched prefill ------------------------------------------------------
 * lisa_q4_gemm: C[m][n] (f32, row stride ldc) = A[m][k] (bf16) . deq(W)[n][k]
 * with deq = bf16(fma(scale, q, bias)) (gemm.metal:238-266), bf16 MFMA with f32
 * accumulation. Grid (ceil(n / LISA_GEMM_TILE_N), ceil(m / LISA_GEMM_TILE_M)) x 256;
 * k multiple of 64. lisa_q4_gemm_wide: same contract, 256 x LISA_GEMM_TILE_N_WIDE
 * tiles, LISA_GEMM_THREADS_WIDE threads. */
#define LISA_GEMM_TILE_M 256
#define LISA_GEMM_TILE_M_SMALL 128 /* lisa_q4_gemm_m128: 128 x LISA_GEMM_TILE_N tiles, 256 threads */
#define LISA_GEMM_TILE_N 128
#define LISA_GEMM_TILE_N_WIDE 256
#define LISA_GEMM_THREADS_WIDE 512

typedef struct LisaGemmParams {
  const uint16_t* a;
  const uint32_t* w;
  const uint32_t* sb;
  float* c;
  uint32_t m, n, k, ldc;
  /* lisa_q4_gemm_swiglu (the MLP's gate/up pair, gemm.metal:273-341): w, sb
   * are the gate projection, w2, sb2 the up projection (both n x k), and
   * act[m][n] (row stride ldc) receives bf16(silu(bf16 g) * bf16 u); c is
   * unused. Grid (ceil(n / 128), ceil(m / 256)) x LISA_GEMM_THREADS_WIDE. */
  const uint32_t* w2;
  const uint32_t* sb2;
  uint16_t* act;
} LisaGemmParams;

/* lisa_rows: per-row kernels of the prefill, grid (x, m) x 256. */
enum {
  LISA_ROWS_EMBED = 0,   /* r_out[t] = q4 embedding row of tokens[t] (bf16) */
  LISA_ROWS_NORM = 1,    /* x_out[t] = RMSNorm(h_in[t]) */
  LISA_ROWS_RESNORM = 2, /* r = bf16(h_in + bf16(o_in)) -> r_out; x_out = RMSNorm(r) */
  LISA_ROWS_SILU = 3,    /* act[t][j] = bf16(silu(bf16 g) * bf16 u), j < width */
  LISA_ROWS_ARGMAX = 4   /* argmax_out[t] = argmax over logits[t][0..vocab) (lowest index) */
};
typedef struct LisaRowsParams {
  const uint16_t* h_in;
  const float* o_in;
  const uint16_t* norm_w;
  uint16_t* r_out;
  uint16_t* x_out;
  const uint32_t* tokens;
  const uint32_t* emb_w;
  const uint32_t* emb_sb;
  const float* g_in;
  const float* u_in;
  uint16_t* act_out;
  const float* logits;
  uint32_t* argmax_out;
  uint32_t width; /* SILU row width; ARGMAX vocabulary */
  uint32_t mode;
  /* NORM / RESNORM: elements between normalized rows t and t + 1 of x_out
   * (0 = 5120); 10240 writes one half of the MTP fc input rows
   * (rms_norm_rows_stride, norm.metal:142-181). RESNORM with h_in null takes
   * r = bf16(o) (the MTP fc output cast). */
  uint32_t x_stride;
  uint32_t pad0;
} LisaRowsParams;

/* lisa_attn_partial_rows takes LISA_ATT_ROWS_PER_WG rows per workgroup:
 * grid (s_max, 4, ceil(m / LISA_ATT_ROWS_PER_WG)) x LISA_ATT_ROWS_THREADS. */
#define LISA_ATT_ROWS_PER_WG 16
#define LISA_ATT_ROWS_THREADS 1024

/* lisa_gdn_conv_rows: causal conv + SiLU over m rows per channel with the
 * carried history, grid (ceil(10240/256), ceil(m/64)) x 256. */
typedef struct LisaConvRowsParams {
  const float* qkv;        /* f32 [m][10240] */
  const uint16_t* conv_w;  /* bf16 [10240][4] */
  uint16_t* conv_state;    /* bf16 [3][10240], updated */
  float* conv_out;         /* f32 [m][10240] */
  uint32_t m_rows;
  uint32_t pad0;
} LisaConvRowsParams;

/* ---- device copy (norm.metal:109-130 copy_bytes) ---------------------------
 * Kernel: lisa_copy_bytes, grid-stride over 16-byte units; src and dst 16-byte
 * aligned. Also the plain-copy reference of the HBM traffic counters. */
typedef struct LisaCopyParams {
  const void* src;
  void* dst;
  uint64_t n16; /* 16-byte units */
} LisaCopyParams;

#endif /* LISA_KERNELS_H */
