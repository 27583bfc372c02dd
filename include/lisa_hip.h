/*
 * lisa_hip.h — C ABI of liblisa_hip.so, the MI355X replacement for the
 * reference's Metal device bridge (src/device/metal.rs) and for the runner
 * methods the speculative loop and the CLI call (src/model/runner.rs,
 * src/speculative/mod.rs).
 *
 * Conventions (shared by every entry point):
 *   - every call returns int: 0 on success, otherwise a negative LISA_E_* code
 *     or a positive hipError_t value; lisa_last_error() gives the message of the
 *     most recent failure on the calling thread. The reference panics on Metal
 *     failures (metal.rs:153,195,240-245) and returns Result<_, String> from the
 *     runner; a Rust binding maps non-zero returns to exactly those.
 *   - handles are opaque; one stream per device handle, in-order, so a runner
 *     or encoder may be driven by one thread at a time (the reference serializes
 *     its Model behind a Mutex, src/serve/mod.rs:37-39).
 *   - byte offsets are bytes (AGENTS.md:380-381 of the reference).
 */
#ifndef LISA_HIP_H
#define LISA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LISA_OK = 0,
  LISA_E_ARG = -1,       /* invalid argument / shape */
  LISA_E_STATE = -2,     /* call not valid in the current state */
  LISA_E_CAPACITY = -3,  /* KV capacity exhausted */
  LISA_E_VOCAB = -4,     /* token outside the vocabulary */
  LISA_E_NOMODULE = -5,  /* kernel code object missing or unloadable */
  LISA_E_NOMEM = -6
};

const char* lisa_last_error(void);

/* ======================= device bridge (metal.rs) ======================== */
typedef struct LisaDevice LisaDevice;
typedef struct LisaBuffer LisaBuffer;
typedef struct LisaModule LisaModule;
typedef struct LisaFunction LisaFunction;
typedef struct LisaEncoder LisaEncoder;
typedef struct LisaGraph LisaGraph;
typedef struct LisaEvent LisaEvent;

/* MetalDevice::default (metal.rs:150-156): device `ordinal` with one stream. */
int lisa_device_create(int ordinal, LisaDevice** out);
void lisa_device_free(LisaDevice* dev);
/* MetalDevice::name (metal.rs:159-167) */
int lisa_device_name(LisaDevice* dev, char* buf, size_t len);
/* recommendedMaxWorkingSetSize (metal.rs:169-173): total HBM bytes. */
uint64_t lisa_device_max_working_set(LisaDevice* dev);
/* new_buffer / new_untracked_buffer (metal.rs:175-197): hipMalloc'd,
 * zero-filled. There is no hazard tracking: the stream is in order. */
int lisa_buffer_alloc(LisaDevice* dev, size_t len, LisaBuffer** out);
/* Drop for MetalBuffer (metal.rs:414-420). */
void lisa_buffer_free(LisaBuffer* buf);
uint64_t lisa_buffer_device_ptr(const LisaBuffer* buf);
size_t lisa_buffer_len(const LisaBuffer* buf);
/* write_bytes / read_bytes (metal.rs:396-409): synchronous with the stream. */
int lisa_buffer_write(LisaBuffer* buf, size_t offset, const void* src, size_t len);
int lisa_buffer_read(LisaBuffer* buf, size_t offset, void* dst, size_t len);
/* Device-to-device copy on the stream (copy_bytes, norm.metal:118-130). */
int lisa_buffer_copy(LisaBuffer* dst, size_t dst_off, const LisaBuffer* src, size_t src_off, size_t len);

/* new_library + function_named (metal.rs:225-277): a gfx950 code object
 * (.hsaco) by path or blob. lisa_module_load_default loads the kernels built
 * with this library (lisa_kernels.hsaco next to liblisa_hip.so). */
int lisa_module_load(LisaDevice* dev, const char* path, LisaModule** out);
int lisa_module_load_data(LisaDevice* dev, const void* blob, size_t len, LisaModule** out);
int lisa_module_load_default(LisaDevice* dev, LisaModule** out);
void lisa_module_free(LisaModule* mod);
int lisa_function_get(LisaModule* mod, const char* name, LisaFunction** out);

/* Command buffer + compute encoder (metal.rs:297-381). Arguments are bound by
 * index: set_buffer binds a device pointer (buffer + byte offset), set_bytes a
 * value blob; a dispatch launches immediately on the device stream
 * (hipModuleLaunchKernel), wait synchronizes the stream. */
int lisa_encoder_begin(LisaDevice* dev, LisaEncoder** out);
int lisa_encoder_set_function(LisaEncoder* enc, LisaFunction* fn);
int lisa_encoder_set_buffer(LisaEncoder* enc, uint32_t index, const LisaBuffer* buf, uint64_t offset);
int lisa_encoder_set_bytes(LisaEncoder* enc, uint32_t index, const void* bytes, size_t len);
/* dispatch_thread_groups (metal.rs:366-376) */
int lisa_encoder_dispatch_groups(LisaEncoder* enc, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t tx,
                                 uint32_t ty, uint32_t tz);
/* dispatch_threads (metal.rs:354-364): total threads, ceil-divided into groups */
int lisa_encoder_dispatch_threads(LisaEncoder* enc, uint32_t nx, uint32_t ny, uint32_t nz, uint32_t tx,
                                  uint32_t ty, uint32_t tz);
/* commit + wait_until_completed (metal.rs:314-320) and end. */
int lisa_encoder_end(LisaEncoder* enc, int wait);

/* hipGraph capture of everything dispatched between begin and end. */
int lisa_capture_begin(LisaDevice* dev);
int lisa_capture_end(LisaDevice* dev, LisaGraph** out);
int lisa_graph_launch(LisaGraph* graph, LisaDevice* dev);
void lisa_graph_free(LisaGraph* graph);
int lisa_device_synchronize(LisaDevice* dev);

/* Timing on the device stream (hipEvent). */
int lisa_event_create(LisaEvent** out);
void lisa_event_free(LisaEvent* ev);
int lisa_event_record(LisaEvent* ev, LisaDevice* dev);
int lisa_event_elapsed_ms(LisaEvent* start, LisaEvent* stop, float* ms);

/* ==================== decode attention (one layer) ======================= */
/* The attention core of one gated-attention decode layer (the partial/merge
 * half of encode_attention, runner.rs:1426-1592; attention.metal:118-319,
 * 520-641) for BASELINE config 2: q/k RMSNorm + partial RoPE, the new K/V rows
 * appended at positions *pos .. *pos + m_rows - 1, split-K slice partials over
 * the live context and their merge with the output gate. All pointers are
 * device addresses. max_pos bounds the last row's position on the host (it
 * sizes the slice grid and the partials); rows past it are not attended. */
typedef struct LisaAttnDecodeArgs {
  const float* q_proj;       /* [m][12288]: per head 256 query then 256 gate, raw */
  const float* k_raw;        /* [m][1024] */
  const float* v_raw;        /* [m][1024] */
  const uint16_t* q_norm_w;  /* bf16[256] */
  const uint16_t* k_norm_w;  /* bf16[256] */
  uint16_t* key_cache;       /* bf16 [4][capacity][256] */
  uint16_t* value_cache;     /* bf16 [4][capacity][256] */
  const uint32_t* pos;       /* device word: position of row 0 */
  uint16_t* gated;           /* out: bf16 [m][6144] */
  uint32_t capacity;
  uint32_t m_rows;           /* 1 (decode) or 3 (block-3 verify) */
  uint32_t max_pos;          /* *pos + m_rows - 1 <= max_pos < capacity */
  uint32_t pad0;
} LisaAttnDecodeArgs;
/* Bytes of slice partials one call needs: m_rows x (max_pos / 64 + 1) x 24 x 258 x 4. */
uint64_t lisa_attention_workspace_bytes(uint32_t m_rows, uint32_t max_pos);
/* `workspace` (nullable) holds the partials; without one the library keeps a
 * workspace per device, allocated and grown with hipMalloc on demand. Queued
 * on the device stream (no wait). */
int lisa_attention_decode(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* args, LisaBuffer* workspace);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (HIP graph capture, tight serving loops, hosts that forbid hipMalloc):
 * lisa_attention_decode with the slice partials in a fixed scratch array of
 * the library (LISA_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends); it calls no allocator. Rejects (LISA_E_ARG) a call whose
 * lisa_attention_workspace_bytes exceed the scratch: up to position 43327 at
 * one row, 14399 at three. Calls that overlap on one GPU share the scratch and
 * race; calls queued on one stream do not. */
#define LISA_NOALLOC_SCRATCH_BYTES (16u << 20)
int lisa_attention_decode_noalloc(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* args);

/* ============================ runner (runner.rs) ========================= */
typedef struct LisaRunner LisaRunner;

typedef struct LisaRunnerConfig {
  int32_t layers;    /* multiple of 4; 64 for the 27B-shaped model */
  int32_t vocab;     /* 248320 for the real vocabulary */
  int32_t capacity;  /* KV capacity in positions (QwenRunner::load, runner.rs:337-417) */
  int32_t with_mtp;  /* also build the 1-layer MTP drafter (MtpRunner::load, runner.rs:2443-2502) */
  uint64_t seed;     /* synthetic checkpoint seed (lisa_synth.h) */
  int32_t use_graph; /* capture the M=1 decode step into a hipGraph */
  int32_t device;    /* device ordinal */
} LisaRunnerConfig;

/* Load: allocate the resident weight arena, generate the synthetic
 * checkpoint in it, allocate state/KV/scratch, reset state. */
int lisa_runner_create(const LisaRunnerConfig* cfg, LisaRunner** out);

/* ============ checkpoint (src/format/safetensor.rs, src/model/weights.rs) ==
 * Host-only (no device call): a snapshot can be opened and validated before a
 * device exists. */
/* Dtype of a safetensors header entry, in the order of the reference's enum
 * (src/format/dtype.rs:3-16). */
enum {
  LISA_DT_BOOL = 0, LISA_DT_U8, LISA_DT_U16, LISA_DT_I16, LISA_DT_F16, LISA_DT_BF16,
  LISA_DT_U32, LISA_DT_I32, LISA_DT_F32, LISA_DT_U64, LISA_DT_F64
};
#define LISA_MAX_DIMS 8
typedef struct LisaWeightIndex LisaWeightIndex;
/* WeightSlot (weights.rs:7-14): shard, byte offset from the start of that
 * shard's data region (the shard's data region starts at data_start of the
 * file: 8 + header length), byte length, dtype, shape. */
typedef struct LisaWeightSlot {
  int32_t shard;
  int32_t dtype;
  int32_t ndim;
  int32_t pad0;
  uint64_t offset;
  uint64_t data_start;
  uint64_t len;
  uint64_t shape[LISA_MAX_DIMS];
} LisaWeightSlot;
/* WeightIndex::open (weights.rs:22-42) over safetensors shards
 * (safetensor.rs:27-89: u64 LE header length, JSON header, data): each shard
 * memory-mapped read-only; "__"-prefixed header keys skipped; a name in two
 * shards is an error ("duplicate tensor <name>"), as are unknown dtypes
 * ("unknown dtype <name>") and byte ranges outside the data region or not
 * equal to dtype size x shape. */
int lisa_weight_index_open(const char* const* paths, int32_t n, LisaWeightIndex** out);
/* The sorted *.safetensors files of a snapshot directory (runner.rs:345-357):
 * "read snapshot <dir>: <error>" / "no safetensors shards in <dir>". */
int lisa_weight_index_open_snapshot(const char* dir, LisaWeightIndex** out);
void lisa_weight_index_free(LisaWeightIndex* idx);
int32_t lisa_weight_index_len(const LisaWeightIndex* idx);         /* WeightIndex::len */
int32_t lisa_weight_index_shard_count(const LisaWeightIndex* idx); /* WeightIndex::shard_count */
/* WeightIndex::slot (weights.rs:44-46); LISA_E_ARG "missing tensor <name>". */
int lisa_weight_index_slot(const LisaWeightIndex* idx, const char* name, LisaWeightSlot* out);
/* The checks of build_layers / q4() / bf16() / slot() (runner.rs:3769-3946)
 * for a model of `layers` layers (0 = 64) and vocabulary `vocab` (0 = 248320)
 * — every tensor the runner reads present with its dtype and shape, messages
 * "missing tensor <name>" / "invalid tensor <name>: <dtype> <shape>, expected
 * <dtype> <shape>" — or, with mtp != 0, those of build_mtp_weights
 * (runner.rs:3861-3928) after MtpRunner::load's count check (runner.rs:2452-2457,
 * "invalid MTP checkpoint: found <n> tensors, expected 31"). */
int lisa_weight_index_validate(const LisaWeightIndex* idx, int32_t layers, int32_t vocab, int32_t mtp);

/* QwenRunner::load (runner.rs:337-417) and, when mtp_snapshot is non-null,
 * MtpRunner::load (runner.rs:2443-2502) sharing the target's embedding and
 * lm_head: the snapshots' shards are validated as above, then copied once
 * into the resident weight arena in the kernels' layout (packed words as
 * stored; each 64-group's bf16 scale and bias interleaved into one 32-bit
 * word). cfg supplies capacity, use_graph and device; cfg->layers and
 * cfg->vocab give the expected geometry (0 = the reference's 64 and 248320);
 * cfg->with_mtp and cfg->seed are ignored. */
int lisa_runner_load(const char* target_snapshot, const char* mtp_snapshot, const LisaRunnerConfig* cfg,
                     LisaRunner** out);
/* MtpRunner::load(target, snapshot, capacity) (runner.rs:2443-2502) on a
 * runner loaded or created without a drafter: validates the snapshot (31
 * tensors), allocates the drafter's weights and KV caches (capacity must equal
 * the target's) and uploads them; the drafter starts at position 0.
 * LISA_E_STATE if the runner already holds one. */
int lisa_mtp_load(LisaRunner* r, const char* mtp_snapshot, int32_t capacity);
void lisa_runner_free(LisaRunner* r);
LisaDevice* lisa_runner_device(LisaRunner* r);
uint32_t lisa_runner_position(LisaRunner* r);
uint64_t lisa_runner_weight_bytes(LisaRunner* r);

/* QwenRunner::reset_state (runner.rs:423-444): zero the target's GDN/conv
 * state and K/V caches, position 0. The drafter's caches and position are
 * kept (MtpRunner::reset_state below clears those). */
int lisa_runner_reset_state(LisaRunner* r);
/* Synthetic context: GDN state N(0,0.01), conv history N(0,1), KV rows
 * [0,filled) N(0,1) (target and drafter), position = filled. */
int lisa_runner_fill_state(LisaRunner* r, uint32_t filled, uint64_t seed);

/* forward_token_decode (runner.rs:555-591): one M=1 step; argmax (lowest
 * index on ties) and optionally the bf16 hidden (before the final norm) as
 * f32[5120]. */
int lisa_runner_forward_token_decode(LisaRunner* r, uint32_t token, uint32_t* argmax, float* hidden);
/* forward_token_with_hidden (runner.rs:510-550): also the f32 logits[vocab]. */
int lisa_runner_forward_token_with_hidden(LisaRunner* r, uint32_t token, uint32_t* argmax, float* hidden,
                                          float* logits);
/* Greedy decode of `steps` tokens from `token` with device-side feedback
 * (argmax -> next embed), replaying the captured step graph; tokens_out
 * receives the `steps` generated tokens. The loop of src/cli/run.rs:69-73. */
int lisa_runner_decode_greedy(LisaRunner* r, uint32_t token, int32_t steps, uint32_t* tokens_out);

/* Per-kernel profile of `steps` eager M=1 steps from `token`: every launch is
 * timed by start/stop events attached to its dispatch (the kernel's execution
 * window, as a kernel trace reports it); kind_ms[k] / kind_count[k]
 * receive the summed duration (ms) and number of launches of kind k. The
 * diagnostic counterpart of profile_token_m1_diagnostic (runner.rs:660-730). */
enum {
  LISA_KIND_GDN_IN = 0,        /* GDN qkv/z/a/b projections (+ residual, norm, conv) */
  LISA_KIND_GDN_RECURRENCE,    /* gated-delta recurrence + gated norm */
  LISA_KIND_GDN_OUT,           /* GDN out_proj */
  LISA_KIND_ATTN_IN,           /* attention q/k/v projections (+ residual, norm) */
  LISA_KIND_ATTN_PARTIAL,      /* norm + RoPE + KV append + split-K slices */
  LISA_KIND_ATTN_MERGE,        /* flash merge + output gate */
  LISA_KIND_ATTN_OUT,          /* o_proj */
  LISA_KIND_MLP_GATE_UP,       /* residual + norm + gate/up + SwiGLU */
  LISA_KIND_MLP_DOWN,          /* down_proj */
  LISA_KIND_LM_HEAD,           /* final residual + norm + lm_head + argmax partials */
  LISA_KIND_FINALIZE,          /* argmax finish + token/position feedback */
  LISA_KIND_COUNT
};
int lisa_runner_profile_step(LisaRunner* r, uint32_t token, int32_t steps, float* kind_ms, int32_t* kind_count);
/* The same per-kind profile of one eager M=3 verify pass (verify_block3's
 * launches with slot capture); leaves the runner as lisa_runner_verify_block3
 * does (position += 3, awaiting commit). No counterpart in the reference, whose
 * diagnostic covers M=1 only. */
int lisa_runner_profile_block3(LisaRunner* r, const uint32_t tokens[3], float* kind_ms, int32_t* kind_count);

/* forward_prefill_with_progress (runner.rs:2129-2230): the `n` prompt tokens
 * in chunks of `chunk` rows (<= 2048; 0 = 2048; the reference's PREFILL_BATCH
 * is 512, and the result is the same for every chunk size)
 * with q4 GEMMs (bf16 MFMA), batched GDN and attention; GDN/conv state and KV
 * carry across chunks. argmax_out[n] (nullable) gets each position's greedy
 * token, hidden_out (nullable) f32[n][5120] the hidden before the final norm.
 * position += n. */
int lisa_runner_forward_prefill(LisaRunner* r, const uint32_t* tokens, int32_t n, int32_t chunk,
                                uint32_t* argmax_out, float* hidden_out);

/* verify_block3_decode (runner.rs:734-909): M=3 pass with GDN/conv capture;
 * argmax[3]; hidden (nullable) f32[3][5120]; logits (nullable) f32[3][vocab].
 * position += 3 until commit. */
int lisa_runner_verify_block3(LisaRunner* r, const uint32_t tokens[3], uint32_t argmax[3], float* hidden,
                              float* logits);
/* commit_verified_prefix (runner.rs:911-944): rows in 1..3. */
int lisa_runner_commit_verified_prefix(LisaRunner* r, int32_t rows);

/* checkpoint_state / restore_state (runner.rs:447-503). Restore rejects a
 * position past the KV capacity (LISA_E_CAPACITY) and a checkpoint taken on a
 * runner with another number of GDN layers (LISA_E_ARG). */
typedef struct LisaCheckpoint LisaCheckpoint;
int lisa_runner_checkpoint_state(LisaRunner* r, LisaCheckpoint** out);
int lisa_runner_restore_state(LisaRunner* r, const LisaCheckpoint* ck);
void lisa_checkpoint_free(LisaCheckpoint* ck);

/* upload_hidden_device (runner.rs:850-858): host f32 hidden -> bf16
 * (truncation, dtype.rs:42-47) into target hidden row `row`, the conditioning
 * row the drafter reads with cond_source 0. */
int lisa_runner_upload_hidden(LisaRunner* r, int32_t row, const float* hidden);
int32_t lisa_runner_vocab(LisaRunner* r);

/* Read back state for tests: GDN state of gdn layer `idx` (f32[48*128*128]),
 * conv history (bf16[3*10240]). */
int lisa_runner_read_gdn_state(LisaRunner* r, int32_t idx, float* out);
int lisa_runner_read_conv_state(LisaRunner* r, int32_t idx, uint16_t* out);

/* MtpRunner (runner.rs:2233-3701). cond_source: 0 = target hidden row
 * `cond_row` (target.hidden_offset, runner.rs:846-848), 1 = the drafter's own
 * last normalized hidden (draft chaining), 2 = the hidden uploaded with
 * lisa_mtp_upload_cond. forward_position_decode_device (runner.rs:2711-2765). */
int lisa_mtp_forward(LisaRunner* r, uint32_t token, int32_t cond_source, int32_t cond_row, uint32_t* argmax);
/* upload_normalized_device (runner.rs:2685-2692): host f32 -> bf16 by
 * truncation into the drafter's normalized-hidden slot (cond_source 1). */
int lisa_mtp_upload_normalized(LisaRunner* r, const float* hidden);
/* A free conditioning hidden (cond_source 2), bf16 bits. */
int lisa_mtp_upload_cond(LisaRunner* r, const uint16_t* hidden);
int lisa_mtp_read_normalized(LisaRunner* r, uint16_t* out);
uint32_t lisa_mtp_position(LisaRunner* r);
int lisa_mtp_trim_state(LisaRunner* r, int32_t count);
/* MtpRunner::reset_state (runner.rs:2508-2520): zero the drafter's K/V caches,
 * drafter position 0; the target's state is kept. LISA_E_STATE without a
 * drafter. */
int lisa_mtp_reset_state(LisaRunner* r);

/* Device-resident conditioning by (buffer, byte offset), as speculative/mod.rs
 * passes it: the target's hidden row `row` sits at lisa_runner_hidden_offset(row)
 * of QwenRunner::scratch() (hidden_offset, runner.rs:846-848), the drafter's own
 * normalized hidden at lisa_mtp_normalized_offset() of MtpRunner::scratch()
 * (normalized_offset, runner.rs:2689-2692). lisa_mtp_resolve_cond maps
 * (cond is the target's scratch, offset) to (cond_source, cond_row) of
 * lisa_mtp_forward, rejecting offsets that address neither (host-only, no
 * device call). lisa_mtp_forward_device is forward_position_decode_device
 * (runner.rs:2711-2765) with that addressing; *normalized_off receives
 * normalized_offset(). */
uint64_t lisa_runner_hidden_offset(int32_t row);
uint64_t lisa_mtp_normalized_offset(void);
int lisa_mtp_resolve_cond(int32_t cond_is_target, uint64_t cond_off, int32_t* cond_source, int32_t* cond_row);
int lisa_mtp_forward_device(LisaRunner* r, uint32_t token, int32_t cond_is_target, uint64_t cond_off,
                            uint32_t* argmax, uint64_t* normalized_off);
/* forward_position_decode (runner.rs:2618-2680): the drafter conditioned on a
 * host hidden f32[5120] (bf16 by truncation); argmax and the normalized hidden
 * (nullable, f32[5120]). */
int lisa_mtp_forward_position_decode(LisaRunner* r, uint32_t token, const float* hidden, uint32_t* argmax,
                                     float* normalized);
/* forward_position_batch_with_progress (runner.rs:3494-3581): n positions of
 * (tokens[t], hiddens f32[t][5120]) in chunks of `chunk` rows (0 = 512) with
 * the prefill kernels (q4 GEMMs on the matrix cores, attention rows);
 * argmax_out[n] and normalized_out f32[n][5120] (both nullable).
 * mtp position += n. A host that reports progress calls it once per chunk. */
int lisa_mtp_forward_batch(LisaRunner* r, const uint32_t* tokens, const float* hiddens, int32_t n, int32_t chunk,
                           uint32_t* argmax_out, float* normalized_out);

/* MtpRunner::checkpoint_state / restore_state (runner.rs:2382-2420): device
 * copies of the drafter's KV caches and its position. Restore rejects a
 * checkpoint position past the capacity (LISA_E_CAPACITY, as the reference
 * does) and a checkpoint of another capacity (LISA_E_ARG). */
typedef struct LisaMtpCheckpoint LisaMtpCheckpoint;
int lisa_mtp_checkpoint_state(LisaRunner* r, LisaMtpCheckpoint** out);
int lisa_mtp_restore_state(LisaRunner* r, const LisaMtpCheckpoint* ck);
void lisa_mtp_checkpoint_free(LisaMtpCheckpoint* ck);

/* ========================= speculative (speculative/mod.rs) ============== */
typedef struct LisaAcceptance {
  int32_t accepted_drafts;
  int32_t emitted_count;
  uint32_t emitted[3];
  int32_t target_trim;
} LisaAcceptance;
/* accept_greedy (speculative/mod.rs:16-32); n_drafts <= 2. */
int lisa_accept_greedy(const uint32_t* drafts, int32_t n_drafts, const uint32_t* target, LisaAcceptance* out);

typedef struct LisaReconcilePlan {
  int32_t trim;
  int32_t replay_count;
  int32_t replay[3]; /* draft index, or -1 for the replacement */
} LisaReconcilePlan;
/* mtp_reconcile_plan (speculative/mod.rs:49-65). */
int lisa_mtp_reconcile_plan(int32_t draft_count, int32_t round_appended, int32_t accepted, LisaReconcilePlan* out);

typedef struct LisaSpecStats {
  int32_t rounds;
  int32_t accepted_drafts;
  int32_t drafted_tokens;
  int32_t target_forwards;
} LisaSpecStats;
/* generate_greedy_block3_prefilled (speculative/mod.rs:384-413, loop
 * :102-198). `bonus` and `target_hidden` (f32[5120]) come from the prefill;
 * mtp_seed_token/mtp_seed_hidden (f32[5120]) seed the drafter. When
 * force_truth is non-null, every draft is replaced before verification by
 * force_truth[j] (the target-only greedy token at that output position) with
 * probability p_accept under the seeded stream force_seed, else by a token
 * that differs from it — a forced acceptance pattern exercising 1, 2 and 3
 * accepted rows. tokens_out receives max_tokens tokens (bonus first). */
int lisa_generate_greedy_block3(LisaRunner* r, uint32_t bonus, const float* target_hidden,
                                uint32_t mtp_seed_token, const float* mtp_seed_hidden, int32_t max_tokens,
                                const uint32_t* force_truth, int32_t force_len, uint64_t force_seed,
                                float p_accept, uint32_t* tokens_out, LisaSpecStats* stats);

/* prefill_prompt_from (speculative/mod.rs:237-311): target prefill of
 * prompt[start..n) (batched from 4 tokens), then the drafter over the shifted
 * tokens conditioned on the target's per-position hidden rows (batched from 4
 * positions). Outputs: the bonus token, the target hidden f32[5120] of the last
 * position and the drafter seed (token, normalized hidden f32[5120]). Both
 * runners must be positioned at `start`. */
int lisa_prefill_prompt(LisaRunner* r, const uint32_t* prompt, int32_t n, int32_t start, uint32_t* bonus,
                        float* target_hidden, uint32_t* mtp_seed_token, float* mtp_seed_hidden);

#ifdef __cplusplus
}
#endif
#endif /* LISA_HIP_H */
