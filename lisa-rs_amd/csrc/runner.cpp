// runner.cpp — the decode-path runner behind include/lisa_hip.h: a C++
// restatement of the reference's QwenRunner / MtpRunner (src/model/runner.rs)
// and greedy block-3 speculative loop (src/speculative/mod.rs), driving the
// gfx950 kernels through the bridge of device.cpp.
//
// Per-token dispatch recipe (one hipGraph for M=1):
//   layer i, GDN      : qmv[in_proj: embed | input RMSNorm -> qkv(conv)|z|a|b]
//                       gdn_recurrence -> gated;  qmv[out_proj + residual add]
//   layer i, attention: qmv[in_proj -> q|k|v];  attn_partial;  attn_merge -> gated;
//                       qmv[o_proj + residual add]
//   every layer       : qmv[post RMSNorm -> gate/up -> SwiGLU];  qmv[down + residual add]
//   final             : qmv[final RMSNorm -> lm_head -> argmax partials];  step_finalize
// A residual-add epilogue updates the residual rows in place; the next launch's
// RMSNorm prologue forms the sum of squares from the residual rows it reads.
// 5 launches per GDN layer, 6 per attention layer, 2 final (338 for 64 layers)
// against the reference's 852 dispatches (runner.rs:568-582, 1248-1592).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "bridge.h"
#include "lisa_hip.h"
#include "loader.h"
#include "lisa_kernels.h"
#include "qmv_launch.h"
#include "lisa_model.h"
#include "lisa_numerics.h"
#include "lisa_synth.h"
#include "spec_round.h"

namespace {

constexpr uint32_t kHistoryCap = 1u << 16;
// Captured decode steps launch attention slices in multiples of this many
// 64-token slices (512 positions), so one graph serves 512 positions and a
// replay dispatches at most 7 slices past the context.
constexpr uint32_t kGraphSliceBucket = 8;

struct Q4Dev {
  uint32_t* w = nullptr;
  uint32_t* sb = nullptr;
  uint32_t n = 0, k = 0;
};

struct LayerDev {
  bool attention = false;
  uint16_t *input_norm = nullptr, *post_norm = nullptr;
  Q4Dev gate, up, down;
  Q4Dev qkv, z, a, b, out;
  uint16_t *conv_w = nullptr, *a_log = nullptr, *dt_bias = nullptr, *gnorm = nullptr;
  int state_index = -1;
  Q4Dev q, k, v, o;
  uint16_t *q_norm = nullptr, *k_norm = nullptr;
  int cache_index = -1;
};

struct MtpDev {
  uint16_t *pre_fc_emb, *pre_fc_hid, *input_norm, *post_norm, *final_norm, *q_norm, *k_norm;
  Q4Dev fc, q, k, v, o, gate, up, down;
};

// Scratch of one forward context (target: rows <= 3; drafter: 1 row).
struct Ctx {
  int rows = 1;
  uint16_t *H, *gated, *act, *xnorm, *cond;  // H: residual rows, updated in place
  float *B, *conv_out, *z, *a, *b, *gate_ab, *q_proj, *k_raw, *v_raw, *part_o, *part_ml, *logits, *am_val;
  uint32_t *am_idx, *tokens, *argmax, *pos, *step, *history, *pf_sink;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Bump allocator over one device buffer; a first pass with base==nullptr
// only measures.
struct Arena {
  char* base = nullptr;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    used = align256(used);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
};

}  // namespace

struct LisaCheckpoint {
  LisaBuffer* gdn = nullptr;
  LisaBuffer* conv = nullptr;
  uint32_t position = 0;
  // geometry of the runner that took it: a restore into a runner of another
  // depth would copy past its state arenas
  int32_t gdn_layers = 0;
};

// MtpCheckpoint (runner.rs:2375-2380): the drafter's KV caches and position.
struct LisaMtpCheckpoint {
  LisaBuffer* key = nullptr;
  LisaBuffer* value = nullptr;
  uint32_t position = 0;
  int32_t capacity = 0;
};

struct LisaRunner {
  LisaRunnerConfig cfg{};
  LisaDevice* dev = nullptr;
  // GDN recurrence launches carry L2 prefetch workgroups for the out_proj
  // weights, l2_prefetch per XCD (environment LISA_L2_PREFETCH, 0 = none,
  // else 20..26), after a sleep of l2_prefetch_delay x 512 cycles
  // (LISA_L2_PREFETCH_DELAY)
  uint32_t l2_prefetch = 20;
  uint32_t l2_prefetch_delay = 0;
  LisaModule* mod = nullptr;
  // kernels
  LisaFunction *qmv[2][5][7] = {};  // [m3][K index][prologue mode]
  LisaFunction *qmv_epi[2][7][5] = {};  // K = 5120 with a fixed epilogue: [m3][prologue][epilogue]
  LisaFunction *qmv_gateup_wide[2] = {};  // MLP gate/up, PRENORM: 17 tiles per 16-wave workgroup [m3]
  LisaFunction *qmv_inproj_wide[2][2] = {};  // in-projections, PRENORM: one tile per wave [m3][NW 7, 8]
  LisaFunction *qmv_x_wide = nullptr;  // one-row LOADX STORE launches of 2049..2304 tiles, 9 waves
  LisaFunction *gdn[2] = {}, *attn_part[2] = {}, *attn_merge[2] = {}, *finalize = nullptr, *synth = nullptr;
  // batched prefill
  LisaFunction *gemm = nullptr, *gemm_m128 = nullptr, *gemm_wide = nullptr, *gemm_swiglu = nullptr, *rows = nullptr, *conv_rows = nullptr, *gdn_prep_rows = nullptr, *gdn_scan_rows = nullptr,
               *gdn_out_rows = nullptr, *attn_store_rows = nullptr,
               *attn_partial_rows = nullptr, *attn_merge_rows = nullptr;
  // memory
  LisaBuffer *weights = nullptr, *state = nullptr, *scratch = nullptr;
  // a drafter loaded after the target (lisa_mtp_load): its weights and KV
  LisaBuffer *mtp_weights = nullptr, *mtp_state = nullptr;
  std::vector<LayerDev> layers;
  Q4Dev embed, head;
  uint16_t* final_norm = nullptr;
  MtpDev mtp{};
  int gdn_layers = 0, attn_layers = 0;
  uint32_t s_max = 0;
  // GDN and conv state in three rotating buffers: buffer `live` holds the
  // state, the other two (in index order) receive a verification's rows 1
  // and 2, and committing one or two rows makes that buffer the live one
  // instead of copying it back (the derived pointers follow set_live)
  float* gdn_buf[3] = {};
  uint16_t* conv_buf[3] = {};
  int live = 0;
  float* gdn_state = nullptr;
  uint16_t* conv_state = nullptr;
  float* gdn_slots = nullptr;  // slot 0; slot 1 is gdn_slot_stride floats further
  uint16_t* conv_slots = nullptr;
  uint64_t gdn_slot_stride = 0, conv_slot_stride = 0;
  uint16_t *key_cache = nullptr, *value_cache = nullptr;
  uint16_t *mtp_key = nullptr, *mtp_value = nullptr;
  Ctx tgt{}, drf{};
  // prefill scratch, allocated at the first prefill call (runner.rs:378 sizes it
  // for PREFILL_BATCH rows)
  struct Prefill {
    LisaBuffer* buf = nullptr;
    uint32_t att_rows = 0;  // rows per attention sub-block (bounds the slice partials)
    uint32_t *tokens = nullptr, *argmax = nullptr, *pos = nullptr;
    uint16_t *H = nullptr, *X = nullptr, *gated = nullptr, *act = nullptr;
    float* query = nullptr;
    float *B = nullptr, *qkv = nullptr, *conv_out = nullptr, *z = nullptr, *a = nullptr, *b = nullptr;
    float *q_proj = nullptr, *k_raw = nullptr, *v_raw = nullptr, *logits = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;
    float *gdn_qk = nullptr, *gdn_gates = nullptr, *gdn_y = nullptr;
  } pf;
  // host mirrors
  uint32_t position = 0;
  int64_t verify_base = -1;
  uint32_t mtp_position = 0;
  // captured M=1 steps keyed by the attention slices they launch (a multiple
  // of kGraphSliceBucket): a replay covers every position whose context fits
  std::map<uint32_t, LisaGraph*> step_graphs;
  // captured M=3 verifications by slice bucket, and captured drafter steps by
  // (condition source, slice bucket)
  std::map<uint32_t, LisaGraph*> verify_graphs;
  std::map<uint32_t, LisaGraph*> mtp_graphs;
  // pinned host staging of the speculative loop's rounds (spec_round.h)
  uint32_t* pinned = nullptr;
  // per-launch timing of eager steps (lisa_runner_profile_step)
  std::vector<LisaProfRec> prof;
};

namespace {

int k_index(uint32_t k) {
  switch (k) {
    case 5120: return 0;
    case 6144: return 1;
    case 10240: return 2;
    case 17408: return 3;
    case 1024: return 4;
    default: return -1;
  }
}

// q4 launch geometry: 8-row tiles (4 outputs for gate/up pairs); K = 5120 runs
// one tile per wave (4 per workgroup), every other K splits each tile's group
// iterations over the four waves of one workgroup.
bool qmv_split(uint32_t k) { return k != LISA_HIDDEN; }

uint32_t qmv_grid(uint32_t k, uint32_t tiles) { return qmv_split(k) ? tiles : (tiles + 3) / 4; }

// Attention slices a launch covers: every 64-token slice up to the position
// of its last row (the reference sizes its slice grid to the live context,
// runner.rs:1498-1500); a captured step rounds up to kGraphSliceBucket.
uint32_t att_slices(const LisaRunner* r, uint32_t last_pos, bool bucket) {
  uint32_t s = last_pos / LISA_ATT_SLICE + 1;
  if (bucket) s = (s + kGraphSliceBucket - 1) / kGraphSliceBucket * kGraphSliceBucket;
  return std::min(s, r->s_max);
}

// workgroups of the lm_head launch = number of argmax partials per row
int lm_head_grid(const LisaRunner* r) {
  return (int)std::max<uint32_t>(1, qmv_grid(LISA_HIDDEN, ((uint32_t)r->cfg.vocab + 7) / 8));
}

int upload_u32(LisaRunner* r, uint32_t* dst, const uint32_t* src, size_t n) {
  return lisa_hip_check(hipMemcpyAsync(dst, src, n * 4, hipMemcpyHostToDevice, r->dev->stream), "H2D");
}

int sync(LisaRunner* r) { return lisa_hip_check(hipStreamSynchronize(r->dev->stream), "hipStreamSynchronize"); }

// ---- synthetic checkpoint ----------------------------------------------------
int fill(LisaRunner* r, void* out, uint64_t n, uint32_t kind, uint64_t key, uint64_t key2, uint32_t dist, float a,
         float b, uint32_t capacity = 0, uint32_t filled = 0) {
  LisaSynthParams p{};
  p.out = out;
  p.n = n;
  p.key = key;
  p.key2 = key2;
  p.kind = kind;
  p.dist = dist;
  p.a = a;
  p.b = b;
  p.capacity = capacity;
  p.filled = filled;
  const uint64_t groups = std::min<uint64_t>((n + 255) / 256, 65536);
  return lisa_launch(r->dev, r->synth, &p, sizeof p, (uint32_t)std::max<uint64_t>(groups, 1), 1, 1, 256, 1, 1);
}

uint64_t key_of(const LisaRunner* r, int scope, int kind, int part) {
  return lisa_stream_key(r->cfg.seed, lisa_tensor_id(scope, kind, part));
}

int gen_q4(LisaRunner* r, const Q4Dev& q, int scope, int kind) {
  LISA_TRY(fill(r, q.w, (uint64_t)q.n * q.k / 8, LISA_FILL_WORDS, key_of(r, scope, kind, 0), 0, 0, 0, 0));
  return fill(r, q.sb, (uint64_t)q.n * q.k / 64, LISA_FILL_SB, key_of(r, scope, kind, 1), key_of(r, scope, kind, 2), 0,
              0, 0);
}

int gen_vec(LisaRunner* r, uint16_t* v, uint64_t n, int scope, int kind, float lo, float hi) {
  return fill(r, v, n, LISA_FILL_BF16, key_of(r, scope, kind, 0), 0, LISA_DIST_UNIFORM, lo, hi);
}

Q4Dev take_q4(Arena& A, uint32_t n, uint32_t k) {
  Q4Dev q;
  q.n = n;
  q.k = k;
  q.w = A.take<uint32_t>((size_t)n * k / 8);
  q.sb = A.take<uint32_t>((size_t)n * k / 64);
  return q;
}

void plan_mtp_weights(LisaRunner* r, Arena& A);

void plan_weights(LisaRunner* r, Arena& A) {
  const int L = r->cfg.layers;
  r->layers.assign(L, LayerDev());
  r->gdn_layers = r->attn_layers = 0;
  for (int i = 0; i < L; ++i) {
    LayerDev& l = r->layers[i];
    l.attention = lisa_layer_is_attention(i);
    l.input_norm = A.take<uint16_t>(LISA_HIDDEN);
    l.post_norm = A.take<uint16_t>(LISA_HIDDEN);
    l.gate = take_q4(A, LISA_INTER, LISA_HIDDEN);
    l.up = take_q4(A, LISA_INTER, LISA_HIDDEN);
    l.down = take_q4(A, LISA_HIDDEN, LISA_INTER);
    if (l.attention) {
      l.q = take_q4(A, LISA_ATT_Q_OUT, LISA_HIDDEN);
      l.k = take_q4(A, LISA_ATT_KV_OUT, LISA_HIDDEN);
      l.v = take_q4(A, LISA_ATT_KV_OUT, LISA_HIDDEN);
      l.o = take_q4(A, LISA_HIDDEN, LISA_ATT_OUT);
      l.q_norm = A.take<uint16_t>(LISA_ATT_HD);
      l.k_norm = A.take<uint16_t>(LISA_ATT_HD);
      l.cache_index = r->attn_layers++;
    } else {
      l.qkv = take_q4(A, LISA_GDN_CONV_DIM, LISA_HIDDEN);
      l.z = take_q4(A, LISA_GDN_VALUE_DIM, LISA_HIDDEN);
      l.a = take_q4(A, LISA_GDN_VH, LISA_HIDDEN);
      l.b = take_q4(A, LISA_GDN_VH, LISA_HIDDEN);
      l.out = take_q4(A, LISA_HIDDEN, LISA_GDN_VALUE_DIM);
      l.conv_w = A.take<uint16_t>(LISA_GDN_CONV_DIM * 4);
      l.a_log = A.take<uint16_t>(LISA_GDN_VH);
      l.dt_bias = A.take<uint16_t>(LISA_GDN_VH);
      l.gnorm = A.take<uint16_t>(LISA_GDN_HD);
      l.state_index = r->gdn_layers++;
    }
  }
  r->embed = take_q4(A, r->cfg.vocab, LISA_HIDDEN);
  r->head = take_q4(A, r->cfg.vocab, LISA_HIDDEN);
  r->final_norm = A.take<uint16_t>(LISA_HIDDEN);
  if (r->cfg.with_mtp) plan_mtp_weights(r, A);
}

// The drafter's own tensors (MtpWeights, runner.rs:2452-2457); it shares the
// target's embedding and lm_head.
void plan_mtp_weights(LisaRunner* r, Arena& A) {
  {
    MtpDev& t = r->mtp;
    t.pre_fc_emb = A.take<uint16_t>(LISA_HIDDEN);
    t.pre_fc_hid = A.take<uint16_t>(LISA_HIDDEN);
    t.input_norm = A.take<uint16_t>(LISA_HIDDEN);
    t.post_norm = A.take<uint16_t>(LISA_HIDDEN);
    t.final_norm = A.take<uint16_t>(LISA_HIDDEN);
    t.q_norm = A.take<uint16_t>(LISA_ATT_HD);
    t.k_norm = A.take<uint16_t>(LISA_ATT_HD);
    t.fc = take_q4(A, LISA_HIDDEN, 2 * LISA_HIDDEN);
    t.q = take_q4(A, LISA_ATT_Q_OUT, LISA_HIDDEN);
    t.k = take_q4(A, LISA_ATT_KV_OUT, LISA_HIDDEN);
    t.v = take_q4(A, LISA_ATT_KV_OUT, LISA_HIDDEN);
    t.o = take_q4(A, LISA_HIDDEN, LISA_ATT_OUT);
    t.gate = take_q4(A, LISA_INTER, LISA_HIDDEN);
    t.up = take_q4(A, LISA_INTER, LISA_HIDDEN);
    t.down = take_q4(A, LISA_HIDDEN, LISA_INTER);
  }
}

int generate_weights(LisaRunner* r) {
  for (int i = 0; i < r->cfg.layers; ++i) {
    const LayerDev& l = r->layers[i];
    const int sc = i + 1;
    LISA_TRY(gen_vec(r, l.input_norm, LISA_HIDDEN, sc, LISA_T_INPUT_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, l.post_norm, LISA_HIDDEN, sc, LISA_T_POST_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_q4(r, l.gate, sc, LISA_T_MLP_GATE));
    LISA_TRY(gen_q4(r, l.up, sc, LISA_T_MLP_UP));
    LISA_TRY(gen_q4(r, l.down, sc, LISA_T_MLP_DOWN));
    if (l.attention) {
      LISA_TRY(gen_q4(r, l.q, sc, LISA_T_ATT_Q));
      LISA_TRY(gen_q4(r, l.k, sc, LISA_T_ATT_K));
      LISA_TRY(gen_q4(r, l.v, sc, LISA_T_ATT_V));
      LISA_TRY(gen_q4(r, l.o, sc, LISA_T_ATT_O));
      LISA_TRY(gen_vec(r, l.q_norm, LISA_ATT_HD, sc, LISA_T_ATT_Q_NORM, 0.9f, 1.1f));
      LISA_TRY(gen_vec(r, l.k_norm, LISA_ATT_HD, sc, LISA_T_ATT_K_NORM, 0.9f, 1.1f));
    } else {
      LISA_TRY(gen_q4(r, l.qkv, sc, LISA_T_GDN_QKV));
      LISA_TRY(gen_q4(r, l.z, sc, LISA_T_GDN_Z));
      LISA_TRY(gen_q4(r, l.a, sc, LISA_T_GDN_A));
      LISA_TRY(gen_q4(r, l.b, sc, LISA_T_GDN_B));
      LISA_TRY(gen_q4(r, l.out, sc, LISA_T_GDN_OUT));
      LISA_TRY(gen_vec(r, l.conv_w, LISA_GDN_CONV_DIM * 4, sc, LISA_T_GDN_CONV_W, -0.5f, 0.5f));
      LISA_TRY(gen_vec(r, l.a_log, LISA_GDN_VH, sc, LISA_T_GDN_A_LOG, -2.0f, 0.0f));
      LISA_TRY(gen_vec(r, l.dt_bias, LISA_GDN_VH, sc, LISA_T_GDN_DT_BIAS, -1.0f, 1.0f));
      LISA_TRY(gen_vec(r, l.gnorm, LISA_GDN_HD, sc, LISA_T_GDN_NORM, 0.9f, 1.1f));
    }
  }
  LISA_TRY(gen_q4(r, r->embed, 0, LISA_T_EMBED));
  LISA_TRY(gen_q4(r, r->head, 0, LISA_T_LM_HEAD));
  LISA_TRY(gen_vec(r, r->final_norm, LISA_HIDDEN, 0, LISA_T_FINAL_NORM, 0.9f, 1.1f));
  if (r->cfg.with_mtp) {
    const int sc = LISA_SCOPE_MTP;
    const MtpDev& t = r->mtp;
    LISA_TRY(gen_vec(r, t.pre_fc_emb, LISA_HIDDEN, sc, LISA_T_MTP_PRE_FC_EMB, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.pre_fc_hid, LISA_HIDDEN, sc, LISA_T_MTP_PRE_FC_HID, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.input_norm, LISA_HIDDEN, sc, LISA_T_INPUT_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.post_norm, LISA_HIDDEN, sc, LISA_T_POST_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.final_norm, LISA_HIDDEN, sc, LISA_T_FINAL_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.q_norm, LISA_ATT_HD, sc, LISA_T_ATT_Q_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_vec(r, t.k_norm, LISA_ATT_HD, sc, LISA_T_ATT_K_NORM, 0.9f, 1.1f));
    LISA_TRY(gen_q4(r, t.fc, sc, LISA_T_MTP_FC));
    LISA_TRY(gen_q4(r, t.q, sc, LISA_T_ATT_Q));
    LISA_TRY(gen_q4(r, t.k, sc, LISA_T_ATT_K));
    LISA_TRY(gen_q4(r, t.v, sc, LISA_T_ATT_V));
    LISA_TRY(gen_q4(r, t.o, sc, LISA_T_ATT_O));
    LISA_TRY(gen_q4(r, t.gate, sc, LISA_T_MLP_GATE));
    LISA_TRY(gen_q4(r, t.up, sc, LISA_T_MLP_UP));
    LISA_TRY(gen_q4(r, t.down, sc, LISA_T_MLP_DOWN));
  }
  return sync(r);
}

// ---- real checkpoint ---------------------------------------------------------
// One tensor the runner reads, under its checkpoint name: a q4 linear (the
// prefix of its .weight / .scales / .biases, q4() of runner.rs:3906-3928) or
// a bf16 tensor of a fixed shape (bf16(), :3930-3932).
struct WeightEntry {
  std::string name;
  const Q4Dev* q = nullptr;  // q4 destination (its n, k give the shapes)
  uint16_t* vec = nullptr;   // bf16 destination
  std::vector<uint64_t> shape;
};

void cat_q4(std::vector<WeightEntry>& c, const std::string& name, const Q4Dev& q) {
  WeightEntry e;
  e.name = name;
  e.q = &q;
  c.push_back(e);
}

void cat_vec(std::vector<WeightEntry>& c, const std::string& name, uint16_t* v, std::vector<uint64_t> shape) {
  WeightEntry e;
  e.name = name;
  e.vec = v;
  e.shape = std::move(shape);
  c.push_back(e);
}

// The target's tensors in the order the reference resolves them: build_layers
// (runner.rs:3769-3860), then embed_tokens, norm, lm_head (:359-361).
std::vector<WeightEntry> target_catalogue(const LisaRunner* r) {
  std::vector<WeightEntry> c;
  const uint64_t H = LISA_HIDDEN;
  for (int i = 0; i < r->cfg.layers; ++i) {
    const LayerDev& l = r->layers[i];
    const std::string pre = "language_model.model.layers." + std::to_string(i);
    cat_vec(c, pre + ".input_layernorm.weight", l.input_norm, {H});
    cat_vec(c, pre + ".post_attention_layernorm.weight", l.post_norm, {H});
    cat_q4(c, pre + ".mlp.gate_proj", l.gate);
    cat_q4(c, pre + ".mlp.up_proj", l.up);
    cat_q4(c, pre + ".mlp.down_proj", l.down);
    if (!l.attention) {
      const std::string p = pre + ".linear_attn";
      cat_q4(c, p + ".in_proj_qkv", l.qkv);
      cat_q4(c, p + ".in_proj_z", l.z);
      cat_q4(c, p + ".in_proj_a", l.a);
      cat_q4(c, p + ".in_proj_b", l.b);
      cat_q4(c, p + ".out_proj", l.out);
      cat_vec(c, p + ".conv1d.weight", l.conv_w, {LISA_GDN_CONV_DIM, LISA_GDN_CONV_K, 1});
      cat_vec(c, p + ".A_log", l.a_log, {LISA_GDN_VH});
      cat_vec(c, p + ".dt_bias", l.dt_bias, {LISA_GDN_VH});
      cat_vec(c, p + ".norm.weight", l.gnorm, {LISA_GDN_HD});
    } else {
      const std::string p = pre + ".self_attn";
      cat_q4(c, p + ".q_proj", l.q);
      cat_q4(c, p + ".k_proj", l.k);
      cat_q4(c, p + ".v_proj", l.v);
      cat_q4(c, p + ".o_proj", l.o);
      cat_vec(c, p + ".q_norm.weight", l.q_norm, {LISA_ATT_HD});
      cat_vec(c, p + ".k_norm.weight", l.k_norm, {LISA_ATT_HD});
    }
  }
  cat_q4(c, "language_model.model.embed_tokens", r->embed);
  cat_vec(c, "language_model.model.norm.weight", r->final_norm, {H});
  cat_q4(c, "language_model.lm_head", r->head);
  return c;
}

// The drafter's 31 tensors (build_mtp_weights, runner.rs:3861-3928).
std::vector<WeightEntry> mtp_catalogue(const LisaRunner* r) {
  std::vector<WeightEntry> c;
  const uint64_t H = LISA_HIDDEN;
  const MtpDev& t = r->mtp;
  cat_vec(c, "pre_fc_norm_embedding.weight", t.pre_fc_emb, {H});
  cat_vec(c, "pre_fc_norm_hidden.weight", t.pre_fc_hid, {H});
  cat_q4(c, "fc", t.fc);
  cat_vec(c, "layers.0.input_layernorm.weight", t.input_norm, {H});
  cat_q4(c, "layers.0.self_attn.q_proj", t.q);
  cat_q4(c, "layers.0.self_attn.k_proj", t.k);
  cat_q4(c, "layers.0.self_attn.v_proj", t.v);
  cat_q4(c, "layers.0.self_attn.o_proj", t.o);
  cat_vec(c, "layers.0.self_attn.q_norm.weight", t.q_norm, {LISA_ATT_HD});
  cat_vec(c, "layers.0.self_attn.k_norm.weight", t.k_norm, {LISA_ATT_HD});
  cat_vec(c, "layers.0.post_attention_layernorm.weight", t.post_norm, {H});
  cat_q4(c, "layers.0.mlp.gate_proj", t.gate);
  cat_q4(c, "layers.0.mlp.up_proj", t.up);
  cat_q4(c, "layers.0.mlp.down_proj", t.down);
  cat_vec(c, "norm.weight", t.final_norm, {H});
  return c;
}

constexpr int kMtpTensors = 31;  // MtpRunner::load (runner.rs:2452-2457)

// slot() checks of every entry: q4 = U32 [out, in/8] + BF16 [out, in/64] twice.
int check_catalogue(const LisaWeightIndex* idx, const std::vector<WeightEntry>& cat) {
  for (const WeightEntry& e : cat) {
    if (e.q) {
      const uint64_t n = e.q->n, k = e.q->k;
      LISA_TRY(lisa_index_expect(idx, e.name + ".weight", LISA_DT_U32, {n, k / 8}, nullptr));
      LISA_TRY(lisa_index_expect(idx, e.name + ".scales", LISA_DT_BF16, {n, k / 64}, nullptr));
      LISA_TRY(lisa_index_expect(idx, e.name + ".biases", LISA_DT_BF16, {n, k / 64}, nullptr));
    } else {
      LISA_TRY(lisa_index_expect(idx, e.name, LISA_DT_BF16, e.shape, nullptr));
    }
  }
  return LISA_OK;
}

// Copies every entry into the planned arena: packed words and bf16 tensors as
// stored, scales and biases interleaved into the kernels' one word per group
// (scale | bias << 16).
int upload_catalogue(LisaRunner* r, const LisaWeightIndex* idx, const std::vector<WeightEntry>& cat) {
  std::vector<uint32_t> sb;
  for (const WeightEntry& e : cat) {
    if (e.q) {
      const LisaSlotInfo *w, *s, *b;
      const uint64_t n = e.q->n, k = e.q->k;
      LISA_TRY(lisa_index_expect(idx, e.name + ".weight", LISA_DT_U32, {n, k / 8}, &w));
      LISA_TRY(lisa_index_expect(idx, e.name + ".scales", LISA_DT_BF16, {n, k / 64}, &s));
      LISA_TRY(lisa_index_expect(idx, e.name + ".biases", LISA_DT_BF16, {n, k / 64}, &b));
      LISA_TRY(lisa_hip_check(hipMemcpy(e.q->w, lisa_index_bytes(idx, *w), w->len, hipMemcpyHostToDevice),
                              "upload q4 words"));
      const uint16_t* sp = reinterpret_cast<const uint16_t*>(lisa_index_bytes(idx, *s));
      const uint16_t* bp = reinterpret_cast<const uint16_t*>(lisa_index_bytes(idx, *b));
      const size_t groups = (size_t)(n * k / 64);
      sb.resize(groups);
      for (size_t g = 0; g < groups; ++g) {
        uint16_t sv, bv;  // the mapping carries no alignment guarantee
        std::memcpy(&sv, sp + g, 2);
        std::memcpy(&bv, bp + g, 2);
        sb[g] = (uint32_t)sv | ((uint32_t)bv << 16);
      }
      LISA_TRY(lisa_hip_check(hipMemcpy(e.q->sb, sb.data(), groups * 4, hipMemcpyHostToDevice),
                              "upload q4 scales/biases"));
    } else {
      const LisaSlotInfo* v;
      LISA_TRY(lisa_index_expect(idx, e.name, LISA_DT_BF16, e.shape, &v));
      LISA_TRY(lisa_hip_check(hipMemcpy(e.vec, lisa_index_bytes(idx, *v), v->len, hipMemcpyHostToDevice),
                              "upload bf16 tensor"));
    }
  }
  return LISA_OK;
}

void plan_mtp_state(LisaRunner* r, Arena& A);

// The verification slots of live buffer k: the other two buffers, in index order.
int slot_buf(int k, int row) { return row == 0 ? (k == 0 ? 1 : 0) : (k == 2 ? 1 : 2); }

void set_live(LisaRunner* r, int k) {
  const int s0 = slot_buf(k, 0), s1 = slot_buf(k, 1);
  r->live = k;
  r->gdn_state = r->gdn_buf[k];
  r->conv_state = r->conv_buf[k];
  r->gdn_slots = r->gdn_buf[s0];
  r->conv_slots = r->conv_buf[s0];
  r->gdn_slot_stride = (uint64_t)(s1 - s0) * r->gdn_layers * LISA_GDN_STATE;
  r->conv_slot_stride = (uint64_t)(s1 - s0) * r->gdn_layers * 3 * LISA_GDN_CONV_DIM;
}

void plan_state(LisaRunner* r, Arena& A) {
  const size_t cap = (size_t)r->cfg.capacity;
  const size_t gs = (size_t)r->gdn_layers * LISA_GDN_STATE, cs = (size_t)r->gdn_layers * 3 * LISA_GDN_CONV_DIM;
  float* g = A.take<float>(3 * gs);
  uint16_t* c = A.take<uint16_t>(3 * cs);
  for (int k = 0; k < 3; ++k) {
    r->gdn_buf[k] = g ? g + k * gs : nullptr;
    r->conv_buf[k] = c ? c + k * cs : nullptr;
  }
  set_live(r, 0);
  r->key_cache = A.take<uint16_t>((size_t)r->attn_layers * LISA_ATT_KVH * cap * LISA_ATT_HD);
  r->value_cache = A.take<uint16_t>((size_t)r->attn_layers * LISA_ATT_KVH * cap * LISA_ATT_HD);
  if (r->cfg.with_mtp) plan_mtp_state(r, A);
}

// The drafter's KV caches (MtpRunner::load, runner.rs:2469-2476).
void plan_mtp_state(LisaRunner* r, Arena& A) {
  const size_t cap = (size_t)r->cfg.capacity;
  r->mtp_key = A.take<uint16_t>((size_t)LISA_ATT_KVH * cap * LISA_ATT_HD);
  r->mtp_value = A.take<uint16_t>((size_t)LISA_ATT_KVH * cap * LISA_ATT_HD);
}

void plan_ctx(LisaRunner* r, Arena& A, Ctx& c, int rows) {
  c.rows = rows;
  c.H = A.take<uint16_t>((size_t)3 * LISA_HIDDEN);
  c.B = A.take<float>((size_t)rows * LISA_HIDDEN);
  c.conv_out = A.take<float>((size_t)rows * LISA_GDN_CONV_DIM);
  c.z = A.take<float>((size_t)rows * LISA_GDN_VALUE_DIM);
  c.a = A.take<float>((size_t)rows * LISA_GDN_VH);
  c.b = A.take<float>((size_t)rows * LISA_GDN_VH);
  c.gate_ab = A.take<float>((size_t)rows * LISA_GDN_VH * LISA_GDN_GATE_FLOATS);
  c.gated = A.take<uint16_t>((size_t)rows * LISA_ATT_OUT);
  c.act = A.take<uint16_t>((size_t)rows * LISA_INTER);
  c.q_proj = A.take<float>((size_t)rows * LISA_ATT_Q_OUT);
  c.k_raw = A.take<float>((size_t)rows * LISA_ATT_KV_OUT);
  c.v_raw = A.take<float>((size_t)rows * LISA_ATT_KV_OUT);
  c.part_o = A.take<float>((size_t)rows * LISA_ATT_QH * r->s_max * LISA_ATT_HD);
  c.part_ml = A.take<float>((size_t)rows * LISA_ATT_QH * r->s_max * 2);
  c.logits = A.take<float>((size_t)rows * r->cfg.vocab);
  c.am_val = A.take<float>((size_t)rows * lm_head_grid(r));
  c.am_idx = A.take<uint32_t>((size_t)rows * lm_head_grid(r));
  c.xnorm = A.take<uint16_t>((size_t)rows * LISA_HIDDEN);
  c.cond = A.take<uint16_t>(LISA_HIDDEN);
  c.tokens = A.take<uint32_t>(4);
  c.argmax = A.take<uint32_t>(4);
  c.pos = A.take<uint32_t>(4);
  c.step = A.take<uint32_t>(4);
  c.history = A.take<uint32_t>(kHistoryCap);
  c.pf_sink = A.take<uint32_t>(64);
}

// ---- launch helpers --------------------------------------------------------------
int prof_mark(LisaRunner* r, int kind);
struct MatSpec {
  const Q4Dev* w;
  const Q4Dev* w2;  // GATEUP
  void* out;
  uint32_t kind;
};

int launch_qmv(LisaRunner* r, int m_rows, uint32_t K, LisaQmvParams& p, const std::vector<MatSpec>& mats) {
  const int ki = k_index(K);
  if (ki < 0) return lisa_fail(LISA_E_ARG, "no q4 kernel for K=%u", K);
  if (mats.empty() || mats.size() > LISA_QMV_MAX_MATS) return lisa_fail(LISA_E_ARG, "q4 launch of %zu matrices", mats.size());
  if (p.pro_mode > LISA_PRO_PRENORM) return lisa_fail(LISA_E_ARG, "bad q4 prologue mode %u", p.pro_mode);
  if (p.gate_ab && (K != LISA_HIDDEN || p.pro_mode == LISA_PRO_LOADX || !p.gate_a_w || !p.gate_a_sb ||
                    !p.gate_b_w || !p.gate_b_sb))
    return lisa_fail(LISA_E_ARG, "gate contributions need K=%u, a normalizing prologue and both gate matrices",
                     (unsigned)LISA_HIDDEN);
  LisaFunction* fn = r->qmv[m_rows == 3 ? 1 : 0][ki][p.pro_mode];
  // a launch whose matrices all share one epilogue uses the specialized kernel when there is one
  bool same_kind = !mats.empty();
  for (const MatSpec& s : mats) same_kind = same_kind && s.kind == mats[0].kind;
  if (K == LISA_HIDDEN && same_kind && mats[0].kind < 5) {
    if (LisaFunction* f = r->qmv_epi[m_rows == 3 ? 1 : 0][p.pro_mode][mats[0].kind]) fn = f;
  }
  if (!fn) return lisa_fail(LISA_E_ARG, "no q4 kernel for K=%u M=%d prologue %u", K, m_rows, p.pro_mode);
  p.n_mats = (uint32_t)mats.size();
  uint32_t tiles = 0, rows_total = 0;
  for (size_t e = 0; e < mats.size(); ++e) {
    const MatSpec& s = mats[e];
    if (s.w->k != K) return lisa_fail(LISA_E_ARG, "q4 launch mixes K");
    LisaQ4Mat& m = p.mats[e];
    m.w = s.w->w;
    m.sb = s.w->sb;
    m.w2 = s.w2 ? s.w2->w : nullptr;
    m.sb2 = s.w2 ? s.w2->sb : nullptr;
    m.out = s.out;
    m.rows = s.w->n;
    m.kind = s.kind;
    p.tile_start[e] = tiles;
    const bool pair = s.kind == LISA_EPI_GATEUP;
    tiles += pair ? (s.w->n + 3) / 4 : (s.w->n + 7) / 8;
    rows_total += pair ? 2 * s.w->n : s.w->n;
  }
  p.tile_start[mats.size()] = tiles;
  (void)rows_total;
  p.ksplit = qmv_split(K) ? 4 : 1;
  uint32_t kinds[LISA_QMV_MAX_MATS];
  for (size_t e = 0; e < mats.size(); ++e) kinds[e] = mats[e].kind;
  const LisaQmvShape sh = lisa_qmv_shape(K, m_rows, p.pro_mode, kinds, (int)mats.size(), tiles, p.gate_ab != nullptr,
                                         p.am_val != nullptr);
  const int mi = m_rows == 3 ? 1 : 0;
  switch (sh.family) {
    case LISA_QMV_GATEUP_WIDE: fn = r->qmv_gateup_wide[mi]; break;
    case LISA_QMV_INPROJ_WIDE: fn = r->qmv_inproj_wide[mi][sh.nw - 7]; break;
    case LISA_QMV_X_WIDE: fn = r->qmv_x_wide; break;
    default: break;
  }
  return lisa_launch(r->dev, fn, &p, sizeof p, sh.grid, 1, 1, sh.block, 1, 1);
}

// Consumer of the residual rows: x = RMSNorm(c.H), the statistic from 8-row
// tile partials of the updated rows.
LisaQmvParams pro_prenorm(Ctx& c, const uint16_t* w) {
  LisaQmvParams p{};
  p.pro_mode = LISA_PRO_PRENORM;
  p.h_in = c.H;
  p.norm_w = w;
  return p;
}

// Producer of the residual rows: c.H += y (bf16 residual add, runner.rs
// encode_residual).
int launch_resid(LisaRunner* r, Ctx& c, int m, uint32_t K, const uint16_t* x, const Q4Dev& w) {
  LisaQmvParams p{};
  p.pro_mode = LISA_PRO_LOADX;
  p.x_in = x;
  p.h_in = c.H;
  return launch_qmv(r, m, K, p, {{&w, nullptr, nullptr, LISA_EPI_RESID}});
}

// `slices`: the partial grid (att_slices); slices past the context exit.
int launch_attention(LisaRunner* r, Ctx& c, int m, uint32_t slices, const uint16_t* qn, const uint16_t* kn,
                     uint16_t* kc, uint16_t* vc) {
  LisaAttnParams a{};
  a.q_proj = c.q_proj;
  a.k_raw = c.k_raw;
  a.v_raw = c.v_raw;
  a.q_norm_w = qn;
  a.k_norm_w = kn;
  a.key_cache = kc;
  a.value_cache = vc;
  a.part_o = c.part_o;
  a.part_ml = c.part_ml;
  a.pos = c.pos;
  a.gated = c.gated;
  a.capacity = (uint32_t)r->cfg.capacity;
  a.s_max = r->s_max;
  const int mi = m == 3 ? 1 : 0;
  LISA_TRY(prof_mark(r, LISA_KIND_ATTN_PARTIAL));
  if (slices == 0 || slices > r->s_max) return lisa_fail(LISA_E_ARG, "attention grid of %u slices", slices);
  LISA_TRY(lisa_launch(r->dev, r->attn_part[mi], &a, sizeof a, slices, LISA_ATT_KVH, 1, LISA_ATT_PARTIAL_THREADS(m),
                       1, 1));
  LISA_TRY(prof_mark(r, LISA_KIND_ATTN_MERGE));
  return lisa_launch(r->dev, r->attn_merge[mi], &a, sizeof a, LISA_ATT_QH, m, 1, 256, 1, 1);
}

int launch_mlp(LisaRunner* r, Ctx& c, int m, const uint16_t* post_norm, const Q4Dev& gate, const Q4Dev& up,
               const Q4Dev& down) {
  LisaQmvParams p = pro_prenorm(c, post_norm);
  LISA_TRY(prof_mark(r, LISA_KIND_MLP_GATE_UP));
  LISA_TRY(launch_qmv(r, m, LISA_HIDDEN, p, {{&gate, &up, c.act, LISA_EPI_GATEUP}}));
  LISA_TRY(prof_mark(r, LISA_KIND_MLP_DOWN));
  return launch_resid(r, c, m, LISA_INTER, c.act, down);
}

// Final norm + lm_head; x_out (nullable) receives the normalized rows. The
// hidden rows (before the final norm) are c.H.
int launch_lm_head(LisaRunner* r, Ctx& c, int m, const uint16_t* norm, uint16_t* x_out) {
  LisaQmvParams p = pro_prenorm(c, norm);
  p.x_out = x_out;
  p.am_val = c.am_val;
  p.am_idx = c.am_idx;
  return launch_qmv(r, m, LISA_HIDDEN, p, {{&r->head, nullptr, c.logits, LISA_EPI_ARGMAX}});
}

int launch_finalize(LisaRunner* r, Ctx& c, int m, bool feedback, uint32_t advance) {
  LisaFinalizeParams f{};
  f.am_val = c.am_val;
  f.am_idx = c.am_idx;
  f.argmax_out = c.argmax;
  f.next_token = feedback ? c.tokens : nullptr;
  f.history = feedback ? c.history : nullptr;
  f.step = feedback ? c.step : nullptr;
  f.pos = c.pos;
  f.n_part = (uint32_t)lm_head_grid(r);
  f.m_rows = (uint32_t)m;
  f.pos_advance = advance;
  f.history_cap = kHistoryCap;
  return lisa_launch(r->dev, r->finalize, &f, sizeof f, 1, 1, 1, 1024, 1, 1);
}

// One target forward of m rows (runner.rs:555-591 for m=1, 866-909 for m=3).
// prof_mark(kind) is recorded before each launch (and a final -1 mark after
// the last) when an eager profile step is running.
// `slices`: attention slices per launch (att_slices of the last row's position).
int encode_target(LisaRunner* r, int m, bool capture, bool feedback, uint32_t slices) {
  Ctx& c = r->tgt;
  const float inv = 1.0f / lisa_sqrt((float)LISA_GDN_HD);  // runner.rs:1316-1317
  for (int i = 0; i < r->cfg.layers; ++i) {
    const LayerDev& l = r->layers[i];
    LisaQmvParams p{};
    if (i == 0) {
      p.pro_mode = LISA_PRO_EMBED;
      p.tokens = c.tokens;
      p.emb_w = r->embed.w;
      p.emb_sb = r->embed.sb;
      p.norm_w = l.input_norm;
      p.r_out = c.H;
    } else {
      p = pro_prenorm(c, l.input_norm);
    }
    if (!l.attention) {
      const int si = l.state_index;
      p.conv_w = l.conv_w;
      p.conv_state = r->conv_state + (size_t)si * 3 * LISA_GDN_CONV_DIM;
      p.conv_slots = capture ? r->conv_slots + (size_t)si * 3 * LISA_GDN_CONV_DIM : nullptr;
      p.conv_slot_stride = r->conv_slot_stride;
      p.capture = capture ? 1 : 0;
      // a and b leave the tile list: the first 48 workgroups form their group
      // contributions, which the recurrence sums (512 workgroups, not 515)
      p.gate_a_w = l.a.w;
      p.gate_a_sb = l.a.sb;
      p.gate_b_w = l.b.w;
      p.gate_b_sb = l.b.sb;
      p.gate_ab = c.gate_ab;
      LISA_TRY(prof_mark(r, LISA_KIND_GDN_IN));
      LISA_TRY(launch_qmv(r, m, LISA_HIDDEN, p,
                          {{&l.qkv, nullptr, c.conv_out, LISA_EPI_CONV}, {&l.z, nullptr, c.z, LISA_EPI_STORE}}));
      LisaGdnParams g{};
      g.conv_out = c.conv_out;
      g.z = c.z;
      g.gate_ab = c.gate_ab;
      g.a_log = l.a_log;
      g.dt_bias = l.dt_bias;
      g.norm_w = l.gnorm;
      g.state = r->gdn_state + (size_t)si * LISA_GDN_STATE;
      g.slots = capture ? r->gdn_slots + (size_t)si * LISA_GDN_STATE : nullptr;
      g.slot_stride = r->gdn_slot_stride;
      g.gated = c.gated;
      g.q_scale = inv * inv;
      g.k_scale = inv;
      g.capture = capture ? 1 : 0;
      // more workgroups per XCD load the out_proj's 640 tiles (4 each at most)
      // into the L2 that its workgroups will read them from
      uint32_t grid = LISA_GDN_VH;
      if (r->l2_prefetch) {
        g.pf_w = l.out.w;
        g.pf_sb = l.out.sb;
        g.pf_sink = c.pf_sink;
        g.pf_tiles = l.out.n / 8;
        g.pf_k = l.out.k;
        g.pf_delay = r->l2_prefetch_delay;
        grid += 8 * r->l2_prefetch;
        if (g.pf_tiles > 32 * r->l2_prefetch || l.out.k % 64 != 0 || l.out.k > 7168)
          return lisa_fail(LISA_E_ARG, "out_proj of %u x %u does not fit the prefetch workgroups", l.out.n, l.out.k);
      }
      LISA_TRY(prof_mark(r, LISA_KIND_GDN_RECURRENCE));
      LISA_TRY(lisa_launch(r->dev, r->gdn[m == 3 ? 1 : 0], &g, sizeof g, grid, 1, 1, 512, 1, 1));
      LISA_TRY(prof_mark(r, LISA_KIND_GDN_OUT));
      LISA_TRY(launch_resid(r, c, m, LISA_GDN_VALUE_DIM, c.gated, l.out));
    } else {
      LISA_TRY(prof_mark(r, LISA_KIND_ATTN_IN));
      LISA_TRY(launch_qmv(r, m, LISA_HIDDEN, p,
                          {{&l.q, nullptr, c.q_proj, LISA_EPI_STORE},
                           {&l.k, nullptr, c.k_raw, LISA_EPI_STORE},
                           {&l.v, nullptr, c.v_raw, LISA_EPI_STORE}}));
      const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * r->cfg.capacity * LISA_ATT_HD;
      LISA_TRY(launch_attention(r, c, m, slices, l.q_norm, l.k_norm, r->key_cache + off, r->value_cache + off));
      LISA_TRY(prof_mark(r, LISA_KIND_ATTN_OUT));
      LISA_TRY(launch_resid(r, c, m, LISA_ATT_OUT, c.gated, l.o));
    }
    LISA_TRY(launch_mlp(r, c, m, l.post_norm, l.gate, l.up, l.down));
  }
  LISA_TRY(prof_mark(r, LISA_KIND_LM_HEAD));
  LISA_TRY(launch_lm_head(r, c, m, r->final_norm, nullptr));
  LISA_TRY(prof_mark(r, LISA_KIND_FINALIZE));
  LISA_TRY(launch_finalize(r, c, m, feedback, (uint32_t)m));
  return prof_mark(r, -1);
}

// MTP drafter step (runner.rs:2711-2765, attention/MLP encoders :3097-3271).
int encode_mtp(LisaRunner* r, const uint16_t* cond, uint32_t slices) {
  Ctx& c = r->drf;
  const MtpDev& t = r->mtp;
  LisaQmvParams p{};
  p.pro_mode = LISA_PRO_MTPFC;
  p.tokens = c.tokens;
  p.emb_w = r->embed.w;
  p.emb_sb = r->embed.sb;
  p.norm_w = t.pre_fc_emb;
  p.norm_w2 = t.pre_fc_hid;
  p.x_in = cond;
  LISA_TRY(launch_qmv(r, 1, 2 * LISA_HIDDEN, p, {{&t.fc, nullptr, c.B, LISA_EPI_STORE}}));
  LisaQmvParams q{};
  q.pro_mode = LISA_PRO_CAST;  // f32_to_bf16 of the fc output (norm.metal:132-137)
  q.o_in = c.B;
  q.norm_w = t.input_norm;
  q.r_out = c.H;
  LISA_TRY(launch_qmv(r, 1, LISA_HIDDEN, q,
                      {{&t.q, nullptr, c.q_proj, LISA_EPI_STORE},
                       {&t.k, nullptr, c.k_raw, LISA_EPI_STORE},
                       {&t.v, nullptr, c.v_raw, LISA_EPI_STORE}}));
  LISA_TRY(launch_attention(r, c, 1, slices, t.q_norm, t.k_norm, r->mtp_key, r->mtp_value));
  LISA_TRY(launch_resid(r, c, 1, LISA_ATT_OUT, c.gated, t.o));
  LISA_TRY(launch_mlp(r, c, 1, t.post_norm, t.gate, t.up, t.down));
  LISA_TRY(launch_lm_head(r, c, 1, t.final_norm, c.xnorm));
  return launch_finalize(r, c, 1, false, 1);
}

// Launch-kind tags of the per-kernel profile (LISA_KIND_* in lisa_hip.h).
// Tags the launches that follow (until the next mark) with a profile kind.
int prof_mark(LisaRunner* r, int kind) {
  r->dev->prof_kind = kind;
  return LISA_OK;
}

int write_pos(LisaRunner* r, Ctx& c, uint32_t pos) {
  return lisa_hip_check(hipMemcpyAsync(c.pos, &pos, 4, hipMemcpyHostToDevice, r->dev->stream), "H2D pos");
}

int read_hidden(LisaRunner* r, const uint16_t* src, int rows, float* out) {
  std::vector<uint16_t> h((size_t)rows * LISA_HIDDEN);
  LISA_TRY(lisa_hip_check(
      hipMemcpyAsync(h.data(), src, h.size() * 2, hipMemcpyDeviceToHost, r->dev->stream), "D2H hidden"));
  LISA_TRY(sync(r));
  for (size_t i = 0; i < h.size(); ++i) out[i] = lisa_bf16_to_f32(h[i]);
  return LISA_OK;
}

int check_token(const LisaRunner* r, uint32_t token) {
  if (token >= (uint32_t)r->cfg.vocab) return lisa_fail(LISA_E_VOCAB, "token %u is outside vocabulary", token);
  return LISA_OK;
}

// The graph of `cache` under `key`, captured from encode() on first use.
// Every captured launch reads its token, position and state through device
// buffers, so a replay serves every call whose attention context fits the
// slice bucket the graph was captured with.
template <class Encode>
int cached_graph(LisaRunner* r, std::map<uint32_t, LisaGraph*>& cache, uint32_t key, Encode encode,
                 LisaGraph** out) {
  auto it = cache.find(key);
  if (it != cache.end()) {
    *out = it->second;
    return LISA_OK;
  }
  LISA_TRY(lisa_capture_begin(r->dev));
  const int rc = encode();
  LisaGraph* g = nullptr;
  const int re = lisa_capture_end(r->dev, &g);
  if (rc) {
    if (g) lisa_graph_free(g);
    return rc;
  }
  LISA_TRY(re);
  cache[key] = g;
  *out = g;
  return LISA_OK;
}

// The captured M=1 step (device-side token/position feedback) that covers
// position `pos`: recorded on first use for its slice bucket.
int step_graph_for(LisaRunner* r, uint32_t pos, LisaGraph** out) {
  const uint32_t slices = att_slices(r, pos, true);
  // the captured pointers name the live state buffer: one graph per buffer
  return cached_graph(r, r->step_graphs, slices * 4 + (uint32_t)r->live,
                      [&] { return encode_target(r, 1, false, true, slices); }, out);
}

// The captured M=3 verification whose last row sits at `last_pos`.
int verify_graph_for(LisaRunner* r, uint32_t last_pos, LisaGraph** out) {
  const uint32_t slices = att_slices(r, last_pos, true);
  return cached_graph(r, r->verify_graphs, slices * 4 + (uint32_t)r->live,
                      [&] { return encode_target(r, 3, true, false, slices); }, out);
}

// The captured drafter step at the drafter's position, conditioned on `cond`
// (cond_key names it: target rows 0..2, the drafter's normalized output, the
// uploaded condition).
int mtp_graph_for(LisaRunner* r, const uint16_t* cond, uint32_t cond_key, LisaGraph** out) {
  const uint32_t slices = att_slices(r, r->mtp_position, true);
  return cached_graph(r, r->mtp_graphs, cond_key << 24 | slices, [&] { return encode_mtp(r, cond, slices); }, out);
}

// The M=3 verification of the tokens in tgt.tokens at the current position
// (captured or eager); the host position advances by 3.
int launch_verify(LisaRunner* r) {
  if (r->position + 3 > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted", r->cfg.capacity);
  if (r->cfg.use_graph) {
    LisaGraph* g = nullptr;
    LISA_TRY(verify_graph_for(r, r->position + 2, &g));
    LISA_TRY(lisa_graph_launch(g, r->dev));
  } else {
    LISA_TRY(encode_target(r, 3, true, false, att_slices(r, r->position + 2, false)));
  }
  r->verify_base = r->position;
  r->position += 3;
  return LISA_OK;
}

// commit_verified_prefix's host work: the GDN and conv states of row rows - 1
// are already in their slot buffer, which becomes the live one (no device
// copy); the caller writes the device position.
int commit_enqueue(LisaRunner* r, int32_t rows) {
  if (r->verify_base < 0) return lisa_fail(LISA_E_STATE, "no pending block-3 verification");
  if (rows < 1 || rows > 3) {
    r->verify_base = -1;
    return lisa_fail(LISA_E_ARG, "verified prefix must contain 1 to 3 rows");
  }
  const uint32_t base = (uint32_t)r->verify_base;
  r->verify_base = -1;
  if (rows < 3) set_live(r, slot_buf(r->live, rows - 1));
  r->position = base + (uint32_t)rows;
  return LISA_OK;
}

// The drafter's conditioning row: target rows 0..2 (source 0), the drafter's
// own normalized output (1), the uploaded condition (2).
int mtp_cond(LisaRunner* r, int32_t cond_source, int32_t cond_row, const uint16_t** cond, uint32_t* key) {
  switch (cond_source) {
    case 0:
      if (cond_row < 0 || cond_row > 2) return lisa_fail(LISA_E_ARG, "cond_row must be 0..2");
      *cond = r->tgt.H + (size_t)cond_row * LISA_HIDDEN;
      *key = (uint32_t)cond_row;
      return LISA_OK;
    case 1: *cond = r->drf.xnorm; *key = 3; return LISA_OK;
    case 2: *cond = r->drf.cond; *key = 4; return LISA_OK;
    default: return lisa_fail(LISA_E_ARG, "bad cond_source %d", cond_source);
  }
}

int check_mtp_step(LisaRunner* r, int32_t cond_source, int32_t cond_row) {
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner was created without the MTP drafter");
  if (r->mtp_position >= (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "MTP KV capacity %d exhausted", r->cfg.capacity);
  const uint16_t* cond = nullptr;
  uint32_t key = 0;
  return mtp_cond(r, cond_source, cond_row, &cond, &key);
}

// One drafter step on the token in drf.tokens (captured or eager); the host
// position advances by 1.
int launch_mtp(LisaRunner* r, int32_t cond_source, int32_t cond_row) {
  const uint16_t* cond = nullptr;
  uint32_t key = 0;
  LISA_TRY(mtp_cond(r, cond_source, cond_row, &cond, &key));
  if (r->cfg.use_graph) {
    LisaGraph* g = nullptr;
    LISA_TRY(mtp_graph_for(r, cond, key, &g));
    LISA_TRY(lisa_graph_launch(g, r->dev));
  } else {
    LISA_TRY(encode_mtp(r, cond, att_slices(r, r->mtp_position, false)));
  }
  r->mtp_position += 1;
  return LISA_OK;
}

int do_decode(LisaRunner* r, uint32_t token, uint32_t* argmax, float* hidden, float* logits) {
  LISA_TRY(check_token(r, token));
  if (r->position >= (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted", r->cfg.capacity);
  Ctx& c = r->tgt;
  LISA_TRY(upload_u32(r, c.tokens, &token, 1));
  if (r->cfg.use_graph) {
    LisaGraph* g = nullptr;
    LISA_TRY(step_graph_for(r, r->position, &g));
    LISA_TRY(lisa_graph_launch(g, r->dev));
  } else {
    LISA_TRY(encode_target(r, 1, false, true, att_slices(r, r->position, false)));
  }
  uint32_t am = 0;
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(&am, c.argmax, 4, hipMemcpyDeviceToHost, r->dev->stream), "D2H argmax"));
  LISA_TRY(sync(r));
  if (argmax) *argmax = am;
  if (hidden) LISA_TRY(read_hidden(r, c.H, 1, hidden));
  if (logits)
    LISA_TRY(lisa_hip_check(hipMemcpy(logits, c.logits, (size_t)r->cfg.vocab * 4, hipMemcpyDeviceToHost), "D2H logits"));
  r->position += 1;
  r->verify_base = -1;
  return LISA_OK;
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================
namespace {

// Everything of a runner but its weights' contents: device, kernels, the
// planned weight arena, state, KV caches and scratch (QwenRunner::load,
// runner.rs:337-417, after the checkpoint is resolved).
int runner_init(const LisaRunnerConfig* cfg, std::unique_ptr<LisaRunner>& out) {
  if (cfg->layers <= 0 || cfg->layers % 4 != 0)
    return lisa_fail(LISA_E_ARG, "layers must be a positive multiple of 4 (got %d)", cfg->layers);
  if (cfg->vocab <= 0 || cfg->vocab % 8 != 0) return lisa_fail(LISA_E_ARG, "vocab must be a positive multiple of 8");
  if (cfg->capacity <= 0) return lisa_fail(LISA_E_ARG, "KV capacity must be greater than zero");
  if (cfg->capacity > 64 * 1024) return lisa_fail(LISA_E_ARG, "KV capacity above 65536 is not supported");
  std::unique_ptr<LisaRunner> r(new LisaRunner());
  r->cfg = *cfg;
  if (const char* e = std::getenv("LISA_L2_PREFETCH")) {
    const int n = std::atoi(e);
    r->l2_prefetch = n <= 0 ? 0 : (uint32_t)std::min(std::max(n, 20), 26);
  }
  if (const char* e = std::getenv("LISA_L2_PREFETCH_DELAY")) r->l2_prefetch_delay = (uint32_t)std::min(std::max(std::atoi(e), 0), 64);
  LISA_TRY(lisa_device_create(cfg->device, &r->dev));
  LISA_TRY(lisa_module_load_default(r->dev, &r->mod));
  // lisa_qmv_k<K>_m<M>_<prologue>; combinations the module does not hold stay null
  static const char* knames[5] = {"5120", "6144", "10240", "17408", "1024"};
  static const char* pnames[7] = {"x", "resnorm", "embed", "cast", "norm", "mtpfc", "prenorm"};
  for (int mi = 0; mi < 2; ++mi)
    for (int ki = 0; ki < 5; ++ki)
      for (int pi = 0; pi < 7; ++pi) {
        const std::string name = std::string("lisa_qmv_k") + knames[ki] + (mi ? "_m3_" : "_m1_") + pnames[pi];
        hipFunction_t hf;
        if (hipModuleGetFunction(&hf, r->mod->mod, name.c_str()) == hipSuccess)
          r->qmv[mi][ki][pi] = new LisaFunction{hf, name};
        static const char* enames[5] = {"store", "gateup", "conv", "argmax", "resid"};
        for (int ei = 0; ki == 0 && ei < 5; ++ei) {
          const std::string en = name + "_" + enames[ei];
          if (hipModuleGetFunction(&hf, r->mod->mod, en.c_str()) == hipSuccess)
            r->qmv_epi[mi][pi][ei] = new LisaFunction{hf, en};
        }
      }
  (void)hipGetLastError();  // the probes of absent combinations leave an error behind
  for (int mi = 0; mi < 2; ++mi) {
    const char* sfx = mi ? "_m3" : "_m1";
    LISA_TRY(lisa_function_get(r->mod, (std::string("lisa_gdn_recurrence") + sfx).c_str(), &r->gdn[mi]));
    LISA_TRY(lisa_function_get(r->mod, (std::string("lisa_attn_partial") + sfx).c_str(), &r->attn_part[mi]));
    LISA_TRY(lisa_function_get(r->mod, (std::string("lisa_attn_merge") + sfx).c_str(), &r->attn_merge[mi]));
    LISA_TRY(lisa_function_get(r->mod, (std::string("lisa_qmv_k5120") + sfx + "_prenorm_gateup_wide").c_str(),
                               &r->qmv_gateup_wide[mi]));
    for (int wi = 0; wi < 2; ++wi)
      LISA_TRY(lisa_function_get(r->mod, (std::string("lisa_qmv_k5120") + sfx + "_prenorm_wide" + (wi ? "8" : "7")).c_str(),
                                 &r->qmv_inproj_wide[mi][wi]));
    if (mi == 0) LISA_TRY(lisa_function_get(r->mod, "lisa_qmv_k5120_m1_x_wide9", &r->qmv_x_wide));
  }
  LISA_TRY(lisa_function_get(r->mod, "lisa_step_finalize", &r->finalize));
  LISA_TRY(lisa_function_get(r->mod, "lisa_synth_fill", &r->synth));
  LISA_TRY(lisa_function_get(r->mod, "lisa_q4_gemm", &r->gemm));
  LISA_TRY(lisa_function_get(r->mod, "lisa_q4_gemm_wide", &r->gemm_wide));
  LISA_TRY(lisa_function_get(r->mod, "lisa_q4_gemm_m128", &r->gemm_m128));
  LISA_TRY(lisa_function_get(r->mod, "lisa_q4_gemm_swiglu", &r->gemm_swiglu));
  LISA_TRY(lisa_function_get(r->mod, "lisa_rows", &r->rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_gdn_conv_rows", &r->conv_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_gdn_prep_rows", &r->gdn_prep_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_gdn_scan_rows", &r->gdn_scan_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_gdn_out_rows", &r->gdn_out_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_attn_store_rows", &r->attn_store_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_attn_partial_rows", &r->attn_partial_rows));
  LISA_TRY(lisa_function_get(r->mod, "lisa_attn_merge_rows", &r->attn_merge_rows));
  r->s_max = ((uint32_t)cfg->capacity + LISA_ATT_SLICE - 1) / LISA_ATT_SLICE;

  Arena wa;
  plan_weights(r.get(), wa);
  LISA_TRY(lisa_buffer_alloc(r->dev, wa.used, &r->weights));
  wa.base = (char*)r->weights->ptr;
  wa.used = 0;
  plan_weights(r.get(), wa);

  Arena sa;
  plan_state(r.get(), sa);
  LISA_TRY(lisa_buffer_alloc(r->dev, sa.used, &r->state));
  sa.base = (char*)r->state->ptr;
  sa.used = 0;
  plan_state(r.get(), sa);

  Arena xa;
  plan_ctx(r.get(), xa, r->tgt, 3);
  plan_ctx(r.get(), xa, r->drf, 1);
  LISA_TRY(lisa_buffer_alloc(r->dev, xa.used, &r->scratch));
  xa.base = (char*)r->scratch->ptr;
  xa.used = 0;
  plan_ctx(r.get(), xa, r->tgt, 3);
  plan_ctx(r.get(), xa, r->drf, 1);

  out = std::move(r);
  return LISA_OK;
}

// The weight plan of a runner of this geometry without a device (pointers
// null): the catalogue's shapes for host-only validation.
void plan_host(LisaRunner& r, int32_t layers, int32_t vocab, bool mtp) {
  r.cfg.layers = layers;
  r.cfg.vocab = vocab;
  r.cfg.with_mtp = mtp ? 1 : 0;
  Arena a;
  plan_weights(&r, a);
}

struct IndexCloser {
  void operator()(LisaWeightIndex* i) const { lisa_weight_index_free(i); }
};
using IndexPtr = std::unique_ptr<LisaWeightIndex, IndexCloser>;

int check_geometry(int32_t layers, int32_t vocab) {
  if (layers <= 0 || layers % 4 != 0) return lisa_fail(LISA_E_ARG, "layers must be a positive multiple of 4 (got %d)", layers);
  if (vocab <= 0 || vocab % 8 != 0) return lisa_fail(LISA_E_ARG, "vocab must be a positive multiple of 8");
  return LISA_OK;
}

// Clears the target's and the drafter's state (defined with the reset entry points).
int reset_all(LisaRunner* r);

}  // namespace

extern "C" int lisa_runner_create(const LisaRunnerConfig* cfg, LisaRunner** out) {
  if (!cfg || !out) return lisa_fail(LISA_E_ARG, "lisa_runner_create: null argument");
  std::unique_ptr<LisaRunner> r;
  LISA_TRY(runner_init(cfg, r));
  LISA_TRY(generate_weights(r.get()));
  LISA_TRY(reset_all(r.get()));
  *out = r.release();
  return LISA_OK;
}

extern "C" int lisa_weight_index_validate(const LisaWeightIndex* idx, int32_t layers, int32_t vocab, int32_t mtp) {
  if (!idx) return lisa_fail(LISA_E_ARG, "lisa_weight_index_validate: null index");
  layers = layers ? layers : LISA_LAYERS;
  vocab = vocab ? vocab : LISA_VOCAB;
  LISA_TRY(check_geometry(layers, vocab));
  LisaRunner plan;
  plan_host(plan, layers, vocab, mtp != 0);
  if (mtp) {
    const int32_t n = lisa_weight_index_len(idx);
    if (n != kMtpTensors)
      return lisa_fail(LISA_E_ARG, "invalid MTP checkpoint: found %d tensors, expected %d", n, kMtpTensors);
    return check_catalogue(idx, mtp_catalogue(&plan));
  }
  return check_catalogue(idx, target_catalogue(&plan));
}

extern "C" int lisa_runner_load(const char* target_snapshot, const char* mtp_snapshot, const LisaRunnerConfig* cfg,
                                LisaRunner** out) {
  if (!target_snapshot || !cfg || !out) return lisa_fail(LISA_E_ARG, "lisa_runner_load: null argument");
  if (cfg->capacity <= 0) return lisa_fail(LISA_E_ARG, "KV capacity must be greater than zero");
  LisaRunnerConfig c = *cfg;
  c.layers = c.layers ? c.layers : LISA_LAYERS;
  c.vocab = c.vocab ? c.vocab : LISA_VOCAB;
  c.with_mtp = mtp_snapshot ? 1 : 0;
  c.seed = 0;
  LISA_TRY(check_geometry(c.layers, c.vocab));
  LisaWeightIndex* raw = nullptr;
  LISA_TRY(lisa_weight_index_open_snapshot(target_snapshot, &raw));
  IndexPtr tgt(raw);
  LISA_TRY(lisa_weight_index_validate(tgt.get(), c.layers, c.vocab, 0));
  IndexPtr drf;
  if (mtp_snapshot) {
    raw = nullptr;
    LISA_TRY(lisa_weight_index_open_snapshot(mtp_snapshot, &raw));
    drf.reset(raw);
    LISA_TRY(lisa_weight_index_validate(drf.get(), c.layers, c.vocab, 1));
  }
  std::unique_ptr<LisaRunner> r;
  LISA_TRY(runner_init(&c, r));
  LISA_TRY(upload_catalogue(r.get(), tgt.get(), target_catalogue(r.get())));
  if (drf) LISA_TRY(upload_catalogue(r.get(), drf.get(), mtp_catalogue(r.get())));
  LISA_TRY(reset_all(r.get()));
  *out = r.release();
  return LISA_OK;
}

extern "C" int lisa_mtp_load(LisaRunner* r, const char* mtp_snapshot, int32_t capacity) {
  if (!r || !mtp_snapshot) return lisa_fail(LISA_E_ARG, "lisa_mtp_load: null argument");
  if (capacity <= 0) return lisa_fail(LISA_E_ARG, "MTP KV capacity must be greater than zero");
  if (capacity != r->cfg.capacity)
    return lisa_fail(LISA_E_ARG, "MTP KV capacity %d differs from the target's %d", capacity, r->cfg.capacity);
  if (r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner already holds an MTP drafter");
  LisaWeightIndex* raw = nullptr;
  LISA_TRY(lisa_weight_index_open_snapshot(mtp_snapshot, &raw));
  IndexPtr drf(raw);
  LISA_TRY(lisa_weight_index_validate(drf.get(), r->cfg.layers, r->cfg.vocab, 1));
  Arena wa;
  plan_mtp_weights(r, wa);
  Arena ka;
  plan_mtp_state(r, ka);
  LisaBuffer *wb = nullptr, *kb = nullptr;
  LISA_TRY(lisa_buffer_alloc(r->dev, wa.used, &wb));
  if (int rc = lisa_buffer_alloc(r->dev, ka.used, &kb)) {
    lisa_buffer_free(wb);
    return rc;
  }
  wa.base = (char*)wb->ptr;
  wa.used = 0;
  plan_mtp_weights(r, wa);
  ka.base = (char*)kb->ptr;
  ka.used = 0;
  plan_mtp_state(r, ka);
  r->mtp_weights = wb;
  r->mtp_state = kb;
  r->cfg.with_mtp = 1;
  int rc = upload_catalogue(r, drf.get(), mtp_catalogue(r));
  if (!rc) rc = lisa_hip_check(hipMemsetAsync(kb->ptr, 0, kb->len, r->dev->stream), "memset MTP KV");
  if (!rc) rc = write_pos(r, r->drf, 0);
  if (!rc) rc = sync(r);
  if (rc) {
    r->cfg.with_mtp = 0;
    r->mtp = MtpDev{};
    r->mtp_key = r->mtp_value = nullptr;
    r->mtp_weights = r->mtp_state = nullptr;
    lisa_buffer_free(wb);
    lisa_buffer_free(kb);
    return rc;
  }
  r->mtp_position = 0;
  return LISA_OK;
}

extern "C" void lisa_runner_free(LisaRunner* r) {
  if (!r) return;
  if (r->dev) (void)hipStreamSynchronize(r->dev->stream);
  for (auto* m : {&r->step_graphs, &r->verify_graphs, &r->mtp_graphs})
    for (auto& kv : *m) lisa_graph_free(kv.second);
  if (r->pinned) (void)hipHostFree(r->pinned);
  for (auto& a : r->qmv)
    for (auto& b : a)
      for (LisaFunction* f : b) delete f;
  for (auto& a : r->qmv_epi)
    for (auto& b : a)
      for (LisaFunction* f : b) delete f;
  for (LisaFunction* f : {r->gdn[0], r->gdn[1], r->attn_part[0], r->attn_part[1], r->attn_merge[0], r->attn_merge[1],
                          r->qmv_gateup_wide[0], r->qmv_gateup_wide[1], r->qmv_inproj_wide[0][0],
                          r->qmv_inproj_wide[0][1], r->qmv_inproj_wide[1][0], r->qmv_inproj_wide[1][1], r->qmv_x_wide,
                          r->finalize, r->synth, r->gemm, r->gemm_m128, r->gemm_wide, r->gemm_swiglu, r->rows, r->conv_rows, r->gdn_prep_rows, r->gdn_scan_rows, r->gdn_out_rows, r->attn_store_rows,
                          r->attn_partial_rows, r->attn_merge_rows})
    delete f;
  lisa_buffer_free(r->pf.buf);
  lisa_buffer_free(r->scratch);
  lisa_buffer_free(r->state);
  lisa_buffer_free(r->weights);
  lisa_buffer_free(r->mtp_state);
  lisa_buffer_free(r->mtp_weights);
  lisa_module_free(r->mod);
  lisa_device_free(r->dev);
  delete r;
}

extern "C" LisaDevice* lisa_runner_device(LisaRunner* r) { return r ? r->dev : nullptr; }
extern "C" uint32_t lisa_runner_position(LisaRunner* r) { return r ? r->position : 0; }
extern "C" uint64_t lisa_runner_weight_bytes(LisaRunner* r) { return r && r->weights ? r->weights->len : 0; }

namespace {

// The target's recurrent state, verify slots and K/V caches: one contiguous
// range of the state arena (plan_state), zeroed and the position rewound.
int clear_target(LisaRunner* r) {
  const size_t kv = (size_t)r->attn_layers * LISA_ATT_KVH * (size_t)r->cfg.capacity * LISA_ATT_HD;
  char* lo = reinterpret_cast<char*>(r->gdn_buf[0]);
  char* hi = reinterpret_cast<char*>(r->value_cache + kv);
  LISA_TRY(lisa_hip_check(hipMemsetAsync(lo, 0, (size_t)(hi - lo), r->dev->stream), "memset state"));
  LISA_TRY(write_pos(r, r->tgt, 0));
  r->position = 0;
  r->verify_base = -1;
  return LISA_OK;
}

// The drafter's K/V caches (in the state arena of a runner created with the
// drafter, in their own arena after lisa_mtp_load) and its position.
int clear_drafter(LisaRunner* r) {
  const size_t kv = (size_t)LISA_ATT_KVH * (size_t)r->cfg.capacity * LISA_ATT_HD * sizeof(uint16_t);
  LISA_TRY(lisa_hip_check(hipMemsetAsync(r->mtp_key, 0, kv, r->dev->stream), "memset MTP keys"));
  LISA_TRY(lisa_hip_check(hipMemsetAsync(r->mtp_value, 0, kv, r->dev->stream), "memset MTP values"));
  LISA_TRY(write_pos(r, r->drf, 0));
  r->mtp_position = 0;
  return LISA_OK;
}

// Both halves: a new runner, a loaded one, a synthetic context.
int reset_all(LisaRunner* r) {
  LISA_TRY(clear_target(r));
  if (r->cfg.with_mtp) LISA_TRY(clear_drafter(r));
  return sync(r);
}

}  // namespace

// QwenRunner::reset_state (runner.rs:423-444) clears the target's GDN, conv
// and K/V state only; the drafter keeps its caches and position.
extern "C" int lisa_runner_reset_state(LisaRunner* r) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  LISA_TRY(clear_target(r));
  return sync(r);
}

// MtpRunner::reset_state (runner.rs:2508-2520): the drafter's K/V and position.
extern "C" int lisa_mtp_reset_state(LisaRunner* r) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner holds no MTP drafter");
  LISA_TRY(clear_drafter(r));
  return sync(r);
}

extern "C" int lisa_runner_fill_state(LisaRunner* r, uint32_t filled, uint64_t seed) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  if (filled > (uint32_t)r->cfg.capacity) return lisa_fail(LISA_E_CAPACITY, "fill beyond KV capacity");
  LISA_TRY(reset_all(r));
  const uint32_t cap = (uint32_t)r->cfg.capacity;
  for (int i = 0; i < r->cfg.layers; ++i) {
    const LayerDev& l = r->layers[i];
    const int sc = i + 1;
    if (!l.attention) {
      LISA_TRY(fill(r, r->gdn_state + (size_t)l.state_index * LISA_GDN_STATE, LISA_GDN_STATE, LISA_FILL_F32,
                    lisa_stream_key(seed, lisa_tensor_id(sc, LISA_T_GDN_STATE, 0)), 0, LISA_DIST_NORMAL, 0.0f, 0.01f));
      LISA_TRY(fill(r, r->conv_state + (size_t)l.state_index * 3 * LISA_GDN_CONV_DIM, 3 * LISA_GDN_CONV_DIM,
                    LISA_FILL_BF16, lisa_stream_key(seed, lisa_tensor_id(sc, LISA_T_CONV_STATE, 0)), 0,
                    LISA_DIST_NORMAL, 0.0f, 1.0f));
    } else if (filled) {
      const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * cap * LISA_ATT_HD;
      const uint64_t n = (uint64_t)LISA_ATT_KVH * filled * LISA_ATT_HD;
      LISA_TRY(fill(r, r->key_cache + off, n, LISA_FILL_KV, lisa_stream_key(seed, lisa_tensor_id(sc, LISA_T_KEY_CACHE, 0)),
                    0, 0, 0, 0, cap, filled));
      LISA_TRY(fill(r, r->value_cache + off, n, LISA_FILL_KV,
                    lisa_stream_key(seed, lisa_tensor_id(sc, LISA_T_VALUE_CACHE, 0)), 0, 0, 0, 0, cap, filled));
    }
  }
  if (r->cfg.with_mtp && filled) {
    const uint64_t n = (uint64_t)LISA_ATT_KVH * filled * LISA_ATT_HD;
    LISA_TRY(fill(r, r->mtp_key, n, LISA_FILL_KV, lisa_stream_key(seed, lisa_tensor_id(LISA_SCOPE_MTP, LISA_T_KEY_CACHE, 0)),
                  0, 0, 0, 0, cap, filled));
    LISA_TRY(fill(r, r->mtp_value, n, LISA_FILL_KV,
                  lisa_stream_key(seed, lisa_tensor_id(LISA_SCOPE_MTP, LISA_T_VALUE_CACHE, 0)), 0, 0, 0, 0, cap, filled));
  }
  LISA_TRY(write_pos(r, r->tgt, filled));
  LISA_TRY(write_pos(r, r->drf, r->cfg.with_mtp ? filled : 0));
  LISA_TRY(sync(r));
  r->position = filled;
  r->mtp_position = r->cfg.with_mtp ? filled : 0;
  return LISA_OK;
}

extern "C" int lisa_runner_forward_token_decode(LisaRunner* r, uint32_t token, uint32_t* argmax, float* hidden) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  return do_decode(r, token, argmax, hidden, nullptr);
}

extern "C" int lisa_runner_forward_token_with_hidden(LisaRunner* r, uint32_t token, uint32_t* argmax, float* hidden,
                                                     float* logits) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  return do_decode(r, token, argmax, hidden, logits);
}

extern "C" int lisa_runner_decode_greedy(LisaRunner* r, uint32_t token, int32_t steps, uint32_t* tokens_out) {
  if (!r || steps < 0 || (steps && !tokens_out)) return lisa_fail(LISA_E_ARG, "lisa_runner_decode_greedy: bad argument");
  if (!steps) return LISA_OK;
  LISA_TRY(check_token(r, token));
  if (r->position + (uint32_t)steps > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted by %d steps", r->cfg.capacity, steps);
  if ((uint32_t)steps > kHistoryCap) return lisa_fail(LISA_E_ARG, "at most %u steps per call", kHistoryCap);
  Ctx& c = r->tgt;
  const uint32_t zero = 0;
  LISA_TRY(upload_u32(r, c.tokens, &token, 1));
  LISA_TRY(upload_u32(r, c.step, &zero, 1));
  for (int s = 0; s < steps; ++s) {
    const uint32_t pos = r->position + (uint32_t)s;
    if (r->cfg.use_graph) {
      LisaGraph* g = nullptr;
      LISA_TRY(step_graph_for(r, pos, &g));
      LISA_TRY(lisa_graph_launch(g, r->dev));
    } else {
      LISA_TRY(encode_target(r, 1, false, true, att_slices(r, pos, false)));
    }
  }
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(tokens_out, c.history, (size_t)steps * 4, hipMemcpyDeviceToHost, r->dev->stream),
                          "D2H history"));
  LISA_TRY(sync(r));
  r->position += (uint32_t)steps;
  r->verify_base = -1;
  return LISA_OK;
}

namespace {

// Timed eager passes (every launch between start/stop events attached to its
// dispatch), summed per launch kind.
int profile_pass(LisaRunner* r, int m, int32_t steps, float* kind_ms, int32_t* kind_count) {
  for (int k = 0; k < LISA_KIND_COUNT; ++k) {
    kind_ms[k] = 0.0f;
    kind_count[k] = 0;
  }
  r->prof.clear();
  r->dev->prof = &r->prof;
  int rc = LISA_OK;
  for (int s = 0; s < steps && !rc; ++s)
    rc = m == 1 ? encode_target(r, 1, false, true, att_slices(r, r->position + s, false))
                : encode_target(r, 3, true, false, att_slices(r, r->position + 2, false));
  r->dev->prof = nullptr;
  r->dev->prof_kind = -1;
  if (!rc) rc = sync(r);
  for (const LisaProfRec& rec : r->prof) {
    if (rc || rec.kind < 0 || rec.kind >= LISA_KIND_COUNT) continue;
    float ms = 0.0f;
    rc = lisa_hip_check(hipEventElapsedTime(&ms, rec.start, rec.stop), "hipEventElapsedTime");
    kind_ms[rec.kind] += ms;
    kind_count[rec.kind] += 1;
  }
  for (const LisaProfRec& rec : r->prof) {
    (void)hipEventDestroy(rec.start);
    (void)hipEventDestroy(rec.stop);
  }
  r->prof.clear();
  return rc;
}

}  // namespace

extern "C" int lisa_runner_profile_step(LisaRunner* r, uint32_t token, int32_t steps, float* kind_ms,
                                        int32_t* kind_count) {
  if (!r || steps <= 0 || !kind_ms || !kind_count) return lisa_fail(LISA_E_ARG, "lisa_runner_profile_step: bad argument");
  LISA_TRY(check_token(r, token));
  if (r->position + (uint32_t)steps > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted by %d steps", r->cfg.capacity, steps);
  LISA_TRY(upload_u32(r, r->tgt.tokens, &token, 1));
  LISA_TRY(profile_pass(r, 1, steps, kind_ms, kind_count));
  r->position += (uint32_t)steps;
  r->verify_base = -1;
  return LISA_OK;
}

extern "C" int lisa_runner_profile_block3(LisaRunner* r, const uint32_t tokens[3], float* kind_ms,
                                          int32_t* kind_count) {
  if (!r || !tokens || !kind_ms || !kind_count) return lisa_fail(LISA_E_ARG, "lisa_runner_profile_block3: bad argument");
  for (int i = 0; i < 3; ++i) LISA_TRY(check_token(r, tokens[i]));
  if (r->position + 3 > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted", r->cfg.capacity);
  LISA_TRY(upload_u32(r, r->tgt.tokens, tokens, 3));
  LISA_TRY(profile_pass(r, 3, 1, kind_ms, kind_count));
  r->verify_base = r->position;
  r->position += 3;
  return LISA_OK;
}

extern "C" int lisa_runner_verify_block3(LisaRunner* r, const uint32_t tokens[3], uint32_t argmax[3], float* hidden,
                                         float* logits) {
  if (!r || !tokens) return lisa_fail(LISA_E_ARG, "lisa_runner_verify_block3: bad argument");
  for (int i = 0; i < 3; ++i) LISA_TRY(check_token(r, tokens[i]));
  if (r->position + 3 > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted", r->cfg.capacity);
  Ctx& c = r->tgt;
  LISA_TRY(upload_u32(r, c.tokens, tokens, 3));
  LISA_TRY(launch_verify(r));
  uint32_t am[3];
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(am, c.argmax, 12, hipMemcpyDeviceToHost, r->dev->stream), "D2H argmax"));
  LISA_TRY(sync(r));
  if (argmax) std::memcpy(argmax, am, 12);
  if (hidden) LISA_TRY(read_hidden(r, c.H, 3, hidden));
  if (logits)
    LISA_TRY(lisa_hip_check(hipMemcpy(logits, c.logits, (size_t)3 * r->cfg.vocab * 4, hipMemcpyDeviceToHost),
                            "D2H logits"));
  return LISA_OK;
}

extern "C" int lisa_runner_commit_verified_prefix(LisaRunner* r, int32_t rows) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  if (r->verify_base < 0) return lisa_fail(LISA_E_STATE, "no pending block-3 verification");
  LISA_TRY(commit_enqueue(r, rows));
  LISA_TRY(write_pos(r, r->tgt, r->position));
  return sync(r);
}

extern "C" int lisa_runner_checkpoint_state(LisaRunner* r, LisaCheckpoint** out) {
  if (!r || !out) return lisa_fail(LISA_E_ARG, "lisa_runner_checkpoint_state: bad argument");
  std::unique_ptr<LisaCheckpoint> ck(new LisaCheckpoint());
  const size_t gs = (size_t)r->gdn_layers * LISA_GDN_STATE * 4, cs = (size_t)r->gdn_layers * 3 * LISA_GDN_CONV_DIM * 2;
  LISA_TRY(lisa_buffer_alloc(r->dev, gs, &ck->gdn));
  LISA_TRY(lisa_buffer_alloc(r->dev, cs, &ck->conv));
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(ck->gdn->ptr, r->gdn_state, gs, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(ck->conv->ptr, r->conv_state, cs, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  LISA_TRY(sync(r));
  ck->position = r->position;
  ck->gdn_layers = r->gdn_layers;
  *out = ck.release();
  return LISA_OK;
}

extern "C" int lisa_runner_restore_state(LisaRunner* r, const LisaCheckpoint* ck) {
  if (!r || !ck) return lisa_fail(LISA_E_ARG, "lisa_runner_restore_state: bad argument");
  if (ck->position > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "checkpoint position %u exceeds KV capacity %d", ck->position, r->cfg.capacity);
  const size_t gs = (size_t)r->gdn_layers * LISA_GDN_STATE * 4, cs = (size_t)r->gdn_layers * 3 * LISA_GDN_CONV_DIM * 2;
  if (ck->gdn_layers != r->gdn_layers || !ck->gdn || !ck->conv || ck->gdn->len != gs || ck->conv->len != cs)
    return lisa_fail(LISA_E_ARG, "checkpoint of %d GDN layers does not fit a runner of %d", ck->gdn_layers,
                     r->gdn_layers);
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(r->gdn_state, ck->gdn->ptr, ck->gdn->len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(r->conv_state, ck->conv->ptr, ck->conv->len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  r->position = ck->position;
  r->verify_base = -1;
  LISA_TRY(write_pos(r, r->tgt, r->position));
  return sync(r);
}

extern "C" void lisa_checkpoint_free(LisaCheckpoint* ck) {
  if (!ck) return;
  lisa_buffer_free(ck->gdn);
  lisa_buffer_free(ck->conv);
  delete ck;
}

extern "C" int lisa_runner_read_gdn_state(LisaRunner* r, int32_t idx, float* out) {
  if (!r || !out || idx < 0 || idx >= r->gdn_layers) return lisa_fail(LISA_E_ARG, "bad GDN layer index");
  LISA_TRY(lisa_hip_check(hipMemcpy(out, r->gdn_state + (size_t)idx * LISA_GDN_STATE, LISA_GDN_STATE * 4,
                                    hipMemcpyDeviceToHost), "D2H state"));
  return LISA_OK;
}

extern "C" int lisa_runner_read_conv_state(LisaRunner* r, int32_t idx, uint16_t* out) {
  if (!r || !out || idx < 0 || idx >= r->gdn_layers) return lisa_fail(LISA_E_ARG, "bad GDN layer index");
  LISA_TRY(lisa_hip_check(hipMemcpy(out, r->conv_state + (size_t)idx * 3 * LISA_GDN_CONV_DIM, 3 * LISA_GDN_CONV_DIM * 2,
                                    hipMemcpyDeviceToHost), "D2H conv"));
  return LISA_OK;
}

// ---- MTP drafter --------------------------------------------------------------
extern "C" int lisa_mtp_forward(LisaRunner* r, uint32_t token, int32_t cond_source, int32_t cond_row,
                                uint32_t* argmax) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner was created without the MTP drafter");
  LISA_TRY(check_token(r, token));
  LISA_TRY(check_mtp_step(r, cond_source, cond_row));
  Ctx& c = r->drf;
  LISA_TRY(upload_u32(r, c.tokens, &token, 1));
  LISA_TRY(launch_mtp(r, cond_source, cond_row));
  uint32_t am = 0;
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(&am, c.argmax, 4, hipMemcpyDeviceToHost, r->dev->stream), "D2H argmax"));
  LISA_TRY(sync(r));
  if (argmax) *argmax = am;
  return LISA_OK;
}

namespace {
int upload_bf16_trunc(LisaRunner* r, uint16_t* dst, const float* hidden) {
  std::vector<uint16_t> h(LISA_HIDDEN);
  for (int i = 0; i < LISA_HIDDEN; ++i) h[i] = lisa_f32_to_bf16_trunc(hidden[i]);
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(dst, h.data(), LISA_HIDDEN * 2, hipMemcpyHostToDevice, r->dev->stream), "H2D"));
  return sync(r);
}
}  // namespace

extern "C" int lisa_runner_upload_hidden(LisaRunner* r, int32_t row, const float* hidden) {
  if (!r || !hidden || row < 0 || row > 2) return lisa_fail(LISA_E_ARG, "lisa_runner_upload_hidden: bad argument");
  return upload_bf16_trunc(r, r->tgt.H + (size_t)row * LISA_HIDDEN, hidden);
}

extern "C" int32_t lisa_runner_vocab(LisaRunner* r) { return r ? r->cfg.vocab : 0; }

extern "C" int lisa_mtp_upload_normalized(LisaRunner* r, const float* hidden) {
  if (!r || !hidden) return lisa_fail(LISA_E_ARG, "lisa_mtp_upload_normalized: bad argument");
  return upload_bf16_trunc(r, r->drf.xnorm, hidden);
}

extern "C" int lisa_mtp_upload_cond(LisaRunner* r, const uint16_t* hidden) {
  if (!r || !hidden) return lisa_fail(LISA_E_ARG, "lisa_mtp_upload_cond: bad argument");
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(r->drf.cond, hidden, LISA_HIDDEN * 2, hipMemcpyHostToDevice, r->dev->stream), "H2D"));
  return sync(r);
}

extern "C" int lisa_mtp_read_normalized(LisaRunner* r, uint16_t* out) {
  if (!r || !out) return lisa_fail(LISA_E_ARG, "lisa_mtp_read_normalized: bad argument");
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(out, r->drf.xnorm, LISA_HIDDEN * 2, hipMemcpyDeviceToHost, r->dev->stream), "D2H"));
  return sync(r);
}

extern "C" uint32_t lisa_mtp_position(LisaRunner* r) { return r ? r->mtp_position : 0; }

extern "C" int lisa_mtp_trim_state(LisaRunner* r, int32_t count) {
  if (!r) return lisa_fail(LISA_E_ARG, "null runner");
  if (count < 0 || (uint32_t)count > r->mtp_position)
    return lisa_fail(LISA_E_ARG, "cannot trim %d MTP positions from %u", count, r->mtp_position);
  r->mtp_position -= (uint32_t)count;
  LISA_TRY(write_pos(r, r->drf, r->mtp_position));
  return sync(r);
}

// ---- stream-ordered round pieces (spec_round.h) ----------------------------
int round_pinned(LisaRunner* r, uint32_t** out) {
  if (!r->pinned) {
    void* p = nullptr;
    LISA_TRY(lisa_hip_check(hipHostMalloc(&p, ROUND_PIN_WORDS * sizeof(uint32_t), hipHostMallocDefault),
                            "hipHostMalloc round staging"));
    r->pinned = static_cast<uint32_t*>(p);
    std::memset(r->pinned, 0, ROUND_PIN_WORDS * sizeof(uint32_t));
  }
  *out = r->pinned;
  return LISA_OK;
}

namespace {
int pinned_copy(LisaRunner* r, void* dst, const void* src, size_t n, hipMemcpyKind kind, const char* what) {
  return lisa_hip_check(hipMemcpyAsync(dst, src, n, kind, r->dev->stream), what);
}
int need_pinned(LisaRunner* r) {
  return r->pinned ? LISA_OK : lisa_fail(LISA_E_STATE, "round staging not allocated");
}
}  // namespace

int round_mtp(LisaRunner* r, bool token_on_host, int32_t cond_source, int32_t cond_row) {
  LISA_TRY(need_pinned(r));
  LISA_TRY(check_mtp_step(r, cond_source, cond_row));
  Ctx& c = r->drf;
  if (token_on_host) {
    LISA_TRY(check_token(r, r->pinned[ROUND_PIN_MTP_TOKEN]));
    LISA_TRY(pinned_copy(r, c.tokens, r->pinned + ROUND_PIN_MTP_TOKEN, 4, hipMemcpyHostToDevice, "H2D token"));
  } else {
    LISA_TRY(pinned_copy(r, c.tokens, c.argmax, 4, hipMemcpyDeviceToDevice, "D2D token"));
  }
  return launch_mtp(r, cond_source, cond_row);
}

int round_forward_draft(LisaRunner* r, int slot, int host_word) {
  LISA_TRY(need_pinned(r));
  if (slot < 1 || slot > 2 || host_word >= ROUND_PIN_WORDS) return lisa_fail(LISA_E_ARG, "bad draft slot");
  LISA_TRY(pinned_copy(r, r->tgt.tokens + slot, r->drf.argmax, 4, hipMemcpyDeviceToDevice, "D2D draft"));
  if (host_word >= 0)
    LISA_TRY(pinned_copy(r, r->pinned + host_word, r->drf.argmax, 4, hipMemcpyDeviceToHost, "D2H draft"));
  return LISA_OK;
}

int round_set_verify_tokens(LisaRunner* r, int first, int n) {
  LISA_TRY(need_pinned(r));
  if (first < 0 || n < 1 || first + n > 3) return lisa_fail(LISA_E_ARG, "bad verify token range");
  for (int i = first; i < first + n; ++i) LISA_TRY(check_token(r, r->pinned[ROUND_PIN_BONUS + i]));
  return pinned_copy(r, r->tgt.tokens + first, r->pinned + ROUND_PIN_BONUS + first, 4 * (size_t)n,
                     hipMemcpyHostToDevice, "H2D verify tokens");
}

int round_verify(LisaRunner* r) {
  LISA_TRY(need_pinned(r));
  LISA_TRY(launch_verify(r));
  return pinned_copy(r, r->pinned + ROUND_PIN_TARGET, r->tgt.argmax, 12, hipMemcpyDeviceToHost, "D2H argmax");
}

int round_commit(LisaRunner* r, int32_t rows) {
  LISA_TRY(need_pinned(r));
  LISA_TRY(commit_enqueue(r, rows));
  r->pinned[ROUND_PIN_TPOS] = r->position;
  return pinned_copy(r, r->tgt.pos, r->pinned + ROUND_PIN_TPOS, 4, hipMemcpyHostToDevice, "H2D pos");
}

int round_trim(LisaRunner* r, int32_t count) {
  LISA_TRY(need_pinned(r));
  if (count < 0 || (uint32_t)count > r->mtp_position)
    return lisa_fail(LISA_E_ARG, "cannot trim %d MTP positions from %u", count, r->mtp_position);
  r->mtp_position -= (uint32_t)count;
  r->pinned[ROUND_PIN_DPOS] = r->mtp_position;
  return pinned_copy(r, r->drf.pos, r->pinned + ROUND_PIN_DPOS, 4, hipMemcpyHostToDevice, "H2D pos");
}

int round_sync(LisaRunner* r) { return sync(r); }

// MtpRunner::checkpoint_state / restore_state (runner.rs:2382-2420): the
// drafter's KV caches (device-to-device copies of the whole capacity) and its
// logical position.
extern "C" int lisa_mtp_checkpoint_state(LisaRunner* r, LisaMtpCheckpoint** out) {
  if (!r || !out) return lisa_fail(LISA_E_ARG, "lisa_mtp_checkpoint_state: bad argument");
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner was created without the MTP drafter");
  const size_t len = (size_t)LISA_ATT_KVH * r->cfg.capacity * LISA_ATT_HD * 2;
  std::unique_ptr<LisaMtpCheckpoint> ck(new LisaMtpCheckpoint());
  auto release = [](LisaMtpCheckpoint* c) {
    lisa_buffer_free(c->key);
    lisa_buffer_free(c->value);
    c->key = c->value = nullptr;
  };
  int rc = lisa_buffer_alloc(r->dev, len, &ck->key);
  if (!rc) rc = lisa_buffer_alloc(r->dev, len, &ck->value);
  if (!rc) rc = lisa_hip_check(hipMemcpyAsync(ck->key->ptr, r->mtp_key, len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D");
  if (!rc)
    rc = lisa_hip_check(hipMemcpyAsync(ck->value->ptr, r->mtp_value, len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D");
  if (!rc) rc = sync(r);
  if (rc) {
    release(ck.get());
    return rc;
  }
  ck->position = r->mtp_position;
  ck->capacity = r->cfg.capacity;
  *out = ck.release();
  return LISA_OK;
}

extern "C" int lisa_mtp_restore_state(LisaRunner* r, const LisaMtpCheckpoint* ck) {
  if (!r || !ck) return lisa_fail(LISA_E_ARG, "lisa_mtp_restore_state: bad argument");
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner was created without the MTP drafter");
  if (ck->position > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "MTP checkpoint position %u exceeds capacity %d", ck->position, r->cfg.capacity);
  const size_t len = (size_t)LISA_ATT_KVH * r->cfg.capacity * LISA_ATT_HD * 2;
  if (ck->capacity != r->cfg.capacity || !ck->key || !ck->value || ck->key->len != len || ck->value->len != len)
    return lisa_fail(LISA_E_ARG, "MTP checkpoint of capacity %d does not fit a runner of capacity %d", ck->capacity,
                     r->cfg.capacity);
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(r->mtp_key, ck->key->ptr, len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(r->mtp_value, ck->value->ptr, len, hipMemcpyDeviceToDevice, r->dev->stream), "D2D"));
  r->mtp_position = ck->position;
  LISA_TRY(write_pos(r, r->drf, r->mtp_position));
  return sync(r);
}

extern "C" void lisa_mtp_checkpoint_free(LisaMtpCheckpoint* ck) {
  if (!ck) return;
  lisa_buffer_free(ck->key);
  lisa_buffer_free(ck->value);
  delete ck;
}

// Device-resident conditioning of the drafter, as the reference addresses it:
// a (buffer, byte offset) pair. The target's hidden rows sit at
// lisa_runner_hidden_offset(row) of its scratch (hidden_offset, runner.rs:846-848);
// the drafter's own normalized hidden at lisa_mtp_normalized_offset() of its
// scratch (normalized_offset, runner.rs:2689-2692).
extern "C" uint64_t lisa_runner_hidden_offset(int32_t row) { return (uint64_t)row * LISA_HIDDEN * 2; }
extern "C" uint64_t lisa_mtp_normalized_offset(void) { return 0; }

extern "C" int lisa_mtp_resolve_cond(int32_t cond_is_target, uint64_t cond_off, int32_t* cond_source,
                                     int32_t* cond_row) {
  if (!cond_source || !cond_row) return lisa_fail(LISA_E_ARG, "lisa_mtp_resolve_cond: null output");
  if (cond_is_target) {
    const uint64_t row_bytes = (uint64_t)LISA_HIDDEN * 2;
    if (cond_off % row_bytes != 0 || cond_off / row_bytes > 2)
      return lisa_fail(LISA_E_ARG, "offset %llu is not a target hidden row", (unsigned long long)cond_off);
    *cond_source = 0;
    *cond_row = (int32_t)(cond_off / row_bytes);
    return LISA_OK;
  }
  if (cond_off != lisa_mtp_normalized_offset())
    return lisa_fail(LISA_E_ARG, "offset %llu is not the drafter's normalized hidden", (unsigned long long)cond_off);
  *cond_source = 1;
  *cond_row = 0;
  return LISA_OK;
}

extern "C" int lisa_mtp_forward_device(LisaRunner* r, uint32_t token, int32_t cond_is_target, uint64_t cond_off,
                                       uint32_t* argmax, uint64_t* normalized_off) {
  int32_t src = 0, row = 0;
  LISA_TRY(lisa_mtp_resolve_cond(cond_is_target, cond_off, &src, &row));
  LISA_TRY(lisa_mtp_forward(r, token, src, row, argmax));
  if (normalized_off) *normalized_off = lisa_mtp_normalized_offset();
  return LISA_OK;
}

// forward_position_decode (runner.rs:2618-2680): the drafter conditioned on a
// host hidden f32[5120] (uploaded as bf16 by truncation, dtype.rs:42-47);
// returns the argmax and the normalized hidden as f32.
extern "C" int lisa_mtp_forward_position_decode(LisaRunner* r, uint32_t token, const float* hidden, uint32_t* argmax,
                                                float* normalized) {
  if (!r || !hidden) return lisa_fail(LISA_E_ARG, "lisa_mtp_forward_position_decode: bad argument");
  std::vector<uint16_t> h(LISA_HIDDEN);
  for (int i = 0; i < LISA_HIDDEN; ++i) h[i] = lisa_f32_to_bf16_trunc(hidden[i]);
  LISA_TRY(lisa_mtp_upload_cond(r, h.data()));
  LISA_TRY(lisa_mtp_forward(r, token, 2, 0, argmax));
  if (normalized) LISA_TRY(read_hidden(r, r->drf.xnorm, 1, normalized));
  return LISA_OK;
}

// =============================================================================
// batched prefill: forward_prefill_with_progress (runner.rs:2129-2230)
// =============================================================================
namespace {

// Rows per prefill chunk. The reference uses 512 (PREFILL_BATCH, runner.rs:51);
// the result does not depend on the chunk (the recurrent state and the KV cache
// carry across chunks), and 2048-row GEMMs keep the matrix cores far busier.
constexpr uint32_t kPrefillRows = 2048;

void plan_prefill(LisaRunner* r, Arena& A) {
  auto& P = r->pf;
  const size_t c = kPrefillRows;
  P.tokens = A.take<uint32_t>(c);
  P.argmax = A.take<uint32_t>(c);
  P.pos = A.take<uint32_t>(c + 1);
  P.H = A.take<uint16_t>(c * LISA_HIDDEN);
  P.X = A.take<uint16_t>(c * LISA_HIDDEN);
  P.B = A.take<float>(c * LISA_HIDDEN);
  P.qkv = A.take<float>(c * LISA_GDN_CONV_DIM);
  P.conv_out = A.take<float>(c * LISA_GDN_CONV_DIM);
  P.z = A.take<float>(c * LISA_GDN_VALUE_DIM);
  P.a = A.take<float>(c * LISA_GDN_VH);
  P.b = A.take<float>(c * LISA_GDN_VH);
  P.gated = A.take<uint16_t>(c * LISA_ATT_OUT);
  P.q_proj = A.take<float>(c * LISA_ATT_Q_OUT);
  P.k_raw = A.take<float>(c * LISA_ATT_KV_OUT);
  P.v_raw = A.take<float>(c * LISA_ATT_KV_OUT);
  P.query = A.take<float>(c * LISA_ATT_OUT);
  P.act = A.take<uint16_t>(c * LISA_INTER);
  P.logits = A.take<float>(c * (size_t)r->cfg.vocab);
  P.gdn_qk = A.take<float>(c * 2 * LISA_GDN_KEY_DIM);
  P.gdn_gates = A.take<float>(c * 2 * LISA_GDN_VH);
  P.gdn_y = A.take<float>(c * LISA_GDN_VALUE_DIM);
  // slice partials of one attention sub-block: at most ~1 GiB
  const size_t per_row = (size_t)LISA_ATT_QH * r->s_max * (LISA_ATT_HD + 2) * sizeof(float);
  const uint32_t rb = LISA_ATT_ROWS_PER_WG;
  uint32_t ar = (uint32_t)std::min<size_t>(kPrefillRows, std::max<size_t>(rb, (size_t(1) << 30) / per_row));
  P.att_rows = ar / rb * rb;
  P.part_o = A.take<float>((size_t)P.att_rows * LISA_ATT_QH * r->s_max * LISA_ATT_HD);
  P.part_ml = A.take<float>((size_t)P.att_rows * LISA_ATT_QH * r->s_max * 2);
}

int ensure_prefill(LisaRunner* r) {
  if (r->pf.buf) return LISA_OK;
  Arena a;
  plan_prefill(r, a);
  LisaBuffer* buf = nullptr;
  LISA_TRY(lisa_buffer_alloc(r->dev, a.used, &buf));
  r->pf.buf = buf;
  a.base = (char*)buf->ptr;
  a.used = 0;
  plan_prefill(r, a);
  return LISA_OK;
}

// C[m][w.n] = A[m][w.k] . deq(w)^T
int launch_gemm(LisaRunner* r, const uint16_t* a, uint32_t m, const Q4Dev& w, float* c) {
  LisaGemmParams g{};
  g.a = a;
  g.w = w.w;
  g.sb = w.sb;
  g.c = c;
  g.m = m;
  g.n = w.n;
  g.k = w.k;
  g.ldc = w.n;
  // One workgroup per CU: a launch runs in rounds of `cus` tiles. A 256-wide
  // tile (eight waves) takes about 1.5x a 128-wide one; take it unless its
  // rounds cost more.
  const uint32_t gm = (m + LISA_GEMM_TILE_M - 1) / LISA_GEMM_TILE_M;
  const uint32_t gn = (w.n + LISA_GEMM_TILE_N - 1) / LISA_GEMM_TILE_N;
  const uint32_t gw = (w.n + LISA_GEMM_TILE_N_WIDE - 1) / LISA_GEMM_TILE_N_WIDE;
  const uint32_t cus = r->dev->cu_count > 0 ? (uint32_t)r->dev->cu_count : 256;
  const uint32_t rn = (gn * gm + cus - 1) / cus, rw = (gw * gm + cus - 1) / cus;
  // a projection whose 256-row tiles would fill at most half the CUs (the GDN
  // a and b, attention k and v): 128-row tiles, twice the workgroups
  if (gn * gm * 2 <= cus)
    return lisa_launch(r->dev, r->gemm_m128, &g, sizeof g, gn, (m + LISA_GEMM_TILE_M_SMALL - 1) / LISA_GEMM_TILE_M_SMALL,
                       1, 256, 1, 1);
  if (rw * 3 <= rn * 2) return lisa_launch(r->dev, r->gemm_wide, &g, sizeof g, gw, gm, 1, LISA_GEMM_THREADS_WIDE, 1, 1);
  return lisa_launch(r->dev, r->gemm, &g, sizeof g, gn, gm, 1, 256, 1, 1);
}

// act[m][gate.n] = bf16(silu(bf16(A . deq(gate)^T)) * bf16(A . deq(up)^T)) in
// one launch (the MLP's gate/up pair with the SwiGLU epilogue).
int launch_gemm_swiglu(LisaRunner* r, const uint16_t* a, uint32_t m, const Q4Dev& gate, const Q4Dev& up,
                       uint16_t* act) {
  if (gate.n != up.n || gate.k != up.k) return lisa_fail(LISA_E_ARG, "gate and up projections differ in shape");
  LisaGemmParams g{};
  g.a = a;
  g.w = gate.w;
  g.sb = gate.sb;
  g.w2 = up.w;
  g.sb2 = up.sb;
  g.act = act;
  g.m = m;
  g.n = gate.n;
  g.k = gate.k;
  g.ldc = gate.n;
  const uint32_t gm = (m + LISA_GEMM_TILE_M - 1) / LISA_GEMM_TILE_M;
  const uint32_t gn = (gate.n + LISA_GEMM_TILE_N_WIDE / 2 - 1) / (LISA_GEMM_TILE_N_WIDE / 2);
  return lisa_launch(r->dev, r->gemm_swiglu, &g, sizeof g, gn, gm, 1, LISA_GEMM_THREADS_WIDE, 1, 1);
}

int launch_rows(LisaRunner* r, LisaRowsParams& p, uint32_t gx, uint32_t m) {
  return lisa_launch(r->dev, r->rows, &p, sizeof p, gx, m, 1, 256, 1, 1);
}

int rows_norm(LisaRunner* r, uint32_t m, const uint16_t* h, const float* o, const uint16_t* w, uint16_t* r_out,
              uint16_t* x_out) {
  LisaRowsParams p{};
  p.mode = o ? LISA_ROWS_RESNORM : LISA_ROWS_NORM;
  p.h_in = h;
  p.o_in = o;
  p.norm_w = w;
  p.r_out = r_out;
  p.x_out = x_out;
  return launch_rows(r, p, 1, m);
}

// Attention over m prefill rows at positions [base, base + m) against one
// layer's caches (the rows are split into sub-blocks that bound the slice
// partials); q/k/v projections in P.q_proj / P.k_raw / P.v_raw, output P.gated.
int prefill_attention(LisaRunner* r, uint32_t m, uint32_t base, const uint16_t* qn, const uint16_t* kn, uint16_t* kc,
                      uint16_t* vc) {
  auto& P = r->pf;
  LisaAttnParams a{};
  a.q_proj = P.q_proj;
  a.k_raw = P.k_raw;
  a.v_raw = P.v_raw;
  a.q_norm_w = qn;
  a.k_norm_w = kn;
  a.key_cache = kc;
  a.value_cache = vc;
  a.part_o = P.part_o;
  a.part_ml = P.part_ml;
  a.pos = P.pos;
  a.gated = P.gated;
  a.capacity = (uint32_t)r->cfg.capacity;
  a.s_max = r->s_max;
  a.query = P.query;
  a.m_rows = m;
  LISA_TRY(lisa_launch(r->dev, r->attn_store_rows, &a, sizeof a, m, 7, 1, 256, 1, 1));
  for (uint32_t r0 = 0; r0 < m; r0 += P.att_rows) {
    const uint32_t ms = std::min(P.att_rows, m - r0);
    LisaAttnParams b = a;
    b.q_proj = P.q_proj + (size_t)r0 * LISA_ATT_Q_OUT;
    b.query = P.query + (size_t)r0 * LISA_ATT_OUT;
    b.gated = P.gated + (size_t)r0 * LISA_ATT_OUT;
    b.pos = P.pos + 1 + r0 / P.att_rows;
    b.m_rows = ms;
    const uint32_t slices = (base + r0 + ms + LISA_ATT_SLICE - 1) / LISA_ATT_SLICE;
    LISA_TRY(lisa_launch(r->dev, r->attn_partial_rows, &b, sizeof b, slices, LISA_ATT_KVH,
                         (ms + LISA_ATT_ROWS_PER_WG - 1) / LISA_ATT_ROWS_PER_WG, LISA_ATT_ROWS_THREADS, 1, 1));
    LISA_TRY(lisa_launch(r->dev, r->attn_merge_rows, &b, sizeof b, LISA_ATT_QH, ms, 1, 256, 1, 1));
  }
  return LISA_OK;
}

// Uploads the positions the attention row kernels read: pos[0] = base, then
// the first position of every attention sub-block.
int upload_prefill_pos(LisaRunner* r, uint32_t m, uint32_t base) {
  auto& P = r->pf;
  std::vector<uint32_t> pos(1 + (m + P.att_rows - 1) / P.att_rows);
  pos[0] = base;
  for (size_t j = 1; j < pos.size(); ++j) pos[j] = base + (uint32_t)(j - 1) * P.att_rows;
  return upload_u32(r, P.pos, pos.data(), pos.size());
}

// One chunk of the drafter's batched prefill (runner.rs:3494-3581) at drafter
// positions [r->mtp_position, + m): tokens in P.tokens, the target hidden rows
// (bf16) in P.gated; leaves argmax in P.argmax and the final normalized rows
// in P.X. The fc input [m][10240] is staged in P.act.
int mtp_prefill_chunk(LisaRunner* r, uint32_t m) {
  auto& P = r->pf;
  const MtpDev& t = r->mtp;
  uint16_t* fc_in = P.act;
  {
    LisaRowsParams e{};
    e.mode = LISA_ROWS_EMBED;
    e.tokens = P.tokens;
    e.emb_w = r->embed.w;
    e.emb_sb = r->embed.sb;
    e.r_out = P.H;
    LISA_TRY(launch_rows(r, e, 1, m));
  }
  // [RMSNorm(embed, pre_fc_norm_embedding) | RMSNorm(hidden, pre_fc_norm_hidden)]
  LisaRowsParams nh{};
  nh.mode = LISA_ROWS_NORM;
  nh.h_in = P.H;
  nh.norm_w = t.pre_fc_emb;
  nh.x_out = fc_in;
  nh.x_stride = 2 * LISA_HIDDEN;
  LISA_TRY(launch_rows(r, nh, 1, m));
  nh.h_in = P.gated;
  nh.norm_w = t.pre_fc_hid;
  nh.x_out = fc_in + LISA_HIDDEN;
  LISA_TRY(launch_rows(r, nh, 1, m));
  LISA_TRY(launch_gemm(r, fc_in, m, t.fc, P.B));
  // hidden = bf16(fc output); normalized = RMSNorm(hidden, input_norm)
  LISA_TRY(rows_norm(r, m, nullptr, P.B, t.input_norm, P.H, P.X));
  LISA_TRY(launch_gemm(r, P.X, m, t.q, P.q_proj));
  LISA_TRY(launch_gemm(r, P.X, m, t.k, P.k_raw));
  LISA_TRY(launch_gemm(r, P.X, m, t.v, P.v_raw));
  LISA_TRY(prefill_attention(r, m, r->mtp_position, t.q_norm, t.k_norm, r->mtp_key, r->mtp_value));
  LISA_TRY(launch_gemm(r, P.gated, m, t.o, P.B));
  LISA_TRY(rows_norm(r, m, P.H, P.B, t.post_norm, P.H, P.X));
  LISA_TRY(launch_gemm_swiglu(r, P.X, m, t.gate, t.up, P.act));
  LISA_TRY(launch_gemm(r, P.act, m, t.down, P.B));
  LISA_TRY(rows_norm(r, m, P.H, P.B, t.final_norm, P.H, P.X));
  LISA_TRY(launch_gemm(r, P.X, m, r->head, P.logits));
  LisaRowsParams am{};
  am.mode = LISA_ROWS_ARGMAX;
  am.logits = P.logits;
  am.width = (uint32_t)r->cfg.vocab;
  am.argmax_out = P.argmax;
  return launch_rows(r, am, 1, m);
}

// One prefill chunk of m rows at positions [r->position, r->position + m).
int prefill_chunk(LisaRunner* r, uint32_t m) {
  auto& P = r->pf;
  const float inv = 1.0f / lisa_sqrt((float)LISA_GDN_HD);  // runner.rs:1316-1317
  {
    LisaRowsParams e{};
    e.mode = LISA_ROWS_EMBED;
    e.tokens = P.tokens;
    e.emb_w = r->embed.w;
    e.emb_sb = r->embed.sb;
    e.r_out = P.H;
    LISA_TRY(launch_rows(r, e, 1, m));
  }
  for (int i = 0; i < r->cfg.layers; ++i) {
    const LayerDev& l = r->layers[i];
    LISA_TRY(rows_norm(r, m, P.H, i == 0 ? nullptr : P.B, l.input_norm, P.H, P.X));
    if (!l.attention) {
      const int si = l.state_index;
      LISA_TRY(launch_gemm(r, P.X, m, l.qkv, P.qkv));
      LISA_TRY(launch_gemm(r, P.X, m, l.z, P.z));
      LISA_TRY(launch_gemm(r, P.X, m, l.a, P.a));
      LISA_TRY(launch_gemm(r, P.X, m, l.b, P.b));
      LisaConvRowsParams cv{};
      cv.qkv = P.qkv;
      cv.conv_w = l.conv_w;
      cv.conv_state = r->conv_state + (size_t)si * 3 * LISA_GDN_CONV_DIM;
      cv.conv_out = P.conv_out;
      cv.m_rows = m;
      LISA_TRY(lisa_launch(r->dev, r->conv_rows, &cv, sizeof cv, (LISA_GDN_CONV_DIM + 255) / 256, (m + 63) / 64, 1, 256, 1,
                              1));
      LisaGdnParams g{};
      g.conv_out = P.conv_out;
      g.z = P.z;
      g.a = P.a;
      g.b = P.b;
      g.a_log = l.a_log;
      g.dt_bias = l.dt_bias;
      g.norm_w = l.gnorm;
      g.state = r->gdn_state + (size_t)si * LISA_GDN_STATE;
      g.gated = P.gated;
      g.q_scale = inv * inv;
      g.k_scale = inv;
      g.m_rows = m;
      g.qk = P.gdn_qk;
      g.gates = P.gdn_gates;
      g.y_out = P.gdn_y;
      LISA_TRY(lisa_launch(r->dev, r->gdn_prep_rows, &g, sizeof g, m, 9, 1, 256, 1, 1));
      LISA_TRY(lisa_launch(r->dev, r->gdn_scan_rows, &g, sizeof g, LISA_GDN_VH, 8, 1, 256, 1, 1));
      LISA_TRY(lisa_launch(r->dev, r->gdn_out_rows, &g, sizeof g, m, LISA_GDN_VH, 1, 128, 1, 1));
      LISA_TRY(launch_gemm(r, P.gated, m, l.out, P.B));
    } else {
      LISA_TRY(launch_gemm(r, P.X, m, l.q, P.q_proj));
      LISA_TRY(launch_gemm(r, P.X, m, l.k, P.k_raw));
      LISA_TRY(launch_gemm(r, P.X, m, l.v, P.v_raw));
      const size_t off = (size_t)l.cache_index * LISA_ATT_KVH * r->cfg.capacity * LISA_ATT_HD;
      LISA_TRY(prefill_attention(r, m, r->position, l.q_norm, l.k_norm, r->key_cache + off, r->value_cache + off));
      LISA_TRY(launch_gemm(r, P.gated, m, l.o, P.B));
    }
    LISA_TRY(rows_norm(r, m, P.H, P.B, l.post_norm, P.H, P.X));
    LISA_TRY(launch_gemm_swiglu(r, P.X, m, l.gate, l.up, P.act));
    LISA_TRY(launch_gemm(r, P.act, m, l.down, P.B));
  }
  LISA_TRY(rows_norm(r, m, P.H, P.B, r->final_norm, P.H, P.X));
  LISA_TRY(launch_gemm(r, P.X, m, r->head, P.logits));
  LisaRowsParams am{};
  am.mode = LISA_ROWS_ARGMAX;
  am.logits = P.logits;
  am.width = (uint32_t)r->cfg.vocab;
  am.argmax_out = P.argmax;
  return launch_rows(r, am, 1, m);
}

}  // namespace

extern "C" int lisa_runner_forward_prefill(LisaRunner* r, const uint32_t* tokens, int32_t n, int32_t chunk,
                                           uint32_t* argmax_out, float* hidden_out) {
  if (!r || n < 0 || (n && !tokens)) return lisa_fail(LISA_E_ARG, "lisa_runner_forward_prefill: bad argument");
  for (int32_t i = 0; i < n; ++i) LISA_TRY(check_token(r, tokens[i]));
  if (!n) return LISA_OK;
  if (r->position + (uint32_t)n > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "KV capacity %d exhausted by prefill of %d tokens", r->cfg.capacity, n);
  const uint32_t rows = (chunk <= 0 || (uint32_t)chunk > kPrefillRows) ? kPrefillRows : (uint32_t)chunk;
  LISA_TRY(ensure_prefill(r));
  auto& P = r->pf;
  std::vector<uint16_t> h;
  for (uint32_t b = 0; b < (uint32_t)n; b += rows) {
    const uint32_t m = std::min(rows, (uint32_t)n - b);
    LISA_TRY(upload_u32(r, P.tokens, tokens + b, m));
    LISA_TRY(upload_prefill_pos(r, m, r->position));
    LISA_TRY(prefill_chunk(r, m));
    if (argmax_out)
      LISA_TRY(lisa_hip_check(hipMemcpyAsync(argmax_out + b, P.argmax, (size_t)m * 4, hipMemcpyDeviceToHost,
                                             r->dev->stream), "D2H argmax"));
    if (hidden_out) {
      h.resize((size_t)m * LISA_HIDDEN);
      LISA_TRY(lisa_hip_check(hipMemcpyAsync(h.data(), P.H, h.size() * 2, hipMemcpyDeviceToHost, r->dev->stream),
                              "D2H hidden"));
    }
    LISA_TRY(sync(r));  // the host staging above is reused by the next chunk
    if (hidden_out)
      for (size_t i = 0; i < h.size(); ++i) hidden_out[(size_t)b * LISA_HIDDEN + i] = lisa_bf16_to_f32(h[i]);
    r->position += m;
  }
  r->verify_base = -1;
  LISA_TRY(write_pos(r, r->tgt, r->position));
  return sync(r);
}


// MtpRunner::forward_position_batch_with_progress (runner.rs:3494-3581): the
// drafter over n (token, target hidden) positions at [mtp_position,
// mtp_position + n), in chunks of `chunk` rows (0 = 512, the reference's
// PREFILL_BATCH; at most the prefill scratch's 2048), with the prefill kernels.
extern "C" int lisa_mtp_forward_batch(LisaRunner* r, const uint32_t* tokens, const float* hiddens, int32_t n,
                                      int32_t chunk, uint32_t* argmax_out, float* normalized_out) {
  if (!r || n < 0 || (n && (!tokens || !hiddens))) return lisa_fail(LISA_E_ARG, "lisa_mtp_forward_batch: bad argument");
  if (!r->cfg.with_mtp) return lisa_fail(LISA_E_STATE, "runner was created without the MTP drafter");
  for (int32_t i = 0; i < n; ++i) LISA_TRY(check_token(r, tokens[i]));
  if (!n) return LISA_OK;
  if (r->mtp_position + (uint32_t)n > (uint32_t)r->cfg.capacity)
    return lisa_fail(LISA_E_CAPACITY, "MTP KV capacity %d exhausted by prefill of %d positions", r->cfg.capacity, n);
  const uint32_t rows = (chunk <= 0) ? 512u : std::min<uint32_t>((uint32_t)chunk, kPrefillRows);
  LISA_TRY(ensure_prefill(r));
  auto& P = r->pf;
  std::vector<uint16_t> hb, xn;
  for (uint32_t b = 0; b < (uint32_t)n; b += rows) {
    const uint32_t m = std::min(rows, (uint32_t)n - b);
    LISA_TRY(upload_u32(r, P.tokens, tokens + b, m));
    hb.resize((size_t)m * LISA_HIDDEN);
    for (size_t i = 0; i < hb.size(); ++i) hb[i] = lisa_f32_to_bf16_trunc(hiddens[(size_t)b * LISA_HIDDEN + i]);
    LISA_TRY(lisa_hip_check(hipMemcpyAsync(P.gated, hb.data(), hb.size() * 2, hipMemcpyHostToDevice, r->dev->stream),
                            "H2D hidden rows"));
    LISA_TRY(upload_prefill_pos(r, m, r->mtp_position));
    LISA_TRY(mtp_prefill_chunk(r, m));
    if (argmax_out)
      LISA_TRY(lisa_hip_check(hipMemcpyAsync(argmax_out + b, P.argmax, (size_t)m * 4, hipMemcpyDeviceToHost,
                                             r->dev->stream), "D2H argmax"));
    if (normalized_out) {
      xn.resize((size_t)m * LISA_HIDDEN);
      LISA_TRY(lisa_hip_check(hipMemcpyAsync(xn.data(), P.X, xn.size() * 2, hipMemcpyDeviceToHost, r->dev->stream),
                              "D2H normalized"));
    }
    LISA_TRY(sync(r));  // hb and xn are reused by the next chunk
    if (normalized_out)
      for (size_t i = 0; i < xn.size(); ++i) normalized_out[(size_t)b * LISA_HIDDEN + i] = lisa_bf16_to_f32(xn[i]);
    r->mtp_position += m;
  }
  LISA_TRY(write_pos(r, r->drf, r->mtp_position));
  return sync(r);
}
