// spec.cpp — greedy block-3 speculative decoding over the runner
// (src/speculative/mod.rs): accept_greedy, mtp_reconcile_plan and the
// device-resident-hidden loop run_block3_loop.
#include <cstring>
#include <vector>

#include "bridge.h"
#include "lisa_hip.h"
#include "lisa_synth.h"
#include "spec_round.h"

// speculative/mod.rs:16-32
extern "C" int lisa_accept_greedy(const uint32_t* drafts, int32_t n, const uint32_t* target, LisaAcceptance* out) {
  if (!drafts || !target || !out || n < 0 || n > 2) return lisa_fail(LISA_E_ARG, "lisa_accept_greedy: bad argument");
  int accepted = 0;
  while (accepted < n && drafts[accepted] == target[accepted]) ++accepted;
  out->accepted_drafts = accepted;
  out->emitted_count = accepted + 1;
  for (int i = 0; i < accepted; ++i) out->emitted[i] = drafts[i];
  out->emitted[accepted] = target[accepted];
  out->target_trim = (n + 1) - out->emitted_count;
  return LISA_OK;
}

// speculative/mod.rs:49-65
extern "C" int lisa_mtp_reconcile_plan(int32_t draft_count, int32_t round_appended, int32_t accepted,
                                       LisaReconcilePlan* out) {
  if (!out || accepted < 0 || accepted > draft_count || round_appended < 0 || round_appended > draft_count ||
      draft_count > 2)
    return lisa_fail(LISA_E_ARG, "lisa_mtp_reconcile_plan: bad argument");
  const int keep = accepted < round_appended ? accepted : round_appended;
  out->replay_count = 0;
  for (int i = keep; i < accepted; ++i) out->replay[out->replay_count++] = i;
  out->replay[out->replay_count++] = -1;
  out->trim = round_appended - keep;
  return LISA_OK;
}

// run_block3_loop (speculative/mod.rs:102-198) after
// generate_greedy_block3_prefilled (:384-413). A round is enqueued without
// waiting for the device until its verification: the drafter's argmaxes
// reach the verify tokens and the next drafter step on the device, and the
// host reads them, with the verified rows, after one wait per round. The
// tokens, acceptance, commits and trims are those of the step-by-step loop
// (lisa_mtp_forward, lisa_runner_verify_block3, ... in turn).
extern "C" int lisa_generate_greedy_block3(LisaRunner* r, uint32_t bonus, const float* target_hidden,
                                           uint32_t mtp_seed_token, const float* mtp_seed_hidden,
                                           int32_t max_tokens, const uint32_t* force_truth, int32_t force_len,
                                           uint64_t force_seed, float p_accept, uint32_t* tokens_out,
                                           LisaSpecStats* stats) {
  if (!r || !target_hidden || !mtp_seed_hidden || max_tokens < 0 || (max_tokens && !tokens_out))
    return lisa_fail(LISA_E_ARG, "lisa_generate_greedy_block3: bad argument");
  LisaSpecStats st{};
  std::vector<uint32_t> out;
  if (max_tokens == 0) {
    if (stats) *stats = st;
    return LISA_OK;
  }
  out.push_back(bonus);
  // target.upload_hidden_device(0, ...) and mtp.upload_normalized_device(seed)
  // (speculative/mod.rs:117-122)
  LISA_TRY(lisa_runner_upload_hidden(r, 0, target_hidden));
  LISA_TRY(lisa_mtp_upload_normalized(r, mtp_seed_hidden));
  uint32_t* pin = nullptr;
  LISA_TRY(round_pinned(r, &pin));
  // the round's first draft: the seed token on the host (first round), else
  // the argmax of the drafter step that closed the previous round
  bool seed_on_device = false;
  uint32_t seed_token = mtp_seed_token;
  const uint64_t force_key = lisa_stream_key(force_seed, 0x5eedull);
  uint64_t force_ctr = 0;
  const uint32_t vocab = (uint32_t)lisa_runner_vocab(r);
  while ((int32_t)out.size() < max_tokens) {
    const int remaining = max_tokens - (int32_t)out.size();
    if (remaining < 3) {
      for (int i = 0; i < remaining; ++i) {
        uint32_t next = 0;
        LISA_TRY(lisa_runner_forward_token_decode(r, bonus, &next, nullptr));
        st.target_forwards += 1;
        bonus = next;
        out.push_back(next);
      }
      break;
    }
    // drafts: the seed, then one drafter step from it (conditioned on the
    // drafter's own normalized output)
    if (seed_on_device) {
      LISA_TRY(round_forward_draft(r, 1, ROUND_PIN_SEED));
      LISA_TRY(round_mtp(r, false, 1, 0));
    } else {
      pin[ROUND_PIN_DRAFTS] = seed_token;
      LISA_TRY(round_set_verify_tokens(r, 1, 1));
      pin[ROUND_PIN_MTP_TOKEN] = seed_token;
      LISA_TRY(round_mtp(r, true, 1, 0));
    }
    LISA_TRY(round_forward_draft(r, 2, ROUND_PIN_D1));
    const int round_appended = 1;
    // forced drafts replace the drafter's on the device before the verification
    bool forced[2] = {false, false};
    uint32_t forced_tok[2] = {0, 0};
    if (force_truth) {
      for (int j = 0; j < 2; ++j) {
        const size_t idx = out.size() + (size_t)j;
        if ((int64_t)idx < force_len) {
          const float u = lisa_rand_unit(lisa_rand64(force_key, force_ctr++));
          const uint32_t truth = force_truth[idx];
          forced[j] = true;
          forced_tok[j] = (u < p_accept) ? truth : (truth + 1u) % vocab;
          pin[ROUND_PIN_DRAFTS + j] = forced_tok[j];
          LISA_TRY(round_set_verify_tokens(r, 1 + j, 1));
        }
      }
    }
    pin[ROUND_PIN_BONUS] = bonus;
    LISA_TRY(round_set_verify_tokens(r, 0, 1));
    LISA_TRY(round_verify(r));
    LISA_TRY(round_sync(r));
    st.target_forwards += 1;
    uint32_t drafts[2] = {seed_on_device ? pin[ROUND_PIN_SEED] : seed_token, pin[ROUND_PIN_D1]};
    for (int j = 0; j < 2; ++j)
      if (forced[j]) drafts[j] = forced_tok[j];
    const uint32_t target[3] = {pin[ROUND_PIN_TARGET], pin[ROUND_PIN_TARGET + 1], pin[ROUND_PIN_TARGET + 2]};
    LisaAcceptance acc;
    LISA_TRY(lisa_accept_greedy(drafts, 2, target, &acc));
    LISA_TRY(round_commit(r, acc.accepted_drafts + 1));
    LisaReconcilePlan plan;
    LISA_TRY(lisa_mtp_reconcile_plan(2, round_appended, acc.accepted_drafts, &plan));
    LISA_TRY(round_trim(r, plan.trim));
    // only the last replay entry is forwarded (speculative/mod.rs:169-183);
    // its argmax seeds the next round on the device
    const int last = plan.replay[plan.replay_count - 1];
    pin[ROUND_PIN_MTP_TOKEN] = last >= 0 ? drafts[last] : acc.emitted[acc.emitted_count - 1];
    const int cond_row = last >= 0 ? last : acc.accepted_drafts;
    LISA_TRY(round_mtp(r, true, 0, cond_row));
    seed_on_device = true;
    bonus = acc.emitted[acc.emitted_count - 1];
    for (int i = 0; i < acc.emitted_count; ++i) out.push_back(acc.emitted[i]);
    st.rounds += 1;
    st.accepted_drafts += acc.accepted_drafts;
    st.drafted_tokens += 2;
  }
  LISA_TRY(round_sync(r));
  std::memcpy(tokens_out, out.data(), sizeof(uint32_t) * (size_t)max_tokens);
  if (stats) *stats = st;
  return LISA_OK;
}

// prefill_prompt_from_with_progress (speculative/mod.rs:237-311): the target
// runs prompt[start..n) (batched prefill for 4 or more tokens, M=1 decode
// steps otherwise), then the drafter replays the shifted tokens
// (prompt[start+1..n) followed by the bonus) conditioned on the target's
// per-position hidden rows (batched for 4 or more positions). Returns the
// bonus token, the target hidden of the last prompt position, and the drafter
// seed (its last argmax and normalized hidden). The runners must already be
// positioned at `start` (a restored session checkpoint, or 0).
extern "C" int lisa_prefill_prompt(LisaRunner* r, const uint32_t* prompt, int32_t n, int32_t start, uint32_t* bonus,
                                   float* target_hidden, uint32_t* mtp_seed_token, float* mtp_seed_hidden) {
  if (!r || !bonus || !target_hidden || !mtp_seed_token || !mtp_seed_hidden)
    return lisa_fail(LISA_E_ARG, "lisa_prefill_prompt: bad argument");
  if (n <= 0 || !prompt) return lisa_fail(LISA_E_ARG, "cannot prefill an empty prompt");
  if (start < 0 || start > n) return lisa_fail(LISA_E_ARG, "prefill start %d exceeds prompt length %d", start, n);
  const int32_t len = n - start;
  if (len == 0) return lisa_fail(LISA_E_ARG, "prefill start %d leaves no prompt token to run", start);
  const uint32_t* seg = prompt + start;
  std::vector<uint32_t> am((size_t)len);
  std::vector<float> hidden((size_t)len * 5120);
  if (len >= 4) {
    LISA_TRY(lisa_runner_forward_prefill(r, seg, len, 0, am.data(), hidden.data()));
  } else {
    for (int32_t t = 0; t < len; ++t)
      LISA_TRY(lisa_runner_forward_token_decode(r, seg[t], &am[(size_t)t], hidden.data() + (size_t)t * 5120));
  }
  const uint32_t b = am[(size_t)len - 1];
  std::vector<uint32_t> tokens((size_t)len);
  for (int32_t t = 0; t < len; ++t) {
    const int32_t global = start + t;
    tokens[(size_t)t] = global + 1 < n ? prompt[global + 1] : b;
  }
  uint32_t seed = 0;
  if (len >= 4) {
    std::vector<uint32_t> mam((size_t)len);
    std::vector<float> xn((size_t)len * 5120);
    LISA_TRY(lisa_mtp_forward_batch(r, tokens.data(), hidden.data(), len, 0, mam.data(), xn.data()));
    seed = mam[(size_t)len - 1];
    std::memcpy(mtp_seed_hidden, xn.data() + (size_t)(len - 1) * 5120, 5120 * sizeof(float));
  } else {
    for (int32_t t = 0; t < len; ++t)
      LISA_TRY(lisa_mtp_forward_position_decode(r, tokens[(size_t)t], hidden.data() + (size_t)t * 5120, &seed,
                                                mtp_seed_hidden));
  }
  *bonus = b;
  *mtp_seed_token = seed;
  std::memcpy(target_hidden, hidden.data() + (size_t)(len - 1) * 5120, 5120 * sizeof(float));
  return LISA_OK;
}
