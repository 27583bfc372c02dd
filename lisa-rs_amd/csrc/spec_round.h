// spec_round.h — stream-ordered pieces of one block-3 speculative round, for
// the loop of spec.cpp. Each piece enqueues its work on the runner's stream
// and returns without waiting for the device; host values travel through a
// small pinned staging array (round_pinned), so the copies are asynchronous
// too. A round then waits once (round_sync), after which the staged
// device-to-host results are valid. The host bookkeeping (positions, the
// pending verification) follows each piece at once, as the synchronous entry
// points of lisa_hip.h do.
#ifndef LISA_SPEC_ROUND_H
#define LISA_SPEC_ROUND_H

#include <cstdint>

struct LisaRunner;

// Words of the pinned staging array.
enum {
  ROUND_PIN_BONUS = 0,     // verify token 0
  ROUND_PIN_DRAFTS = 1,    // verify tokens 1, 2 (host-chosen drafts)
  ROUND_PIN_MTP_TOKEN = 3, // drafter input token
  ROUND_PIN_TPOS = 4,      // target position after a commit
  ROUND_PIN_DPOS = 5,      // drafter position after a trim
  ROUND_PIN_TARGET = 8,    // verify argmax rows 0..2 (device to host)
  ROUND_PIN_SEED = 12,     // drafter argmax that seeded the round (device to host)
  ROUND_PIN_D1 = 13,       // drafter argmax of the round's second draft (device to host)
  ROUND_PIN_WORDS = 16
};

// The runner's pinned staging array (allocated on first use, freed with the runner).
int round_pinned(LisaRunner* r, uint32_t** out);
// One drafter step (lisa_mtp_forward without its wait): the input token is
// pinned[ROUND_PIN_MTP_TOKEN] when token_on_host, else the drafter's previous
// argmax, copied on the device.
int round_mtp(LisaRunner* r, bool token_on_host, int32_t cond_source, int32_t cond_row);
// The drafter's last argmax into verify token `slot` (1 or 2) on the device,
// and to pinned word `host_word` (or none when negative).
int round_forward_draft(LisaRunner* r, int slot, int host_word);
// Verify tokens [first, first + n) from the pinned words ROUND_PIN_BONUS + first.
int round_set_verify_tokens(LisaRunner* r, int first, int n);
// lisa_runner_verify_block3 without its wait: argmax rows to ROUND_PIN_TARGET.
int round_verify(LisaRunner* r);
// lisa_runner_commit_verified_prefix and lisa_mtp_trim_state without their waits.
int round_commit(LisaRunner* r, int32_t rows);
int round_trim(LisaRunner* r, int32_t count);
// Waits for the round's work; errors of the enqueued work surface here.
int round_sync(LisaRunner* r);

#endif
