// Request-level decide at the token level: question blocks, option-order passes, slot scoring.
//
// Host code above the batched GPU prefill.  It restates, over token ids instead of text, the
// reference's decision layer (src/models/openthai/decision.rs): question validation (:20-107),
// pass count (:140-162), option orders (:125-139), prompt layout and answer positions
// (:169-233), slot softmax with abstain and pass averaging (:268-279), final normalisation,
// confidence, choice and score (:297-336).  The tokenizer is not part of this path, so each
// text piece of a request arrives as token ids and the control tokens come from the model.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "lg.h"

namespace lg {

class Gguf;

// Control tokens and budgets of the decide layout.
// laya-decoder models: laya.decide.* metadata when the model has it; otherwise the top of the
// vocabulary: slot s (s < 255: option marker s, 255: abstain) = V - 256 + s, then state,
// question, the three kind markers, answer, newline and colon below it.  The scored head rows
// are the slot tokens' rows of the language-model head.
// OpenThai models: the special tokens of the embedded tokenizer (<|ts_opt_s|>, <|ts_state|>,
// <|ts_q|>, <|ts_choice|>, <|ts_score|>, <|ts_noul|>, byte-level newline, ":"), the config's
// answer_token_id, openthai.context_length / state_length; the scored rows are the 256 rows of
// the slot head (src/models/openthai/decision.rs:185-224, model.rs:116-132).
struct DecideSpec {
  int32_t slot[256];
  int32_t head_row[256];  // head row scored for slot s
  int32_t state = 0, question = 0, kind[3] = {0, 0, 0}, answer = 0, newline = 0, colon = 0;
  float temperature[3] = {1.0f, 1.0f, 1.0f};  // per question kind (choice, score, noul)
  int max_tokens = 0;                         // prompt budget (context_length)
  int max_state = 0;                          // state budget (state_length)
  int vocab = 0;
  std::string error;  // non-empty: the model cannot encode decide prompts (reported on use)
};

DecideSpec decide_spec(const Gguf &g);

struct Encoded {
  std::vector<int32_t> ids;
  std::vector<int32_t> positions;           // one answer position per question
  std::vector<std::vector<int>> order;      // per question: option index shown at each slot
  bool truncated = false;
};

// Validation of a request (throws lg::Error with the reference's wording where it applies).
void decide_validate(const DecideSpec &s, const lg_decide_request &r);
// Number of option-order passes (decision.rs:140-162).
int decide_passes(const lg_decide_request &r);
// Cyclic option orders for k options over n passes (decision.rs:125-139).
std::vector<std::vector<int>> decide_orders(int k, int n);
// Token layout of one pass (decision.rs:169-233).
Encoded decide_encode(const DecideSpec &s, const lg_decide_request &r, int npasses, int pass);
// Aggregate slot logits [npasses][nq][256] into the result (decision.rs:268-279,297-336).
void decide_aggregate(const DecideSpec &s, const lg_decide_request &r, int npasses,
                      const std::vector<Encoded> &enc, const float *slot_logits, lg_decide_result &out);

}  // namespace lg
