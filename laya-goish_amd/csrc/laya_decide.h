// The Laya decision layer at the token level (host side): restates src/models/laya/decision.rs
// (questions :19-99, encode :100-154, confidence :155-167, decide :168-318) over token ids.  The
// tokenizer is not on this path: a question's instruction tokens stand for the encoded
// "<kind> question: <instructions>" text and an option's name + description tokens for the
// encoded " <option text>".  One forward per question (Model::forward(ids, markers, qtype)).
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "lg.h"

namespace lg {

class Gguf;

struct LayaSpec {
  int vocab = 0, max_len = 512, head_max = 192;
  int32_t mask = 50284, sep = 50282, cls = 50281;
  bool has_temp = false;
  float temp[3] = {1.0f, 1.0f, 1.0f};        // laya.temperature (per question kind)
  std::map<std::string, float> buckets;      // laya.temperature_by_options ("choice:3-5" -> T)
};

LayaSpec laya_spec(const Gguf &g);

struct LayaEncoded {
  std::vector<int32_t> ids, markers;
};

// decision.rs:19-99 at the token level (question and option counts per kind).
void laya_validate(const LayaSpec &s, const lg_decide_request &r);
// decision.rs:100-154: [cls] head [sep] ([mask] option)... [sep] state [sep], cut to max_len.
LayaEncoded laya_encode(const LayaSpec &s, const lg_decide_request &r, int question);
// decision.rs:185-298: temperature bucket, softmax, act probability (stored in out.abstain),
// choice (ties to the lower index), expected score, confidence (noul: max(p, 1 - p)).
// logits: the k option logits of every question concatenated; act: [n_questions][2].
void laya_aggregate(const LayaSpec &s, const lg_decide_request &r, const float *logits, const float *act,
                    int input_tokens, lg_decide_result &out);

}  // namespace lg
