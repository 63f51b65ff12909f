// Laya decision layer over token ids; see laya_decide.h.
#include "laya_decide.h"

#include <algorithm>
#include <cmath>

#include "common.h"
#include "gguf.h"
#include "json.h"

namespace lg {

LayaSpec laya_spec(const Gguf &g) {
  LayaSpec s;
  const TensorInfo *et = g.tensor("tok_emb.weight");
  s.vocab = et && et->dims.size() > 1 ? int(et->dims[1]) : 0;
  s.max_len = int(g.num("laya.max_len", 512));
  s.head_max = int(g.num("laya.head_max_len", 192));
  s.mask = int32_t(g.num("laya.mask_token_id", 50284));
  s.sep = int32_t(g.num("laya.sep_token_id", 50282));
  s.cls = int32_t(g.num("laya.cls_token_id", 50281));
  // decision.rs:181-182: unparsable metadata counts as absent
  try {
    const Json t = Json::parse(g.str("laya.temperature"), "laya.temperature");
    if (t.kind == Json::Arr) {
      s.has_temp = true;
      for (int i = 0; i < 3; ++i) s.temp[i] = i < int(t.size()) ? float(t.at(size_t(i)).num()) : 1.0f;
      // decision.rs:209: a missing entry counts as 1
      for (int i = int(t.size()); i < 3; ++i) s.temp[i] = 1.0f;
    }
  } catch (const Error &) {
  }
  try {
    const Json b = Json::parse(g.str("laya.temperature_by_options"), "laya.temperature_by_options");
    for (const auto &kv : b.o)
      if (kv.second.kind != Json::Null) s.buckets[kv.first] = float(kv.second.num());
  } catch (const Error &) {
  }
  return s;
}

void laya_validate(const LayaSpec &s, const lg_decide_request &r) {
  if (r.n_questions < 1 || r.n_questions > 256 || !r.questions)
    fail(LG_ERR_INVALID, "questions must contain 1..256 named questions");
  for (int qi = 0; qi < r.n_questions; ++qi) {
    const lg_question &q = r.questions[qi];
    if (q.kind != LG_Q_CHOICE && q.kind != LG_Q_SCORE && q.kind != LG_Q_NOUL)
      fail(LG_ERR_INVALID, "question %d: type must be choice, score, or noul", qi);
    if (q.kind == LG_Q_CHOICE && q.n_options < 1) fail(LG_ERR_INVALID, "question %d: choice requires a criteria object", qi);
    if (q.kind == LG_Q_SCORE && q.n_options < 2)
      fail(LG_ERR_INVALID, "question %d: score requires at least two ordered criteria", qi);
    if (q.kind == LG_Q_NOUL && q.n_options != 2) fail(LG_ERR_INVALID, "question %d: noul has exactly two options", qi);
    if (q.n_options < 1 || q.n_options > 16) fail(LG_ERR_INVALID, "question %d: requires 1..16 options", qi);
    if (q.n_instruction < 0 || (q.n_instruction > 0 && !q.instruction) || !q.names || !q.name_len)
      fail(LG_ERR_INVALID, "question %d: tokens missing", qi);
  }
  if (r.n_state < 0 || (r.n_state > 0 && !r.state)) fail(LG_ERR_INVALID, "state tokens missing");
  // decision.rs:107-109, checked by encode after the questions parse
  if (s.head_max < 32 || s.head_max >= s.max_len) fail(LG_ERR_FORMAT, "invalid sequence budgets");
}

LayaEncoded laya_encode(const LayaSpec &s, const lg_decide_request &r, int qi) {
  const lg_question &q = r.questions[qi];
  std::vector<int32_t> head(q.instruction, q.instruction + q.n_instruction);
  std::vector<std::vector<int32_t>> opts;
  for (int i = 0; i < q.n_options; ++i) {
    std::vector<int32_t> tok(q.names[i], q.names[i] + q.name_len[i]);
    if (q.desc_len && q.descs && q.descs[i]) tok.insert(tok.end(), q.descs[i], q.descs[i] + q.desc_len[i]);
    if (tok.size() > 48) tok.resize(48);  // decision.rs:121-122
    std::vector<int32_t> v{s.mask};
    v.insert(v.end(), tok.begin(), tok.end());
    opts.push_back(std::move(v));
  }
  size_t sum = 0;
  for (const auto &o : opts) sum += o.size();
  if (int64_t(s.head_max) - int64_t(sum) < 16) {  // decision.rs:126-133
    const size_t per = std::max<size_t>(size_t(s.head_max - 16) / opts.size(), 4);
    for (auto &o : opts)
      if (o.size() > per) o.resize(per);
    sum = 0;
    for (const auto &o : opts) sum += o.size();
  }
  const size_t keep = std::max<size_t>(size_t(s.head_max) > sum ? size_t(s.head_max) - sum : 0, 8);
  if (head.size() > keep) head.resize(keep);
  LayaEncoded e;
  e.ids.push_back(s.cls);
  e.ids.insert(e.ids.end(), head.begin(), head.end());
  e.ids.push_back(s.sep);
  for (const auto &o : opts) {
    e.markers.push_back(int32_t(e.ids.size()));
    e.ids.insert(e.ids.end(), o.begin(), o.end());
  }
  e.ids.push_back(s.sep);
  const size_t room = size_t(s.max_len) > e.ids.size() + 1 ? size_t(s.max_len) - (e.ids.size() + 1) : 0;
  const size_t ns = std::min(size_t(std::max(0, r.n_state)), room);
  e.ids.insert(e.ids.end(), r.state, r.state + ns);
  e.ids.push_back(s.sep);
  if (e.ids.size() > size_t(s.max_len)) e.ids.resize(size_t(s.max_len));
  for (int32_t m : e.markers)
    if (size_t(m) >= e.ids.size()) fail(LG_ERR_INVALID, "option markers exceed context");
  return e;
}

void laya_aggregate(const LayaSpec &s, const lg_decide_request &r, const float *logits, const float *act,
                    int input_tokens, lg_decide_result &out) {
  static const char *kinds[3] = {"choice", "score", "noul"};
  int at = 0;
  for (int qi = 0; qi < r.n_questions; ++qi) {
    const lg_question &q = r.questions[qi];
    const int k = q.n_options;
    const float *z = logits + at;
    const std::string bucket = std::string(kinds[q.kind]) + ":" + (k <= 2 ? "2" : k <= 5 ? "3-5" : k <= 10 ? "6-10" : "11+");
    auto it = s.buckets.find(bucket);
    float T = it != s.buckets.end() ? it->second : s.has_temp ? s.temp[q.kind] : 1.0f;
    T = std::max(T, 1e-3f);
    // tensor::softmax (src/tensor.rs:132-140) over z / T
    std::vector<float> v(k), p(k);
    float m = -INFINITY;
    for (int i = 0; i < k; ++i) {
      v[i] = z[i] / T;
      m = std::max(m, v[i]);
    }
    float sum = -0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] = std::exp(v[i] - m);
      sum = sum + p[i];
    }
    for (int i = 0; i < k; ++i) p[i] = p[i] / sum;
    // act probability: softmax(act)[0]
    const float a0 = act[2 * qi], a1 = act[2 * qi + 1], am = std::max(a0, a1);
    const float e0 = std::exp(a0 - am), e1 = std::exp(a1 - am);
    out.abstain[qi] = e0 / (e0 + e1);
    int best = 0;  // max_by with ties to the lower index (decision.rs:227-230)
    for (int i = 1; i < k; ++i)
      if (p[i] > p[best]) best = i;
    double score = 0.0;
    for (int i = 0; i < k; ++i) score += double(i) * double(p[i]);
    float conf;
    if (q.kind == LG_Q_NOUL) {
      conf = std::max(p[1], 1.0f - p[1]);
    } else if (k < 2) {
      conf = 1.0f;
    } else {  // decision.rs:155-167 in f64
      double e = -0.0;
      for (int i = 0; i < k; ++i) {
        const double x = std::max(double(p[i]), 1e-12);
        e += x * std::log(x);
      }
      conf = float(std::min(1.0, std::max(0.0, 1.0 - (-e) / std::log(double(k)))));
    }
    out.choice[qi] = best;
    out.confidence[qi] = conf;
    out.score[qi] = q.kind == LG_Q_SCORE ? float(score) : 0.0f;
    for (int i = 0; i < k; ++i) out.probs[at + i] = p[i];
    at += k;
  }
  out.input_tokens = input_tokens;
  out.permutations = 1;
  out.truncated = 0;
}

}  // namespace lg
