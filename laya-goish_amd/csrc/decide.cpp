// Request-level decide over token ids (host side).  Restates src/models/openthai/decision.rs
// (questions :20-107, orders :125-139, permutations :140-162, encode :169-233, decide :243-390)
// with token ids in place of text and the model's control tokens in place of the special
// tokens of its tokenizer.  Arithmetic of the aggregation follows the reference's f32 order.
#include "decide.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <set>

#include "common.h"
#include "gguf.h"
#include "json.h"

namespace lg {

namespace {

void read_temperatures(const Gguf &g, DecideSpec &s) {
  // expf of a 3-element F32 tensor log_temperature when the model has one, as
  // src/models/openthai/model.rs:175-178; else metadata; else 1
  s.temperature[0] = float(g.num("laya.decide.temperature_choice", 1.0));
  s.temperature[1] = float(g.num("laya.decide.temperature_score", 1.0));
  s.temperature[2] = float(g.num("laya.decide.temperature_noul", 1.0));
  if (const TensorInfo *t = g.tensor("log_temperature")) {
    if (t->kind != LG_F32 || t->cols() * t->rows() != 3) fail(LG_ERR_FORMAT, "log_temperature must be F32 [3]");
    const float *v = reinterpret_cast<const float *>(g.data(*t));
    for (int i = 0; i < 3; ++i) s.temperature[i] = std::exp(v[i]);
  }
  for (float T : s.temperature)
    if (!(T > 0.0f) || !std::isfinite(T)) fail(LG_ERR_FORMAT, "decide temperatures must be positive");
}

DecideSpec openthai_spec(const Gguf &g) {
  DecideSpec s;
  const Json cfg = Json::parse(g.str("openthai.config"), "openthai.config");
  s.vocab = int(cfg.get("text_config").get("vocab_size").num());
  s.answer = int(cfg.get("answer_token_id").num());
  s.max_tokens = int(g.num("openthai.context_length", 4096));
  s.max_state = int(g.num("openthai.state_length", 2048));
  for (int i = 0; i < 256; ++i) s.head_row[i] = i;
  read_temperatures(g, s);
  const MetaValue *tv = g.meta("tokenizer.ggml.tokens");
  if (!tv || tv->strs.empty()) {
    s.error = "OpenThai model has no tokenizer.ggml.tokens to take its decide control tokens from";
    return s;
  }
  std::map<std::string, int32_t> index;
  for (size_t i = 0; i < tv->strs.size(); ++i) index.emplace(tv->strs[i], int32_t(i));
  auto find = [&](const std::string &tok, int32_t &dst) {
    auto it = index.find(tok);
    if (it == index.end()) {
      if (s.error.empty()) s.error = "OpenThai tokenizer lacks the decide control token " + tok;
      dst = 0;
    } else {
      dst = it->second;
    }
  };
  for (int i = 0; i < 255; ++i) find("<|ts_opt_" + std::to_string(i) + "|>", s.slot[i]);
  s.slot[255] = s.slot[254];  // the abstain slot has no prompt marker
  find("<|ts_state|>", s.state);
  find("<|ts_q|>", s.question);
  find("<|ts_choice|>", s.kind[0]);
  find("<|ts_score|>", s.kind[1]);
  find("<|ts_noul|>", s.kind[2]);
  find("\xc4\x8a", s.newline);  // byte-level BPE spelling of "\n"
  find(":", s.colon);
  int32_t answer_tok = 0;
  find("<|ts_answer|>", answer_tok);
  if (s.error.empty() && answer_tok != s.answer) s.error = "missing OpenThai answer token";
  return s;
}

}  // namespace

DecideSpec decide_spec(const Gguf &g) {
  if (g.str("general.architecture") == "openthai_systemone") return openthai_spec(g);
  if (g.str("general.architecture") == "ggmlc" && g.str("laya.model_name") != "laya-decoder") {
    DecideSpec s;
    for (int i = 0; i < 256; ++i) s.slot[i] = s.head_row[i] = 0;
    s.error = "a Laya encoder decides per question through lg_laya_forward, not the slot layout of lg_decide";
    return s;
  }
  DecideSpec s;
  const int V = int(g.num("laya.decoder.vocab_size", 0));
  const int ctx = int(g.num("laya.decoder.context_length", 0));
  s.vocab = V;
  const int base = int(g.num("laya.decide.slot_base", V - 256));
  for (int i = 0; i < 256; ++i) s.slot[i] = base + i;
  s.state = int(g.num("laya.decide.state_id", V - 257));
  s.question = int(g.num("laya.decide.question_id", V - 258));
  s.kind[0] = int(g.num("laya.decide.choice_id", V - 259));
  s.kind[1] = int(g.num("laya.decide.score_id", V - 260));
  s.kind[2] = int(g.num("laya.decide.noul_id", V - 261));
  s.answer = int(g.num("laya.decide.answer_id", V - 262));
  s.newline = int(g.num("laya.decide.newline_id", V - 263));
  s.colon = int(g.num("laya.decide.colon_id", V - 264));
  for (int i = 0; i < 256; ++i) s.head_row[i] = s.slot[i];
  read_temperatures(g, s);
  s.max_tokens = int(g.num("laya.decide.context_length", ctx));
  s.max_state = int(g.num("laya.decide.state_length", std::min(2048, ctx)));
  return s;
}

namespace {

void check_ids(const DecideSpec &s, const int32_t *ids, int n, const char *what, int q) {
  if (n < 0) fail(LG_ERR_INVALID, "question %d: negative %s length", q, what);
  if (n > 0 && !ids) fail(LG_ERR_INVALID, "question %d: %s tokens missing", q, what);
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= s.vocab)
      fail(LG_ERR_INVALID, "question %d: %s token %d outside the vocabulary", q, what, ids[i]);
}

int desc_len(const lg_question &q, int i) { return q.desc_len && q.descs && q.descs[i] ? q.desc_len[i] : 0; }

}  // namespace

void decide_validate(const DecideSpec &s, const lg_decide_request &r) {
  if (!s.error.empty()) fail(LG_ERR_FORMAT, "%s", s.error.c_str());
  for (int32_t id : {s.state, s.question, s.kind[0], s.kind[1], s.kind[2], s.answer, s.newline, s.colon})
    if (id < 0 || id >= s.vocab) fail(LG_ERR_FORMAT, "decide control token %d outside the vocabulary of %d", id, s.vocab);
  for (int32_t id : s.slot)
    if (id < 0 || id >= s.vocab) fail(LG_ERR_FORMAT, "decide control token %d outside the vocabulary of %d", id, s.vocab);
  if (r.n_questions < 1 || r.n_questions > 256 || !r.questions)
    fail(LG_ERR_INVALID, "questions must contain 1..256 named questions");
  if (r.n_state < 0 || (r.n_state > 0 && !r.state)) fail(LG_ERR_INVALID, "state tokens missing");
  for (int i = 0; i < r.n_state; ++i)
    if (r.state[i] < 0 || r.state[i] >= s.vocab)
      fail(LG_ERR_INVALID, "state token %d outside the vocabulary", r.state[i]);
  for (int qi = 0; qi < r.n_questions; ++qi) {
    const lg_question &q = r.questions[qi];
    switch (q.kind) {
      case LG_Q_CHOICE:
        if (q.n_options < 1 || q.n_options > 255) fail(LG_ERR_INVALID, "question %d: choice requires 1..255 options", qi);
        break;
      case LG_Q_SCORE:
        if (q.n_options < 2 || q.n_options > 10) fail(LG_ERR_INVALID, "question %d: score requires 2..10 levels", qi);
        break;
      case LG_Q_NOUL:
        if (q.n_options != 2) fail(LG_ERR_INVALID, "question %d: noul has exactly two options (no, yes)", qi);
        break;
      default: fail(LG_ERR_INVALID, "question %d: invalid question type", qi);
    }
    check_ids(s, q.instruction, q.n_instruction, "instruction", qi);
    if (!q.names || !q.name_len) fail(LG_ERR_INVALID, "question %d: option names missing", qi);
    for (int o = 0; o < q.n_options; ++o) {
      if (q.kind == LG_Q_CHOICE && q.name_len[o] <= 0) fail(LG_ERR_INVALID, "question %d: option name is empty", qi);
      check_ids(s, q.names[o], q.name_len[o], "option name", qi);
      check_ids(s, q.descs ? q.descs[o] : nullptr, desc_len(q, o), "description", qi);
    }
  }
  if (r.order_invariant < -1 || r.order_invariant > 1) fail(LG_ERR_INVALID, "order_invariant must be boolean");
  if (r.permutations != 0 && (r.permutations < 1 || r.permutations > 32))
    fail(LG_ERR_INVALID, "permutations must be 1..32");
}

// src/models/openthai/decision.rs:140-162
int decide_passes(const lg_decide_request &r) {
  int k = 1;
  bool any = false;
  for (int i = 0; i < r.n_questions; ++i)
    if (r.questions[i].kind == LG_Q_CHOICE) {
      k = any ? std::max(k, r.questions[i].n_options) : r.questions[i].n_options;
      any = true;
    }
  int n;
  if (r.permutations > 0) n = r.permutations;
  else if (r.order_invariant == 0) n = 1;
  else if (r.order_invariant == 1) n = 8;
  else n = k >= 11 ? 8 : 1;
  return std::max(std::min(n, k), 1);
}

// src/models/openthai/decision.rs:125-139: offsets j*k/n rounded half to even, deduplicated,
// in increasing order; each order is a rotation of the options by its offset.
std::vector<std::vector<int>> decide_orders(int k, int n) {
  n = std::max(std::min(n, k), 1);
  std::set<int> offsets;
  for (int j = 0; j < n; ++j) {
    const int a = j * k, d = a / n, rem = a % n;
    offsets.insert((d + int(rem * 2 > n || (rem * 2 == n && d % 2 == 1))) % k);
  }
  std::vector<std::vector<int>> out;
  for (int off : offsets) {
    std::vector<int> o(k);
    for (int i = 0; i < k; ++i) o[i] = (i + off) % k;
    out.push_back(o);
  }
  return out;
}

// src/models/openthai/decision.rs:169-233.  Block of question q at the token level:
//   question, kind marker, instruction..., newline,
//   per slot: option marker(slot), name..., [colon, description...], newline,
//   answer, newline
// The state block is: state marker, state..., newline, cut to the state budget by keeping its
// first token and its tail.
Encoded decide_encode(const DecideSpec &s, const lg_decide_request &r, int npasses, int pass) {
  Encoded e;
  std::vector<std::vector<int32_t>> blocks;
  size_t total = 0;
  for (int qi = 0; qi < r.n_questions; ++qi) {
    const lg_question &q = r.questions[qi];
    std::vector<int> ord(q.n_options);
    if (q.kind == LG_Q_CHOICE) {
      const auto all = decide_orders(q.n_options, npasses);
      ord = all[size_t(pass) % all.size()];
    } else {
      for (int i = 0; i < q.n_options; ++i) ord[i] = i;
    }
    std::vector<int32_t> b;
    b.push_back(s.question);
    b.push_back(s.kind[q.kind]);
    b.insert(b.end(), q.instruction, q.instruction + q.n_instruction);
    b.push_back(s.newline);
    for (int slot = 0; slot < q.n_options; ++slot) {
      const int i = ord[slot];
      b.push_back(s.slot[slot]);
      b.insert(b.end(), q.names[i], q.names[i] + q.name_len[i]);
      if (desc_len(q, i) > 0) {
        b.push_back(s.colon);
        b.insert(b.end(), q.descs[i], q.descs[i] + desc_len(q, i));
      }
      b.push_back(s.newline);
    }
    b.push_back(s.answer);
    b.push_back(s.newline);
    total += b.size();
    blocks.push_back(std::move(b));
    e.order.push_back(ord);
  }
  if (total >= size_t(s.max_tokens)) fail(LG_ERR_INVALID, "question tokens exceed the context budget");
  std::vector<int32_t> &ids = e.ids;
  ids.push_back(s.state);
  ids.insert(ids.end(), r.state, r.state + r.n_state);
  ids.push_back(s.newline);
  const size_t budget = std::min(size_t(s.max_state), size_t(s.max_tokens) - total);
  e.truncated = ids.size() > budget;
  if (e.truncated) {
    std::vector<int32_t> tail(ids.end() - (budget - 1), ids.end());
    ids.resize(1);
    ids.insert(ids.end(), tail.begin(), tail.end());
  }
  for (auto &b : blocks) {
    size_t p = b.size();
    while (p > 0 && b[p - 1] != s.answer) --p;  // last answer marker of the block
    if (p == 0) fail(LG_ERR_INVALID, "missing answer token");
    e.positions.push_back(int32_t(ids.size() + p - 1));
    ids.insert(ids.end(), b.begin(), b.end());
  }
  return e;
}

// src/models/openthai/decision.rs:268-279 (per pass) and :297-336 (per question), f32 in the
// reference's operation order; tensor::softmax is src/tensor.rs:132-140.
void decide_aggregate(const DecideSpec &s, const lg_decide_request &r, int n, const std::vector<Encoded> &enc,
                      const float *slot_logits, lg_decide_result &out) {
  const int nq = r.n_questions;
  std::vector<std::vector<float>> probs(nq);
  std::vector<float> abstain(nq, 0.0f);
  for (int i = 0; i < nq; ++i) probs[i].assign(r.questions[i].n_options, 0.0f);
  for (int pass = 0; pass < n; ++pass) {
    for (int i = 0; i < nq; ++i) {
      const lg_question &q = r.questions[i];
      const int k = q.n_options;
      const float *row = slot_logits + (int64_t(pass) * nq + i) * 256;
      const float T = s.temperature[q.kind];
      std::vector<float> v(k + 1);
      for (int j = 0; j < k; ++j) v[j] = row[j] / T;
      v[k] = row[255] / T;
      float m = -INFINITY;
      for (float x : v) m = std::fmax(m, x);
      float sum_e = 0.0f;
      for (float &x : v) {
        x = std::exp(x - m);
        sum_e += x;
      }
      for (float &x : v) x /= sum_e;
      float sum = 0.0f;
      for (int j = 0; j < k; ++j) sum += v[j];
      sum = std::fmax(sum, 1e-12f);
      for (int slot = 0; slot < k; ++slot) probs[i][enc[pass].order[i][slot]] += v[slot] / sum / float(n);
      abstain[i] += v[k] / float(n);
    }
  }
  float *pout = out.probs;
  for (int i = 0; i < nq; ++i) {
    const lg_question &q = r.questions[i];
    std::vector<float> &p = probs[i];
    const int k = int(p.size());
    float sum = 0.0f;
    for (float x : p) sum += x;
    sum = std::fmax(sum, 1e-12f);
    for (float &x : p) x /= sum;
    float ent = 0.0f;
    for (float x : p) {
      const float c = std::fmax(x, 1e-12f);
      ent += c * std::log(c);
    }
    ent = -ent;
    float conf = 1.0f;
    if (k > 1) conf = std::min(std::max(1.0f - ent / std::log(float(k)), 0.0f), 1.0f);
    int best = 0;
    for (int j = 1; j < k; ++j)
      if (p[j] > p[best]) best = j;
    float score = 0.0f;
    for (int j = 0; j < k; ++j) score += float(j) * p[j];
    for (int j = 0; j < k; ++j) *pout++ = p[j];
    if (out.abstain) out.abstain[i] = q.kind == LG_Q_CHOICE ? abstain[i] : 0.0f;
    if (out.confidence) out.confidence[i] = conf;
    if (out.score) out.score[i] = q.kind == LG_Q_SCORE ? score : 0.0f;
    if (out.choice) out.choice[i] = best;
  }
  out.permutations = n;
  out.input_tokens = int32_t(enc[0].ids.size());
  bool trunc = false;
  for (const Encoded &e : enc) trunc = trunc || e.truncated;
  out.truncated = trunc ? 1 : 0;
}

}  // namespace lg
