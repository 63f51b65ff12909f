// extern "C" surface of include/lg.h.  Every entry point converts library exceptions into
// an LG_ERR_* status and a thread-local message; nothing escapes as a C++ exception and no
// call aborts the process.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "common.h"
#include "decide.h"
#include "engine.h"
#include "gguf.h"
#include "kernels.h"
#include "lg.h"
#include "registry.h"

namespace lg {
void synth_image(const char *preset, uint64_t seed, int n_layers, uint8_t **out, uint64_t *out_len);
}  // namespace lg

struct lg_gguf {
  lg::Gguf *g;
};
struct lg_engine {
  lg::Engine *e;
};
struct lg_batch {
  lg::BatchPlan *b;
};

namespace {

thread_local std::string g_err;

template <class F>
int guard(F &&f) {
  try {
    f();
    g_err.clear();
    return LG_OK;
  } catch (const lg::Error &e) {
    g_err = e.what();
    return e.code;
  } catch (const std::bad_alloc &) {
    g_err = "out of host memory";
    return LG_ERR_OOM;
  } catch (const std::exception &e) {
    g_err = e.what();
    return LG_ERR_INVALID;
  } catch (...) {
    g_err = "unknown error";
    return LG_ERR_INVALID;
  }
}

#define NEED(p, what) \
  if (!(p)) ::lg::fail(LG_ERR_INVALID, "%s must not be null", what)

}  // namespace

extern "C" {

const char *lg_last_error(void) { return g_err.c_str(); }

const char *lg_version(void) { return "laya-mi355x 0.1.0 gfx950"; }

int lg_layout(uint32_t kind, uint64_t *block, uint64_t *bytes) {
  return guard([&] {
    if (!lg::layout(kind, block, bytes))
      lg::fail(LG_ERR_UNSUPPORTED, "unsupported GGML tensor type %u; supported F32/F16/Q4_0/Q8_0/Q4_K/Q6_K", kind);
  });
}

float lg_half(uint16_t bits) { return lg::half_to_float(bits); }

int lg_probe_read(uint64_t bytes, int launches, double *us_per_launch) {
  return guard([&] {
    NEED(us_per_launch, "us_per_launch");
    *us_per_launch = lg::probe_read_chain(size_t(bytes), launches);
  });
}

int lg_gguf_open(const char *path, lg_gguf **out) {
  return guard([&] {
    NEED(path, "path");
    NEED(out, "out");
    *out = nullptr;
    lg::Gguf *g = lg::Gguf::open_file(path);
    *out = new lg_gguf{g};
  });
}

int lg_gguf_open_memory(const void *bytes, uint64_t len, lg_gguf **out) {
  return guard([&] {
    NEED(out, "out");
    *out = nullptr;
    if (!bytes && len) lg::fail(LG_ERR_INVALID, "bytes must not be null");
    lg::Gguf *g = lg::Gguf::open_memory(static_cast<const uint8_t *>(bytes), len);
    *out = new lg_gguf{g};
  });
}

void lg_gguf_close(lg_gguf *g) {
  if (!g) return;
  delete g->g;
  delete g;
}

int lg_gguf_tensor_count(const lg_gguf *g) { return g ? int(g->g->tensors().size()) : 0; }

const char *lg_gguf_tensor_name(const lg_gguf *g, int i) {
  if (!g || i < 0 || i >= int(g->g->tensors().size())) return nullptr;
  return g->g->tensors()[i].name.c_str();
}

int lg_gguf_tensor(const lg_gguf *g, const char *name, uint32_t *kind, uint64_t dims[4], int *nd,
                   const void **data, uint64_t *len) {
  return guard([&] {
    NEED(g, "g");
    NEED(name, "name");
    const lg::TensorInfo *t = g->g->tensor(name);
    if (!t) lg::fail(LG_ERR_INVALID, "missing tensor %s", name);
    if (kind) *kind = t->kind;
    if (dims) {
      for (int i = 0; i < 4; ++i) dims[i] = i < int(t->dims.size()) ? t->dims[i] : 1;
    }
    if (nd) *nd = int(t->dims.size());
    if (data) *data = g->g->data(*t);
    if (len) *len = t->len;
  });
}

int lg_gguf_meta_num(const lg_gguf *g, const char *key, double *value, int *found) {
  return guard([&] {
    NEED(g, "g");
    NEED(key, "key");
    const lg::MetaValue *v = g->g->meta(key);
    if (found) *found = v != nullptr;
    if (value) *value = v ? g->g->num(key, 0) : 0.0;
  });
}

int lg_gguf_meta_str(const lg_gguf *g, const char *key, const char **value, int *found) {
  return guard([&] {
    NEED(g, "g");
    NEED(key, "key");
    const lg::MetaValue *v = g->g->meta(key);
    if (found) *found = v != nullptr;
    if (value) *value = v ? v->str.c_str() : "";
  });
}

int lg_dequant(uint32_t kind, const void *src, uint64_t len, float *dst) {
  return guard([&] {
    uint64_t block, size;
    if (!lg::layout(kind, &block, &size))
      lg::fail(LG_ERR_UNSUPPORTED, "unsupported GGML tensor type %u; supported F32/F16/Q4_0/Q8_0/Q4_K/Q6_K", kind);
    if (len % size) lg::fail(LG_ERR_INVALID, "length %llu is not a whole number of blocks", (unsigned long long)len);
    if (len == 0) return;
    NEED(src, "src");
    NEED(dst, "dst");
    const uint64_t nblocks = len / size, nelem = nblocks * block;
    lg::DevBuf dsrc, ddst;
    dsrc.ensure(len);
    ddst.ensure(nelem * 4);
    HIP_CHECK(hipMemcpy(dsrc.p, src, len, hipMemcpyHostToDevice));
    if (kind == LG_Q4_0 || kind == LG_F32) {
      lg::launch_dequant(kind, dsrc.as<uint8_t>(), nblocks, ddst.as<float>(), nullptr);
    } else {
      // through the engine's repacked layout: the exact arithmetic the GEMV kernels use
      lg::DevBuf q, s;
      lg::DevMatrix w;
      w.kind = kind;
      w.rows = int(nblocks);
      w.cols = int(block);
      LG_REQUIRE(nblocks < (1ull << 31), "too many blocks");
      const int64_t n = int64_t(nelem);
      const int64_t qb = kind == LG_F16 ? n * 2 : kind == LG_Q4_K ? n / 2 : n;
      const int64_t sb = kind == LG_Q8_0 ? n / 32 * 2 : kind == LG_Q4_K ? n / 32 * 8 : kind == LG_Q6_K ? n / 16 * 4 : 0;
      q.ensure(size_t(qb));
      w.q = q.p;
      if (sb) {
        s.ensure(size_t(sb));
        w.s = s.p;
      }
      lg::launch_repack(kind, dsrc.as<uint8_t>(), w.rows, w.cols, w, nullptr);
      lg::launch_dequant_repacked(w, ddst.as<float>(), nullptr);
    }
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(dst, ddst.p, nelem * 4, hipMemcpyDeviceToHost));
  });
}

int lg_synth_gguf(const char *preset, uint64_t seed, int n_layers, void **image, uint64_t *len) {
  return guard([&] {
    NEED(preset, "preset");
    NEED(image, "image");
    NEED(len, "len");
    uint8_t *img = nullptr;
    lg::synth_image(preset, seed, n_layers, &img, len);
    *image = img;
  });
}

int lg_synth_gguf_file(const char *preset, uint64_t seed, int n_layers, const char *path) {
  return guard([&] {
    NEED(preset, "preset");
    NEED(path, "path");
    uint8_t *img = nullptr;
    uint64_t len = 0;
    lg::synth_image(preset, seed, n_layers, &img, &len);
    FILE *fp = std::fopen(path, "wb");
    if (!fp) {
      std::free(img);
      lg::fail(LG_ERR_INVALID, "cannot write %s", path);
    }
    const size_t w = std::fwrite(img, 1, len, fp);
    std::fclose(fp);
    std::free(img);
    if (w != len) lg::fail(LG_ERR_INVALID, "short write to %s", path);
  });
}

void lg_synth_free(void *image) { std::free(image); }

int lg_model_describe(const lg_gguf *g, lg_model_desc *out) {
  return guard([&] {
    NEED(g, "gguf");
    NEED(out, "out");
    const lg::ModelDesc d = lg::describe(*g->g);
    lg_model_desc r{};
    auto put = [](char *dst, size_t cap, const std::string &v) {
      if (v.size() >= cap) ::lg::fail(LG_ERR_FORMAT, "model name %s is too long", v.c_str());
      std::memcpy(dst, v.c_str(), v.size() + 1);
    };
    put(r.name, sizeof(r.name), d.name);
    put(r.family, sizeof(r.family), d.family);
    put(r.architecture, sizeof(r.architecture), d.architecture);
    put(r.release_date, sizeof(r.release_date), d.release_date);
    for (const std::string &a : d.aliases) put(r.aliases[r.n_aliases++], sizeof(r.aliases[0]), a);
    *out = r;
  });
}

int lg_registry_preflight(const char *const *paths, int n, const char *default_name, int *default_index) {
  return guard([&] {
    NEED(default_index, "default_index");
    LG_REQUIRE(n >= 0 && (n == 0 || paths), "registry: bad path list");
    std::vector<std::string> ps;
    for (int i = 0; i < n; ++i) {
      NEED(paths[i], "path");
      ps.emplace_back(paths[i]);
    }
    *default_index = lg::registry_preflight(ps, default_name);
  });
}

int lg_engine_create(const lg_gguf *g, const lg_engine_opts *opts, lg_engine **out) {
  return guard([&] {
    NEED(g, "g");
    NEED(out, "out");
    *out = nullptr;
    lg_engine_opts o{};
    if (opts) o = *opts;
    lg::Engine *e = new lg::Engine(*g->g, o);
    *out = new lg_engine{e};
  });
}

void lg_engine_destroy(lg_engine *e) {
  if (!e) return;
  try {
    delete e->e;
  } catch (...) {
  }
  delete e;
}

int lg_engine_info(const lg_engine *e, lg_model_info *info) {
  return guard([&] {
    NEED(e, "engine");
    NEED(info, "info");
    *info = e->e->info();
  });
}

int lg_engine_sync(lg_engine *e) {
  return guard([&] {
    NEED(e, "engine");
    e->e->sync();
  });
}

int lg_engine_workspace_bytes(const lg_engine *e, int64_t *bytes) {
  return guard([&] {
    NEED(e, "engine");
    NEED(bytes, "bytes");
    *bytes = int64_t(e->e->workspace_bytes());
  });
}

int lg_matmul(lg_engine *e, const char *tensor, const float *x, int m, const float *bias, float *y) {
  return guard([&] {
    NEED(e, "engine");
    NEED(tensor, "tensor");
    NEED(x, "x");
    NEED(y, "y");
    e->e->matmul(tensor, x, m, bias, y);
  });
}

int lg_seq_create(lg_engine *e, int *seq) {
  return guard([&] {
    NEED(e, "engine");
    NEED(seq, "seq");
    *seq = e->e->seq_create();
  });
}

int lg_seq_fork(lg_engine *e, int parent, int ntokens, int *child) {
  return guard([&] {
    NEED(e, "engine");
    NEED(child, "child");
    *child = e->e->seq_fork(parent, ntokens);
  });
}

int lg_seq_free(lg_engine *e, int seq) {
  return guard([&] {
    NEED(e, "engine");
    e->e->seq_free(seq);
  });
}

int lg_seq_len(lg_engine *e, int seq, int *len) {
  return guard([&] {
    NEED(e, "engine");
    NEED(len, "len");
    *len = e->e->seq_len(seq);
  });
}

int lg_seq_kv_read(lg_engine *e, int seq, int layer, int pos0, int n, float *k, float *v) {
  return guard([&] {
    NEED(e, "engine");
    e->e->seq_kv_read(seq, layer, pos0, n, k, v);
  });
}

int lg_forward(lg_engine *e, int seq, const int32_t *ids, int n, const int32_t *positions, int npos,
               const int32_t *vocab_ids, int nv, float *logits, lg_cancel_fn cancel, void *cancel_arg) {
  return guard([&] {
    NEED(e, "engine");
    if (npos > 0) NEED(logits, "logits");
    if (vocab_ids) LG_REQUIRE(nv > 0 && nv <= 256, "nv must be 1..256 when vocab_ids is given");
    e->e->forward(seq, ids, n, positions, npos, vocab_ids, nv, logits, cancel, cancel_arg);
  });
}

int lg_batch_create(lg_engine *e, const lg_request *reqs, int nreq, lg_batch **out) {
  return guard([&] {
    NEED(e, "engine");
    NEED(out, "out");
    *out = nullptr;
    lg::BatchPlan *b = e->e->batch_create(reqs, nreq);
    *out = new lg_batch{b};
  });
}

void lg_batch_free(lg_engine *e, lg_batch *b) {
  if (!b) return;
  if (e) e->e->batch_free(b->b);
  delete b;
}

int lg_batch_run(lg_engine *e, lg_batch *b, const int32_t *option_ids, int k, float temperature,
                 float *logits, float *probs, float *logprobs, lg_cancel_fn cancel, void *cancel_arg) {
  return guard([&] {
    NEED(e, "engine");
    NEED(b, "batch");
    e->e->batch_run(b->b, option_ids, k, temperature, logits, probs, logprobs, cancel, cancel_arg);
  });
}

int lg_batch_rewind(lg_engine *e, lg_batch *b) {
  return guard([&] {
    NEED(e, "engine");
    NEED(b, "batch");
    e->e->batch_rewind(b->b);
  });
}

int lg_decode(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, float *logits) {
  return guard([&] {
    NEED(e, "engine");
    e->e->decode(seq, first, steps, tokens, logits);
  });
}

int lg_decode_graph(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, double *capture_ms,
                    double *run_ms) {
  return guard([&] {
    NEED(e, "engine");
    e->e->decode_graph(seq, first, steps, tokens, capture_ms, run_ms);
  });
}

int lg_decode_noalloc(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, float *logits) {
  return guard([&] {
    NEED(e, "engine");
    e->e->decode_noalloc(seq, first, steps, tokens, logits);
  });
}

namespace {

// The Laya decide of `reqs` (src/models/laya/decision.rs:168-318, one forward per question):
// every question of every request validated and encoded first, then run through the encoder as
// GPU batches of at most the engine's batch token budget, then aggregated per request.
void laya_decide_many(lg::Engine &E, const lg_decide_request *reqs, int n, lg_decide_result *outs,
                      lg_cancel_fn cancel, void *cancel_arg) {
  const lg::LayaSpec &s = E.laya_decide;
  std::vector<std::vector<lg::LayaEncoded>> enc(n);
  std::vector<int> tokens(n, 0);
  for (int r = 0; r < n; ++r) {
    lg::laya_validate(s, reqs[r]);
    for (int q = 0; q < reqs[r].n_questions; ++q) {
      enc[r].push_back(lg::laya_encode(s, reqs[r], q));
      tokens[r] += int(enc[r].back().ids.size());
    }
  }
  std::vector<lg_laya_input> in;
  std::vector<size_t> koff{0};
  for (int r = 0; r < n; ++r)
    for (int q = 0; q < reqs[r].n_questions; ++q) {
      const lg::LayaEncoded &x = enc[r][q];
      in.push_back({x.ids.data(), int32_t(x.ids.size()), x.markers.data(), int32_t(x.markers.size()),
                    reqs[r].questions[q].kind});
      koff.push_back(koff.back() + x.markers.size());
    }
  std::vector<float> logits(koff.back()), act(2 * in.size());
  const int64_t budget = E.max_batch_tokens();
  size_t i0 = 0;
  while (i0 < in.size()) {
    size_t i1 = i0;
    int64_t toks = 0;
    while (i1 < in.size() && (i1 == i0 || toks + in[i1].n <= budget)) toks += in[i1++].n;
    E.laya_forward(in.data() + i0, int(i1 - i0), logits.data() + koff[i0], act.data() + 2 * i0, cancel, cancel_arg);
    i0 = i1;
  }
  size_t at = 0;
  for (int r = 0; r < n; ++r) {
    lg::laya_aggregate(s, reqs[r], logits.data() + koff[at], act.data() + 2 * at, tokens[r], outs[r]);
    at += size_t(reqs[r].n_questions);
  }
}

// Runs every pass of `reqs` through the engine (GPU batches of at most the engine's batch token
// budget, passes of one request kept in one batch when they fit) and aggregates each request.
void decide_many(lg::Engine &E, const lg_decide_request *reqs, int n, lg_decide_result *outs, lg_cancel_fn cancel,
                 void *cancel_arg) {
  if (E.arch == lg::Arch::Laya) return laya_decide_many(E, reqs, n, outs, cancel, cancel_arg);
  const lg::DecideSpec &s = E.decide;
  std::vector<int> passes(n);
  std::vector<std::vector<lg::Encoded>> enc(n);
  // validate and encode everything before any inference (src/models/openthai/decision.rs:234-241,
  // src/server.rs:259-283)
  for (int r = 0; r < n; ++r) {
    lg::decide_validate(s, reqs[r]);
    passes[r] = lg::decide_passes(reqs[r]);
    for (int p = 0; p < passes[r]; ++p) enc[r].push_back(lg::decide_encode(s, reqs[r], passes[r], p));
    for (const lg::Encoded &x : enc[r])
      LG_REQUIRE(int64_t(x.ids.size()) <= E.ctx, "prompt of %zu tokens exceeds the model context %d", x.ids.size(), E.ctx);
  }
  std::vector<std::vector<float>> logits(n);
  for (int r = 0; r < n; ++r) logits[r].resize(size_t(passes[r]) * reqs[r].n_questions * 256);
  // (request, pass) work in order, packed greedily into batches under the token budget
  struct Item { int r, p; };
  std::vector<Item> items;
  for (int r = 0; r < n; ++r)
    for (int p = 0; p < passes[r]; ++p) items.push_back({r, p});
  const int64_t budget = E.max_batch_tokens();
  size_t i0 = 0;
  while (i0 < items.size()) {
    size_t i1 = i0;
    int64_t toks = 0;
    while (i1 < items.size()) {
      const int64_t t = int64_t(enc[items[i1].r][items[i1].p].ids.size());
      if (i1 > i0 && toks + t > budget) break;
      toks += t;
      ++i1;
    }
    // the sequences and the plan are released whatever happens
    struct Seqs {
      lg::Engine &E;
      std::vector<int> ids;
      lg::BatchPlan *b = nullptr;
      ~Seqs() {
        try {
          if (b) E.batch_free(b);
          for (int q : ids) E.seq_free(q);
        } catch (...) {
        }
      }
    } held{E, {}};
    std::vector<lg_request> rq;
    int rows = 0;
    for (size_t i = i0; i < i1; ++i) {
      const lg::Encoded &x = enc[items[i].r][items[i].p];
      held.ids.push_back(E.seq_create());
      rq.push_back({held.ids.back(), x.ids.data(), int(x.ids.size()), x.positions.data(), int(x.positions.size())});
      rows += int(x.positions.size());
    }
    held.b = E.batch_create(rq.data(), int(rq.size()));
    std::vector<float> out(size_t(rows) * 256);
    E.batch_run(held.b, s.head_row, 256, 1.0f, out.data(), nullptr, nullptr, cancel, cancel_arg);
    size_t row = 0;
    for (size_t i = i0; i < i1; ++i) {
      const int r = items[i].r, nq = reqs[r].n_questions;
      std::copy(out.begin() + row * 256, out.begin() + (row + nq) * 256,
                logits[r].begin() + size_t(items[i].p) * nq * 256);
      row += nq;
    }
    i0 = i1;
  }
  for (int r = 0; r < n; ++r) lg::decide_aggregate(s, reqs[r], passes[r], enc[r], logits[r].data(), outs[r]);
}

}  // namespace

int lg_decide(lg_engine *e, const lg_decide_request *req, lg_decide_result *out, lg_cancel_fn cancel,
              void *cancel_arg) {
  return guard([&] {
    NEED(e, "engine");
    NEED(req, "request");
    NEED(out, "result");
    NEED(out->probs, "result probabilities");
    decide_many(*e->e, req, 1, out, cancel, cancel_arg);
  });
}

int lg_laya_forward(lg_engine *e, const lg_laya_input *in, int n, float *logits, float *act, lg_cancel_fn cancel,
                    void *cancel_arg) {
  return guard([&] {
    NEED(e, "engine");
    e->e->laya_forward(in, n, logits, act, cancel, cancel_arg);
  });
}

int lg_decide_batch(lg_engine *e, const lg_decide_request *reqs, int n, lg_decide_result *outs,
                    lg_cancel_fn cancel, void *cancel_arg) {
  return guard([&] {
    NEED(e, "engine");
    NEED(reqs, "requests");
    NEED(outs, "results");
    LG_REQUIRE(n >= 1 && n <= 256, "states must be an array of 1..256 states");
    int64_t questions = 0;
    for (int r = 0; r < n; ++r) {
      NEED(outs[r].probs, "result probabilities");
      questions += reqs[r].n_questions;
    }
    LG_REQUIRE(questions <= 256, "At most 256 total questions per request");
    decide_many(*e->e, reqs, n, outs, cancel, cancel_arg);
  });
}

int lg_decide_encode(const lg_gguf *g, const lg_decide_request *req, int pass, int32_t *ids, int cap, int *n,
                     int32_t *positions, int32_t *order, int *truncated, int *passes) {
  return guard([&] {
    NEED(g, "gguf");
    NEED(req, "request");
    const lg::DecideSpec s = lg::decide_spec(*g->g);
    lg::decide_validate(s, *req);
    const int np = lg::decide_passes(*req);
    LG_REQUIRE(pass >= 0 && pass < np, "pass %d outside 0..%d", pass, np - 1);
    const lg::Encoded e = lg::decide_encode(s, *req, np, pass);
    if (passes) *passes = np;
    if (n) *n = int(e.ids.size());
    if (truncated) *truncated = e.truncated ? 1 : 0;
    if (ids) {
      LG_REQUIRE(size_t(cap) >= e.ids.size(), "ids capacity %d < %zu tokens", cap, e.ids.size());
      std::copy(e.ids.begin(), e.ids.end(), ids);
    }
    if (positions) std::copy(e.positions.begin(), e.positions.end(), positions);
    if (order)
      for (int q = 0; q < req->n_questions; ++q)
        for (size_t j = 0; j < e.order[q].size(); ++j) order[q * 255 + j] = e.order[q][j];
  });
}

int lg_decide_scores(const lg_gguf *g, const lg_decide_request *req, const float *slot_logits, lg_decide_result *out) {
  return guard([&] {
    NEED(g, "gguf");
    NEED(req, "request");
    NEED(slot_logits, "slot logits");
    NEED(out, "result");
    NEED(out->probs, "result probabilities");
    const lg::DecideSpec s = lg::decide_spec(*g->g);
    lg::decide_validate(s, *req);
    const int n = lg::decide_passes(*req);
    std::vector<lg::Encoded> enc;
    for (int p = 0; p < n; ++p) enc.push_back(lg::decide_encode(s, *req, n, p));
    lg::decide_aggregate(s, *req, n, enc, slot_logits, *out);
  });
}

int lg_laya_decide_encode(const lg_gguf *g, const lg_decide_request *req, int question, int32_t *ids, int cap,
                          int *n, int32_t *markers) {
  return guard([&] {
    NEED(g, "gguf");
    NEED(req, "request");
    const lg::LayaSpec s = lg::laya_spec(*g->g);
    lg::laya_validate(s, *req);
    LG_REQUIRE(question >= 0 && question < req->n_questions, "question %d outside 0..%d", question,
               req->n_questions - 1);
    const lg::LayaEncoded e = lg::laya_encode(s, *req, question);
    if (n) *n = int(e.ids.size());
    if (ids) {
      LG_REQUIRE(size_t(cap) >= e.ids.size(), "ids capacity %d < %zu tokens", cap, e.ids.size());
      std::copy(e.ids.begin(), e.ids.end(), ids);
    }
    if (markers) std::copy(e.markers.begin(), e.markers.end(), markers);
  });
}

int lg_laya_decide_scores(const lg_gguf *g, const lg_decide_request *req, const float *logits, const float *act,
                          lg_decide_result *out) {
  return guard([&] {
    NEED(g, "gguf");
    NEED(req, "request");
    NEED(logits, "logits");
    NEED(act, "act logits");
    NEED(out, "result");
    NEED(out->probs, "result probabilities");
    const lg::LayaSpec s = lg::laya_spec(*g->g);
    lg::laya_validate(s, *req);
    int tokens = 0;
    for (int q = 0; q < req->n_questions; ++q) tokens += int(lg::laya_encode(s, *req, q).ids.size());
    lg::laya_aggregate(s, *req, logits, act, tokens, *out);
  });
}

int lg_option_scores(const float *logits, int k, float temperature, float *probs, float *logprobs) {
  return guard([&] {
    NEED(logits, "logits");
    LG_REQUIRE(k > 0 && k <= 256, "k must be 1..256");
    LG_REQUIRE(temperature > 0 && std::isfinite(temperature), "temperature must be positive");
    float z[256], p[256];
    float m = -INFINITY;
    for (int i = 0; i < k; ++i) {
      z[i] = logits[i] / temperature;
      m = std::fmax(m, z[i]);
    }
    float s = 0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] = std::exp(z[i] - m);
      s += p[i];
    }
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] /= s;
      sum += p[i];
    }
    sum = std::fmax(sum, 1e-12f);
    float s2 = 0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] /= sum;
      s2 += p[i];
    }
    s2 = std::fmax(s2, 1e-12f);
    const float lse = std::log(s);
    for (int i = 0; i < k; ++i) {
      if (probs) probs[i] = p[i] / s2;
      if (logprobs) logprobs[i] = z[i] - m - lse;
    }
  });
}

int lg_option_confidence(const float *probs, int k, int mode, float *confidence) {
  return guard([&] {
    NEED(probs, "probs");
    NEED(confidence, "confidence");
    LG_REQUIRE(k >= 0, "k must be non-negative");
    LG_REQUIRE(mode == LG_CONF_F32 || mode == LG_CONF_F64, "unknown confidence mode %d", mode);
    if (k <= 1) {
      *confidence = 1.0f;
      return;
    }
    if (mode == LG_CONF_F64) {
      double h = -0.0;
      for (int i = 0; i < k; ++i) {
        const double x = std::fmax(double(probs[i]), 1e-12);
        h -= x * std::log(x);
      }
      double c = 1.0 - h / std::log(double(k));
      c = c < 0.0 ? 0.0 : (c > 1.0 ? 1.0 : c);
      *confidence = float(c);
    } else {
      float h = -0.0f;
      for (int i = 0; i < k; ++i) {
        const float x = std::fmax(probs[i], 1e-12f);
        h -= x * std::log(x);
      }
      float c = 1.0f - h / std::log(float(k));
      c = c < 0.0f ? 0.0f : (c > 1.0f ? 1.0f : c);
      *confidence = c;
    }
  });
}

int lg_profile_enable(lg_engine *e, int on) {
  return guard([&] {
    NEED(e, "engine");
    e->e->prof.enable(on != 0);
  });
}

int lg_profile_read(lg_engine *e, const char *cls, int64_t *launches, double *ms, double *bytes,
                    double *flops) {
  return guard([&] {
    NEED(e, "engine");
    NEED(cls, "cls");
    e->e->prof.read(cls, launches, ms, bytes, flops);
  });
}

int lg_profile_reset(lg_engine *e) {
  return guard([&] {
    NEED(e, "engine");
    e->e->prof.reset();
  });
}

}  // extern "C"
