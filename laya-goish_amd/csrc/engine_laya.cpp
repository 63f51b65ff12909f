// The Laya encoder on the engine: load (src/models/laya/model.rs:60-291) and the batched forward
// (model.rs:303-416).  Every input is one reference forward over a fresh sequence: bidirectional
// attention needs the whole input, so there is no cache.  Linears run on the MFMA GEMM with
// hi/lo activation planes (biases in the epilogue; GeGLU and ReLU fused), LayerNorm and attention
// in f32 kernels, the small decision tail on the generic f32 GEMM.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "common.h"
#include "engine.h"
#include "json.h"

namespace lg {

namespace {

const std::string &graph_name(const Json &graph, const Json &id) {
  return graph.get("tensors").get(std::to_string(int64_t(id.num()))).get("name").str();
}

}  // namespace

// model.rs:65-121: the linear's weight [rows][cols] plus the sum of its bias inputs in the graph
// (the opcode-29 node's third input and any opcode-200 add on its output)
LayaLinear Engine::laya_linear(const Gguf &g, const Json &graph, const std::string &key) {
  const std::string weight = key + ".weight";
  const TensorInfo *t = g.tensor(weight);
  if (!t) fail(LG_ERR_FORMAT, "missing tensor %s", weight.c_str());
  for (size_t i = 2; i < t->dims.size(); ++i)
    if (t->dims[i] != 1) fail(LG_ERR_FORMAT, "non-matrix linear");
  const Json *node = nullptr;
  for (const Json &n : graph.get("nodes").a)
    if (n.get("opcode").num() == 29.0 && n.get("inputs").size() > 0 && graph_name(graph, n.get("inputs").at(0)) == weight) {
      node = &n;
      break;
    }
  if (!node) fail(LG_ERR_FORMAT, "graph lacks linear %s", key.c_str());
  std::vector<std::string> biases;
  if (node->get("inputs").size() > 2) biases.push_back(graph_name(graph, node->get("inputs").at(2)));
  const Json &out0 = node->get("outputs").at(0);
  for (const Json &n : graph.get("nodes").a)
    if (n.get("opcode").num() == 200.0 && n.get("inputs").size() > 1 && out0.kind == Json::Num &&
        n.get("inputs").at(0).kind == Json::Num && n.get("inputs").at(0).num() == out0.num())
      biases.push_back(graph_name(graph, n.get("inputs").at(1)));
  LayaLinear l;
  const int cols = int(t->cols()), rows = int(t->dims.size() > 1 ? t->dims[1] : 1);
  if (t->dims.size() >= 2) {
    l.w = upload_matrix(g, {weight}, cols);
  } else {  // a one-row linear stored as a vector: upload it as a [1][cols] matrix
    l.w.kind = t->kind;
    l.w.rows = 1;
    l.w.cols = cols;
    if (t->kind != LG_F16 && t->kind != LG_F32) fail(LG_ERR_UNSUPPORTED, "%s: vector linears must be F16/F32", weight.c_str());
    l.w.q = carve(t->len);
    uploader().bytes(g.data(*t), t->len, l.w.q);
    named_[weight] = l.w;
    weight_bytes_ += int64_t(t->len);
  }
  if (!biases.empty()) {
    std::vector<float> sum(rows, 0.0f);
    for (const std::string &bn : biases) {
      const TensorInfo *bt = g.tensor(bn);
      if (!bt) fail(LG_ERR_FORMAT, "missing tensor %s", bn.c_str());
      uint64_t count = 1;
      for (auto v : bt->dims) count *= v;
      if (int64_t(count) != rows) fail(LG_ERR_FORMAT, "linear bias shape mismatch");
      const uint8_t *src = g.data(*bt);
      for (int i = 0; i < rows; ++i) {
        float v;
        if (bt->kind == LG_F32) std::memcpy(&v, src + 4 * i, 4);
        else if (bt->kind == LG_F16) v = half_to_float(uint16_t(src[2 * i] | (src[2 * i + 1] << 8)));
        else fail(LG_ERR_UNSUPPORTED, "%s: biases must be F32/F16", bn.c_str());
        sum[i] = sum[i] + v;  // tensor::add, in graph order
      }
    }
    float *d = static_cast<float *>(carve(size_t(rows) * 4));
    HIP_CHECK(hipMemcpy(d, sum.data(), size_t(rows) * 4, hipMemcpyHostToDevice));
    l.b = d;
  }
  return l;
}

// model.rs:122-150: layer norm i of the graph (node "layer_norm" / "layer_norm_<i>", opcode 201)
LayaNorm Engine::laya_norm(const Gguf &g, const Json &graph, int i) {
  const std::string key = i == 0 ? "layer_norm" : "layer_norm_" + std::to_string(i);
  const Json *node = nullptr;
  for (const Json &n : graph.get("nodes").a)
    if (n.get("name").str() == key && n.get("opcode").num() == 201.0) {
      node = &n;
      break;
    }
  if (!node) fail(LG_ERR_FORMAT, "missing %s", key.c_str());
  LayaNorm n;
  const Json &ins = node->get("inputs");
  if (ins.size() > 1) n.w = upload_vector_f32(g, graph_name(graph, ins.at(1)), d);
  if (ins.size() > 2) n.b = upload_vector_f32(g, graph_name(graph, ins.at(2)), d);
  n.eps = float(node->get("attributes").get("eps").num());
  if (!(n.eps > 0.0f && n.eps < 0.1f)) fail(LG_ERR_FORMAT, "invalid layer norm epsilon");
  return n;
}

void Engine::load_laya(const Gguf &g) {
  if (g.str("general.architecture") != "ggmlc" || g.str("laya.checkpoint").find("laya") == std::string::npos)
    fail(LG_ERR_FORMAT, "expected a compiled Laya GGUF (Kev and other architectures are outside this port)");
  if (g.num("laya.max_opts", 16) != 16) fail(LG_ERR_FORMAT, "expected 16-option Laya head");
  if (!g.str("ggmlc.decision").empty() &&
      Json::parse(g.str("ggmlc.decision"), "ggmlc.decision").get("kind").str() != "laya")
    fail(LG_ERR_FORMAT, "unsupported decision sequence recipe");
  const Json graph = Json::parse(g.str("ggmlc.graph_spec"), "ggmlc.graph_spec");
  int layers = 0, heads = 0;
  while (g.tensor("qkv." + std::to_string(layers) + ".weight")) ++layers;
  while (g.tensor("head_qkv." + std::to_string(heads) + ".weight")) ++heads;
  if (layers == 0 || layers > 64 || heads != 2) fail(LG_ERR_FORMAT, "unsupported Laya encoder/head layout");
  const TensorInfo *et = g.tensor("tok_emb.weight");
  if (!et) fail(LG_ERR_FORMAT, "missing embedding");
  const TensorInfo *ct = g.tensor("cos_full");
  if (!ct) fail(LG_ERR_FORMAT, "missing RoPE tables");
  L = layers;
  d = int(et->cols());
  V = int(et->dims.size() > 1 ? et->dims[1] : 1);
  hd = int(ct->cols());
  if (d == 0 || hd == 0 || hd % 2 || d % hd) fail(LG_ERR_FORMAT, "invalid attention dimensions");
  if (hd != 64 || d % 128 || d > 4096)
    fail(LG_ERR_UNSUPPORTED, "Laya shape outside the kernels (hidden %d, head_dim %d)", d, hd);
  if (et->kind != LG_F16 && et->kind != LG_F32) fail(LG_ERR_UNSUPPORTED, "Laya embeddings must be F16/F32");
  hq = hkv = d / hd;
  ctx = int(g.num("laya.max_len", 512));
  std::vector<const Json *> attns;
  for (const Json &n : graph.get("nodes").a)
    if (n.get("opcode").num() == 74.0) attns.push_back(&n);
  if (int(attns.size()) != layers + heads) fail(LG_ERR_FORMAT, "unexpected attention graph");
  const Json &m0 = attns[0]->get("inputs");
  if (m0.size() == 0) fail(LG_ERR_FORMAT, "attention has no mask");
  const double fullmask = m0.at(m0.size() - 1).num();

  // arena: every tensor but the embedding table as f32 at most (+ summed biases)
  size_t total = 4096;
  for (const auto &t : g.tensors()) {
    if (t.name == "tok_emb.weight") continue;
    uint64_t count = 1;
    for (auto v : t.dims) count *= v;
    total += 2 * (align256(count * 4) + 512);
  }
  arena_size_ = total;
  if (hipMalloc(&arena_, arena_size_) != hipSuccess) {
    arena_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %zu bytes of weights", arena_size_);
  }
  emb_kind = et->kind;
  if (hipMalloc(&emb_, et->len) != hipSuccess) {
    emb_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %llu bytes of embeddings", (unsigned long long)et->len);
  }
  uploader().bytes(g.data(*et), et->len, emb_);
  weight_bytes_ += int64_t(et->len);

  auto layer = [&](int i, bool head) {
    LayaLayer y;
    const std::string s = std::to_string(i);
    if (!head) {
      y.has_n1 = i > 0;
      if (y.has_n1) y.n1 = laya_norm(g, graph, 2 * i);
      y.qkv = laya_linear(g, graph, "qkv." + s);
      y.wo = laya_linear(g, graph, "wo." + s);
      y.n2 = laya_norm(g, graph, 2 * i + 1);
      y.wi = laya_linear(g, graph, "mlp_wi." + s);
      y.down = laya_linear(g, graph, "mlp_wo." + s);
      const Json &ins = attns[i]->get("inputs");
      y.full = ins.at(ins.size() - 1).num() == fullmask;
    } else {
      y.has_n1 = true;
      y.n1 = laya_norm(g, graph, 2 * layers + 1 + 2 * i);
      y.qkv = laya_linear(g, graph, "head_qkv." + s);
      y.wo = laya_linear(g, graph, "head_wo." + s);
      y.n2 = laya_norm(g, graph, 2 * layers + 2 + 2 * i);
      y.wi = laya_linear(g, graph, "head_fc1." + s);
      y.down = laya_linear(g, graph, "head_fc2." + s);
      y.full = true;
    }
    // model.rs:238-259
    if (y.qkv.w.cols != d || y.qkv.w.rows != 3 * d || y.wo.w.cols != d || y.wo.w.rows != d || y.wi.w.cols != d ||
        y.down.w.rows != d || y.wi.w.rows != y.down.w.cols * (head ? 1 : 2))
      fail(LG_ERR_FORMAT, "inconsistent layer dimensions");
    // the large-batch 256 x 256 GEMM's operand form (for F16 the weights themselves)
    for (LayaLinear *x : {&y.qkv, &y.wo, &y.wi, &y.down}) add_prefill_copy(x->w);
    return y;
  };
  laya_embnorm_ = laya_norm(g, graph, 0);
  for (int i = 0; i < layers; ++i) laya_trunk_.push_back(layer(i, false));
  laya_finalnorm_ = laya_norm(g, graph, 2 * layers);
  for (int i = 0; i < heads; ++i) laya_head_.push_back(layer(i, true));
  laya_scorenorm_ = laya_norm(g, graph, 2 * layers + 1 + 2 * heads);
  laya_type_emb_ = upload_vector_f32(g, "type_emb.weight", int64_t(3) * d);
  laya_score1_ = laya_linear(g, graph, "scorer_fc1");
  laya_score2_ = laya_linear(g, graph, "scorer_fc2");
  laya_act1_ = laya_linear(g, graph, "act_fc1");
  laya_act2_ = laya_linear(g, graph, "act_fc2");
  if (laya_score1_.w.cols != d || laya_score1_.w.rows != d || laya_score2_.w.cols != d || laya_score2_.w.rows != 1 ||
      laya_act1_.w.cols != d + 4 || laya_act2_.w.cols != laya_act1_.w.rows || laya_act2_.w.rows != 2)
    fail(LG_ERR_FORMAT, "decision head shape mismatch");
  f = laya_trunk_[0].down.w.cols;
  laya_f_ = f;
  laya_head_f_ = laya_head_[0].wi.w.rows;
  for (const LayaLayer &y : laya_trunk_)
    if (y.wi.b || y.down.w.cols != f) fail(LG_ERR_UNSUPPORTED, "Laya MLP with a gate|up bias or varying width");
  for (const LayaLayer &y : laya_head_)
    if (y.wi.w.rows != laya_head_f_) fail(LG_ERR_UNSUPPORTED, "Laya head MLPs of different widths");
  // RoPE tables [max_len][hd] f32
  const int64_t tab = int64_t(ctx) * hd;
  laya_cos_full_ = upload_vector_f32(g, "cos_full", tab);
  laya_sin_full_ = upload_vector_f32(g, "sin_full", tab);
  laya_cos_slide_ = upload_vector_f32(g, "cos_slide", tab);
  laya_sin_slide_ = upload_vector_f32(g, "sin_slide", tab);
}

void Engine::run_laya(BatchPlan &b, const int32_t *qtype_dev, lg_cancel_fn cancel, void *arg) {
  const int T = b.T, planes = split() ? 2 : 1;
  const int fw = std::max(laya_f_, laya_head_f_);
  ws_x_.ensure(size_t(T) * d * 4);
  ws_ot_o_.ensure(size_t(T) * d * 4);
  ws_h16_.ensure(size_t(T) * d * 2 * planes);
  ws_qkv_.ensure(size_t(T) * 3 * d * 4);
  ws_att16_.ensure(size_t(T) * d * 2 * planes);
  ws_act16_.ensure(size_t(T) * fw * 2 * planes);
  auto lo = [&](DevBuf &buf, int64_t n) { return split() ? buf.as<_Float16>() + n : nullptr; };
  float *h = ws_x_.as<float>(), *tmp = ws_ot_o_.as<float>(), *qkv = ws_qkv_.as<float>();
  _Float16 *x16 = ws_h16_.as<_Float16>(), *x16lo = lo(ws_h16_, int64_t(T) * d);
  _Float16 *att = ws_att16_.as<_Float16>(), *attlo = lo(ws_att16_, int64_t(T) * d);
  _Float16 *act = ws_act16_.as<_Float16>(), *actlo = lo(ws_act16_, int64_t(T) * fw);
  prof.begin("embed", stream);
  launch_embed(emb_, emb_kind, b.ids, T, d, V, tmp, stream);
  launch_layer_norm(tmp, nullptr, T, d, laya_embnorm_.w, laya_embnorm_.b, laya_embnorm_.eps, nullptr, nullptr, nullptr,
                    nullptr, nullptr, h, stream);
  prof.end(double(T) * d * 12, 0, stream);
  auto attention = [&](const LayaLayer &y, bool rope) {
    const float *cosT = y.full ? laya_cos_full_ : laya_cos_slide_, *sinT = y.full ? laya_sin_full_ : laya_sin_slide_;
    // the 256 x 256 GEMM rotates q and k in its epilogue (the same bits as the RoPE kernel after it)
    const bool fused = rope && x16lo && hd == 64 && (d / hd) % 2 == 0 && gemm_wide_takes(T, y.qkv.w, Epi::F32);
    if (fused) {
      const _Float16 *ks = chunk_sums(x16, x16lo, T, y.qkv.w);
      prof.begin_kernel("gemm");
      launch_gemm_wide_laya_rope(x16, x16lo, T, y.qkv.w, y.qkv.b, cosT, sinT, b.tok_pos, d / hd, qkv, 3 * d, stream, ks);
      prof.end_kernel(double(y.qkv.w.bytes()) + double(T) * d * 2, 2.0 * T * double(y.qkv.w.rows) * d);
    } else {
      gemm(x16, x16lo, T, y.qkv.w, Epi::F32, qkv, nullptr, nullptr, 3 * d, y.qkv.b);
    }
    prof.begin("laya_attn", stream);
    if (rope && !fused) launch_laya_rope(qkv, T, d, hd, cosT, sinT, b.tok_pos, stream);
    launch_laya_attn(qkv, d, hd, y.full ? -1 : 64, b.tile_row0, b.tile_pos0, b.tile_n, b.tile_seq, b.seq_n, b.ntiles,
                     att, attlo, stream);
    prof.end(0, 0, stream);
    gemm(att, attlo, T, y.wo.w, Epi::ADD, h, nullptr, nullptr, d, y.wo.b);
  };
  auto norm_planes = [&](const LayaNorm &n) {
    prof.begin("layer_norm", stream);
    launch_layer_norm(h, nullptr, T, d, n.w, n.b, n.eps, nullptr, nullptr, nullptr, x16, x16lo, nullptr, stream);
    prof.end(double(T) * d * (4 + 2 * planes), 0, stream);
  };
  for (const LayaLayer &y : laya_trunk_) {
    if (cancel && cancel(arg)) fail(LG_ERR_CANCELED, "request canceled");
    if (y.has_n1) norm_planes(y.n1);
    else launch_cvt_f16(h, int64_t(T) * d, x16, x16lo, stream);
    attention(y, true);
    norm_planes(y.n2);
    gemm(x16, x16lo, T, y.wi.w, Epi::GEGLU, nullptr, act, actlo, laya_f_, nullptr);
    gemm(act, actlo, T, y.down.w, Epi::ADD, h, nullptr, nullptr, d, y.down.b);
  }
  // final norm, then the question type's row (model.rs:369-372)
  launch_layer_norm(h, nullptr, T, d, laya_finalnorm_.w, laya_finalnorm_.b, laya_finalnorm_.eps, laya_type_emb_,
                    b.tok_seq, qtype_dev, nullptr, nullptr, tmp, stream);
  HIP_CHECK(hipMemcpyAsync(h, tmp, size_t(T) * d * 4, hipMemcpyDeviceToDevice, stream));
  for (const LayaLayer &y : laya_head_) {
    if (cancel && cancel(arg)) fail(LG_ERR_CANCELED, "request canceled");
    norm_planes(y.n1);
    attention(y, false);
    norm_planes(y.n2);
    gemm(x16, x16lo, T, y.wi.w, Epi::RELU16, nullptr, act, actlo, laya_head_f_, y.wi.b);
    gemm(act, actlo, T, y.down.w, Epi::ADD, h, nullptr, nullptr, d, y.down.b);
  }
}

void Engine::laya_forward(const lg_laya_input *in, int n, float *logits, float *act, lg_cancel_fn cancel, void *arg) {
  if (arch != Arch::Laya) fail(LG_ERR_UNSUPPORTED, "laya forward: the model is not a Laya encoder");
  LG_REQUIRE(in && n > 0 && logits && act, "laya forward: need inputs and outputs");
  int R = 0;
  for (int i = 0; i < n; ++i) {  // model.rs:311-335
    const lg_laya_input &q = in[i];
    if (q.n < 1 || q.n > ctx || q.qtype < 0 || q.qtype >= 3 || q.k < 1 || q.k > 16 || !q.ids || !q.markers)
      fail(LG_ERR_INVALID, "invalid inference input shape");
    for (int j = 0; j < q.k; ++j)
      if (q.markers[j] < 0 || q.markers[j] >= q.n) fail(LG_ERR_INVALID, "invalid inference input shape");
    for (int j = 0; j < q.n; ++j)
      if (q.ids[j] < 0 || q.ids[j] >= V) fail(LG_ERR_INVALID, "token ID out of range");
    R += q.k;
  }
  // fresh sequences, released whatever happens
  struct Held {
    Engine &E;
    std::vector<int> seqs;
    BatchPlan *b = nullptr;
    ~Held() {
      try {
        if (b) E.batch_free(b);
        for (int s : seqs) E.seq_free(s);
      } catch (...) {
      }
    }
  } held{*this, {}};
  std::vector<lg_request> reqs(n);
  std::vector<int32_t> meta;  // qtype per input, first logit row per input, markers per input
  for (int i = 0; i < n; ++i) {
    held.seqs.push_back(seq_create());
    reqs[i] = {held.seqs.back(), in[i].ids, in[i].n, in[i].markers, in[i].k};
  }
  held.b = batch_create(reqs.data(), n);
  BatchPlan &b = *held.b;
  int first = 0;
  for (int i = 0; i < n; ++i) meta.push_back(in[i].qtype);
  for (int i = 0; i < n; ++i) {
    meta.push_back(first);
    first += in[i].k;
  }
  for (int i = 0; i < n; ++i) meta.push_back(in[i].k);
  const int dd = d, a1 = laya_act1_.w.rows;
  // tail workspace: marker rows normalised, scorer hidden, logits, pooled, act hidden, act
  const size_t tail = size_t(R) * dd * 2 + R + size_t(n) * (dd + 4) + size_t(n) * a1 + size_t(n) * 2 + 64;
  ws_out_.ensure(tail * 4 + meta.size() * 4 + 1024);
  float *gn = ws_out_.as<float>(), *s1 = gn + size_t(R) * dd, *lg = s1 + size_t(R) * dd;
  float *pooled = lg + R, *xa = pooled + size_t(n) * (dd + 4), *ac = xa + size_t(n) * a1;
  int32_t *dm = reinterpret_cast<int32_t *>(ac + size_t(n) * 2 + 64);
  HIP_CHECK(hipMemcpyAsync(dm, meta.data(), meta.size() * 4, hipMemcpyHostToDevice, stream));
  const int32_t *qt = dm, *lgf = dm + n, *lgc = dm + 2 * n;
  run_laya(b, qt, cancel, arg);
  for (size_t r = 0; r < b.seqs.size(); ++r) seq(b.seqs[r]).len += b.n[r];
  b.ran = true;
  prof.begin("laya_tail", stream);
  // model.rs:384-403: marker rows -> norm -> fc1 -> gelu -> fc2 (option logits); act features
  launch_layer_norm(ws_x_.as<float>(), b.gather, R, dd, laya_scorenorm_.w, laya_scorenorm_.b, laya_scorenorm_.eps,
                    nullptr, nullptr, nullptr, nullptr, nullptr, gn, stream);
  launch_gemm_generic(gn, R, laya_score1_.w, laya_score1_.b, s1, stream);
  launch_gelu_inplace(s1, int64_t(R) * dd, stream);
  launch_gemm_generic(s1, R, laya_score2_.w, laya_score2_.b, lg, stream);
  launch_laya_act_features(ws_x_.as<float>(), dd, b.seq_row0, lgf, lgc, lg, n, pooled, stream);
  launch_gemm_generic(pooled, n, laya_act1_.w, laya_act1_.b, xa, stream);
  launch_gelu_inplace(xa, int64_t(n) * a1, stream);
  launch_gemm_generic(xa, n, laya_act2_.w, laya_act2_.b, ac, stream);
  prof.end(0, 0, stream);
  HIP_CHECK(hipMemcpyAsync(logits, lg, size_t(R) * 4, hipMemcpyDeviceToHost, stream));
  HIP_CHECK(hipMemcpyAsync(act, ac, size_t(n) * 2 * 4, hipMemcpyDeviceToHost, stream));
  sync();
  for (int i = 0; i < R; ++i)
    if (!std::isfinite(logits[i])) fail(LG_ERR_INVALID, "non-finite model output");
  for (int i = 0; i < 2 * n; ++i)
    if (!std::isfinite(act[i])) fail(LG_ERR_INVALID, "non-finite model output");
}

}  // namespace lg
