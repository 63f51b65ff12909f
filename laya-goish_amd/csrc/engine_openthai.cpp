// OpenThai-SystemOne on the engine: load (src/models/openthai/model.rs:96-191) and the batched
// forward over fresh sequences (model.rs:192-241, Full::run :244-299, Delta::run :302-362).
//
// Every sequence of a batch is one reference forward: the recurrent state and the attention
// keys live only inside the call (model.rs:2), so no KV pages are used.  Projections of one
// mixer are fused into one matrix (full: q|gate, k, v; DeltaNet: q|k|v, z, a, b) and run on the
// MFMA GEMM with hi/lo activation planes; the mixers' own arithmetic runs in f32 kernels.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "common.h"
#include "engine.h"
#include "json.h"

namespace lg {

void Engine::load_openthai(const Gguf &g) {
  const Json cfg = Json::parse(g.str("openthai.config"), "openthai.config");
  const Json &c = cfg.get("text_config");
  // model.rs:99-115 pins every size to the 0.8B checkpoint.  The head geometry below is what
  // the kernels are built for; hidden/ffn/layer/head counts and the vocabulary come from the
  // config, so smaller models of the same family load too.
  static const std::pair<const char *, int> fixed[] = {
      {"head_dim", 256}, {"linear_conv_kernel_dim", 4}, {"linear_key_head_dim", 128}, {"linear_value_head_dim", 128}};
  for (const auto &kv : fixed)
    if (c.get(kv.first).num() != kv.second) fail(LG_ERR_UNSUPPORTED, "unsupported OpenThai config %s", kv.first);
  d = int(c.get("hidden_size").num());
  f = int(c.get("intermediate_size").num());
  L = int(c.get("num_hidden_layers").num());
  hq = int(c.get("num_attention_heads").num());
  hkv = int(c.get("num_key_value_heads").num());
  nh = int(c.get("linear_num_value_heads").num());
  V = int(c.get("vocab_size").num());
  hd = 256;
  if (c.get("linear_num_key_heads").num() != nh) fail(LG_ERR_UNSUPPORTED, "unsupported OpenThai config linear_num_key_heads");
  if (L < 1 || hq < 1 || hkv < 1 || hq % hkv || V < 1)
    fail(LG_ERR_FORMAT, "invalid OpenThai dimensions");
  if (d < 128 || d % 128 || f < 64 || f % 64 || nh < 1 || nh > 32)
    fail(LG_ERR_UNSUPPORTED, "OpenThai sizes outside the kernels' shapes (hidden %d, ffn %d, linear heads %d)", d, f, nh);
  const Json &rp = c.get("rope_parameters");
  const int answer = int(cfg.get("answer_token_id").num());
  if (cfg.get("n_slots").num() != 256 || cfg.get("abstain_slot").num() != 255 || answer < 0 || answer >= V ||
      c.get("rms_norm_eps").num() != 1e-6 || rp.get("rope_theta").num() != 10000000.0 ||
      rp.get("partial_rotary_factor").num() != 0.25 || rp.get("rope_type").str() != "default")
    fail(LG_ERR_UNSUPPORTED, "unsupported OpenThai head/normalization/rotary configuration");
  eps = 1e-6f;
  ctx = int(g.num("openthai.context_length", 4096));
  const int state = int(g.num("openthai.state_length", 2048));
  if (ctx < 32 || ctx > 8192 || state < 1 || state > ctx) fail(LG_ERR_FORMAT, "invalid OpenThai sequence budgets");
  const TensorInfo *emb = g.tensor("model.embed_tokens.weight");
  if (!emb || emb->dims.size() != 2 || emb->cols() != uint64_t(d) || emb->rows() != uint64_t(V) ||
      (emb->kind != LG_F16 && emb->kind != LG_F32))
    fail(LG_ERR_FORMAT, "OpenThai embeddings must be F32/F16 with shape [%d,%d]", V, d);
  const Json &types = c.get("layer_types");
  ot_.resize(L);
  for (int l = 0; l < L; ++l) {
    const std::string &t = types.at(size_t(l)).str();
    if (t == "full_attention") ot_[l].full = true;
    else if (t != "linear_attention") fail(LG_ERR_UNSUPPORTED, "unsupported OpenThai layer type");
  }
  const int lw = nh * 128, cd = 3 * lw;
  ldp_full_ = (2 * hq + 2 * hkv) * 256;
  // padded to a multiple of 256 rows, the 256 x 256 GEMM's tile width
  ldp_delta_ = (cd + lw + 2 * nh + 255) / 256 * 256;

  // weight arena: every tensor but the embedding table as f32 at most, plus the pad rows of
  // the DeltaNet projections and the RoPE tables
  size_t total = 0;
  for (const auto &t : g.tensors()) {
    if (t.name == "model.embed_tokens.weight") continue;
    uint64_t count = 1;
    for (auto v : t.dims) count *= v;
    total += align256(count * 4) + 512;
  }
  total += size_t(L) * (align256(size_t(256) * d * 4) + 512) + 2 * (align256(size_t(ctx) * 32 * 4) + 512) + 4096;
  arena_size_ = total;
  if (hipMalloc(&arena_, arena_size_) != hipSuccess) {
    arena_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %zu bytes of weights", arena_size_);
  }
  emb_kind = emb->kind;
  if (hipMalloc(&emb_, emb->len) != hipSuccess) {
    emb_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %llu bytes of embeddings", (unsigned long long)emb->len);
  }
  uploader().bytes(g.data(*emb), emb->len, emb_);
  weight_bytes_ += int64_t(emb->len);

  for (int l = 0; l < L; ++l) {
    OtLayer &y = ot_[l];
    const std::string p = "model.layers." + std::to_string(l) + ".";
    y.n1 = upload_vector_f32(g, p + "input_layernorm.weight", d, 1.0f);
    y.n2 = upload_vector_f32(g, p + "post_attention_layernorm.weight", d, 1.0f);
    if (y.full) {
      y.proj = upload_matrix(g, {p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight", p + "self_attn.v_proj.weight"}, d);
      if (y.proj.rows != ldp_full_ || named_[p + "self_attn.q_proj.weight"].rows != 2 * hq * 256 ||
          named_[p + "self_attn.k_proj.weight"].rows != hkv * 256)
        fail(LG_ERR_FORMAT, "%sself_attn: unexpected matrix shape", p.c_str());
      y.out = upload_matrix(g, {p + "self_attn.o_proj.weight"}, hq * 256);
      y.qn1 = upload_vector_f32(g, p + "self_attn.q_norm.weight", 256, 1.0f);
      y.kn1 = upload_vector_f32(g, p + "self_attn.k_norm.weight", 256, 1.0f);
    } else {
      const std::string a = p + "linear_attn.";
      y.proj = upload_matrix(g, {a + "in_proj_qkv.weight", a + "in_proj_z.weight", a + "in_proj_a.weight", a + "in_proj_b.weight"},
                             d, 256);
      if (y.proj.rows != ldp_delta_ || named_[a + "in_proj_qkv.weight"].rows != cd || named_[a + "in_proj_z.weight"].rows != lw ||
          named_[a + "in_proj_a.weight"].rows != nh)
        fail(LG_ERR_FORMAT, "%slinear_attn: unexpected matrix shape", p.c_str());
      y.out = upload_matrix(g, {a + "out_proj.weight"}, lw);
      y.conv = upload_vector_f32(g, a + "conv1d.weight", int64_t(cd) * 4);
      y.dt = upload_vector_f32(g, a + "dt_bias", nh);
      y.alog = upload_vector_f32(g, a + "A_log", nh);
      y.norm = upload_vector_f32(g, a + "norm.weight", 128);
    }
    if (y.out.rows != d) fail(LG_ERR_FORMAT, "%s: unexpected matrix shape", (p + (y.full ? "self_attn.o_proj" : "linear_attn.out_proj")).c_str());
    y.wi = upload_matrix(g, {p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"}, d);
    if (y.wi.rows != 2 * f) fail(LG_ERR_FORMAT, "%smlp.gate_proj.weight: unexpected matrix shape", p.c_str());
    y.wd = upload_matrix(g, {p + "mlp.down_proj.weight"}, f);
    if (y.wd.rows != d) fail(LG_ERR_FORMAT, "%smlp.down_proj.weight: unexpected matrix shape", p.c_str());
    // F16 matrices are their own operand form for the large-batch 256 x 256 GEMM (nothing allocated)
    for (DevMatrix *m : {&y.proj, &y.out, &y.wi, &y.wd})
      if (m->kind == LG_F16) add_prefill_copy(*m);
  }
  final_norm_ = upload_vector_f32(g, "model.norm.weight", d, 1.0f);
  head_ = upload_matrix(g, {"slot_head.weight"}, d);
  if (head_.rows != 256) fail(LG_ERR_FORMAT, "slot_head.weight: unexpected matrix shape");
  head_bias_ = upload_vector_f32(g, "slot_head.bias", 256);
  // partial RoPE angles of model.rs:264-266, angle = i / 1e7^(2j/64) in f32 with the host's
  // powf/cosf/sinf, shared by every full-attention layer: tables [ctx][32]
  std::vector<float> cs(size_t(ctx) * 32), sn(size_t(ctx) * 32);
  for (int i = 0; i < ctx; ++i)
    for (int j = 0; j < 32; ++j) {
      const float angle = float(i) / powf(10000000.0f, float(2 * j) / 64.0f);
      cs[size_t(i) * 32 + j] = cosf(angle);
      sn[size_t(i) * 32 + j] = sinf(angle);
    }
  cos_ = static_cast<float *>(carve(cs.size() * 4));
  sin_ = static_cast<float *>(carve(sn.size() * 4));
  HIP_CHECK(hipMemcpy(cos_, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(sin_, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
}

void Engine::run_openthai(BatchPlan &b, lg_cancel_fn cancel, void *arg) {
  const int T = b.T, lw = nh * 128, qw = hq * 256, kvw = hkv * 256;
  const int nseq = int(b.seqs.size());
  const int planes = split() ? 2 : 1;
  const int ldp = std::max(ldp_full_, ldp_delta_);
  const int mix = std::max(qw, lw);
  ws_x_.ensure(size_t(T) * d * 4);
  ws_h16_.ensure(size_t(T) * d * 2 * planes);
  ws_qkv_.ensure(size_t(T) * ldp * 4);
  ws_att16_.ensure(size_t(T) * mix * 2 * planes);
  ws_act16_.ensure(size_t(T) * f * 2 * planes);
  ws_ot_qk_.ensure(size_t(T) * std::max(2 * lw, qw) * 4);
  ws_ot_v_.ensure(size_t(T) * std::max(lw, kvw) * 4);
  ws_ot_gb_.ensure(size_t(T) * nh * 2 * 4);
  ws_ot_o_.ensure(size_t(T) * lw * 4);
  ws_ot_chunk_.ensure(ot_delta_chunk_floats(T, nseq, nh) * 4);
  const int max_n = *std::max_element(b.n.begin(), b.n.end());
  auto lo = [&](DevBuf &buf, int64_t n) { return split() ? buf.as<_Float16>() + n : nullptr; };
  float *x = ws_x_.as<float>(), *proj = ws_qkv_.as<float>();
  _Float16 *h16 = ws_h16_.as<_Float16>(), *h16lo = lo(ws_h16_, int64_t(T) * d);
  _Float16 *att = ws_att16_.as<_Float16>();
  _Float16 *act = ws_act16_.as<_Float16>(), *actlo = lo(ws_act16_, int64_t(T) * f);
  float *qk = ws_ot_qk_.as<float>(), *vb = ws_ot_v_.as<float>(), *gb = ws_ot_gb_.as<float>(), *o = ws_ot_o_.as<float>();
  prof.begin("embed", stream);
  launch_embed(emb_, emb_kind, b.ids, T, d, V, x, stream);
  prof.end(double(T) * d * (emb_kind == LG_F16 ? 6 : 8), 0, stream);
  for (int l = 0; l < L; ++l) {
    if (cancel && cancel(arg)) fail(LG_ERR_CANCELED, "request canceled");
    const OtLayer &y = ot_[l];
    prof.begin("rmsnorm", stream);
    launch_rmsnorm_f16(x, T, d, y.n1, eps, h16, h16lo, stream);
    prof.end(double(T) * d * (4 + 2 * planes), 0, stream);
    if (y.full) {
      _Float16 *attlo = lo(ws_att16_, int64_t(T) * qw);
      gemm(h16, h16lo, T, y.proj, Epi::F32, proj, nullptr, nullptr, ldp_full_, nullptr);
      prof.begin("ot_attn_prep", stream);
      launch_ot_attn_prep(proj, ldp_full_, T, hq, hkv, b.tok_pos, y.qn1, y.kn1, cos_, sin_, qk, vb, stream);
      prof.end(double(T) * (qw + kvw) * 8, 0, stream);
      prof.begin("ot_attn", stream);
      if ((hq / hkv) % 4 == 0) {
        ws_ot_part_.ensure(size_t(ot_attn_part_floats(b.nitems, hq)) * 4);
        launch_ot_attn_mfma(qk, vb, proj, ldp_full_, hq, hkv, b.it_row0, b.it_pos0, b.it_nq, b.it_klo, b.it_khi,
                            b.nitems, b.cb_row0, b.cb_nq, b.cb_first, b.cb_n, b.ncomb, ws_ot_part_.as<float>(), att,
                            attlo, stream);
      } else {
        launch_ot_attn(qk, vb, proj, ldp_full_, hq, hkv, b.tile_row0, b.tile_pos0, b.tile_n, b.ntiles, att, attlo,
                       stream);
      }
      prof.end(0, 0, stream);
      gemm(att, attlo, T, y.out, Epi::ADD, x, nullptr, nullptr, d, nullptr);
    } else {
      _Float16 *attlo = lo(ws_att16_, int64_t(T) * lw);
      gemm(h16, h16lo, T, y.proj, Epi::F32, proj, nullptr, nullptr, ldp_delta_, nullptr);
      prof.begin("ot_delta_prep", stream);
      launch_ot_delta_prep(proj, ldp_delta_, T, b.tok_pos, y.conv, y.alog, y.dt, nh, qk, vb, gb, stream);
      prof.end(double(T) * (3 * lw * 4 * 2 + lw * 4 + nh * 8), 0, stream);
      prof.begin("ot_delta_scan", stream);
      launch_ot_delta_scan(qk, vb, gb, b.seq_row0, b.seq_n, nseq, T, max_n, nh, ws_ot_chunk_.as<float>(), o, stream);
      prof.end(double(T) * (3 * lw + 2 * nh + lw) * 4, 4.0 * double(T) * nh * 128 * 128, stream);
      prof.begin("ot_delta_out", stream);
      launch_ot_delta_out(o, T, nh, y.norm, proj, ldp_delta_, 3 * lw, att, attlo, stream);
      prof.end(double(T) * lw * (8 + 2 * planes), 0, stream);
      gemm(att, attlo, T, y.out, Epi::ADD, x, nullptr, nullptr, d, nullptr);
    }
    prof.begin("rmsnorm", stream);
    launch_rmsnorm_f16(x, T, d, y.n2, eps, h16, h16lo, stream);
    prof.end(double(T) * d * (4 + 2 * planes), 0, stream);
    gemm(h16, h16lo, T, y.wi, Epi::SWIGLU, nullptr, act, actlo, f, nullptr);
    gemm(act, actlo, T, y.wd, Epi::ADD, x, nullptr, nullptr, d, nullptr);
  }
}

}  // namespace lg
