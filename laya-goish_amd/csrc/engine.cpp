// Engine: model upload, paged KV cache, batched prefill and greedy decode drivers.
#include "engine.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>

#include "common.h"
#include "noalloc.h"

namespace lg {

// ------------------------------------------------------------------ DevBuf / Profiler
void DevBuf::ensure(size_t bytes) {
  if (bytes <= n) return;
  if (p) HIP_CHECK(hipFree(p));
  p = nullptr;
  n = 0;
  const size_t want = std::max(bytes, size_t(256));
  if (hipMalloc(&p, want) != hipSuccess) {
    p = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %zu bytes of workspace", want);
  }
  n = want;
}

DevBuf::~DevBuf() {
  if (p) (void)hipFree(p);
}

KernelTimer *&kernel_timer() {
  thread_local KernelTimer *t = nullptr;
  return t;
}

hipEvent_t Profiler::take() {
  if (pool_.empty()) {
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    pool_.push_back(e);
  }
  hipEvent_t e = pool_.back();
  pool_.pop_back();
  return e;
}

void Profiler::begin_kernel(const char *cls) {
  if (!on_) return;
  cur_ = cls;
  cur_a_ = take();
  cur_b_ = take();
  timer_.start = cur_a_;
  timer_.stop = cur_b_;
  kernel_timer() = &timer_;
}

void Profiler::end_kernel(double bytes, double flops) {
  if (!on_) return;
  kernel_timer() = nullptr;
  open_.push_back({cur_, cur_a_, cur_b_, bytes, flops});
  if (open_.size() > 4096) drain();
}

void Profiler::begin(const char *cls, hipStream_t st) {
  if (!on_) return;
  cur_ = cls;
  if (pool_.empty()) {
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    pool_.push_back(e);
  }
  cur_a_ = pool_.back();
  pool_.pop_back();
  HIP_CHECK(hipEventRecord(cur_a_, st));
}

void Profiler::end(double bytes, double flops, hipStream_t st) {
  if (!on_) return;
  if (pool_.empty()) {
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    pool_.push_back(e);
  }
  hipEvent_t b = pool_.back();
  pool_.pop_back();
  HIP_CHECK(hipEventRecord(b, st));
  open_.push_back({cur_, cur_a_, b, bytes, flops});
  if (open_.size() > 4096) drain();
}

void Profiler::drain() {
  for (auto &r : open_) {
    HIP_CHECK(hipEventSynchronize(r.b));
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
    Sum &s = sums_[r.cls];
    s.launches += 1;
    s.ms += ms;
    s.bytes += r.bytes;
    s.flops += r.flops;
    pool_.push_back(r.a);
    pool_.push_back(r.b);
  }
  open_.clear();
}

void Profiler::read(const std::string &cls, int64_t *launches, double *ms, double *bytes, double *flops) {
  drain();
  Sum s;
  auto it = sums_.find(cls);
  if (it != sums_.end()) s = it->second;
  if (launches) *launches = s.launches;
  if (ms) *ms = s.ms;
  if (bytes) *bytes = s.bytes;
  if (flops) *flops = s.flops;
}

void Profiler::reset() {
  drain();
  sums_.clear();
}

Profiler::~Profiler() {
  for (auto &r : open_) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : pool_) (void)hipEventDestroy(e);
}

// ------------------------------------------------------------------ helpers
int64_t q_row_bytes(uint32_t kind, int cols) {
  switch (kind) {
    case LG_F32: return int64_t(cols) * 4;
    case LG_F16: return int64_t(cols) * 2;
    case LG_Q8_0: return cols;
    case LG_Q4_K: return cols / 2;
    case LG_Q6_K: return cols;
  }
  return 0;
}
int64_t s_row_bytes(uint32_t kind, int cols) {
  switch (kind) {
    case LG_Q8_0: return int64_t(cols / 32) * 2;
    case LG_Q4_K: return int64_t(cols / 32) * 8;
    case LG_Q6_K: return int64_t(cols / 16) * 4;
  }
  return 0;
}
DevMatrix sub_rows(const DevMatrix &m, int row0, int nrows) {
  DevMatrix s = m;
  s.rows = nrows;
  s.q = static_cast<uint8_t *>(m.q) + q_row_bytes(m.kind, m.cols) * row0;
  if (m.s) s.s = static_cast<uint8_t *>(m.s) + s_row_bytes(m.kind, m.cols) * row0;
  return s;
}
size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// ------------------------------------------------------------------ streamed upload
Uploader::Uploader(hipStream_t st) : st_(st) {
  for (int i = 0; i < 2; ++i) {
    if (hipHostMalloc(&host_[i], kChunk, hipHostMallocDefault) != hipSuccess) {
      host_[i] = nullptr;
      (void)hipGetLastError();
      fail(LG_ERR_OOM, "cannot allocate %zu bytes of pinned upload staging", kChunk);
    }
    if (hipMalloc(&dev_[i], kChunk) != hipSuccess) {
      dev_[i] = nullptr;
      (void)hipGetLastError();
      fail(LG_ERR_OOM, "cannot allocate %zu bytes of upload staging", kChunk);
    }
    HIP_CHECK(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming));
  }
}

Uploader::~Uploader() {
  if (st_) (void)hipStreamSynchronize(st_);
  for (int i = 0; i < 2; ++i) {
    if (done_[i]) (void)hipEventDestroy(done_[i]);
    if (host_[i]) (void)hipHostFree(host_[i]);
    if (dev_[i]) (void)hipFree(dev_[i]);
  }
}

int Uploader::take() {
  const int s = next_;
  next_ ^= 1;
  if (used_[s]) HIP_CHECK(hipEventSynchronize(done_[s]));
  used_[s] = true;
  return s;
}

void Uploader::bytes(const uint8_t *src, size_t n, void *dst) {
  for (size_t off = 0; off < n; off += kChunk) {
    const size_t c = std::min(kChunk, n - off);
    const int s = take();
    std::memcpy(host_[s], src + off, c);
    HIP_CHECK(hipMemcpyAsync(static_cast<uint8_t *>(dst) + off, host_[s], c, hipMemcpyHostToDevice, st_));
    HIP_CHECK(hipEventRecord(done_[s], st_));
  }
}

void Uploader::matrix(uint32_t kind, const uint8_t *src, int rows, size_t row_bytes, const DevMatrix &m) {
  LG_REQUIRE(row_bytes > 0 && row_bytes <= kChunk, "upload: %zu-byte rows do not fit the staging", row_bytes);
  const int per = int(std::min<size_t>(kChunk / row_bytes, size_t(rows)));
  for (int r0 = 0; r0 < rows; r0 += per) {
    const int n = std::min(per, rows - r0);
    const size_t c = size_t(n) * row_bytes;
    const int s = take();
    std::memcpy(host_[s], src + size_t(r0) * row_bytes, c);
    HIP_CHECK(hipMemcpyAsync(dev_[s], host_[s], c, hipMemcpyHostToDevice, st_));
    DevMatrix part = sub_rows(m, r0, n);
    launch_repack(kind, static_cast<const uint8_t *>(dev_[s]), n, m.cols, part, st_);
    HIP_CHECK(hipEventRecord(done_[s], st_));
  }
}

void Uploader::finish() { HIP_CHECK(hipStreamSynchronize(st_)); }

Uploader &Engine::uploader() {
  if (!up_) up_ = new Uploader(stream);
  return *up_;
}

void Engine::finish_upload() {
  if (up_) {
    up_->finish();
    delete up_;
    up_ = nullptr;
  }
  HIP_CHECK(hipStreamSynchronize(stream));
}

// ------------------------------------------------------------------ construction
Engine::Engine(const Gguf &g, const lg_engine_opts &opts) {
  const auto t_load = std::chrono::steady_clock::now();
  device = opts.device;
  int ndev = 0;
  HIP_CHECK(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) fail(LG_ERR_INVALID, "device %d out of range (%d devices)", device, ndev);
  HIP_CHECK(hipSetDevice(device));
  max_batch_tokens_ = opts.max_batch_tokens > 0 ? opts.max_batch_tokens : 65536;
  if (opts.precision != LG_PREC_EXACT && opts.precision != LG_PREC_FAST && opts.precision != LG_PREC_KV16)
    fail(LG_ERR_INVALID, "unknown precision mode %d", opts.precision);
  precision = opts.precision;
  try {
    if (g.str("general.architecture") == "openthai_systemone") {
      arch = Arch::OpenThai;
      HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
      load_openthai(g);
      decide = decide_spec(g);
      finish_upload();
      load_s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_load).count();
      return;
    }
    if (g.str("general.architecture") == "ggmlc" && g.str("laya.model_name") != "laya-decoder" &&
        g.meta("ggmlc.graph_spec")) {
      arch = Arch::Laya;
      HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
      load_laya(g);
      decide = decide_spec(g);
      laya_decide = laya_spec(g);
      finish_upload();
      load_s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_load).count();
      return;
    }
    load_decoder(g, opts);
    load_s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_load).count();
  } catch (...) {
    release();
    throw;
  }
}

void Engine::load_decoder(const Gguf &g, const lg_engine_opts &opts) {
  if (g.str("general.architecture") != "ggmlc" || g.str("laya.model_name") != "laya-decoder")
    fail(LG_ERR_FORMAT, "unsupported ggmlc model %s", g.str("laya.model_name").c_str());
  L = int(g.num("laya.decoder.block_count", 0));
  d = int(g.num("laya.decoder.embedding_length", 0));
  hq = int(g.num("laya.decoder.head_count", 0));
  hkv = int(g.num("laya.decoder.head_count_kv", 0));
  hd = int(g.num("laya.decoder.key_length", 0));
  f = int(g.num("laya.decoder.feed_forward_length", 0));
  V = int(g.num("laya.decoder.vocab_size", 0));
  ctx = int(g.num("laya.decoder.context_length", 0));
  eps = float(g.num("laya.decoder.layer_norm_rms_epsilon", 1e-5));
  decide = decide_spec(g);
  if (L < 1 || d < 1 || hq < 1 || hkv < 1 || hq % hkv || hd < 2 || hd % 2 || f < 1 || V < 1 || ctx < 1)
    fail(LG_ERR_FORMAT, "invalid laya-decoder dimensions");
  if (d % 64 || (hd != 64 && hd != 128))
    fail(LG_ERR_UNSUPPORTED, "d_model %d / head_dim %d outside the kernels' shapes", d, hd);
  HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  upload(g);
  finish_upload();
  // KV pool: [L][npages][hkv][64][hd] elements (hi/lo f16 planes in EXACT mode, f16 in KV16 and
  // FAST) for K, then V
  int64_t pages = opts.kv_pages;
  if (pages <= 0) {
    const int64_t toks = opts.kv_tokens > 0 ? opts.kv_tokens : 65536;
    pages = toks / 64 + (toks % 64 != 0);
  }
  page_stride_ = int64_t(hkv) * 64 * hd;
  // bytes of the pool; anything past 2^47 (128 TiB) is no device's memory and is refused up front
  const double want = 2.0 * double(L) * double(pages) * double(page_stride_) * kv_elem();
  if (pages > (1 << 30) || want > double(int64_t(1) << 47))
    fail(LG_ERR_OOM, "cannot allocate %.3g bytes of KV pages (%lld pages)", want, (long long)pages);
  npages_ = int(pages);
  const size_t kv_bytes = size_t(2) * L * npages_ * page_stride_ * kv_elem();
  if (hipMalloc(&kv_, kv_bytes) != hipSuccess) {
    kv_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %zu bytes of KV pages", kv_bytes);
  }
  // zero once so never-written slots hold finite values (masked keys multiply V by 0)
  HIP_CHECK(hipMemsetAsync(kv_, 0, kv_bytes, stream));
  refcnt_.assign(npages_, 0);
  free_pages_.resize(npages_);
  for (int i = 0; i < npages_; ++i) free_pages_[i] = npages_ - 1 - i;
  HIP_CHECK(hipStreamSynchronize(stream));
}

Engine::~Engine() { release(); }

void Engine::release() {
  if (stream) (void)hipStreamSynchronize(stream);
  delete up_;
  up_ = nullptr;
  if (arena_) (void)hipFree(arena_);
  if (emb_) (void)hipFree(emb_);
  if (kv_) (void)hipFree(kv_);
  if (stream) (void)hipStreamDestroy(stream);
  arena_ = emb_ = kv_ = nullptr;
  stream = nullptr;
}

void *Engine::carve(size_t bytes) {
  bytes = align256(bytes);
  if (arena_used_ + bytes > arena_size_) fail(LG_ERR_OOM, "weight arena exhausted");
  void *p = static_cast<uint8_t *>(arena_) + arena_used_;
  arena_used_ += bytes;
  return p;
}

float *Engine::upload_vector_f32(const Gguf &g, const std::string &name, int64_t n, float offset) {
  const TensorInfo *t = g.tensor(name);
  if (!t) fail(LG_ERR_FORMAT, "missing tensor %s", name.c_str());
  uint64_t count = 1;
  for (auto v : t->dims) count *= v;
  if (int64_t(count) != n) fail(LG_ERR_FORMAT, "%s: unexpected vector shape", name.c_str());
  std::vector<float> h(n);
  const uint8_t *src = g.data(*t);
  if (t->kind == LG_F32) std::memcpy(h.data(), src, n * 4);
  else if (t->kind == LG_F16)
    for (int64_t i = 0; i < n; ++i) h[i] = half_to_float(uint16_t(src[2 * i] | (src[2 * i + 1] << 8)));
  else fail(LG_ERR_UNSUPPORTED, "%s: vectors must be F32/F16", name.c_str());
  if (offset != 0.0f)
    for (int64_t i = 0; i < n; ++i) h[i] = offset + h[i];
  float *dptr = static_cast<float *>(carve(n * 4));
  HIP_CHECK(hipMemcpy(dptr, h.data(), n * 4, hipMemcpyHostToDevice));
  return dptr;
}

// Upload one or more GGUF matrices with equal kind and row length as one row-concatenated
// device matrix (q|k|v or gate|up): row blocks of the same layout are contiguous.
DevMatrix Engine::upload_matrix(const Gguf &g, const std::vector<std::string> &names, int cols, int pad_to) {
  DevMatrix m;
  std::vector<const TensorInfo *> ts;
  int rows = 0;
  for (const auto &nm : names) {
    const TensorInfo *t = g.tensor(nm);
    if (!t) fail(LG_ERR_FORMAT, "missing tensor %s", nm.c_str());
    if (t->dims.size() != 2 || t->cols() != uint64_t(cols))
      fail(LG_ERR_FORMAT, "%s: unexpected matrix shape", nm.c_str());
    if (!ts.empty() && t->kind != ts[0]->kind) fail(LG_ERR_FORMAT, "%s: mixed kinds in one projection", nm.c_str());
    ts.push_back(t);
    rows += int(t->rows());
  }
  m.kind = ts[0]->kind;
  m.rows = rows;
  m.cols = cols;
  if (m.kind == LG_Q4_0) fail(LG_ERR_UNSUPPORTED, "Q4_0 matrices have no device kernel");
  if ((m.kind == LG_Q4_K || m.kind == LG_Q6_K) && cols % 256)
    fail(LG_ERR_FORMAT, "invalid quantized row alignment");
  const int alloc_rows = pad_to > 0 ? (rows + pad_to - 1) / pad_to * pad_to : rows;
  m.q = carve(size_t(q_row_bytes(m.kind, cols)) * alloc_rows);
  if (s_row_bytes(m.kind, cols)) m.s = carve(size_t(s_row_bytes(m.kind, cols)) * alloc_rows);
  int row0 = 0;
  for (size_t i = 0; i < ts.size(); ++i) {
    const TensorInfo *t = ts[i];
    DevMatrix part = sub_rows(m, row0, int(t->rows()));
    uploader().matrix(t->kind, g.data(*t), part.rows, size_t(t->len / t->rows()), part);
    named_[names[i]] = part;
    row0 += part.rows;
  }
  weight_bytes_ += m.gguf_bytes();
  if (alloc_rows > rows) {  // zero weights in the pad rows: their outputs are 0 and never read
    DevMatrix pad = sub_rows(m, rows, alloc_rows - rows);
    HIP_CHECK(hipMemsetAsync(pad.q, 0, size_t(q_row_bytes(m.kind, cols)) * pad.rows, stream));
    if (pad.s) HIP_CHECK(hipMemsetAsync(pad.s, 0, size_t(s_row_bytes(m.kind, cols)) * pad.rows, stream));
    m.rows = alloc_rows;
  }
  return m;
}

void Engine::add_prefill_copy(DevMatrix &m) {
  if (!split()) return;
  const size_t n = size_t(m.rows) * m.cols;
  if (m.kind == LG_F16) {
    m.pc = static_cast<_Float16 *>(m.q);
    return;
  }
  if (m.kind == LG_Q8_0) {
    m.pc = static_cast<_Float16 *>(carve(n * 2));
    m.pcs = static_cast<float *>(carve(size_t(m.rows) * (m.cols / 32) * 4));
  } else if (m.kind == LG_Q4_K) {  // two-pass form: codes, sub-block scales, correction planes
    m.pkp = ksum_cols(m.cols);
    m.pc = static_cast<_Float16 *>(carve(n * 2));
    m.pcs = static_cast<float *>(carve(size_t(m.rows) * (m.cols / 32) * 4));
    m.pcl = static_cast<_Float16 *>(carve(size_t(m.rows) * m.pkp * 4));
    m.pcr = static_cast<float *>(carve(size_t(m.rows) * 4));
  } else if (m.kind == LG_Q6_K) {
    m.pc = static_cast<_Float16 *>(carve(n * 2));
    m.pcl = static_cast<_Float16 *>(carve(n * 2));
  } else {
    return;
  }
  launch_prefill_copy(m, stream);
}

void Engine::upload(const Gguf &g) {
  // size the arena: every matrix/vector tensor except the embedding table, + 256 B slack each
  size_t total = 0;
  for (const auto &t : g.tensors()) {
    if (t.name == "tok_emb.weight") continue;
    const uint64_t n = t.cols() * t.rows();
    size_t need;
    if (t.dims.size() == 1) need = n * 8;  // vectors: f32 copy, plus a fused-bias copy
    else if (t.name == "cos_full" || t.name == "sin_full") need = n * 4;
    else need = size_t(q_row_bytes(t.kind, int(t.cols())) + s_row_bytes(t.kind, int(t.cols()))) * t.rows();
    if (split() && t.dims.size() == 2 && t.name != "output.weight")
      need += prefill_copy_bytes(t.kind, int(t.rows()), int(t.cols())) + 1024;  // up to four 256-B aligned carves
    total += align256(need) + 512;
  }
  arena_size_ = total;
  if (hipMalloc(&arena_, arena_size_) != hipSuccess) {
    arena_ = nullptr;
    (void)hipGetLastError();
    fail(LG_ERR_OOM, "cannot allocate %zu bytes of weights", arena_size_);
  }
  // embedding table: raw F16/F32 rows [V][d]
  const TensorInfo *emb = g.tensor("tok_emb.weight");
  if (!emb || emb->cols() != uint64_t(d) || emb->rows() != uint64_t(V) ||
      (emb->kind != LG_F16 && emb->kind != LG_F32))
    fail(LG_ERR_FORMAT, "tok_emb.weight must be F32/F16 [d, vocab]");
  emb_kind = emb->kind;
  HIP_CHECK(hipMalloc(&emb_, emb->len));
  uploader().bytes(g.data(*emb), emb->len, emb_);
  weight_bytes_ += int64_t(emb->len);

  const int qw = hq * hd, kvw = hkv * hd;
  layers_.resize(L);
  for (int l = 0; l < L; ++l) {
    Layer &ly = layers_[l];
    const std::string i = std::to_string(l);
    ly.attn_norm = upload_vector_f32(g, "attn_norm." + i + ".weight", d);
    ly.ffn_norm = upload_vector_f32(g, "ffn_norm." + i + ".weight", d);
    if (g.tensor("qkv." + i + ".weight")) {
      ProjPart p;
      p.w = upload_matrix(g, {"qkv." + i + ".weight"}, d);
      if (p.w.rows != qw + 2 * kvw) fail(LG_ERR_FORMAT, "qkv.%d.weight: unexpected matrix shape", l);
      if (g.tensor("qkv." + i + ".bias")) p.bias = upload_vector_f32(g, "qkv." + i + ".bias", qw + 2 * kvw);
      ly.qkv.push_back(p);
    } else {
      // separate q/k/v: fuse runs of equal kind into one device matrix (one GEMM / GEMV each)
      const std::string nm[3] = {"q." + i + ".weight", "k." + i + ".weight", "v." + i + ".weight"};
      const std::string bn[3] = {"q." + i + ".bias", "k." + i + ".bias", "v." + i + ".bias"};
      const int rows[3] = {qw, kvw, kvw};
      uint32_t kinds[3];
      int nbias = 0;
      for (int j = 0; j < 3; ++j) {
        const TensorInfo *t = g.tensor(nm[j]);
        if (!t) fail(LG_ERR_FORMAT, "missing tensor %s", nm[j].c_str());
        kinds[j] = t->kind;
        nbias += g.tensor(bn[j]) ? 1 : 0;
      }
      if (nbias != 0 && nbias != 3) fail(LG_ERR_FORMAT, "layer %d: q/k/v biases must all be present or all absent", l);
      int j = 0, col = 0;
      while (j < 3) {
        int e = j + 1;
        while (e < 3 && kinds[e] == kinds[j]) ++e;
        ProjPart p;
        p.w = upload_matrix(g, std::vector<std::string>(nm + j, nm + e), d);
        int nrows = 0;
        for (int t = j; t < e; ++t) nrows += rows[t];
        if (p.w.rows != nrows) fail(LG_ERR_FORMAT, "%s: unexpected matrix shape", nm[j].c_str());
        p.col0 = col;
        if (nbias) {
          p.bias = static_cast<float *>(carve(size_t(nrows) * 4));
          int off = 0;
          for (int t = j; t < e; ++t) {
            float *tmp = upload_vector_f32(g, bn[t], rows[t]);
            HIP_CHECK(hipMemcpy(const_cast<float *>(p.bias) + off, tmp, size_t(rows[t]) * 4, hipMemcpyDeviceToDevice));
            off += rows[t];
          }
        }
        ly.qkv.push_back(p);
        col += nrows;
        j = e;
      }
    }
    ly.wo = upload_matrix(g, {"wo." + i + ".weight"}, qw);
    if (ly.wo.rows != d) fail(LG_ERR_FORMAT, "wo.%d.weight: unexpected matrix shape", l);
    if (g.tensor("mlp_wi." + i + ".weight")) ly.wi = upload_matrix(g, {"mlp_wi." + i + ".weight"}, d);
    else ly.wi = upload_matrix(g, {"gate." + i + ".weight", "up." + i + ".weight"}, d);
    if (ly.wi.rows != 2 * f) fail(LG_ERR_FORMAT, "mlp_wi.%d.weight: unexpected matrix shape", l);
    ly.wd = upload_matrix(g, {"mlp_wo." + i + ".weight"}, f);
    if (ly.wd.rows != d) fail(LG_ERR_FORMAT, "mlp_wo.%d.weight: unexpected matrix shape", l);
    for (ProjPart &p : ly.qkv) add_prefill_copy(p.w);
    add_prefill_copy(ly.wo);
    add_prefill_copy(ly.wi);
    add_prefill_copy(ly.wd);
  }
  final_norm_ = upload_vector_f32(g, "final_norm.weight", d);
  head_ = upload_matrix(g, {"output.weight"}, d);
  if (head_.rows != V) fail(LG_ERR_FORMAT, "output.weight: unexpected matrix shape");
  cos_ = upload_vector_f32(g, "cos_full", int64_t(ctx) * hd);
  sin_ = upload_vector_f32(g, "sin_full", int64_t(ctx) * hd);
}

lg_model_info Engine::info() const {
  lg_model_info i{};
  i.layers = L;
  i.d_model = d;
  i.heads = hq;
  i.kv_heads = hkv;
  i.head_dim = hd;
  i.ffn = f;
  i.vocab = V;
  i.context = ctx;
  i.kind_attn = !layers_.empty() ? layers_[0].wo.kind : !ot_.empty() ? ot_[0].out.kind : 0;
  i.kind_ffn = !layers_.empty() ? layers_[0].wd.kind : !ot_.empty() ? ot_[0].wd.kind : 0;
  i.kind_head = head_.kind;
  i.weight_bytes = weight_bytes_;
  i.kv_bytes = int64_t(2) * L * npages_ * page_stride_ * kv_elem();
  i.kv_pages = npages_;
  i.kv_page_tokens = 64;
  i.precision = precision;
  i.kv_elem_bytes = kv_elem();
  i.arch = int(arch);
  i.linear_heads = nh;
  i.full_layers = 0;
  for (const OtLayer &y : ot_) i.full_layers += y.full ? 1 : 0;
  i.load_seconds = load_s_;
  return i;
}

void Engine::sync() { HIP_CHECK(hipStreamSynchronize(stream)); }

KvGeom Engine::geom() const {
  KvGeom g;
  g.page_tokens = 64;
  g.hkv = hkv;
  g.hd = hd;
  g.page_stride = page_stride_;
  g.layer_stride = int64_t(npages_) * page_stride_;
  g.split = kv_split() ? 1 : 0;
  return g;
}
void *Engine::kpool(int layer) const {
  return static_cast<uint8_t *>(kv_) + int64_t(layer) * npages_ * page_stride_ * kv_elem();
}
void *Engine::vpool(int layer) const {
  return static_cast<uint8_t *>(kv_) + (int64_t(L) + layer) * npages_ * page_stride_ * kv_elem();
}

// ------------------------------------------------------------------ kernels with profiling
const _Float16 *Engine::chunk_sums(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W) {
  if (!A_lo || !needs_ksum(W)) return nullptr;
  ws_ksum_.ensure(size_t(M) * W.pkp * 4);
  prof.begin("ksum", stream);
  launch_chunk_sums(A, A_lo, M, W.cols, W.pkp, ws_ksum_.as<_Float16>(), stream);
  prof.end(double(M) * W.cols * 4 + double(M) * W.pkp * 4, double(M) * W.cols * 2, stream);
  return ws_ksum_.as<_Float16>();
}

void Engine::gemm(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W, Epi epi, float *C,
                  _Float16 *C16, _Float16 *C16_lo, int ldc, const float *bias) {
  const _Float16 *ks = chunk_sums(A, A_lo, M, W);
  prof.begin_kernel("gemm");
  launch_gemm(A, A_lo, M, W, epi, C, C16, C16_lo, ldc, bias, stream, ks);
  prof.end_kernel(double(W.bytes()) + double(M) * W.cols * 2, 2.0 * M * double(W.rows) * W.cols);
}

void Engine::gemv(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                  const float *norm_w) {
  prof.begin_kernel("gemv");
  launch_gemv(x, W, epi, y, bias, norm_w, eps, stream);
  // algorithmic bytes: the GGUF-encoded weight bytes of the matrix
  prof.end_kernel(double(W.gguf_bytes()), 2.0 * double(W.rows) * W.cols);
}

// ------------------------------------------------------------------ matmul drop-in
void Engine::matmul(const std::string &name, const float *x, int m, const float *bias, float *y) {
  auto it = named_.find(name);
  if (it == named_.end()) fail(LG_ERR_INVALID, "missing tensor %s", name.c_str());
  const DevMatrix &W = it->second;
  LG_REQUIRE(m > 0, "matmul: m must be positive");
  const size_t xb = size_t(m) * W.cols * 4, yb = size_t(m) * W.rows * 4;
  DevBuf dx, dy, db, dh;
  dx.ensure(xb);
  dy.ensure(yb);
  HIP_CHECK(hipMemcpyAsync(dx.p, x, xb, hipMemcpyHostToDevice, stream));
  const float *dbias = nullptr;
  if (bias) {
    db.ensure(size_t(W.rows) * 4);
    HIP_CHECK(hipMemcpyAsync(db.p, bias, size_t(W.rows) * 4, hipMemcpyHostToDevice, stream));
    dbias = db.as<float>();
  }
  const bool tiled = W.kind != LG_F32 && W.cols % 64 == 0 && W.rows % 128 == 0;
  if (m == 1 && W.cols % 16 == 0 && W.cols * 4 <= 64 * 1024 && W.kind != LG_F32) {
    gemv(dx.as<float>(), W, Epi::F32, dy.as<float>(), dbias, nullptr);
  } else if (tiled && m > 1) {
    const int64_t n = int64_t(m) * W.cols;
    dh.ensure(size_t(n) * 4);
    _Float16 *hi = dh.as<_Float16>(), *lo = split() ? hi + n : nullptr;
    launch_cvt_f16(dx.as<float>(), n, hi, lo, stream);
    gemm(hi, lo, m, W, Epi::F32, dy.as<float>(), nullptr, nullptr, W.rows, dbias);
  } else {
    launch_gemm_generic(dx.as<float>(), m, W, dbias, dy.as<float>(), stream);
  }
  HIP_CHECK(hipMemcpyAsync(y, dy.p, yb, hipMemcpyDeviceToHost, stream));
  HIP_CHECK(hipStreamSynchronize(stream));
}

// ------------------------------------------------------------------ sequences / pages
Seq &Engine::seq(int id) {
  auto it = seqs_.find(id);
  if (it == seqs_.end()) fail(LG_ERR_INVALID, "unknown sequence %d", id);
  return it->second;
}

int Engine::seq_create() {
  const int id = next_seq_++;
  seqs_[id] = Seq{};
  return id;
}

int Engine::alloc_page() {
  if (free_pages_.empty()) fail(LG_ERR_OOM, "KV cache exhausted (%d pages)", npages_);
  const int p = free_pages_.back();
  free_pages_.pop_back();
  refcnt_[p] = 1;
  return p;
}

void Engine::release_page(int p) {
  if (--refcnt_[p] == 0) free_pages_.push_back(p);
}

void Engine::reserve_pages(Seq &s, int upto) {
  if (upto > ctx) fail(LG_ERR_INVALID, "sequence of %d tokens exceeds the context length %d", upto, ctx);
  const int need = (upto + 63) / 64;
  const int extra = need - int(s.pages.size());
  if (extra > int(free_pages_.size()))
    fail(LG_ERR_OOM, "KV cache exhausted: need %d more pages, %zu free", extra, free_pages_.size());
  while (int(s.pages.size()) < need) s.pages.push_back(alloc_page());
}

int Engine::seq_fork(int parent, int ntokens) {
  if (fresh_only()) fail(LG_ERR_UNSUPPORTED, "fork: sequences of this model keep no cache to share");
  Seq &p = seq(parent);
  LG_REQUIRE(ntokens >= 0 && ntokens <= p.len, "fork: %d tokens outside the parent's %d", ntokens, p.len);
  Seq c;
  c.len = ntokens;
  const int full = ntokens / 64, rem = ntokens % 64;
  for (int i = 0; i < full; ++i) {
    c.pages.push_back(p.pages[i]);
    ++refcnt_[p.pages[i]];
  }
  if (rem) {  // private copy of the partly filled page, all layers, K and V
    const int np = alloc_page();
    for (int l = 0; l < L; ++l) {
      const size_t bytes = size_t(page_stride_) * kv_elem();
      uint8_t *kb = static_cast<uint8_t *>(kpool(l)), *vb = static_cast<uint8_t *>(vpool(l));
      HIP_CHECK(hipMemcpyAsync(kb + np * bytes, kb + p.pages[full] * bytes, bytes, hipMemcpyDeviceToDevice, stream));
      HIP_CHECK(hipMemcpyAsync(vb + np * bytes, vb + p.pages[full] * bytes, bytes, hipMemcpyDeviceToDevice, stream));
    }
    c.pages.push_back(np);
  }
  const int id = next_seq_++;
  seqs_[id] = std::move(c);
  return id;
}

void Engine::seq_free(int id) {
  Seq &s = seq(id);
  for (int p : s.pages) release_page(p);
  seqs_.erase(id);
}

int Engine::seq_len(int id) const {
  auto it = seqs_.find(id);
  if (it == seqs_.end()) fail(LG_ERR_INVALID, "unknown sequence %d", id);
  return it->second.len;
}

void Engine::seq_kv_read(int id, int layer, int pos0, int n, float *k, float *v) {
  LG_REQUIRE(arch == Arch::Decoder, "kv read: the model keeps no KV cache");
  const Seq &s = seq(id);
  LG_REQUIRE(layer >= 0 && layer < L, "kv read: layer %d outside 0..%d", layer, L - 1);
  LG_REQUIRE(pos0 >= 0 && n >= 0 && int64_t(pos0) + n <= s.len, "kv read: positions [%d, %d) outside the sequence's %d",
             pos0, pos0 + n, s.len);
  LG_REQUIRE(k && v, "kv read: missing output");
  const int kvw = hkv * hd, es = kv_elem();
  std::vector<uint8_t> kp(size_t(page_stride_) * es), vp(size_t(page_stride_) * es);
  HIP_CHECK(hipStreamSynchronize(stream));
  int loaded = -1;
  for (int i = 0; i < n; ++i) {
    const int pos = pos0 + i, pi = pos / 64, slot = pos % 64;
    if (pi != loaded) {
      const size_t off = size_t(s.pages[pi]) * page_stride_ * es;
      HIP_CHECK(hipMemcpy(kp.data(), static_cast<uint8_t *>(kpool(layer)) + off, kp.size(), hipMemcpyDeviceToHost));
      HIP_CHECK(hipMemcpy(vp.data(), static_cast<uint8_t *>(vpool(layer)) + off, vp.size(), hipMemcpyDeviceToHost));
      loaded = pi;
    }
    for (int h = 0; h < hkv; ++h)
      for (int j = 0; j < hd; ++j) {
        // K rows, V columns; a split page holds per kv head an f16 hi plane then an f16 lo plane
        const size_t plane = size_t(64) * hd, npl = es == 4 ? 2 : 1;
        const size_t ki = h * npl * plane + size_t(slot) * hd + j, vi = h * npl * plane + size_t(j) * 64 + slot;
        _Float16 kh, vh, kl = 0, vl = 0;
        std::memcpy(&kh, kp.data() + ki * 2, 2);
        std::memcpy(&vh, vp.data() + vi * 2, 2);
        if (npl == 2) {
          std::memcpy(&kl, kp.data() + (ki + plane) * 2, 2);
          std::memcpy(&vl, vp.data() + (vi + plane) * 2, 2);
        }
        const float kf = float(kh) + float(kl), vf = float(vh) + float(vl);
        k[size_t(i) * kvw + h * hd + j] = kf;
        v[size_t(i) * kvw + h * hd + j] = vf;
      }
  }
}

// ------------------------------------------------------------------ batched prefill
BatchPlan *Engine::batch_create(const lg_request *reqs, int nreq) {
  LG_REQUIRE(nreq > 0 && reqs, "batch: no requests");
  auto *b = new BatchPlan();
  const bool ot = arch == Arch::OpenThai, fresh = fresh_only();
  try {
    std::vector<int32_t> ids, tseq, tpos, tpage, tiles_s, tiles_r, tiles_p, tiles_n, gather, grp_f, grp_c, srow0, sn;
    std::vector<int32_t> it_r, it_p, it_n, it_lo, it_hi, cb_r, cb_n, cb_f, cb_c;
    int max_pages = 0, max_len = 0;  // max_len: the longest sequence of the batch once its tokens are in
    for (int r = 0; r < nreq; ++r) {
      const lg_request &q = reqs[r];
      Seq &s = seq(q.seq);
      for (int j = 0; j < r; ++j)
        if (reqs[j].seq == q.seq) fail(LG_ERR_INVALID, "sequence %d appears twice in one batch", q.seq);
      LG_REQUIRE(q.n > 0 && q.ids, "request %d: empty token sequence", r);
      LG_REQUIRE(q.npos >= 0 && (q.npos == 0 || q.positions), "request %d: bad positions", r);
      for (int i = 0; i < q.n; ++i)
        if (q.ids[i] < 0 || q.ids[i] >= V) fail(LG_ERR_INVALID, "request %d: token id %d outside the vocabulary", r, q.ids[i]);
      for (int i = 0; i < q.npos; ++i)
        if (q.positions[i] < 0 || q.positions[i] >= q.n) fail(LG_ERR_INVALID, "request %d: answer position %d outside the request", r, q.positions[i]);
      if (fresh && s.len != 0)  // OpenThai: the recurrent state lives only inside one forward (model.rs:2); Laya: bidirectional
        fail(LG_ERR_INVALID, "request %d: sequence %d already holds %d tokens; a forward of this model starts from an empty sequence",
             r, q.seq, s.len);
      if (s.len + q.n > ctx) fail(LG_ERR_INVALID, "request %d: %d tokens exceed the context length %d", r, s.len + q.n, ctx);
      if (!fresh) max_pages = std::max(max_pages, (s.len + q.n + 63) / 64);
      max_len = std::max(max_len, s.len + q.n);
    }
    const int gtiles = arch == Arch::Decoder ? attn_prefill_group_tiles(hq, hkv, max_len) : 4;
    b->gtiles = gtiles;
    const int64_t T = std::accumulate(reqs, reqs + nreq, int64_t(0), [](int64_t a, const lg_request &q) { return a + q.n; });
    if (T > max_batch_tokens_) fail(LG_ERR_INVALID, "batch of %lld tokens exceeds max_batch_tokens %lld", (long long)T, (long long)max_batch_tokens_);
    // reserve pages (all or nothing)
    int need = 0;
    for (int r = 0; r < nreq && !fresh; ++r) {
      const Seq &s = seq(reqs[r].seq);
      need += std::max(0, (s.len + reqs[r].n + 63) / 64 - int(s.pages.size()));
    }
    if (need > int(free_pages_.size())) fail(LG_ERR_OOM, "KV cache exhausted: batch needs %d pages, %zu free", need, free_pages_.size());
    std::vector<int32_t> ptab(size_t(nreq) * max_pages, 0);
    int row = 0;
    for (int r = 0; r < nreq; ++r) {
      const lg_request &q = reqs[r];
      Seq &s = seq(q.seq);
      if (!fresh) {
        reserve_pages(s, s.len + q.n);
        for (size_t p = 0; p < s.pages.size(); ++p) ptab[size_t(r) * max_pages + p] = s.pages[p];
      }
      srow0.push_back(row);
      sn.push_back(q.n);
      for (int i = 0; i < q.n; ++i) {
        ids.push_back(q.ids[i]);
        tseq.push_back(r);
        tpos.push_back(s.len + i);
        tpage.push_back(fresh ? 0 : ptab[size_t(r) * max_pages + (s.len + i) / 64]);
      }
      // attention groups of <= gtiles consecutive tiles, cut from the request's end and listed last
      // first: the leftover short group is the one nearest the start (the fewest pages), not a
      // group of one or two tiles that reads every page with most of its waves idle
      const int t_first = int(tiles_s.size()), ntl = (q.n + 31) / 32;
      for (int e = ntl; e > 0; e -= gtiles) {
        const int b = std::max(0, e - gtiles);
        grp_f.push_back(t_first + b);
        grp_c.push_back(e - b);
      }
      for (int i = 0; i < q.n; i += 32) {
        tiles_s.push_back(r);
        tiles_r.push_back(row + i);
        tiles_p.push_back(s.len + i);
        tiles_n.push_back(std::min(32, q.n - i));
      }
      if (ot)  // attention work of a fresh sequence: 16 query rows x key ranges of <= 256
        for (int i = 0; i < q.n; i += 16) {
          const int nq = std::min(16, q.n - i), kend = i + nq;
          cb_r.push_back(row + i);
          cb_n.push_back(nq);
          cb_f.push_back(int32_t(it_r.size()));
          cb_c.push_back((kend + 255) / 256);
          for (int k0 = 0; k0 < kend; k0 += 256) {
            it_r.push_back(row + i);
            it_p.push_back(i);
            it_n.push_back(nq);
            it_lo.push_back(k0);
            it_hi.push_back(std::min(kend, k0 + 256));
          }
        }
      for (int i = 0; i < q.npos; ++i) gather.push_back(row + q.positions[i]);
      b->seqs.push_back(q.seq);
      b->start_len.push_back(s.len);
      b->n.push_back(q.n);
      b->npos.push_back(q.npos);
      row += q.n;
    }
    b->T = int(T);
    b->R = int(gather.size());
    b->ntiles = int(tiles_s.size());
    b->ngroups = int(grp_f.size());
    b->max_pages = max_pages;
    const size_t nints = ids.size() * 4 + ptab.size() + tiles_s.size() * 4 + grp_f.size() * 2 + gather.size() +
                         srow0.size() * 2 + it_r.size() * 5 + cb_r.size() * 4 + 64;
    b->meta.ensure(nints * 4 + 34 * 256);
    int32_t *base = b->meta.as<int32_t>();
    // every table goes into one host image at its 256-byte aligned offset, uploaded by one copy
    std::vector<int32_t> image;
    image.reserve(nints + 34 * 64);
    size_t off = 0;
    auto put = [&](const std::vector<int32_t> &v, int32_t *&dst) {
      dst = base + off;
      image.insert(image.end(), v.begin(), v.end());
      off += (v.size() + 63) & ~size_t(63);
      image.resize(off, 0);
    };
    put(ids, b->ids);
    put(tseq, b->tok_seq);
    put(tpos, b->tok_pos);
    put(tpage, b->tok_page);
    put(ptab, b->pages);
    put(tiles_s, b->tile_seq);
    put(tiles_r, b->tile_row0);
    put(tiles_p, b->tile_pos0);
    put(tiles_n, b->tile_n);
    put(grp_f, b->grp_first);
    put(grp_c, b->grp_count);
    put(gather, b->gather);
    put(srow0, b->seq_row0);
    put(sn, b->seq_n);
    put(it_r, b->it_row0);
    put(it_p, b->it_pos0);
    put(it_n, b->it_nq);
    put(it_lo, b->it_klo);
    put(it_hi, b->it_khi);
    put(cb_r, b->cb_row0);
    put(cb_n, b->cb_nq);
    put(cb_f, b->cb_first);
    put(cb_c, b->cb_n);
    LG_REQUIRE(image.size() * 4 <= b->meta.n, "batch: metadata image exceeds its buffer");
    if (!image.empty()) HIP_CHECK(hipMemcpyAsync(base, image.data(), image.size() * 4, hipMemcpyHostToDevice, stream));
    b->nitems = int(it_r.size());
    b->ncomb = int(cb_r.size());
    HIP_CHECK(hipStreamSynchronize(stream));
  } catch (...) {
    delete b;
    throw;
  }
  return b;
}

void Engine::batch_free(BatchPlan *b) { delete b; }

void Engine::batch_rewind(BatchPlan *b) {
  LG_REQUIRE(b, "batch: null");
  for (size_t r = 0; r < b->seqs.size(); ++r) {
    Seq &s = seq(b->seqs[r]);
    if (b->ran && s.len != b->start_len[r] + b->n[r])
      fail(LG_ERR_INVALID, "batch: sequence %d changed since the batch ran", b->seqs[r]);
    s.len = b->start_len[r];
  }
  b->ran = false;
}

void Engine::run_layers_prefill(BatchPlan &b, lg_cancel_fn cancel, void *arg) {
  const int T = b.T, qw = hq * hd, kvw = hkv * hd, qkvw = qw + 2 * kvw;
  const int planes = split() ? 2 : 1;  // hi (+ lo) f16 planes per activation
  ws_x_.ensure(size_t(T) * d * 4);
  ws_h16_.ensure(size_t(T) * d * 2 * planes);
  // q|k|v projections whose GEMM also rotates and stores q, k and v (the 256 x 256 exact GEMM's
  // fused epilogue) leave no f32 q|k|v rows to stage
  bool fused = split() && hd == 128;
  for (int l = 0; l < L && fused; ++l)
    for (const ProjPart &p : layers_[l].qkv) fused = fused && p.col0 % 128 == 0 && gemm_wide_takes(T, p.w, Epi::F32);
  if (!fused) ws_qkv_.ensure(size_t(T) * qkvw * 4);
  ws_q16_.ensure(size_t(T) * qw * 2 * planes);
  ws_att16_.ensure(size_t(T) * qw * 2 * planes);
  ws_act16_.ensure(size_t(T) * f * 2 * planes);
  auto lo = [&](DevBuf &buf, int64_t n) { return split() ? buf.as<_Float16>() + n : nullptr; };
  float *x = ws_x_.as<float>();
  _Float16 *h16 = ws_h16_.as<_Float16>(), *h16lo = lo(ws_h16_, int64_t(T) * d);
  _Float16 *q16 = ws_q16_.as<_Float16>(), *q16lo = lo(ws_q16_, int64_t(T) * qw);
  _Float16 *att = ws_att16_.as<_Float16>(), *attlo = lo(ws_att16_, int64_t(T) * qw);
  _Float16 *act = ws_act16_.as<_Float16>(), *actlo = lo(ws_act16_, int64_t(T) * f);
  float *qkv = fused ? nullptr : ws_qkv_.as<float>();
  const KvGeom g = geom();
  prof.begin("embed", stream);
  launch_embed(emb_, emb_kind, b.ids, T, d, V, x, stream);
  prof.end(double(T) * d * (emb_kind == LG_F16 ? 6 : 8), 0, stream);
  for (int l = 0; l < L; ++l) {
    if (cancel && cancel(arg)) fail(LG_ERR_CANCELED, "request canceled");
    const Layer &ly = layers_[l];
    prof.begin("rmsnorm", stream);
    launch_rmsnorm_f16(x, T, d, ly.attn_norm, eps, h16, h16lo, stream);
    prof.end(double(T) * d * (4 + 2 * planes), 0, stream);
    RopeKvOut ro;
    ro.cosT = cos_;
    ro.sinT = sin_;
    ro.tok_pos = b.tok_pos;
    ro.tok_page = b.tok_page;
    ro.q16 = q16;
    ro.q16lo = q16lo;
    ro.kpool = static_cast<_Float16 *>(kpool(l));
    ro.vpool = static_cast<_Float16 *>(vpool(l));
    ro.page_stride = g.page_stride;
    ro.hq = hq;
    ro.hkv = hkv;
    ro.hd = hd;
    ro.page_tokens = g.page_tokens;
    ro.qscale = attn_q_scale(hd);
    ro.kv_planes = kv_split() ? 2 : 1;
    // short batches of F16 / Q8_0 weights: the small-tile q|k|v GEMM rotates and stores q, k and v too
    // (no f32 q|k|v rows, no RoPE launch: C1's 144-token request 0.42 -> 0.40 ms, the same bits)
    bool small_rope = split();
    for (const ProjPart &p : ly.qkv) small_rope = small_rope && p.col0 % hd == 0 && gemm_small_rope_takes(T, p.w, hd);
    if (fused) {
      for (const ProjPart &p : ly.qkv) {
        ro.col0 = p.col0;
        const _Float16 *ks = chunk_sums(h16, h16lo, T, p.w);
        prof.begin_kernel("gemm");
        if (!launch_gemm_wide_rope(h16, h16lo, T, p.w, p.bias, ro, stream, ks))
          fail(LG_ERR_UNSUPPORTED, "gemm: fused q|k|v launch refused");
        prof.end_kernel(double(p.w.bytes()) + double(T) * p.w.cols * 2, 2.0 * T * double(p.w.rows) * p.w.cols);
      }
    } else if (small_rope) {
      for (const ProjPart &p : ly.qkv) {
        ro.col0 = p.col0;
        prof.begin_kernel("gemm");
        if (!launch_gemm_small_rope(h16, h16lo, T, p.w, p.bias, ro, stream))
          fail(LG_ERR_UNSUPPORTED, "gemm: short q|k|v launch refused");
        prof.end_kernel(double(p.w.bytes()) + double(T) * p.w.cols * 2, 2.0 * T * double(p.w.rows) * p.w.cols);
      }
    } else {
      for (const ProjPart &p : ly.qkv)
        gemm(h16, h16lo, T, p.w, Epi::F32, qkv + p.col0, nullptr, nullptr, qkvw, p.bias);
      prof.begin("rope_kv", stream);
      launch_rope_kv_tiles(qkv, hq, g, cos_, sin_, b.pages, b.max_pages, b.tile_seq, b.tile_row0,
                           b.tile_pos0, b.tile_n, b.ntiles, q16, q16lo, kpool(l), vpool(l), stream);
      prof.end(double(T) * (qkvw * 4 + qw * 2 * planes + 2 * kvw * kv_elem()), 0, stream);
    }
    prof.begin("attn_prefill", stream);
    launch_attn_prefill(q16, q16lo, T, hq, g, kpool(l), vpool(l), b.pages, b.max_pages, b.tile_seq,
                        b.tile_row0, b.tile_pos0, b.tile_n, b.ntiles, b.grp_first, b.grp_count,
                        b.ngroups, b.gtiles, att, attlo, stream);
    prof.end(0, 0, stream);
    gemm(att, attlo, T, ly.wo, Epi::ADD, x, nullptr, nullptr, d, nullptr);
    prof.begin("rmsnorm", stream);
    launch_rmsnorm_f16(x, T, d, ly.ffn_norm, eps, h16, h16lo, stream);
    prof.end(double(T) * d * (4 + 2 * planes), 0, stream);
    gemm(h16, h16lo, T, ly.wi, Epi::SWIGLU, nullptr, act, actlo, f, nullptr);
    gemm(act, actlo, T, ly.wd, Epi::ADD, x, nullptr, nullptr, d, nullptr);
  }
}

void Engine::batch_run(BatchPlan *b, const int32_t *option_ids, int k, float temperature,
                       float *logits, float *probs, float *logprobs, lg_cancel_fn cancel, void *arg) {
  LG_REQUIRE(b, "batch: null");
  LG_REQUIRE(!b->ran, "batch: already run (stage a new batch)");
  LG_REQUIRE(k > 0 && k <= 256 && option_ids, "batch: need 1..256 head rows");
  LG_REQUIRE(k <= 32 || (!probs && !logprobs), "batch: option scores need 1..32 option ids");
  LG_REQUIRE(temperature > 0 && std::isfinite(temperature), "batch: temperature must be positive");
  for (int j = 0; j < k; ++j)
    if (option_ids[j] < 0 || option_ids[j] >= head_rows())
      fail(LG_ERR_INVALID, arch == Arch::OpenThai ? "slot %d outside the 256 slots" : "option id %d outside the vocabulary",
           option_ids[j]);
  if (arch == Arch::Laya) fail(LG_ERR_UNSUPPORTED, "batch: a Laya encoder scores option markers; use lg_laya_forward");
  // sequences must still exist and not have moved since staging
  for (size_t r = 0; r < b->seqs.size(); ++r) seq(b->seqs[r]);
  if (arch == Arch::OpenThai) run_openthai(*b, cancel, arg);
  else run_layers_prefill(*b, cancel, arg);
  for (size_t r = 0; r < b->seqs.size(); ++r) seq(b->seqs[r]).len += b->n[r];
  b->ran = true;
  const int R = b->R;
  if (R == 0) {
    sync();
    return;
  }
  ws_out_.ensure(size_t(R) * k * 12 + size_t(k) * 4 + 256);  // logits, probs, logprobs, then the k ids
  float *dl = ws_out_.as<float>(), *dp = dl + size_t(R) * k, *dlp = dp + size_t(R) * k;
  int32_t *dids = reinterpret_cast<int32_t *>(dlp + size_t(R) * k);
  HIP_CHECK(hipMemcpyAsync(dids, option_ids, size_t(k) * 4, hipMemcpyHostToDevice, stream));
  prof.begin("head", stream);
  launch_head_rows(ws_x_.as<float>(), b->gather, R, d, final_norm_, eps, head_, head_bias_, dids, k, dl, stream);
  if (k <= 32) launch_option_scores(dl, R, k, temperature, dp, dlp, stream);
  prof.end(0, 0, stream);
  std::vector<float> staged;
  float *hl = logits;
  if (!hl) {
    staged.resize(size_t(R) * k);
    hl = staged.data();
  }
  HIP_CHECK(hipMemcpyAsync(hl, dl, size_t(R) * k * 4, hipMemcpyDeviceToHost, stream));
  if (probs) HIP_CHECK(hipMemcpyAsync(probs, dp, size_t(R) * k * 4, hipMemcpyDeviceToHost, stream));
  if (logprobs) HIP_CHECK(hipMemcpyAsync(logprobs, dlp, size_t(R) * k * 4, hipMemcpyDeviceToHost, stream));
  sync();
  // a non-finite output is an error, as the reference's Laya forward makes it
  // (src/models/laya/model.rs:412-414); the sequences go back to their lengths before this batch.
  // The OpenThai forward returns its slot logits as they are (src/models/openthai/model.rs:232-240:
  // no such check), so its decide sees what the reference's would.
  for (size_t i = 0; arch != Arch::OpenThai && i < size_t(R) * k; ++i)
    if (!std::isfinite(hl[i])) {
      for (size_t r = 0; r < b->seqs.size(); ++r) seq(b->seqs[r]).len -= b->n[r];
      b->ran = false;
      fail(LG_ERR_INVALID, "non-finite model output");
    }
}

void Engine::forward(int sq, const int32_t *ids, int n, const int32_t *positions, int npos,
                     const int32_t *vocab_ids, int nv, float *logits, lg_cancel_fn cancel, void *arg) {
  lg_request r{sq, ids, n, positions, npos};
  BatchPlan *b = batch_create(&r, 1);
  struct Guard { Engine *e; BatchPlan *b; ~Guard() { e->batch_free(b); } } guard{this, b};
  if (vocab_ids) {
    batch_run(b, vocab_ids, nv, 1.0f, logits, nullptr, nullptr, cancel, arg);
    return;
  }
  if (arch == Arch::OpenThai) {  // every slot row of the slot head
    int32_t slots[256];
    for (int i = 0; i < 256; ++i) slots[i] = i;
    batch_run(b, slots, 256, 1.0f, logits, nullptr, nullptr, cancel, arg);
    return;
  }
  if (arch == Arch::Laya) fail(LG_ERR_UNSUPPORTED, "forward: a Laya encoder scores option markers; use lg_laya_forward");
  // full vocabulary: prefill, then one fused-norm GEMV over the head per answer row
  for (size_t i = 0; i < b->seqs.size(); ++i) seq(b->seqs[i]);
  run_layers_prefill(*b, cancel, arg);
  seq(sq).len += n;
  b->ran = true;
  if (npos == 0) {
    sync();
    return;
  }
  ws_out_.ensure(size_t(V) * 4);
  std::vector<int32_t> rows(npos);
  for (int i = 0; i < npos; ++i) rows[i] = positions[i];
  for (int i = 0; i < npos; ++i) {
    gemv(ws_x_.as<float>() + size_t(rows[i]) * d, head_, Epi::F32, ws_out_.as<float>(), nullptr, final_norm_);
    HIP_CHECK(hipMemcpyAsync(logits + size_t(i) * V, ws_out_.p, size_t(V) * 4, hipMemcpyDeviceToHost, stream));
    sync();
    for (int j = 0; j < V; ++j)
      if (!std::isfinite(logits[size_t(i) * V + j])) {
        seq(sq).len -= n;
        fail(LG_ERR_INVALID, "non-finite model output");
      }
  }
}

size_t Engine::workspace_bytes() const {
  size_t n = 0;
  for (const DevBuf *b : {&ws_x_, &ws_h16_, &ws_qkv_, &ws_q16_, &ws_att16_, &ws_act16_, &ws_ksum_, &ws_meta_, &ws_out_, &ws_dec_,
                          &ws_ot_qk_, &ws_ot_v_, &ws_ot_gb_, &ws_ot_o_, &ws_ot_part_})
    n += b->n;
  return n;
}

// ------------------------------------------------------------------ greedy decode
void Engine::decode_check(const Seq &s, int32_t first, int steps, const int32_t *tokens) const {
  if (arch != Arch::Decoder) fail(LG_ERR_UNSUPPORTED, "decode: this model has a decision head, not a language-model head");
  LG_REQUIRE(steps > 0 && tokens, "decode: need steps > 0 and an output");
  LG_REQUIRE(first >= 0 && first < V, "decode: token id %d outside the vocabulary", first);
  if (int64_t(s.len) + steps > ctx)
    fail(LG_ERR_INVALID, "sequence of %lld tokens exceeds the context length %d", (long long)s.len + steps, ctx);
  // the decode attention combines at most 1024 pages (65,536 tokens) of context; refused here,
  // before any page is reserved or any step runs
  const int64_t last_pages = (int64_t(s.len) + steps - 1) / 64 + 1;
  if (last_pages > 1024)
    fail(LG_ERR_INVALID, "decode: a context of %lld tokens exceeds the decode attention's 65536", (long long)s.len + steps);
}

// Workspace of a decode run over a sequence holding `npages` pages (its whole page table, which a
// canceled forward can leave longer than the tokens need): x, q|k|v, attention output, SwiGLU
// output, logits, argmax partial maxima, attention page partials (f32, laid out by the page table's
// length), then the token slots, the page table and the argmax partial indices.
size_t Engine::decode_ws_bytes(int npages, int steps) const {
  const int qw = hq * hd, qkvw = qw + 2 * hkv * hd;
  const size_t part_floats = size_t(attn_decode_scratch_floats(hq, hd, npages));
  const size_t floats = size_t(d) + qkvw + qw + f + V + 64 + part_floats;
  return floats * 4 + (size_t(steps) + 1 + npages) * 4 + 64 * 4 + 256;
}

void Engine::decode(int sq, int32_t first, int steps, int32_t *tokens, float *logits) {
  Seq &s = seq(sq);
  decode_check(s, first, steps, tokens);
  reserve_pages(s, s.len + steps);
  ws_dec_.ensure(decode_ws_bytes(int(s.pages.size()), steps));
  decode_run(s, first, steps, tokens, logits, ws_dec_.p);
}

void Engine::decode_noalloc(int sq, int32_t first, int steps, int32_t *tokens, float *logits) {
  Seq &s = seq(sq);
  decode_check(s, first, steps, tokens);
  // the page table as reserve_pages below leaves it (checked first, so a refusal reserves nothing)
  const int npages = std::max(int(s.pages.size()), (s.len + steps + 63) / 64);
  const size_t need = decode_ws_bytes(npages, steps);
  if (need > kNoAllocScratchBytes)
    fail(LG_ERR_INVALID,
         "decode_noalloc: %d steps after %d tokens need %zu bytes of scratch; the per-GPU limit is %zu "
         "(use lg_decode for longer contexts)",
         steps, s.len, need, kNoAllocScratchBytes);
  // one user of this GPU's scratch at a time, from the first launch until the stream has drained
  std::lock_guard<std::mutex> lock(noalloc_mutex(device));
  void *ws = noalloc_scratch(device);
  reserve_pages(s, s.len + steps);
  try {
    decode_run(s, first, steps, tokens, logits, ws);
  } catch (...) {
    (void)hipStreamSynchronize(stream);  // launches already queued still use the scratch
    throw;
  }
}

void Engine::decode_graph(int sq, int32_t first, int steps, int32_t *tokens, double *capture_ms, double *run_ms) {
  Seq &s = seq(sq);
  decode_check(s, first, steps, tokens);
  LG_REQUIRE(capture_ms && run_ms, "decode_graph: need both time outputs");
  LG_REQUIRE(!prof.on(), "decode_graph: turn kernel profiling off first");
  reserve_pages(s, s.len + steps);
  ws_dec_.ensure(decode_ws_bytes(int(s.pages.size()), steps));
  decode_run(s, first, steps, tokens, nullptr, ws_dec_.p, capture_ms, run_ms);
}

// With capture_ms / run_ms set, the step loop (kernels only: no copies, no memsets) is captured into a
// HIP graph after the metadata upload and launched once.
void Engine::decode_run(Seq &s, int32_t first, int steps, int32_t *tokens, float *logits, void *ws,
                        double *capture_ms, double *run_ms) {
  const bool graph = capture_ms != nullptr;
  const int pos0 = s.len;
  const int qw = hq * hd, kvw = hkv * hd, qkvw = qw + 2 * kvw;
  const int max_pages = int(s.pages.size());
  // device metadata, uploaded once: token slots (step i reads slot i, its argmax goes to slot
  // i + 1) and the page table; positions and context lengths travel as kernel arguments
  std::vector<int32_t> meta;
  meta.push_back(first);
  meta.resize(steps + 1, 0);
  for (int p : s.pages) meta.push_back(p);
  const size_t part_floats = size_t(attn_decode_scratch_floats(hq, hd, max_pages));
  float *x = static_cast<float *>(ws);
  float *qkv = x + d, *att = qkv + qkvw, *act = att + qw, *lg = act + f;
  float *part_v = lg + V;
  float *part = part_v + 64;
  int32_t *dm = reinterpret_cast<int32_t *>(part + part_floats);
  int32_t *tok = dm, *pt = dm + steps + 1;
  int32_t *part_i = pt + max_pages;
  HIP_CHECK(hipMemcpyAsync(dm, meta.data(), meta.size() * 4, hipMemcpyHostToDevice, stream));
  const KvGeom g = geom();
  hipGraph_t hg = nullptr;
  hipGraphExec_t hx = nullptr;
  std::chrono::steady_clock::time_point t0;
  if (graph) {
    sync();
    t0 = std::chrono::steady_clock::now();
    HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  }
  auto step_loop = [&] {
    for (int i = 0; i < steps; ++i) {
      if (i == 0) {  // later steps' rows come from the previous step's argmax launch
        prof.begin("embed", stream);
        launch_embed(emb_, emb_kind, tok + i, 1, d, V, x, stream);
        prof.end(double(d) * 6, 0, stream);
      }
      for (int l = 0; l < L; ++l) {
        const Layer &ly = layers_[l];
        for (const ProjPart &p : ly.qkv) gemv(x, p.w, Epi::F32, qkv + p.col0, p.bias, ly.attn_norm);
        // the position of this step is a kernel argument; RoPE and the k/v write are fused in
        prof.begin("attn_decode", stream);
        launch_attn_decode(qkv, hq, g, cos_, sin_, pos0 + i, kpool(l), vpool(l), pt, max_pages, part, att,
                           stream);
        prof.end(double(pos0 + i + 1) * 2 * kvw * kv_elem(), 4.0 * double(pos0 + i + 1) * qw, stream);
        gemv(att, ly.wo, Epi::ADD, x, nullptr, nullptr);
        gemv(x, ly.wi, Epi::SWIGLU, act, nullptr, ly.ffn_norm);
        gemv(act, ly.wd, Epi::ADD, x, nullptr, nullptr);
      }
      gemv(x, head_, Epi::F32, lg, nullptr, final_norm_);
      prof.begin("argmax", stream);
      if (i + 1 < steps) launch_argmax_embed(lg, V, tok + i + 1, emb_, emb_kind, d, x, stream);
      else launch_argmax(lg, V, tok + i + 1, part_v, part_i, stream);
      prof.end(double(V) * 4, 0, stream);
      if (logits) HIP_CHECK(hipMemcpyAsync(logits + size_t(i) * V, lg, size_t(V) * 4, hipMemcpyDeviceToHost, stream));
    }
  };
  if (!graph) {
    step_loop();
  } else {
    // an error raised while capturing ends the capture first, so the stream stays usable
    try {
      step_loop();
    } catch (...) {
      hipGraph_t dropped = nullptr;
      (void)hipStreamEndCapture(stream, &dropped);
      if (dropped) (void)hipGraphDestroy(dropped);
      throw;
    }
    const hipError_t ce = hipStreamEndCapture(stream, &hg);
    hipError_t ie = hipErrorUnknown;
    if (ce == hipSuccess) ie = hipGraphInstantiate(&hx, hg, nullptr, nullptr, 0);
    if (ce != hipSuccess || ie != hipSuccess) {
      if (hg) (void)hipGraphDestroy(hg);
      fail(LG_ERR_DEVICE, "decode_graph: capture failed (%s)", hipGetErrorString(ce != hipSuccess ? ce : ie));
    }
    const auto t1 = std::chrono::steady_clock::now();
    const hipError_t le = hipGraphLaunch(hx, stream);
    const hipError_t se = hipStreamSynchronize(stream);
    const auto t2 = std::chrono::steady_clock::now();
    (void)hipGraphExecDestroy(hx);
    (void)hipGraphDestroy(hg);
    HIP_CHECK(le);
    HIP_CHECK(se);
    *capture_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    *run_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  }
  HIP_CHECK(hipMemcpyAsync(tokens, tok + 1, size_t(steps) * 4, hipMemcpyDeviceToHost, stream));
  sync();
  // the argmax writes -1 for a step whose logits have no finite maximum
  for (int i = 0; i < steps; ++i)
    if (tokens[i] < 0) fail(LG_ERR_INVALID, "non-finite model output");
  s.len = pos0 + steps;
}

}  // namespace lg
