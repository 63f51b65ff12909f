// The engine: one model on one GPU with its own stream, weight arena and KV page pool.
// Host-side counterpart of the reference's Engine + Backend + Model (src/engine.rs:10-48,
// src/models/mod.rs:13-23, src/models/openthai/model.rs:41-241), for the laya-decoder shape
// and the OpenThai-SystemOne text tower (dispatch on general.architecture, mod.rs:65-71).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "gguf.h"
#include "decide.h"
#include "laya_decide.h"
#include "json.h"
#include "kernels.h"
#include "lg.h"

namespace lg {

// Bytes per row of a repacked matrix: codes/values (q) and scales (s); rows [row0, row0+n) view.
int64_t q_row_bytes(uint32_t kind, int cols);
int64_t s_row_bytes(uint32_t kind, int cols);
DevMatrix sub_rows(const DevMatrix &m, int row0, int nrows);
size_t align256(size_t n);

// A slice of a projection's output columns computed by one device matrix.
struct ProjPart {
  DevMatrix w;
  int col0 = 0;                 // first output column in the fused output
  const float *bias = nullptr;  // device, w.rows entries, or null
};

struct Layer {
  float *attn_norm = nullptr, *ffn_norm = nullptr;  // device f32 [d]
  std::vector<ProjPart> qkv;                        // fused q|k|v output [(hq+2hkv)*hd]
  DevMatrix wo, wi, wd;                             // wi = gate rows then up rows
};

struct Seq {
  std::vector<int> pages;
  int len = 0;
};

// Grow-only device buffer.
struct DevBuf {
  void *p = nullptr;
  size_t n = 0;
  void ensure(size_t bytes);
  ~DevBuf();
  template <class T>
  T *as() const { return static_cast<T *>(p); }
};

class Profiler {
 public:
  void enable(bool on) { on_ = on; }
  bool on() const { return on_; }
  void begin(const char *cls, hipStream_t st);
  void end(double bytes, double flops, hipStream_t st);
  // one timed kernel (GEMV, GEMM): events recorded at the kernel's own start and end
  void begin_kernel(const char *cls);
  void end_kernel(double bytes, double flops);
  void read(const std::string &cls, int64_t *launches, double *ms, double *bytes, double *flops);
  void reset();
  ~Profiler();

 private:
  struct Rec { std::string cls; hipEvent_t a, b; double bytes, flops; };
  struct Sum { int64_t launches = 0; double ms = 0, bytes = 0, flops = 0; };
  void drain();
  bool on_ = false;
  std::vector<Rec> open_;
  std::vector<hipEvent_t> pool_;
  std::map<std::string, Sum> sums_;
  hipEvent_t take();
  std::string cur_;
  hipEvent_t cur_a_ = nullptr, cur_b_ = nullptr;
  KernelTimer timer_;
};

// Planned batch: device metadata for one staged prefill batch.
struct BatchPlan {
  std::vector<int> seqs;        // engine sequence per request
  std::vector<int> n, npos;     // tokens and answer positions per request
  std::vector<int> start_len;   // sequence length at staging time
  int T = 0, R = 0, ntiles = 0, max_pages = 0;
  DevBuf meta;                  // ids, tok_seq, tok_pos, pages, tiles..., gather rows
  int32_t *ids = nullptr, *tok_seq = nullptr, *tok_pos = nullptr, *pages = nullptr;
  int32_t *tok_page = nullptr;  // per batch row: the page its position falls in
  int32_t *tile_seq = nullptr, *tile_row0 = nullptr, *tile_pos0 = nullptr, *tile_n = nullptr;
  int ngroups = 0;              // runs of <= gtiles consecutive tiles of one sequence
  int gtiles = 0;               // attention tiles per group (attn_prefill_group_tiles)
  int32_t *grp_first = nullptr, *grp_count = nullptr;
  int32_t *gather = nullptr;
  int32_t *seq_row0 = nullptr, *seq_n = nullptr;  // first batch row and token count per request
  // OpenThai attention work: items (16 query rows x <= 256 keys) and per-16-row merges
  int nitems = 0, ncomb = 0;
  int32_t *it_row0 = nullptr, *it_pos0 = nullptr, *it_nq = nullptr, *it_klo = nullptr, *it_khi = nullptr;
  int32_t *cb_row0 = nullptr, *cb_nq = nullptr, *cb_first = nullptr, *cb_n = nullptr;
  bool ran = false;
};

enum class Arch { Decoder = 0, OpenThai = 1, Laya = 2 };

// Laya encoder layer (src/models/laya/model.rs:29-40); norms with optional weight and bias
struct LayaNorm {
  const float *w = nullptr, *b = nullptr;
  float eps = 1e-5f;
};
struct LayaLinear {
  DevMatrix w;
  const float *b = nullptr;  // summed biases of the graph, or null
};
struct LayaLayer {
  bool has_n1 = false, full = false;
  LayaNorm n1, n2;
  LayaLinear qkv, wo, wi, down;
};

// One OpenThai-SystemOne layer (src/models/openthai/model.rs:10-40).  Norm weights are stored
// as 1 + w (the zero-centred RMSNorm's offset applied once at upload, an exact f32 add).
struct OtLayer {
  bool full = false;
  float *n1 = nullptr, *n2 = nullptr;
  // full: rows [(q 256 | gate 256) x hq | k 256 x hkv | v 256 x hkv];
  // DeltaNet: rows [q|k|v (3*nh*128) | z (nh*128) | a (nh) | b (nh) | zero rows to a multiple of 128]
  DevMatrix proj;
  DevMatrix out;               // o_proj / out_proj
  DevMatrix wi, wd;            // gate rows then up rows; down
  float *qn1 = nullptr, *kn1 = nullptr;                                      // full: 1 + q_norm, 1 + k_norm
  float *conv = nullptr, *dt = nullptr, *alog = nullptr, *norm = nullptr;  // DeltaNet
};

// Streamed host -> HBM upload of GGUF bytes: two pinned host buffers and two device staging
// buffers of kChunk bytes.  While the DMA engine copies chunk i and the repack kernel converts it,
// the host copies chunk i + 1 out of the (memory-mapped) file into the other pinned buffer.  Large
// matrices (a 152,064-row head) go through in row slices, so staging never exceeds 2 x kChunk.
class Uploader {
 public:
  static constexpr size_t kChunk = size_t(64) << 20;
  explicit Uploader(hipStream_t st);
  ~Uploader();
  Uploader(const Uploader &) = delete;
  Uploader &operator=(const Uploader &) = delete;
  // n bytes of host memory to device memory
  void bytes(const uint8_t *src, size_t n, void *dst);
  // rows of GGUF blocks (row_bytes raw bytes each), repacked into the rows of `m`
  void matrix(uint32_t kind, const uint8_t *src, int rows, size_t row_bytes, const DevMatrix &m);
  void finish();  // everything queued has landed; the host buffers are free

 private:
  int take();  // the next slot, once its previous copy and repack have finished
  hipStream_t st_;
  void *host_[2] = {nullptr, nullptr}, *dev_[2] = {nullptr, nullptr};
  hipEvent_t done_[2] = {nullptr, nullptr};
  bool used_[2] = {false, false};
  int next_ = 0;
};

class Engine {
 public:
  Engine(const Gguf &g, const lg_engine_opts &opts);
  ~Engine();

  lg_model_info info() const;
  void sync();
  // bytes held by the grow-only workspaces (not weights, not the KV pool)
  size_t workspace_bytes() const;

  // Matrix::apply drop-in on a named uploaded matrix (host pointers).
  void matmul(const std::string &name, const float *x, int m, const float *bias, float *y);

  int seq_create();
  int seq_fork(int parent, int ntokens);
  void seq_free(int id);
  int seq_len(int id) const;
  // Cached K (after RoPE) and V rows of positions [pos0, pos0 + n) of one layer, as f32 [n][hkv * hd].
  void seq_kv_read(int id, int layer, int pos0, int n, float *k, float *v);

  BatchPlan *batch_create(const lg_request *reqs, int nreq);
  void batch_free(BatchPlan *b);
  void batch_rewind(BatchPlan *b);
  void batch_run(BatchPlan *b, const int32_t *option_ids, int k, float temperature, float *logits,
                 float *probs, float *logprobs, lg_cancel_fn cancel, void *arg);
  // Single-sequence forward with host ids; vocab_ids == nullptr -> full vocabulary.
  void forward(int seq, const int32_t *ids, int n, const int32_t *positions, int npos,
               const int32_t *vocab_ids, int nv, float *logits, lg_cancel_fn cancel, void *arg);
  void decode(int seq, int32_t first, int steps, int32_t *tokens, float *logits);
  // decode with its workspace in the per-device no-alloc scratch: no device allocation at all
  void decode_noalloc(int seq, int32_t first, int steps, int32_t *tokens, float *logits);
  // decode with the whole step loop captured into one HIP graph, then launched once; wall times of
  // the capture + instantiation and of the graph launch
  void decode_graph(int seq, int32_t first, int steps, int32_t *tokens, double *capture_ms, double *run_ms);
  // Laya Model::forward (src/models/laya/model.rs:303-416) for n inputs as one batch:
  // option logits (k_i per input, concatenated) and act logits [n][2].
  void laya_forward(const lg_laya_input *in, int n, float *logits, float *act, lg_cancel_fn cancel, void *arg);

  Profiler prof;

 private:
  void load_decoder(const Gguf &g, const lg_engine_opts &opts);
  void upload(const Gguf &g);
  void load_openthai(const Gguf &g);
  void load_laya(const Gguf &g);
  LayaLinear laya_linear(const Gguf &g, const Json &graph, const std::string &key);
  LayaNorm laya_norm(const Gguf &g, const Json &graph, int i);
  void release();
  // pad_to > 0: rows rounded up to a multiple of pad_to with zero weights
  DevMatrix upload_matrix(const Gguf &g, const std::vector<std::string> &names, int cols, int pad_to = 0);
  // exact mode: the operand form the large-batch prefill GEMM reads (DevMatrix::pc, pcl, pcs)
  void add_prefill_copy(DevMatrix &m);
  Uploader &uploader();  // created on first use
  void finish_upload();  // waits for the queued upload work and frees the staging
  // offset != 0: stores offset + w (the zero-centred RMSNorm weight)
  float *upload_vector_f32(const Gguf &g, const std::string &name, int64_t n, float offset = 0.0f);
  void *carve(size_t bytes);
  Seq &seq(int id);
  void reserve_pages(Seq &s, int upto_tokens);
  int alloc_page();
  void release_page(int p);
  void run_layers_prefill(BatchPlan &b, lg_cancel_fn cancel, void *arg);
  // decode: argument checks, then the steps with the workspace `ws` (decode_ws_bytes of it)
  void decode_check(const Seq &s, int32_t first, int steps, const int32_t *tokens) const;
  size_t decode_ws_bytes(int npages, int steps) const;
  void decode_run(Seq &s, int32_t first, int steps, int32_t *tokens, float *logits, void *ws,
                  double *capture_ms = nullptr, double *run_ms = nullptr);
  void run_openthai(BatchPlan &b, lg_cancel_fn cancel, void *arg);
  void run_laya(BatchPlan &b, const int32_t *qtype_dev, lg_cancel_fn cancel, void *arg);
  KvGeom geom() const;
  void *kpool(int layer) const;
  void *vpool(int layer) const;

  // prof-wrapped launch helpers
  // A/A_lo and C16/C16_lo are hi/lo planes in EXACT mode (lo == nullptr in FAST mode)
  // exact Q4_K launches (two-pass prefill copy): the activation's chunk sums in ws_ksum_ (nullptr when W
  // does not need them)
  const _Float16 *chunk_sums(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W);
  void gemm(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W, Epi epi, float *C,
            _Float16 *C16, _Float16 *C16_lo, int ldc, const float *bias);
  void gemv(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
            const float *norm_w);

 public:
  int device = 0;
  hipStream_t stream = nullptr;
  Arch arch = Arch::Decoder;
  int L = 0, d = 0, hq = 0, hkv = 0, hd = 0, f = 0, V = 0, ctx = 0;
  int nh = 0;          // OpenThai: gated DeltaNet heads (128-dim)
  int head_rows() const { return arch == Arch::OpenThai ? 256 : V; }
  bool fresh_only() const { return arch != Arch::Decoder; }  // forwards start from empty sequences
  int64_t max_batch_tokens() const { return max_batch_tokens_; }
  float eps = 1e-5f;
  uint32_t emb_kind = 0;
  int precision = LG_PREC_EXACT;
  DecideSpec decide;  // control tokens and budgets of the request-level decide layout
  LayaSpec laya_decide;  // budgets, special ids and temperatures of the Laya decide
  bool split() const { return precision != LG_PREC_FAST; }     // hi/lo activation planes
  bool kv_split() const { return precision == LG_PREC_EXACT; }  // hi/lo KV cache planes
  int kv_elem() const { return kv_split() ? 4 : 2; }

 private:
  // weights
  void *arena_ = nullptr;
  size_t arena_size_ = 0, arena_used_ = 0;
  Uploader *up_ = nullptr;  // live while the constructor uploads weights
  double load_s_ = 0.0;     // wall time of the constructor (upload, repack, prefill copies)
  void *emb_ = nullptr;
  float *cos_ = nullptr, *sin_ = nullptr, *final_norm_ = nullptr;
  std::vector<Layer> layers_;
  DevMatrix head_;
  float *head_bias_ = nullptr;                 // OpenThai slot-head bias [256]
  std::vector<OtLayer> ot_;                    // OpenThai layers
  int ldp_full_ = 0, ldp_delta_ = 0;           // OpenThai projection row widths
  // Laya encoder
  std::vector<LayaLayer> laya_trunk_, laya_head_;
  LayaNorm laya_embnorm_, laya_finalnorm_, laya_scorenorm_;
  const float *laya_type_emb_ = nullptr;
  LayaLinear laya_score1_, laya_score2_, laya_act1_, laya_act2_;
  const float *laya_cos_full_ = nullptr, *laya_sin_full_ = nullptr, *laya_cos_slide_ = nullptr, *laya_sin_slide_ = nullptr;
  int laya_f_ = 0, laya_head_f_ = 0;
  std::map<std::string, DevMatrix> named_;  // GGUF name -> device matrix view
  int64_t weight_bytes_ = 0;
  // KV pool
  void *kv_ = nullptr;
  int npages_ = 0;
  int64_t page_stride_ = 0;  // elements per (layer, page) of K (same for V)
  std::vector<int> free_pages_, refcnt_;
  std::map<int, Seq> seqs_;
  int next_seq_ = 1;
  int64_t max_batch_tokens_ = 65536;
  // workspaces
  DevBuf ws_x_, ws_h16_, ws_qkv_, ws_q16_, ws_att16_, ws_act16_, ws_ksum_, ws_meta_, ws_out_;
  DevBuf ws_dec_;
  DevBuf ws_ot_qk_, ws_ot_v_, ws_ot_gb_, ws_ot_o_;  // OpenThai mixer workspaces
  DevBuf ws_ot_part_;                               // OpenThai attention partials
  DevBuf ws_ot_chunk_;                              // OpenThai DeltaNet chunk records
};

}  // namespace lg
