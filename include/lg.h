/*
 * lg.h -- C ABI of the MI355X (gfx950) Laya decoder engine.
 *
 * Plain pointers, sizes and status codes; no C++ or torch types cross this line.
 * Every call returns LG_OK (0) or an LG_ERR_* code, and on failure sets a
 * thread-local message readable through lg_last_error() -- the counterpart of
 * the reference's `Result<_, String>` (src/models/mod.rs:13-23).  No call aborts
 * the process; a failed call leaves its handle usable.
 *
 * Thread-safety: an lg_engine is not re-entrant (calls on one engine serialise on
 * its HIP stream); distinct engines are independent.  lg_gguf handles are
 * read-only after open and may be shared.
 */
#ifndef LAYA_LG_H
#define LAYA_LG_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LG_OK 0
#define LG_ERR_INVALID 1     /* bad argument, shape or token id */
#define LG_ERR_FORMAT 2      /* GGUF parse / model validation failure */
#define LG_ERR_DEVICE 3      /* HIP runtime error */
#define LG_ERR_OOM 4         /* device arena or KV pages exhausted */
#define LG_ERR_CANCELED 5    /* the cancel callback returned non-zero */
#define LG_ERR_UNSUPPORTED 6 /* tensor kind / shape the engine has no kernel for */

/* GGML tensor kinds accepted by src/gguf.rs:81-93. */
#define LG_F32 0u
#define LG_F16 1u
#define LG_Q4_0 2u
#define LG_Q8_0 8u
#define LG_Q4_K 12u
#define LG_Q6_K 14u

/* Message of the last failing call on this thread ("" if none). */
const char *lg_last_error(void);
/* "laya-mi355x <version> gfx950" */
const char *lg_version(void);

/* ---------------------------------------------------------------- formats */

/* (elements per block, bytes per block) of a tensor kind.
 * Replaces gguf::layout, src/gguf.rs:81-93. */
int lg_layout(uint32_t kind, uint64_t *block, uint64_t *bytes);

/* IEEE binary16 -> f32, exact incl. subnormals, Inf and NaN payloads.
 * Replaces gguf::half, src/gguf.rs:226-246. */
float lg_half(uint16_t bits);

typedef struct lg_gguf lg_gguf;

/* Open and validate a GGUF v3 file through a read-only private mmap.
 * Replaces Gguf::open, src/gguf.rs:95-179 (and io::Mapping::open, src/io.rs:65-88);
 * the error messages are the reference's. */
int lg_gguf_open(const char *path, lg_gguf **out);
/* Same over caller-owned bytes, borrowed until lg_gguf_close. */
int lg_gguf_open_memory(const void *bytes, uint64_t len, lg_gguf **out);
void lg_gguf_close(lg_gguf *g);

int lg_gguf_tensor_count(const lg_gguf *g);
/* Name of tensor i (file order). */
const char *lg_gguf_tensor_name(const lg_gguf *g, int i);
/* Tensor lookup, replaces Gguf::data, src/gguf.rs:193-199.  dims[0] is the row length. */
int lg_gguf_tensor(const lg_gguf *g, const char *name, uint32_t *kind, uint64_t dims[4], int *nd,
                   const void **data, uint64_t *len);
/* Metadata, replaces Gguf::get / Gguf::num, src/gguf.rs:181-189.  *found = 0 when absent. */
int lg_gguf_meta_num(const lg_gguf *g, const char *key, double *value, int *found);
int lg_gguf_meta_str(const lg_gguf *g, const char *key, const char **value, int *found);

/* Dequantise `len` bytes of GGUF blocks of `kind` into `dst` (len/bytes*block floats) on
 * the GPU, bit-identical to gguf::decode, src/gguf.rs:250-336.  Host pointers. */
int lg_dequant(uint32_t kind, const void *src, uint64_t len, float *dst);

/* ------------------------------------------------------------ synthetic models */

/* Seeded synthetic "laya-decoder" GGUF (general.architecture = "ggmlc",
 * laya.model_name = "laya-decoder").  `preset` names a workload shape
 * ("plumbing-f16", "q8-2048", "q4km-7b", "f16-7b", or "tiny-*" test shapes);
 * n_layers > 0 overrides the layer count.  The image is malloc'd; free it with
 * lg_synth_free.  Deterministic in (preset, seed, n_layers). */
int lg_synth_gguf(const char *preset, uint64_t seed, int n_layers, void **image, uint64_t *len);
/* Write the same image to a file. */
int lg_synth_gguf_file(const char *preset, uint64_t seed, int n_layers, const char *path);
void lg_synth_free(void *image);

/* ---------------------------------------------------------------- engine */

typedef struct lg_engine lg_engine;

/* Numeric modes of the prefill path (the decode GEMV always computes in f32):
 * LG_PREC_EXACT: f32-faithful -- activations carried as hi/lo f16 planes into split-precision
 *   MFMA, weights applied exactly, KV cache as hi/lo f16 planes (4 bytes a value, about 22
 *   significant bits).  Matches the f32 reference to its own summation-order spread even on
 *   ill-conditioned models.  The default.
 * LG_PREC_KV16: LG_PREC_EXACT's projections (hi/lo activation planes, exact weights) over an
 *   f16 KV cache (2 bytes a value, k and v rounded to nearest f16): decode attention reads half
 *   the bytes and prefill attention takes two f16 MFMA passes a product instead of three.
 *   Queries and attention probabilities stay hi/lo planes.  Only the decoder family keeps a KV
 *   cache; for the other families this mode is LG_PREC_EXACT.
 * LG_PREC_FAST: one f16 MFMA pass, weights rounded to f16, f16 KV cache. */
#define LG_PREC_EXACT 0
#define LG_PREC_FAST 1
#define LG_PREC_KV16 2

typedef struct {
  int device;              /* HIP device ordinal */
  int kv_pages;            /* 64-token KV pages to reserve (0 = derive from kv_tokens) */
  int64_t kv_tokens;       /* tokens of KV capacity when kv_pages == 0 (0 = 65536) */
  int64_t max_batch_tokens;/* largest prefill batch (0 = 65536) */
  int precision;           /* LG_PREC_EXACT (0), LG_PREC_FAST or LG_PREC_KV16 */
} lg_engine_opts;

typedef struct {
  int layers, d_model, heads, kv_heads, head_dim, ffn, vocab, context;
  uint32_t kind_attn, kind_ffn, kind_head; /* GGML kinds of the uploaded matrices */
  int64_t weight_bytes;    /* HBM bytes of the uploaded weight arena */
  int64_t kv_bytes;        /* HBM bytes of the KV page pool */
  int kv_pages, kv_page_tokens;
  int precision;           /* LG_PREC_* the engine was created with */
  int kv_elem_bytes;       /* 4 (f16 hi + lo planes, exact mode) or 2 (f16: kv16 and fast modes) */
  int arch;                /* LG_ARCH_* */
  int linear_heads;        /* OpenThai: gated DeltaNet heads (128-dim); 0 otherwise */
  int full_layers;         /* OpenThai: full-attention layers (the rest are DeltaNet) */
  double load_seconds;     /* wall time of lg_engine_create: upload, repack, prefill copies, KV pool */
} lg_model_info;

/* Model families (general.architecture): "ggmlc" + laya.model_name "laya-decoder", the
 * "openthai_systemone" text tower, and the compiled Laya encoder ("ggmlc" with a laya.checkpoint
 * and a ggmlc.graph_spec) (src/models/mod.rs:65-71). */
#define LG_ARCH_LAYA_DECODER 0
#define LG_ARCH_OPENTHAI 1
#define LG_ARCH_LAYA 2

/* ---- model description and registry preflight (host only; no weight is read) ---- */
typedef struct {
  char name[128];          /* the registry name: "openthai-systemone", laya.model_name, or the decoder's general.name */
  char family[64];
  char architecture[64];   /* general.architecture */
  char aliases[4][64];
  int n_aliases;
  char release_date[16];   /* "" for the decoder family */
} lg_model_desc;

/* Replaces models::describe, src/models/mod.rs:32-64 ("ggmlc" Laya encoders and
 * "openthai_systemone"), plus the laya-decoder family ("ggmlc" with laya.model_name
 * "laya-decoder", which the reference does not load: named by its general.name, no aliases).
 * Errors (LG_ERR_FORMAT): "unsupported ggmlc model X", "unsupported GGUF architecture X". */
int lg_model_describe(const lg_gguf *g, lg_model_desc *out);

/* Replaces the preflight of Registry::load, src/registry.rs:16-39, run before any weights
 * load: every path is opened (header and tensor table) and described, and an empty list, a
 * name or alias used twice and an unknown default are refused with the reference's messages.
 * On success *default_index is the default model's index (0 when default_name is NULL). */
int lg_registry_preflight(const char *const *paths, int n, const char *default_name, int *default_index);

/* Load a laya-decoder GGUF onto one GPU: validate, upload and repack every matrix into a
 * hipMalloc'd weight arena, reserve the KV page pool, create the engine's stream.
 * Replaces Engine::new / models::load / Model::new (src/engine.rs:16-34,
 * src/models/mod.rs:65-71, src/models/openthai/model.rs:96-191) -- without the F32
 * expansion at load. */
int lg_engine_create(const lg_gguf *g, const lg_engine_opts *opts, lg_engine **out);
void lg_engine_destroy(lg_engine *e);
/* Replaces Backend::layers, src/models/mod.rs:14, plus the shapes. */
int lg_engine_info(const lg_engine *e, lg_model_info *info);
/* Block until all work queued on the engine's stream has finished. */
int lg_engine_sync(lg_engine *e);
/* Device memory held by the engine's grow-only workspaces (activations, the decode workspace, output
 * staging), in bytes: weights and the KV page pool are not counted.  No reference counterpart (the
 * reference holds no device memory); for serving-side memory accounting, and it shows that
 * lg_decode_noalloc grows nothing. */
int lg_engine_workspace_bytes(const lg_engine *e, int64_t *bytes);

/* y[m][rows] = x[m][cols] . W[rows][cols]^T (+ bias[rows]) with W the named uploaded
 * matrix.  Host pointers.  Replaces Matrix::apply, src/tensor.rs:10-39. */
int lg_matmul(lg_engine *e, const char *tensor, const float *x, int m, const float *bias, float *y);

/* ---- sequences over the paged F16 KV cache (no reference counterpart: the reference
 * recomputes every forward from scratch, src/models/openthai/model.rs:192-241) ---- */
int lg_seq_create(lg_engine *e, int *seq);
/* New sequence sharing the first `ntokens` tokens' KV pages of `parent` (whole pages are
 * shared by reference count; a partially filled last page is copied). */
int lg_seq_fork(lg_engine *e, int parent, int ntokens, int *child);
int lg_seq_free(lg_engine *e, int seq);
int lg_seq_len(lg_engine *e, int seq, int *len);
/* Read back the cached keys (after RoPE) and values of positions [pos0, pos0 + n) of one layer of a
 * sequence, as f32 [n][kv_heads * head_dim] each (host).  For tests and debugging: the reference keeps
 * no cache (src/models/openthai/model.rs:276-294 recomputes k and v every forward); this exposes the
 * k/v rows that its attention loop would read. */
int lg_seq_kv_read(lg_engine *e, int seq, int layer, int pos0, int n, float *k, float *v);

typedef int (*lg_cancel_fn)(void *arg); /* non-zero = cancel; polled between layers */

/* Append `n` tokens to `seq`, run them through every layer and return logits at the
 * `npos` positions (indices into the n new tokens) for the head rows `vocab_ids`
 * (NULL = the full vocabulary, nv ignored).  logits is [npos][nv] (host).
 * Replaces Model::forward(ids, positions, canceled), src/models/openthai/model.rs:192-241. */
int lg_forward(lg_engine *e, int seq, const int32_t *ids, int n, const int32_t *positions,
               int npos, const int32_t *vocab_ids, int nv, float *logits, lg_cancel_fn cancel,
               void *cancel_arg);

/* One request of a batched prefill. */
typedef struct {
  int seq;                  /* sequence to append to */
  const int32_t *ids;       /* n token ids */
  int n;
  const int32_t *positions; /* npos answer positions (indices into ids) */
  int npos;
} lg_request;

typedef struct lg_batch lg_batch;

/* Stage a batch of requests in HBM (token ids, positions, page tables).  Replaces the
 * sequential per-request loop of /v1/decide/batch (src/server.rs:301-319) with one GPU
 * batch.  The sequences' KV pages are reserved here. */
int lg_batch_create(lg_engine *e, const lg_request *reqs, int nreq, lg_batch **out);
void lg_batch_free(lg_engine *e, lg_batch *b);
/* Run a staged batch: prefill every request, then option scoring at every answer position
 * over the head rows `option_ids` (k of them, 1..256) with temperature `temperature`.
 * Outputs (host, [sum npos][k], NULL to skip): raw logits, probabilities, log-probabilities
 * (the last two need k <= 32).
 * Probabilities follow src/models/openthai/decision.rs:268-279,297-303; log-probabilities
 * are the option log-softmax of logit/temperature. */
int lg_batch_run(lg_engine *e, lg_batch *b, const int32_t *option_ids, int k, float temperature,
                 float *logits, float *probs, float *logprobs, lg_cancel_fn cancel,
                 void *cancel_arg);
/* Return every sequence of a batch that has run to its length at staging time (its pages
 * stay reserved), so the same staged requests can be executed again. */
int lg_batch_rewind(lg_engine *e, lg_batch *b);

/* Greedy decode: feed `first` and then each argmax for `steps` single-token steps on `seq`
 * (which must hold its prefilled context).  tokens[steps] receives each step's argmax
 * (first maximum wins, src/models/openthai/decision.rs:330-335); logits (optional, host,
 * [steps][vocab]) each step's full-vocabulary logits.  The context after the last step may hold at
 * most 65,536 tokens (the decode attention's 1024 pages); a longer run fails with LG_ERR_INVALID
 * before any step runs. */
int lg_decode(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, float *logits);
/* lg_decode without any device allocation: its workspace (activations, attention page partials,
 * argmax partials, token slots and page table) lives in a fixed 16 MiB scratch array that every GPU
 * the library runs on holds until the process ends, so the call makes no hipMalloc/hipFree.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Results equal lg_decode.
 * A run whose workspace exceeds the scratch fails with LG_ERR_INVALID and changes nothing; the
 * workspace grows by hq x (2 + head_dim) x 4 bytes per 64-token page of context, so the scratch would
 * hold about 70k tokens of context on the 7B shape and 127k on d2048, beyond the 65,536 tokens that
 * decode accepts at all.  Every call on one GPU shares that GPU's scratch: a call holds a per-GPU
 * lock from its first launch until its stream has drained, so calls from engines on several threads
 * run one after another. */
int lg_decode_noalloc(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, float *logits);

/* lg_decode (no logits) with the whole step loop -- every kernel of every step -- captured into one
 * HIP graph after the metadata upload and launched once; the wall time of the capture and
 * instantiation and that of the graph launch (through its completion) are returned.  No reference
 * counterpart: it measures whether launching the decode as a graph changes its GPU time.  Tokens
 * and the sequence's new length equal lg_decode's; kernel profiling must be off. */
int lg_decode_graph(lg_engine *e, int seq, int32_t first, int steps, int32_t *tokens, double *capture_ms,
                    double *run_ms);

/* Launch-floor probe on the current device: `launches` dependent launches of a plain read kernel
 * (16-byte loads, four per thread issued together, nothing written), each over its own zero-filled slice
 * of `bytes` (slices of about 2 GiB in all, so the reads come from HBM rather than the memory-side cache),
 * timed with events on a stream of its own; *us_per_launch receives the average.  No
 * reference counterpart: it measures the fixed cost of a dependent launch and the streaming rate that
 * the decode GEMV's launches are compared against. */
int lg_probe_read(uint64_t bytes, int launches, double *us_per_launch);

/* Option scores over host logits, the CPU side of the same rule (for callers that
 * already hold logits).  Replaces src/models/openthai/decision.rs:268-279. */
int lg_option_scores(const float *logits, int k, float temperature, float *probs,
                     float *logprobs);

/* Decision confidence of k option probabilities: 1 - H(p)/ln k clamped to [0,1] (1 when
 * k <= 1), p floored at 1e-12 inside the entropy.  mode 0 computes in f32 with logf, as
 * src/models/openthai/decision.rs:304-313; mode 1 accumulates in f64, as
 * src/models/laya/decision.rs:155-167. */
#define LG_CONF_F32 0
#define LG_CONF_F64 1
int lg_option_confidence(const float *probs, int k, int mode, float *confidence);

/* ---- request-level decide over token ids ----
 * The reference's decision layer (src/models/openthai/decision.rs) at the token level: the
 * tokenizer is not on this path, so every text piece arrives as token ids and the control
 * tokens (state/question/kind/option/answer markers) come from the model's laya.decide.*
 * metadata, or by default from the top of the vocabulary: option slot s (s < 255) and the
 * abstain slot 255 are ids V-256+s, then V-257 state, V-258 question, V-259..V-261 the
 * choice/score/noul kind markers, V-262 answer, V-263 newline, V-264 colon. */
#define LG_Q_CHOICE 0
#define LG_Q_SCORE 1
#define LG_Q_NOUL 2

typedef struct {
  int32_t kind;                       /* LG_Q_CHOICE (1..255 options), LG_Q_SCORE (2..10 levels),
                                         LG_Q_NOUL (2 options: no, yes) */
  const int32_t *instruction;         /* instruction tokens */
  int32_t n_instruction;
  int32_t n_options;
  const int32_t *const *names;        /* [n_options] option name tokens (score levels may be empty) */
  const int32_t *name_len;
  const int32_t *const *descs;        /* [n_options] description tokens; NULL / 0 length = none */
  const int32_t *desc_len;            /* NULL = no descriptions */
} lg_question;

typedef struct {
  const int32_t *state;               /* state tokens (truncated to the state budget, first kept) */
  int32_t n_state;
  const lg_question *questions;       /* 1..256 */
  int32_t n_questions;
  int32_t permutations;               /* 0 = default rule; else 1..32 passes */
  int32_t order_invariant;            /* -1 unset, 0 false, 1 true */
} lg_decide_request;

typedef struct {
  float *probs;                       /* [sum of n_options], question order (caller-owned) */
  float *abstain;                     /* [n_questions]: abstain slot mass (choice; else 0); for a
                                         Laya encoder the act probability of every question */
  float *confidence;                  /* [n_questions]: 1 - H(p)/ln k */
  float *score;                       /* [n_questions]: sum_j j p_j (score questions; else 0) */
  int32_t *choice;                    /* [n_questions]: first most probable option */
  int32_t input_tokens;               /* tokens of the first pass's prompt */
  int32_t permutations;               /* passes run */
  int32_t truncated;                  /* 1 when the state was cut to its budget */
} lg_decide_result;

/* Decide: encode every option-order pass, prefill all passes as one GPU batch, score the
 * 256 slot rows at each answer position and aggregate.  Replaces Backend::decide / decide,
 * src/models/mod.rs:16-22 and src/models/openthai/decision.rs:243-390 (text encoding aside).
 * For a Laya encoder: one forward per question (src/models/laya/decision.rs:168-318), all the
 * questions as GPU batches; one pass, truncated 0, input_tokens summed over the questions. */
int lg_decide(lg_engine *e, const lg_decide_request *req, lg_decide_result *out, lg_cancel_fn cancel,
              void *cancel_arg);
/* The token layout of pass `pass` of a request for the model in `g` (host only, no GPU):
 * ids[cap] (n written), positions[n_questions], order[n_questions][255] (option index shown at
 * each slot), truncated, and the number of passes.  Replaces encode / permutations,
 * src/models/openthai/decision.rs:140-233. */
int lg_decide_encode(const lg_gguf *g, const lg_decide_request *req, int pass, int32_t *ids, int cap,
                     int *n, int32_t *positions, int32_t *order, int *truncated, int *passes);

/* One input of the Laya encoder: token ids (<= laya.max_len), the positions of the option markers
 * (1..16) and the question type (0 choice, 1 score, 2 noul). */
typedef struct {
  const int32_t *ids;
  int32_t n;
  const int32_t *markers;
  int32_t k;
  int32_t qtype;
} lg_laya_input;

/* Laya Model::forward (src/models/laya/model.rs:303-416) for n inputs as one GPU batch: option
 * logits (k of each input, concatenated, host) and act logits [n][2] (host).  Errors as the
 * reference: "invalid inference input shape", "token ID out of range", "non-finite model output".
 * LG_ERR_UNSUPPORTED on other model families. */
int lg_laya_forward(lg_engine *e, const lg_laya_input *in, int n, float *logits, float *act, lg_cancel_fn cancel,
                    void *cancel_arg);

/* The Laya token layout of question `question` of a request (host only, no GPU): ids[cap] (n
 * written) and markers[n_options] (the [mask] position of each option).  The instruction tokens
 * stand for the encoded "<kind> question: <instructions>" and each option's name + description
 * tokens for its encoded text.  Replaces encode, src/models/laya/decision.rs:100-154. */
int lg_laya_decide_encode(const lg_gguf *g, const lg_decide_request *req, int question, int32_t *ids, int cap,
                          int *n, int32_t *markers);
/* The Laya aggregation over logits the caller already holds (host only): option logits (k of
 * every question, concatenated) and act logits [n_questions][2].  abstain[q] receives the
 * act probability (softmax of the act logits, entry 0).  Replaces decision.rs:185-298. */
int lg_laya_decide_scores(const lg_gguf *g, const lg_decide_request *req, const float *logits, const float *act,
                          lg_decide_result *out);

/* Several decide requests at once: the states of /v1/decide/batch (src/server.rs:235-319, which
 * runs one decide per state while a global busy flag turns other requests away).  Every request
 * is validated and every pass encoded before any inference (at most 256 requests and 256
 * questions in total, as server.rs:238-283); then all passes of all requests run as GPU
 * batches of at most max_batch_tokens tokens (as few batches as the budget allows) and each
 * request is aggregated into its own result.  Results equal lg_decide on each request alone. */
int lg_decide_batch(lg_engine *e, const lg_decide_request *reqs, int n, lg_decide_result *outs,
                    lg_cancel_fn cancel, void *cancel_arg);

/* The aggregation of lg_decide over slot logits the caller already holds ([passes][n_questions]
 * [256], the 256 slot rows at each answer position of each pass), host only.  Replaces the
 * scoring of src/models/openthai/decision.rs:268-279,297-336. */
int lg_decide_scores(const lg_gguf *g, const lg_decide_request *req, const float *slot_logits,
                     lg_decide_result *out);

/* ---- profiling: per-kernel-class HIP event timing on the engine's stream ---- */
/* When on, every launch of the timed kernel classes is bracketed by HIP events. */
int lg_profile_enable(lg_engine *e, int on);
/* Accumulated launches and device milliseconds of one kernel class since the last reset
 * ("gemm", "gemv", "attn_prefill", "attn_decode", "rope_kv", "rmsnorm", "embed", "head"). */
int lg_profile_read(lg_engine *e, const char *cls, int64_t *launches, double *ms,
                    double *bytes, double *flops);
int lg_profile_reset(lg_engine *e);

#ifdef __cplusplus
}
#endif
#endif
