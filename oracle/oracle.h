/*
 * CPU oracle for the Laya decoder forward pass -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU algorithm for the hot path,
 * in the reference's f32 operation order.  Only tests, the smoke check and the
 * bench's CPU-baseline leg may load it, and only to check (or time beside) the GPU
 * path's results: the product path never calls into this library.
 *
 * Each function cites the reference file:line it restates.  Built with
 * -ffp-contract=off so that every multiply and add rounds separately unless the
 * reference itself fuses them (the AVX2 FMA in Matrix::apply).
 */
#ifndef LAYA_ORACLE_H
#define LAYA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14 };

/* src/gguf.rs:81-93 -- (elements per block, bytes per block); -1 if unsupported. */
int or_layout(uint32_t kind, uint64_t *block, uint64_t *size);
/* src/gguf.rs:226-246 -- IEEE binary16 -> f32, exact. */
float or_half(uint16_t x);
/* src/gguf.rs:250-336 -- dequantise `len` bytes of `kind` into len/size*block floats. */
int or_decode(uint32_t kind, const uint8_t *b, uint64_t len, float *out);

/* src/gguf.rs:95-179 -- GGUF v3 parse over caller-owned bytes (borrowed for the handle's life). */
typedef struct or_gguf or_gguf;
or_gguf *or_gguf_open(const uint8_t *bytes, uint64_t n, char *err, int errlen);
void or_gguf_close(or_gguf *g);
int or_gguf_ntensors(const or_gguf *g);
/* 0 if found; dims[0] is the innermost (column) extent as in the file. */
int or_gguf_tensor(const or_gguf *g, const char *name, uint32_t *kind, uint64_t dims[4], int *nd,
                   const uint8_t **data, uint64_t *len);
double or_gguf_num(const or_gguf *g, const char *key, double dflt);
const char *or_gguf_str(const or_gguf *g, const char *key);

/* src/tensor.rs:10-102 -- out[m][rows] = x[m][cols] . W[rows][cols]^T (+ bias), 4-row tiles,
 * 8-lane FMA accumulators, sequential lane sum, separately-rounded tail, then bias. */
void or_apply(const float *w, int rows, int cols, const float *x, int m, const float *bias,
              int threads, float *out);
/* Loop-nest switches (process-wide), none of which changes a result bit: scalar forces the
 * scalar apply; blocked selects the cache-blocked AVX2 apply and the eight-wide attention
 * (for long full-depth parity runs).  The default is the reference's own loop order. */
void or_set_scalar_apply(int on);
void or_set_blocked(int on);
/* src/tensor.rs:193-195 */
float or_dot(const float *a, const float *b, int n);
/* src/tensor.rs:132-140 */
void or_softmax(const float *x, int n, float *p);
/* src/models/openthai/model.rs:84-94 with the offset and eps as parameters. */
void or_rms(const float *x, int rows, int d, const float *w, float offset, float eps, float *y);
/* src/models/openthai/model.rs:71-76 */
float or_silu(float x);

/* ---- assembled decoder (Llama/Qwen2 shape) ---- */
typedef struct or_model or_model;
or_model *or_model_load(const or_gguf *g, int threads, char *err, int errlen);
/* The same model with its layers decoded only while they run: or_prefill decodes layer l's weights
 * to F32 (the same gguf.rs:250-336 decode), runs it and frees it, so a full-depth forward of a 7B
 * shape holds one layer of F32 weights instead of all of them.  Results are bit-identical to
 * or_model_load's.  The GGUF handle must outlive the model. */
or_model *or_model_load_streamed(const or_gguf *g, int threads, char *err, int errlen);
void or_model_free(or_model *m);
/* layers, d_model, heads, kv_heads, head_dim, ffn, vocab, context */
void or_model_dims(const or_model *m, int out[8]);
void or_model_set_threads(or_model *m, int threads);

/* Per-sequence f32 K/V rows (the reference recomputes the whole sequence; rows of K/V
 * depend only on earlier tokens, so a cache reproduces the full recompute bit for bit). */
typedef struct or_cache or_cache;
or_cache *or_cache_new(const or_model *m, int capacity);
or_cache *or_cache_fork(const or_cache *c, int len);
void or_cache_free(or_cache *c);
int or_cache_len(const or_cache *c);
/* Cached K (after RoPE) and V rows [pos0, pos0 + n) of one layer, [n][hkv*hd] each; -1 if outside. */
int or_cache_read(const or_cache *c, int layer, int pos0, int n, float *k, float *v);

/* Run n tokens starting at the cache's current length; append their K/V; return the
 * residual-stream rows at `gather` (indices into the n new tokens), [ngather][d].
 * Layer-loop order follows src/models/openthai/model.rs:214-231. */
/* Causal GQA attention of one layer on caller-held rotated rows: q [n][hq*hd] at positions
 * pos0 .. pos0+n-1, k/v [pos0+n][hkv*hd], out [n][hq*hd] (src/models/openthai/model.rs:276-294). */
int or_attention(const float *q, const float *k, const float *v, int n, int pos0, int hq, int hkv, int hd,
                 int threads, float *out);
int or_prefill(or_model *m, or_cache *c, const int32_t *ids, int n, const int32_t *gather,
               int ngather, float *hidden);
/* Final RMSNorm + head rows `vocab_ids` (NULL = every row), src/models/openthai/model.rs:232-240. */
int or_head(or_model *m, const float *hidden, int rows, const int32_t *vocab_ids, int nv,
            float *logits);
/* First maximum wins (strict >), src/models/openthai/decision.rs:330-335. */
int or_argmax(const float *v, int n);
/* Option scores: z = logit / T; softmax over k (+ abstain logit when has_abstain);
 * probs renormalised over k (max(sum,1e-12)); logprobs = log of probs.
 * src/models/openthai/decision.rs:268-279,297-303. */
void or_option_scores(const float *logits, int k, float abstain_logit, int has_abstain,
                      float temperature, float *probs, float *logprobs, float *abstain);
/* Decision confidence 1 - H(p)/ln k, clamped to [0,1]; 1 when k <= 1.
 * f64 = 0: f32 entropy with logf, src/models/openthai/decision.rs:304-313.
 * f64 = 1: f64 entropy with log, src/models/laya/decision.rs:155-167. */
float or_confidence(const float *p, int k, int f64);

/* ---- OpenThai-SystemOne text tower (openthai.c), src/models/openthai/model.rs ---- */
typedef struct or_openthai or_openthai;
/* dims = {hidden, ffn, layers, heads, kv_heads, linear_heads, vocab}; full[l] != 0 marks a
 * full-attention layer (else gated DeltaNet).  model.rs:96-191. */
or_openthai *or_openthai_load(const or_gguf *g, const int dims[7], const int32_t *full, int threads,
                              char *err, int errlen);
void or_openthai_free(or_openthai *m);
void or_openthai_dims(const or_openthai *m, int out[7]);
void or_openthai_set_threads(or_openthai *m, int threads);
/* model.rs:192-241: slot logits [npos][256] (final norm, slot head + bias). */
int or_openthai_forward(or_openthai *m, const int32_t *ids, int n, const int32_t *pos, int npos,
                        float *logits);
/* Pieces of the forward, exposed for invariant tests:
 * model.rs:306-318 causal conv (kernel 4) + silu over raw[s][ch], conv[ch][4];
 * model.rs:319-358 gated delta rule over conv output qkv[s][3*nh*128], a/b[s][nh] -> out[s][nh*128];
 * model.rs:260-275 partial RoPE (64 of 256 dims) in place over buf[s][heads][256];
 * model.rs:276-294 causal GQA (scores / 16) over q[s][hq][256], k/v[s][hkv][256]. */
void or_ot_conv_silu(const float *raw, int s, int ch, const float *conv, float *out);
void or_ot_gated_delta(const float *qkv, const float *a, const float *b, const float *alog,
                       const float *dt, int s, int nh, int threads, float *out);
void or_ot_rope(float *buf, int s, int heads);
void or_ot_attention(const float *q, const float *k, const float *v, int s, int hq, int hkv, int threads,
                     float *out);

/* ---- Laya encoder (laya.c), src/models/laya/model.rs + src/tensor.rs:103-195 ---- */
typedef struct { const float *w, *b; float eps; } or_ln;             /* w/b NULL = absent */
typedef struct { const float *w, *b; int rows, cols; } or_lin;       /* w [rows][cols]; b NULL = none */
typedef struct { or_ln n1, n2; or_lin qkv, wo, wi, down; int has_n1, full; } or_laya_layer;
typedef struct {
  int layers, d, hd, vocab, max_len, threads;
  const float *emb;                              /* [vocab][d] */
  or_ln embnorm, finalnorm, scorenorm;
  const or_laya_layer *trunk;                    /* [layers] */
  const or_laya_layer *head;                     /* [2] */
  const float *type_emb;                         /* [3][d] */
  or_lin score1, score2, act1, act2;
  const float *cos_full, *sin_full, *cos_slide, *sin_slide; /* [max_len][hd] */
} or_laya;
/* src/tensor.rs:103-122 */
void or_layer_norm(const float *x, int rows, int d, const float *w, const float *b, float eps, float *y);
/* src/tensor.rs:129-131 */
float or_gelu(float x);
/* src/tensor.rs:141-192 over q|k|v rows [s][3d]; cos == NULL: no RoPE; window < 0: all keys */
void or_laya_attention(const float *qkv, int s, int d, int hd, const float *cs, const float *sn, int window,
                       float *out);
/* src/models/laya/model.rs:301-416: option logits [k] and act logits [2]; -1 invalid shape,
 * -2 token out of range, -3 non-finite output. */
int or_laya_forward(const or_laya *m, const int32_t *ids, int s, const int32_t *markers, int k, int qtype,
                    float *logits, float *act);

#ifdef __cplusplus
}
#endif
#endif
