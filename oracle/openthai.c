/*
 * CPU oracle for the OpenThai-SystemOne text tower -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of src/models/openthai/model.rs (Qwen3.5 hybrid: gated DeltaNet and
 * sigmoid-gated full attention layers, zero-centred RMSNorm, SwiGLU, 256-slot head) in the
 * reference's f32 operation order, built with -ffp-contract=off.  Sizes that the reference
 * pins to the 0.8B checkpoint (hidden 1024, 8/2 heads, 16 linear heads, vocab 248339) are
 * parameters here; the head geometry (256-dim attention heads with 64 rotary dims, 128-dim
 * linear heads, conv kernel 4, 256 slots) is fixed as in the reference.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"
#include "oracle.h"

enum { HD = 256, ROT = 32, LK = 128, KC = 4, SLOTS = 256 };

typedef struct {
  int full;
  float *n1, *n2, *gate, *up, *down;
  /* full attention */
  float *q, *k, *v, *o, *qn, *kn;
  /* gated DeltaNet */
  float *qkv, *z, *a, *b, *out, *conv, *dt, *alog, *norm;
} ot_layer;

struct or_openthai {
  int d, f, L, hq, hkv, nh, V, threads;
  uint32_t emb_kind;
  const uint8_t *emb;
  ot_layer *layers;
  float *norm, *head, *bias;
};

static int ot_err(char *err, int errlen, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  if (err && errlen > 0) vsnprintf(err, (size_t)errlen, fmt, ap);
  va_end(ap);
  return -1;
}

/* model.rs:54-70: a matrix must have dims [cols, rows]; a vector only its element count. */
static float *ot_load(const or_gguf *g, const char *name, uint64_t cols, uint64_t rows, int vector,
                      char *err, int errlen) {
  uint32_t kind;
  uint64_t dims[4];
  int nd;
  const uint8_t *data;
  uint64_t len;
  if (or_gguf_tensor(g, name, &kind, dims, &nd, &data, &len)) {
    ot_err(err, errlen, "missing tensor %s", name);
    return NULL;
  }
  uint64_t count = 1;
  for (int i = 0; i < nd; ++i) count *= dims[i];
  int ok = vector ? count == cols * rows : (nd == 2 && dims[0] == cols && dims[1] == rows);
  if (!ok) {
    ot_err(err, errlen, "%s: unexpected %s shape", name, vector ? "vector" : "matrix");
    return NULL;
  }
  float *o = (float *)malloc(count * sizeof(float));
  if (or_decode(kind, data, len, o)) {
    free(o);
    ot_err(err, errlen, "%s: unsupported kind %u", name, kind);
    return NULL;
  }
  return o;
}

void or_openthai_free(or_openthai *m) {
  if (!m) return;
  if (m->layers)
    for (int l = 0; l < m->L; ++l) {
      ot_layer *y = &m->layers[l];
      float *all[] = {y->n1, y->n2, y->gate, y->up, y->down, y->q, y->k, y->v, y->o, y->qn, y->kn,
                      y->qkv, y->z, y->a, y->b, y->out, y->conv, y->dt, y->alog, y->norm};
      for (size_t i = 0; i < sizeof all / sizeof all[0]; ++i) free(all[i]);
    }
  free(m->layers);
  free(m->norm);
  free(m->head);
  free(m->bias);
  free(m);
}

or_openthai *or_openthai_load(const or_gguf *g, const int dims[7], const int32_t *full, int threads,
                              char *err, int errlen) {
  or_openthai *m = (or_openthai *)calloc(1, sizeof(*m));
  m->d = dims[0];
  m->f = dims[1];
  m->L = dims[2];
  m->hq = dims[3];
  m->hkv = dims[4];
  m->nh = dims[5];
  m->V = dims[6];
  m->threads = threads < 1 ? 1 : threads;
  if (m->d < 1 || m->f < 1 || m->L < 1 || m->hq < 1 || m->hkv < 1 || m->hq % m->hkv || m->nh < 1 ||
      m->V < 1) {
    ot_err(err, errlen, "invalid OpenThai dimensions");
    or_openthai_free(m);
    return NULL;
  }
  uint32_t kind;
  uint64_t ed[4];
  int nd;
  uint64_t len;
  if (or_gguf_tensor(g, "model.embed_tokens.weight", &kind, ed, &nd, &m->emb, &len) || nd != 2 ||
      ed[0] != (uint64_t)m->d || ed[1] != (uint64_t)m->V || (kind != OR_F32 && kind != OR_F16)) {
    ot_err(err, errlen, "OpenThai embeddings must be F32/F16 with shape [vocab, hidden]");
    or_openthai_free(m);
    return NULL;
  }
  m->emb_kind = kind;
  m->layers = (ot_layer *)calloc((size_t)m->L, sizeof(ot_layer));
  const uint64_t d = m->d, f = m->f, qw = (uint64_t)m->hq * HD, kvw = (uint64_t)m->hkv * HD;
  const uint64_t lw = (uint64_t)m->nh * LK, cd = 3 * lw;
  char nm[256];
#define LOAD(dst, tail, cols, rows, vec)                                    \
  do {                                                                      \
    snprintf(nm, sizeof nm, "model.layers.%d.%s", l, tail);                 \
    if (!((dst) = ot_load(g, nm, cols, rows, vec, err, errlen))) goto bad;  \
  } while (0)
  for (int l = 0; l < m->L; ++l) {
    ot_layer *y = &m->layers[l];
    y->full = full[l] != 0;
    LOAD(y->n1, "input_layernorm.weight", d, 1, 1);
    LOAD(y->n2, "post_attention_layernorm.weight", d, 1, 1);
    LOAD(y->gate, "mlp.gate_proj.weight", d, f, 0);
    LOAD(y->up, "mlp.up_proj.weight", d, f, 0);
    LOAD(y->down, "mlp.down_proj.weight", f, d, 0);
    if (y->full) {
      LOAD(y->q, "self_attn.q_proj.weight", d, 2 * qw, 0);
      LOAD(y->k, "self_attn.k_proj.weight", d, kvw, 0);
      LOAD(y->v, "self_attn.v_proj.weight", d, kvw, 0);
      LOAD(y->o, "self_attn.o_proj.weight", qw, d, 0);
      LOAD(y->qn, "self_attn.q_norm.weight", HD, 1, 1);
      LOAD(y->kn, "self_attn.k_norm.weight", HD, 1, 1);
    } else {
      LOAD(y->qkv, "linear_attn.in_proj_qkv.weight", d, cd, 0);
      LOAD(y->z, "linear_attn.in_proj_z.weight", d, lw, 0);
      LOAD(y->a, "linear_attn.in_proj_a.weight", d, (uint64_t)m->nh, 0);
      LOAD(y->b, "linear_attn.in_proj_b.weight", d, (uint64_t)m->nh, 0);
      LOAD(y->out, "linear_attn.out_proj.weight", lw, d, 0);
      LOAD(y->conv, "linear_attn.conv1d.weight", cd * KC, 1, 1);
      LOAD(y->dt, "linear_attn.dt_bias", (uint64_t)m->nh, 1, 1);
      LOAD(y->alog, "linear_attn.A_log", (uint64_t)m->nh, 1, 1);
      LOAD(y->norm, "linear_attn.norm.weight", LK, 1, 1);
    }
  }
#undef LOAD
  if (!(m->norm = ot_load(g, "model.norm.weight", d, 1, 1, err, errlen))) goto bad;
  if (!(m->head = ot_load(g, "slot_head.weight", d, SLOTS, 0, err, errlen))) goto bad;
  if (!(m->bias = ot_load(g, "slot_head.bias", SLOTS, 1, 1, err, errlen))) goto bad;
  return m;
bad:
  or_openthai_free(m);
  return NULL;
}

void or_openthai_dims(const or_openthai *m, int out[7]) {
  int v[7] = {m->d, m->f, m->L, m->hq, m->hkv, m->nh, m->V};
  memcpy(out, v, sizeof v);
}

void or_openthai_set_threads(or_openthai *m, int threads) { m->threads = threads < 1 ? 1 : threads; }

/* model.rs:71-83 */
static float ot_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
static float ot_silu(float x) { return x * ot_sigmoid(x); }
static float ot_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* model.rs:306-318: causal depthwise conv over the last 4 projected rows, then silu. */
void or_ot_conv_silu(const float *raw, int s, int ch, const float *conv, float *out) {
  for (int i = 0; i < s; ++i)
    for (int c = 0; c < ch; ++c) {
      float v = 0.0f;
      for (int j = 0; j < KC; ++j)
        if (i + j >= KC - 1) v = v + raw[(size_t)(i + j - (KC - 1)) * ch + c] * conv[(size_t)c * KC + j];
      out[(size_t)i * ch + c] = ot_silu(v);
    }
}

/* model.rs:319-358: per head, a [key, value] = 128 x 128 state; per token: normalise q and k,
 * decay the state, delta = (v - S^T k) * beta, S += k delta^T, o = S^T q. */
typedef struct {
  const float *qkv, *a, *b, *alog, *dt;
  int s, nh;
  float *out;
} delta_ctx;

static void delta_heads(void *p, int lo, int hi) {
  const delta_ctx *c = (const delta_ctx *)p;
  const int nh = c->nh, cd = 3 * nh * LK, lw = nh * LK;
  float *state = (float *)malloc((size_t)LK * LK * sizeof(float));
  for (int h = lo; h < hi; ++h) {
    memset(state, 0, (size_t)LK * LK * sizeof(float));
    for (int i = 0; i < c->s; ++i) {
      const float *q = c->qkv + (size_t)i * cd + (size_t)h * LK;
      const float *k = q + lw;
      const float *v = q + 2 * lw;
      const float qs = 1.0f / sqrtf(or_dot(q, q, LK) + 1e-6f) / sqrtf(128.0f);
      const float ks = 1.0f / sqrtf(or_dot(k, k, LK) + 1e-6f);
      const float decay = expf(-expf(c->alog[h]) * ot_softplus(c->a[(size_t)i * nh + h] + c->dt[h]));
      const float beta = ot_sigmoid(c->b[(size_t)i * nh + h]);
      float delta[LK] = {0};
      for (int e = 0; e < LK * LK; ++e) state[e] = state[e] * decay;
      for (int j = 0; j < LK; ++j) {
        const float key = k[j] * ks;
        for (int d = 0; d < LK; ++d) delta[d] = delta[d] + state[j * LK + d] * key;
      }
      for (int d = 0; d < LK; ++d) delta[d] = (v[d] - delta[d]) * beta;
      float *o = c->out + (size_t)i * lw + (size_t)h * LK;
      for (int j = 0; j < LK; ++j) {
        const float key = k[j] * ks, query = q[j] * qs;
        for (int d = 0; d < LK; ++d) {
          state[j * LK + d] = state[j * LK + d] + key * delta[d];
          o[d] = o[d] + state[j * LK + d] * query;
        }
      }
    }
  }
  free(state);
}

void or_ot_gated_delta(const float *qkv, const float *a, const float *b, const float *alog,
                       const float *dt, int s, int nh, int threads, float *out) {
  memset(out, 0, (size_t)s * nh * LK * sizeof(float));
  delta_ctx c = {qkv, a, b, alog, dt, s, nh, out};
  or_parallel(nh, threads, delta_heads, &c);
}

/* model.rs:260-275: partial rotary embedding of the first 64 dims of every 256-dim head,
 * pairs (j, j + 32), angle = i / 1e7^(2j/64) with i the token index. */
void or_ot_rope(float *buf, int s, int heads) {
  for (int i = 0; i < s; ++i)
    for (int h = 0; h < heads; ++h)
      for (int j = 0; j < ROT; ++j) {
        const float angle = (float)i / powf(10000000.0f, (float)(2 * j) / 64.0f);
        const float co = cosf(angle), si = sinf(angle);
        const size_t p = (size_t)i * heads * HD + (size_t)h * HD + j;
        const float a = buf[p], b = buf[p + ROT];
        buf[p] = a * co - b * si;
        buf[p + ROT] = b * co + a * si;
      }
}

/* model.rs:276-294: causal GQA over normalised, rotated q/k; scores divided by 16. */
typedef struct {
  const float *q, *k, *v;
  int s, hq, hkv;
  float *out;
} fattn_ctx;

static void fattn_heads(void *p, int lo, int hi) {
  const fattn_ctx *c = (const fattn_ctx *)p;
  const int qw = c->hq * HD, kvw = c->hkv * HD, grp = c->hq / c->hkv;
  float *scores = (float *)malloc((size_t)c->s * sizeof(float));
  float *prob = (float *)malloc((size_t)c->s * sizeof(float));
  for (int h = lo; h < hi; ++h) {
    const int kh = h / grp;
    for (int i = 0; i < c->s; ++i) {
      for (int j = 0; j <= i; ++j)
        scores[j] = or_dot(c->q + (size_t)i * qw + (size_t)h * HD, c->k + (size_t)j * kvw + (size_t)kh * HD, HD) / 16.0f;
      or_softmax(scores, i + 1, prob);
      float *o = c->out + (size_t)i * qw + (size_t)h * HD;
      for (int j = 0; j <= i; ++j) {
        const float *v = c->v + (size_t)j * kvw + (size_t)kh * HD;
        for (int d = 0; d < HD; ++d) o[d] = o[d] + prob[j] * v[d];
      }
    }
  }
  free(scores);
  free(prob);
}

void or_ot_attention(const float *q, const float *k, const float *v, int s, int hq, int hkv, int threads,
                     float *out) {
  memset(out, 0, (size_t)s * hq * HD * sizeof(float));
  fattn_ctx c = {q, k, v, s, hq, hkv, out};
  or_parallel(hq, threads, fattn_heads, &c);
}

/* model.rs:244-299 */
static void full_run(const or_openthai *m, const ot_layer *y, const float *x, int s, float *res) {
  const int qw = m->hq * HD, kvw = m->hkv * HD, d = m->d;
  float *qgate = (float *)malloc((size_t)s * 2 * qw * sizeof(float));
  float *q = (float *)malloc((size_t)s * qw * sizeof(float));
  float *gate = (float *)malloc((size_t)s * qw * sizeof(float));
  float *kr = (float *)malloc((size_t)s * kvw * sizeof(float));
  float *k = (float *)malloc((size_t)s * kvw * sizeof(float));
  float *v = (float *)malloc((size_t)s * kvw * sizeof(float));
  float *att = (float *)malloc((size_t)s * qw * sizeof(float));
  or_apply(y->q, 2 * qw, d, x, s, NULL, m->threads, qgate);
  for (int i = 0; i < s; ++i)
    for (int h = 0; h < m->hq; ++h) {
      memcpy(q + (size_t)i * qw + (size_t)h * HD, qgate + (size_t)i * 2 * qw + (size_t)h * 2 * HD, HD * sizeof(float));
      memcpy(gate + (size_t)i * qw + (size_t)h * HD, qgate + (size_t)i * 2 * qw + (size_t)h * 2 * HD + HD,
             HD * sizeof(float));
    }
  or_rms(q, s * m->hq, HD, y->qn, 1.0f, 1e-6f, q);
  or_apply(y->k, kvw, d, x, s, NULL, m->threads, kr);
  or_rms(kr, s * m->hkv, HD, y->kn, 1.0f, 1e-6f, k);
  or_apply(y->v, kvw, d, x, s, NULL, m->threads, v);
  or_ot_rope(q, s, m->hq);
  or_ot_rope(k, s, m->hkv);
  or_ot_attention(q, k, v, s, m->hq, m->hkv, m->threads, att);
  for (size_t e = 0; e < (size_t)s * qw; ++e) att[e] = att[e] * ot_sigmoid(gate[e]);
  or_apply(y->o, d, qw, att, s, NULL, m->threads, res);
  free(qgate); free(q); free(gate); free(kr); free(k); free(v); free(att);
}

/* model.rs:302-362 */
static void delta_run(const or_openthai *m, const ot_layer *y, const float *x, int s, float *res) {
  const int d = m->d, nh = m->nh, lw = nh * LK, cd = 3 * lw;
  float *raw = (float *)malloc((size_t)s * cd * sizeof(float));
  float *qkv = (float *)malloc((size_t)s * cd * sizeof(float));
  float *z = (float *)malloc((size_t)s * lw * sizeof(float));
  float *a = (float *)malloc((size_t)s * nh * sizeof(float));
  float *b = (float *)malloc((size_t)s * nh * sizeof(float));
  float *o = (float *)malloc((size_t)s * lw * sizeof(float));
  float *on = (float *)malloc((size_t)s * lw * sizeof(float));
  or_apply(y->qkv, cd, d, x, s, NULL, m->threads, raw);
  or_apply(y->z, lw, d, x, s, NULL, m->threads, z);
  or_apply(y->a, nh, d, x, s, NULL, m->threads, a);
  or_apply(y->b, nh, d, x, s, NULL, m->threads, b);
  or_ot_conv_silu(raw, s, cd, y->conv, qkv);
  or_ot_gated_delta(qkv, a, b, y->alog, y->dt, s, nh, m->threads, o);
  or_rms(o, s * nh, LK, y->norm, 0.0f, 1e-6f, on);
  for (size_t e = 0; e < (size_t)s * lw; ++e) on[e] = on[e] * ot_silu(z[e]);
  or_apply(y->out, d, lw, on, s, NULL, m->threads, res);
  free(raw); free(qkv); free(z); free(a); free(b); free(o); free(on);
}

/* model.rs:192-241: returns slot logits [npos][256]; -1 on an invalid sequence. */
int or_openthai_forward(or_openthai *m, const int32_t *ids, int n, const int32_t *pos, int npos,
                        float *logits) {
  const int d = m->d, f = m->f;
  if (n < 1) return -1;
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= m->V) return -1;
  for (int i = 0; i < npos; ++i)
    if (pos[i] < 0 || pos[i] >= n) return -1;
  const size_t es = m->emb_kind == OR_F32 ? 4 : 2;
  float *x = (float *)malloc((size_t)n * d * sizeof(float));
  for (int i = 0; i < n; ++i)
    or_decode(m->emb_kind, m->emb + (size_t)ids[i] * d * es, (uint64_t)d * es, x + (size_t)i * d);
  float *h = (float *)malloc((size_t)n * d * sizeof(float));
  float *y = (float *)malloc((size_t)n * d * sizeof(float));
  float *g = (float *)malloc((size_t)n * f * sizeof(float));
  float *u = (float *)malloc((size_t)n * f * sizeof(float));
  for (int l = 0; l < m->L; ++l) {
    const ot_layer *ly = &m->layers[l];
    or_rms(x, n, d, ly->n1, 1.0f, 1e-6f, h);
    if (ly->full) full_run(m, ly, h, n, y);
    else delta_run(m, ly, h, n, y);
    for (size_t e = 0; e < (size_t)n * d; ++e) x[e] = x[e] + y[e];
    or_rms(x, n, d, ly->n2, 1.0f, 1e-6f, h);
    or_apply(ly->gate, f, d, h, n, NULL, m->threads, g);
    or_apply(ly->up, f, d, h, n, NULL, m->threads, u);
    for (size_t e = 0; e < (size_t)n * f; ++e) g[e] = ot_silu(g[e]) * u[e];
    or_apply(ly->down, d, f, g, n, NULL, m->threads, y);
    for (size_t e = 0; e < (size_t)n * d; ++e) x[e] = x[e] + y[e];
  }
  float *ans = (float *)malloc((size_t)(npos ? npos : 1) * d * sizeof(float));
  for (int i = 0; i < npos; ++i) memcpy(ans + (size_t)i * d, x + (size_t)pos[i] * d, (size_t)d * sizeof(float));
  if (npos) {
    or_rms(ans, npos, d, m->norm, 1.0f, 1e-6f, h);
    or_apply(m->head, SLOTS, d, h, npos, m->bias, m->threads, logits);
  }
  free(x); free(h); free(y); free(g); free(u); free(ans);
  return 0;
}
