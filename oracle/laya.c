/*
 * CPU oracle for the Laya encoder (ModernBERT trunk + 2-layer decision head) -- TEST
 * INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of src/models/laya/model.rs:301-416 with src/tensor.rs:103-195 (norm,
 * gelu, softmax, attention, dot) in the reference's f32 operation order, built with
 * -ffp-contract=off.  The caller (pyoracle.Laya) resolves the model's layers from the GGUF's
 * ggmlc.graph_spec as model.rs:60-291 does and hands over decoded f32 weights.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* src/tensor.rs:103-122: (a - mean) * scale * w + b per row; sums left to right from -0.0 */
static void ln_rows(const float *x, int rows, int d, const or_ln *n, float *y) {
  for (int r = 0; r < rows; ++r) {
    const float *a = x + (size_t)r * d;
    float s = -0.0f;
    for (int j = 0; j < d; ++j) s = s + a[j];
    const float mean = s / (float)d;
    float v = -0.0f;
    for (int j = 0; j < d; ++j) {
      const float z = a[j] - mean;
      v = v + z * z;
    }
    const float var = v / (float)d;
    const float scale = 1.0f / sqrtf(var + n->eps);
    float *o = y + (size_t)r * d;
    for (int j = 0; j < d; ++j) o[j] = (a[j] - mean) * scale * (n->w ? n->w[j] : 1.0f) + (n->b ? n->b[j] : 0.0f);
  }
}

void or_layer_norm(const float *x, int rows, int d, const float *w, const float *b, float eps, float *y) {
  or_ln n = {w, b, eps};
  ln_rows(x, rows, d, &n, y);
}

/* src/tensor.rs:129-131 */
float or_gelu(float x) { return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x))); }

static void lin(const or_lin *l, const float *x, int m, int threads, float *y) {
  or_apply(l->w, l->rows, l->cols, x, m, l->b, threads, y);
}

/* src/tensor.rs:141-192: q|k|v rows, table RoPE (pairs j, j + hd/2 at the token's row of the
 * tables), scores dot * (1/sqrt(hd)) over j in [i - window, i + window] (all keys when window
 * < 0), softmax, out += p v. */
void or_laya_attention(const float *qkv, int s, int d, int hd, const float *cs, const float *sn, int window,
                       float *out) {
  const int heads = d / hd;
  float *q = (float *)malloc((size_t)s * d * sizeof(float));
  float *k = (float *)malloc((size_t)s * d * sizeof(float));
  float *v = (float *)malloc((size_t)s * d * sizeof(float));
  for (int i = 0; i < s; ++i) {
    memcpy(q + (size_t)i * d, qkv + (size_t)i * 3 * d, (size_t)d * sizeof(float));
    memcpy(k + (size_t)i * d, qkv + (size_t)i * 3 * d + d, (size_t)d * sizeof(float));
    memcpy(v + (size_t)i * d, qkv + (size_t)i * 3 * d + 2 * d, (size_t)d * sizeof(float));
  }
  if (cs) {
    float *both[2] = {q, k};
    for (int t = 0; t < 2; ++t) {
      float *a = both[t];
      for (int i = 0; i < s; ++i)
        for (int h = 0; h < heads; ++h)
          for (int j = 0; j < hd / 2; ++j) {
            const size_t p = (size_t)i * d + (size_t)h * hd + j;
            const float u = a[p], w = a[p + hd / 2];
            a[p] = u * cs[(size_t)i * hd + j] - w * sn[(size_t)i * hd + j];
            a[p + hd / 2] = w * cs[(size_t)i * hd + j + hd / 2] + u * sn[(size_t)i * hd + j + hd / 2];
          }
    }
  }
  memset(out, 0, (size_t)s * d * sizeof(float));
  const float scale = 1.0f / sqrtf((float)hd);
  float *score = (float *)malloc((size_t)s * sizeof(float));
  float *p = (float *)malloc((size_t)s * sizeof(float));
  for (int h = 0; h < heads; ++h)
    for (int i = 0; i < s; ++i) {
      const int lo = window < 0 ? 0 : (i > window ? i - window : 0);
      const int hi = window < 0 ? s : (i + window + 1 < s ? i + window + 1 : s);
      for (int j = lo; j < hi; ++j)
        score[j] = or_dot(q + (size_t)i * d + (size_t)h * hd, k + (size_t)j * d + (size_t)h * hd, hd) * scale;
      or_softmax(score + lo, hi - lo, p + lo);
      float *o = out + (size_t)i * d + (size_t)h * hd;
      for (int j = lo; j < hi; ++j) {
        const float *vv = v + (size_t)j * d + (size_t)h * hd;
        for (int z = 0; z < hd; ++z) o[z] = o[z] + p[j] * vv[z];
      }
    }
  free(q); free(k); free(v); free(score); free(p);
}

static void add_rows(float *h, const float *y, size_t n) {
  for (size_t e = 0; e < n; ++e) h[e] = h[e] + y[e];
}

/* src/models/laya/model.rs:301-416 */
int or_laya_forward(const or_laya *m, const int32_t *ids, int s, const int32_t *markers, int k, int qtype,
                    float *logits, float *act) {
  const int d = m->d, hd = m->hd;
  if (s < 1 || s > m->max_len || qtype < 0 || qtype >= 3 || k < 1 || k > 16) return -1;
  for (int i = 0; i < k; ++i)
    if (markers[i] < 0 || markers[i] >= s) return -1;
  for (int i = 0; i < s; ++i)
    if (ids[i] < 0 || ids[i] >= m->vocab) return -2;
  float *h = (float *)malloc((size_t)s * d * sizeof(float));
  float *x = (float *)malloc((size_t)s * d * sizeof(float));
  float *y = (float *)malloc((size_t)s * d * sizeof(float));
  float *qkv = (float *)malloc((size_t)s * 3 * d * sizeof(float));
  float *att = (float *)malloc((size_t)s * d * sizeof(float));
  for (int i = 0; i < s; ++i) memcpy(x + (size_t)i * d, m->emb + (size_t)ids[i] * d, (size_t)d * sizeof(float));
  ln_rows(x, s, d, &m->embnorm, h);
  for (int l = 0; l < m->layers; ++l) {
    const or_laya_layer *L = &m->trunk[l];
    if (L->has_n1) ln_rows(h, s, d, &L->n1, x);
    else memcpy(x, h, (size_t)s * d * sizeof(float));
    lin(&L->qkv, x, s, m->threads, qkv);
    or_laya_attention(qkv, s, d, hd, L->full ? m->cos_full : m->cos_slide, L->full ? m->sin_full : m->sin_slide,
                      L->full ? -1 : 64, att);
    lin(&L->wo, att, s, m->threads, y);
    add_rows(h, y, (size_t)s * d);
    ln_rows(h, s, d, &L->n2, x);
    const int f = L->down.cols;
    float *up = (float *)malloc((size_t)s * 2 * f * sizeof(float));
    float *mm = (float *)malloc((size_t)s * f * sizeof(float));
    lin(&L->wi, x, s, m->threads, up);
    for (int i = 0; i < s; ++i)
      for (int j = 0; j < f; ++j)
        mm[(size_t)i * f + j] = or_gelu(up[(size_t)i * 2 * f + j]) * up[(size_t)i * 2 * f + f + j];
    lin(&L->down, mm, s, m->threads, y);
    add_rows(h, y, (size_t)s * d);
    free(up);
    free(mm);
  }
  ln_rows(h, s, d, &m->finalnorm, x);
  memcpy(h, x, (size_t)s * d * sizeof(float));
  for (int i = 0; i < s; ++i) add_rows(h + (size_t)i * d, m->type_emb + (size_t)qtype * d, (size_t)d);
  for (int l = 0; l < 2; ++l) {
    const or_laya_layer *L = &m->head[l];
    ln_rows(h, s, d, &L->n1, x);
    lin(&L->qkv, x, s, m->threads, qkv);
    or_laya_attention(qkv, s, d, hd, NULL, NULL, -1, att);
    lin(&L->wo, att, s, m->threads, y);
    add_rows(h, y, (size_t)s * d);
    ln_rows(h, s, d, &L->n2, x);
    const int f = L->wi.rows;
    float *fc = (float *)malloc((size_t)s * f * sizeof(float));
    lin(&L->wi, x, s, m->threads, fc);
    for (size_t e = 0; e < (size_t)s * f; ++e) fc[e] = fmaxf(fc[e], 0.0f);
    lin(&L->down, fc, s, m->threads, y);
    add_rows(h, y, (size_t)s * d);
    free(fc);
  }
  float *g = (float *)malloc((size_t)k * d * sizeof(float));
  float *gn = (float *)malloc((size_t)k * d * sizeof(float));
  float *s1 = (float *)malloc((size_t)k * d * sizeof(float));
  for (int i = 0; i < k; ++i) memcpy(g + (size_t)i * d, h + (size_t)markers[i] * d, (size_t)d * sizeof(float));
  ln_rows(g, k, d, &m->scorenorm, gn);
  lin(&m->score1, gn, k, m->threads, s1);
  for (size_t e = 0; e < (size_t)k * d; ++e) s1[e] = or_gelu(s1[e]);
  lin(&m->score2, s1, k, m->threads, logits); /* [k][1] */
  float p[16];
  or_softmax(logits, k, p);
  float top1 = 0.0f;
  for (int i = 0; i < k; ++i) top1 = fmaxf(top1, p[i]);
  float top2 = 0.0f;
  for (int i = 0; i < k; ++i) top2 = fmaxf(top2, p[i] * (top1 - p[i]) / ((top1 - p[i]) + 1e-6f));
  const float kk = (float)(k > 2 ? k : 2);
  float es = -0.0f;
  for (int i = 0; i < k; ++i) es = es + p[i] * logf(fmaxf(p[i], 1e-9f));
  const float ent = -es / logf(kk);
  const int a1 = m->act1.rows;
  float *pooled = (float *)malloc((size_t)(d + 4) * sizeof(float));
  float *xa = (float *)malloc((size_t)a1 * sizeof(float));
  memcpy(pooled, h, (size_t)d * sizeof(float));
  pooled[d] = top1;
  pooled[d + 1] = top1 - top2;
  pooled[d + 2] = ent;
  pooled[d + 3] = kk / 255.0f;
  lin(&m->act1, pooled, 1, m->threads, xa);
  for (int i = 0; i < a1; ++i) xa[i] = or_gelu(xa[i]);
  lin(&m->act2, xa, 1, m->threads, act);
  int rc = 0;
  for (int i = 0; i < k; ++i)
    if (!isfinite(logits[i])) rc = -3;
  if (!isfinite(act[0]) || !isfinite(act[1])) rc = -3;
  free(h); free(x); free(y); free(qkv); free(att); free(g); free(gn); free(s1); free(pooled); free(xa);
  return rc;
}
