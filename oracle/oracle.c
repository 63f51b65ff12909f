/*
 * CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).  Restates the reference's
 * CPU algorithm in plain C for parity checks; never linked into the product.
 */
#define _GNU_SOURCE
#include "oracle.h"
#include "internal.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------- */
/* src/gguf.rs:81-93                                                          */
int or_layout(uint32_t kind, uint64_t *block, uint64_t *size) {
  uint64_t b, s;
  switch (kind) {
  case 0: b = 1; s = 4; break;
  case 1: b = 1; s = 2; break;
  case 2: b = 32; s = 18; break;
  case 8: b = 32; s = 34; break;
  case 12: b = 256; s = 144; break;
  case 14: b = 256; s = 210; break;
  default: return -1;
  }
  if (block) *block = b;
  if (size) *size = s;
  return 0;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* src/gguf.rs:226-246 */
float or_half(uint16_t x) {
  uint32_t sign = ((uint32_t)x & 0x8000u) << 16;
  uint32_t e = (x >> 10) & 31u;
  uint32_t m = x & 1023u;
  if (e == 0) {
    if (m == 0) return bits_f32(sign);
    float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

static float h2(const uint8_t *b) { return or_half((uint16_t)(b[0] | (b[1] << 8))); }

/* src/gguf.rs:250-336 */
int or_decode(uint32_t kind, const uint8_t *b, uint64_t len, float *out) {
  uint64_t block, size;
  if (or_layout(kind, &block, &size)) return -1;
  uint64_t nb = len / size;
  switch (kind) {
  case 0:
    for (uint64_t i = 0; i < nb; ++i) memcpy(&out[i], b + 4 * i, 4);
    break;
  case 1:
    for (uint64_t i = 0; i < nb; ++i) out[i] = h2(b + 2 * i);
    break;
  case 8: /* Q8_0: [f16 d][32 x i8], w = d * q  (gguf.rs:264-271) */
    for (uint64_t i = 0; i < nb; ++i) {
      const uint8_t *c = b + 34 * i;
      float d = h2(c);
      for (int j = 0; j < 32; ++j) out[32 * i + j] = d * (float)(int8_t)c[2 + j];
    }
    break;
  case 2: /* Q4_0 (gguf.rs:272-280) */
    for (uint64_t i = 0; i < nb; ++i) {
      const uint8_t *c = b + 18 * i;
      float d = h2(c);
      for (int j = 0; j < 16; ++j) {
        out[32 * i + j] = d * ((float)(c[2 + j] & 15) - 8.0f);
        out[32 * i + j + 16] = d * ((float)(c[2 + j] >> 4) - 8.0f);
      }
    }
    break;
  case 12: /* Q4_K (gguf.rs:281-307): w = ((d*s)*q) - (dm*m) */
    for (uint64_t i = 0; i < nb; ++i) {
      const uint8_t *c = b + 144 * i;
      float d = h2(c), dm = h2(c + 2);
      const uint8_t *sc = c + 4, *qs = c + 16;
      float *o = out + 256 * i;
      for (int g = 0; g < 4; ++g) {
        uint8_t sm[2][2];
        for (int t = 0; t < 2; ++t) {
          int j = g * 2 + t;
          if (j < 4) {
            sm[t][0] = sc[j] & 63;
            sm[t][1] = sc[j + 4] & 63;
          } else {
            sm[t][0] = (uint8_t)((sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4));
            sm[t][1] = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
          }
        }
        for (int j = 0; j < 32; ++j) {
          uint8_t q = qs[g * 32 + j];
          o[g * 64 + j] = d * (float)sm[0][0] * (float)(q & 15) - dm * (float)sm[0][1];
          o[g * 64 + 32 + j] = d * (float)sm[1][0] * (float)(q >> 4) - dm * (float)sm[1][1];
        }
      }
    }
    break;
  case 14: /* Q6_K (gguf.rs:308-332): w = (d*sc)*(q-32) */
    for (uint64_t i = 0; i < nb; ++i) {
      const uint8_t *c = b + 210 * i;
      const uint8_t *ql = c, *qh = c + 128, *sc = c + 192;
      float d = h2(c + 208);
      float *o = out + 256 * i;
      for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
          int lo = n * 64 + l;
          uint8_t hi = qh[n * 32 + l];
          int si = n * 8 + l / 16;
          uint8_t q[4] = {
              (uint8_t)((ql[lo] & 15) | ((hi & 3) << 4)),
              (uint8_t)((ql[lo + 32] & 15) | (((hi >> 2) & 3) << 4)),
              (uint8_t)((ql[lo] >> 4) | (((hi >> 4) & 3) << 4)),
              (uint8_t)((ql[lo + 32] >> 4) | (((hi >> 6) & 3) << 4)),
          };
          for (int j = 0; j < 4; ++j)
            o[n * 128 + j * 32 + l] = d * (float)(int8_t)sc[si + j * 2] * ((float)q[j] - 32.0f);
        }
    }
    break;
  default:
    return -1;
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* GGUF v3 reader, src/gguf.rs:22-179                                         */
typedef struct {
  char *key;
  uint32_t type; /* GGUF metadata kind 0..12 */
  double num;
  char *str;
} or_meta;

typedef struct {
  char *name;
  uint64_t dims[4];
  int nd;
  uint32_t kind;
  uint64_t offset, len;
} or_tensor;

struct or_gguf {
  const uint8_t *bytes;
  uint64_t n;
  or_meta *meta;
  int nmeta;
  or_tensor *t;
  int nt;
};

typedef struct {
  const uint8_t *b;
  uint64_t n, p;
  char *err;
  int errlen;
  int failed;
} rdr;

static void fail(rdr *r, const char *fmt, ...) {
  if (r->failed) return;
  r->failed = 1;
  va_list ap;
  va_start(ap, fmt);
  if (r->err && r->errlen > 0) vsnprintf(r->err, (size_t)r->errlen, fmt, ap);
  va_end(ap);
}

static const uint8_t *take(rdr *r, uint64_t k) {
  if (r->failed) return NULL;
  if (r->p + k < r->p) { fail(r, "GGUF length overflow"); return NULL; }
  if (r->p + k > r->n) { fail(r, "truncated GGUF"); return NULL; }
  const uint8_t *s = r->b + r->p;
  r->p += k;
  return s;
}
static uint32_t rd32(rdr *r) {
  const uint8_t *s = take(r, 4);
  uint32_t v = 0;
  if (s) memcpy(&v, s, 4);
  return v;
}
static uint64_t rd64(rdr *r) {
  const uint8_t *s = take(r, 8);
  uint64_t v = 0;
  if (s) memcpy(&v, s, 8);
  return v;
}

static int utf8_ok(const uint8_t *s, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    uint8_t c = s[i];
    if (c < 0x80) { ++i; continue; }
    int len;
    uint32_t cp;
    if ((c & 0xe0) == 0xc0) { len = 2; cp = c & 0x1f; }
    else if ((c & 0xf0) == 0xe0) { len = 3; cp = c & 0x0f; }
    else if ((c & 0xf8) == 0xf0) { len = 4; cp = c & 0x07; }
    else return 0;
    if (i + (uint64_t)len > n) return 0;
    for (int k = 1; k < len; ++k) {
      if ((s[i + k] & 0xc0) != 0x80) return 0;
      cp = (cp << 6) | (s[i + k] & 0x3f);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
        cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
      return 0;
    i += (uint64_t)len;
  }
  return 1;
}

static char *rdstr(rdr *r) {
  uint64_t n = rd64(r);
  if (r->failed) return NULL;
  if (n > 32u * 1024u * 1024u) { fail(r, "GGUF string too large"); return NULL; }
  const uint8_t *s = take(r, n);
  if (!s) return NULL;
  if (!utf8_ok(s, n)) { fail(r, "invalid GGUF UTF-8"); return NULL; }
  char *o = (char *)malloc(n + 1);
  memcpy(o, s, n);
  o[n] = 0;
  return o;
}

/* src/gguf.rs:48-79; stores numbers/strings of scalar values, skips array contents. */
static void rdvalue(rdr *r, uint32_t t, int depth, or_meta *m) {
  if (depth > 4) { fail(r, "GGUF metadata nesting too deep"); return; }
  const uint8_t *s;
  double v = 0;
  switch (t) {
  case 0: s = take(r, 1); if (s) v = s[0]; break;
  case 1: s = take(r, 1); if (s) v = (int8_t)s[0]; break;
  case 2: s = take(r, 2); if (s) v = (uint16_t)(s[0] | (s[1] << 8)); break;
  case 3: s = take(r, 2); if (s) v = (int16_t)(uint16_t)(s[0] | (s[1] << 8)); break;
  case 4: v = rd32(r); break;
  case 5: v = (int32_t)rd32(r); break;
  case 6: { uint32_t u = rd32(r); v = bits_f32(u); } break;
  case 7: s = take(r, 1); if (s) v = s[0] != 0; break;
  case 8: {
    char *str = rdstr(r);
    if (m && str) { m->str = str; } else free(str);
  } break;
  case 9: {
    uint32_t et = rd32(r);
    uint64_t n = rd64(r);
    if (r->failed) return;
    if (n > 1000000) { fail(r, "GGUF array too large"); return; }
    for (uint64_t i = 0; i < n && !r->failed; ++i) rdvalue(r, et, depth + 1, NULL);
  } break;
  case 10: v = (double)rd64(r); break;
  case 11: v = (double)(int64_t)rd64(r); break;
  case 12: { uint64_t u = rd64(r); memcpy(&v, &u, 8); } break;
  default: fail(r, "unsupported GGUF metadata type %u", t); return;
  }
  if (m) { m->type = t; m->num = v; }
}

void or_gguf_close(or_gguf *g) {
  if (!g) return;
  for (int i = 0; i < g->nmeta; ++i) { free(g->meta[i].key); free(g->meta[i].str); }
  for (int i = 0; i < g->nt; ++i) free(g->t[i].name);
  free(g->meta);
  free(g->t);
  free(g);
}

or_gguf *or_gguf_open(const uint8_t *bytes, uint64_t n, char *err, int errlen) {
  rdr r = {bytes, n, 0, err, errlen, 0};
  or_gguf *g = (or_gguf *)calloc(1, sizeof(*g));
  g->bytes = bytes;
  g->n = n;
  const uint8_t *magic = take(&r, 4);
  if (magic && memcmp(magic, "GGUF", 4) != 0) fail(&r, "not a GGUF file");
  if (!r.failed && rd32(&r) != 3 && !r.failed) fail(&r, "expected GGUF version 3");
  uint64_t nt = rd64(&r), nk = rd64(&r);
  if (!r.failed && (nt > 100000 || nk > 100000)) fail(&r, "GGUF table too large");
  if (!r.failed) {
    g->meta = (or_meta *)calloc(nk ? nk : 1, sizeof(or_meta));
    for (uint64_t i = 0; i < nk && !r.failed; ++i) {
      char *k = rdstr(&r);
      uint32_t t = rd32(&r);
      or_meta m = {0};
      rdvalue(&r, t, 0, &m);
      if (r.failed) { free(k); free(m.str); break; }
      for (int j = 0; j < g->nmeta; ++j)
        if (!strcmp(g->meta[j].key, k)) { fail(&r, "duplicate GGUF metadata key"); break; }
      if (r.failed) { free(k); free(m.str); break; }
      m.key = k;
      g->meta[g->nmeta++] = m;
    }
  }
  if (!r.failed) {
    g->t = (or_tensor *)calloc(nt ? nt : 1, sizeof(or_tensor));
    for (uint64_t i = 0; i < nt && !r.failed; ++i) {
      char *name = rdstr(&r);
      uint32_t nd = rd32(&r);
      if (r.failed) { free(name); break; }
      if (nd < 1 || nd > 4) { fail(&r, "invalid tensor rank"); free(name); break; }
      or_tensor t = {0};
      uint64_t count = 1;
      for (uint32_t d = 0; d < nd && !r.failed; ++d) {
        uint64_t v = rd64(&r);
        if (r.failed) break;
        if (v == 0) { fail(&r, "empty tensor"); break; }
        if (count > UINT64_MAX / v) { fail(&r, "tensor size overflow"); break; }
        count *= v;
        t.dims[d] = v;
      }
      uint32_t kind = rd32(&r);
      uint64_t off = rd64(&r);
      uint64_t block = 0, size = 0;
      if (!r.failed && or_layout(kind, &block, &size))
        fail(&r, "unsupported GGML tensor type %u; supported F32/F16/Q4_0/Q8_0/Q4_K/Q6_K", kind);
      if (!r.failed && t.dims[0] % block) fail(&r, "invalid quantized row alignment");
      if (!r.failed && (count / block) > UINT64_MAX / size) fail(&r, "tensor byte size overflow");
      if (r.failed) { free(name); break; }
      for (int j = 0; j < g->nt; ++j)
        if (!strcmp(g->t[j].name, name)) { fail(&r, "duplicate tensor"); break; }
      if (r.failed) { free(name); break; }
      t.name = name;
      t.nd = (int)nd;
      t.kind = kind;
      t.offset = off;
      t.len = (count / block) * size;
      g->t[g->nt++] = t;
    }
  }
  if (!r.failed) {
    /* `v.num() as usize`, src/gguf.rs:158-165: non-numbers read 0, the cast saturates */
    double a = or_gguf_num(g, "general.alignment", 32);
    uint64_t align = !(a > 0) ? 0 : a >= 18446744073709551616.0 ? UINT64_MAX : (uint64_t)a;
    if (align == 0 || (align & (align - 1)) || align > 4096) fail(&r, "invalid GGUF alignment");
    else {
      uint64_t base = (r.p + align - 1) & ~(align - 1);
      /* the reference walks its BTreeMap, i.e. tensors in name order */
      int *ord = (int *)malloc(sizeof(int) * (size_t)(g->nt ? g->nt : 1));
      for (int i = 0; i < g->nt; ++i) ord[i] = i;
      for (int i = 1; i < g->nt; ++i) /* insertion sort by name (byte order) */
        for (int j = i; j > 0 && strcmp(g->t[ord[j - 1]].name, g->t[ord[j]].name) > 0; --j) {
          int x = ord[j]; ord[j] = ord[j - 1]; ord[j - 1] = x;
        }
      for (int i = 0; i < g->nt && !r.failed; ++i) {
        or_tensor *t = &g->t[ord[i]];
        if (t->offset % align) { fail(&r, "unaligned GGUF tensor"); break; }
        if (t->offset + base < t->offset) { fail(&r, "offset overflow"); break; }
        t->offset += base;
        if (t->offset + t->len < t->offset) { fail(&r, "length overflow"); break; }
        if (t->offset + t->len > n) { fail(&r, "truncated tensor data"); break; }
      }
      free(ord);
    }
  }
  if (r.failed) { or_gguf_close(g); return NULL; }
  return g;
}

int or_gguf_ntensors(const or_gguf *g) { return g->nt; }

int or_gguf_tensor(const or_gguf *g, const char *name, uint32_t *kind, uint64_t dims[4], int *nd,
                   const uint8_t **data, uint64_t *len) {
  for (int i = 0; i < g->nt; ++i)
    if (!strcmp(g->t[i].name, name)) {
      const or_tensor *t = &g->t[i];
      if (kind) *kind = t->kind;
      if (dims) memcpy(dims, t->dims, sizeof(t->dims));
      if (nd) *nd = t->nd;
      if (data) *data = g->bytes + t->offset;
      if (len) *len = t->len;
      return 0;
    }
  return -1;
}

double or_gguf_num(const or_gguf *g, const char *key, double dflt) {
  for (int i = 0; i < g->nmeta; ++i)
    if (!strcmp(g->meta[i].key, key))  /* J::num(): only numbers have a value */
      return g->meta[i].type == 7 || g->meta[i].type == 8 || g->meta[i].type == 9 ? 0 : g->meta[i].num;
  return dflt;
}

const char *or_gguf_str(const or_gguf *g, const char *key) {
  for (int i = 0; i < g->nmeta; ++i)
    if (!strcmp(g->meta[i].key, key)) return g->meta[i].str ? g->meta[i].str : "";
  return "";
}

/* ------------------------------------------------------------------------- */
/* Threading helper: the reference splits token rows over goroutines          */
/* (src/tensor.rs:17-37); per-row arithmetic does not depend on the split.    */
typedef void (*range_fn)(void *ctx, int lo, int hi);
typedef struct { range_fn f; void *ctx; int lo, hi; } job;
static void *job_run(void *p) {
  job *j = (job *)p;
  j->f(j->ctx, j->lo, j->hi);
  return NULL;
}
static void parallel(int n, int workers, range_fn f, void *ctx) {
  if (workers < 1) workers = 1;
  if (workers > n) workers = n;
  if (workers <= 1) { if (n > 0) f(ctx, 0, n); return; }
  int per = (n + workers - 1) / workers;
  pthread_t th[256];
  job jobs[256];
  if (workers > 256) workers = 256;
  int started = 0;
  for (int t = 1; t < workers; ++t) {
    int lo = t * per, hi = lo + per < n ? lo + per : n;
    if (lo >= n) break;
    jobs[t] = (job){f, ctx, lo, hi};
    pthread_create(&th[t], NULL, job_run, &jobs[t]);
    started = t;
  }
  f(ctx, 0, per < n ? per : n);
  for (int t = 1; t <= started; ++t) pthread_join(th[t], NULL);
}
void or_parallel(int n, int workers, void (*f)(void *, int, int), void *ctx) { parallel(n, workers, f, ctx); }

/* ------------------------------------------------------------------------- */
/* src/tensor.rs:59-102: per (r, c): 8 FMA lanes over k in steps of 8, lanes   */
/* summed left to right, tail of k%8 with separate mul and add, then + bias.  */
typedef struct {
  const float *w, *x, *bias;
  float *out;
  int k, n;
} apply_ctx;

static inline float lane_sum(const float a[8]) {
  float v = -0.0f; /* Rust's f32 Sum fold */
  for (int l = 0; l < 8; ++l) v = v + a[l];
  return v;
}

static void apply_rows_scalar(const apply_ctx *a, int start, int end) {
  int k = a->k, n = a->n;
  for (int r = start; r < end; r += 4) {
    int nr = end - r < 4 ? end - r : 4;
    for (int c = 0; c < n; ++c) {
      float acc[4][8] = {{0}};
      int j = 0;
      for (; j + 8 <= k; j += 8)
        for (int t = 0; t < nr; ++t)
          for (int l = 0; l < 8; ++l)
            acc[t][l] = fmaf(a->w[(size_t)c * k + j + l], a->x[(size_t)(r + t) * k + j + l], acc[t][l]);
      for (int t = 0; t < nr; ++t) {
        float v = lane_sum(acc[t]);
        for (int q = j; q < k; ++q) v = v + a->w[(size_t)c * k + q] * a->x[(size_t)(r + t) * k + q];
        if (a->bias) v = v + a->bias[c];
        a->out[(size_t)(r + t) * n + c] = v;
      }
    }
  }
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static void apply_rows_avx2(const apply_ctx *a, int start,
                                                                 int end) {
  int k = a->k, n = a->n;
  for (int r = start; r < end; r += 4) {
    int nr = end - r < 4 ? end - r : 4;
    for (int c = 0; c < n; ++c) {
      __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),
                       _mm256_setzero_ps()};
      int j = 0;
      const float *wr = a->w + (size_t)c * k;
      for (; j + 8 <= k; j += 8) {
        __m256 v = _mm256_loadu_ps(wr + j);
        for (int t = 0; t < nr; ++t)
          acc[t] = _mm256_fmadd_ps(v, _mm256_loadu_ps(a->x + (size_t)(r + t) * k + j), acc[t]);
      }
      for (int t = 0; t < nr; ++t) {
        float lanes[8];
        _mm256_storeu_ps(lanes, acc[t]);
        float v = lane_sum(lanes);
        for (int q = j; q < k; ++q) v = v + wr[q] * a->x[(size_t)(r + t) * k + q];
        if (a->bias) v = v + a->bias[c];
        a->out[(size_t)(r + t) * n + c] = v;
      }
    }
  }
}
#endif

#if defined(__x86_64__)
/* The same per-(r, c) arithmetic as apply_rows_avx2 with a cache-friendly loop nest (the
 * blocked mode, or_set_blocked): columns in blocks whose weight rows stay in L2 while every
 * 4-row tile of the worker passes over them, two columns per pass over a tile's x rows.  Each
 * output still gets its own 8 lane accumulators over k in order, the same fold and the same
 * tail, so the results are bit-identical to the reference loop order; only memory traffic
 * differs.  The reference loop order stays the default (the CPU baseline times it). */
__attribute__((target("avx2,fma"))) static void finish_col(const apply_ctx *a, int r, int nr, int c, int j,
                                                           const __m256 *acc) {
  int k = a->k, n = a->n;
  const float *wr = a->w + (size_t)c * k;
  for (int t = 0; t < nr; ++t) {
    float lanes[8];
    _mm256_storeu_ps(lanes, acc[t]);
    float v = lane_sum(lanes);
    for (int q = j; q < k; ++q) v = v + wr[q] * a->x[(size_t)(r + t) * k + q];
    if (a->bias) v = v + a->bias[c];
    a->out[(size_t)(r + t) * n + c] = v;
  }
}

__attribute__((target("avx2,fma"))) static void apply_block(const apply_ctx *a, int start, int end,
                                                             int col_lo, int col_hi) {
  int k = a->k;
  int cb = 262144 / (4 * (k > 0 ? k : 1));
  if (cb < 2) cb = 2;
  cb &= ~1;
  for (int c0 = col_lo; c0 < col_hi; c0 += cb) {
    int c1 = c0 + cb < col_hi ? c0 + cb : col_hi;
    for (int r = start; r < end; r += 4) {
      int nr = end - r < 4 ? end - r : 4;
      const float *x0 = a->x + (size_t)r * k;
      int c = c0;
      for (; c + 2 <= c1; c += 2) {
        const float *w0 = a->w + (size_t)c * k, *w1 = w0 + k;
        __m256 p[4], q[4];
        for (int t = 0; t < 4; ++t) p[t] = q[t] = _mm256_setzero_ps();
        int j = 0;
        if (nr == 4) {
          for (; j + 8 <= k; j += 8) {
            __m256 v0 = _mm256_loadu_ps(w0 + j), v1 = _mm256_loadu_ps(w1 + j);
            __m256 a0 = _mm256_loadu_ps(x0 + j), a1 = _mm256_loadu_ps(x0 + k + j);
            __m256 a2 = _mm256_loadu_ps(x0 + 2 * (size_t)k + j), a3 = _mm256_loadu_ps(x0 + 3 * (size_t)k + j);
            p[0] = _mm256_fmadd_ps(v0, a0, p[0]);
            q[0] = _mm256_fmadd_ps(v1, a0, q[0]);
            p[1] = _mm256_fmadd_ps(v0, a1, p[1]);
            q[1] = _mm256_fmadd_ps(v1, a1, q[1]);
            p[2] = _mm256_fmadd_ps(v0, a2, p[2]);
            q[2] = _mm256_fmadd_ps(v1, a2, q[2]);
            p[3] = _mm256_fmadd_ps(v0, a3, p[3]);
            q[3] = _mm256_fmadd_ps(v1, a3, q[3]);
          }
        } else {
          for (; j + 8 <= k; j += 8) {
            __m256 v0 = _mm256_loadu_ps(w0 + j), v1 = _mm256_loadu_ps(w1 + j);
            for (int t = 0; t < nr; ++t) {
              __m256 xv = _mm256_loadu_ps(x0 + (size_t)t * k + j);
              p[t] = _mm256_fmadd_ps(v0, xv, p[t]);
              q[t] = _mm256_fmadd_ps(v1, xv, q[t]);
            }
          }
        }
        finish_col(a, r, nr, c, j, p);
        finish_col(a, r, nr, c + 1, j, q);
      }
      for (; c < c1; ++c) {
        const float *w0 = a->w + (size_t)c * k;
        __m256 p[4];
        for (int t = 0; t < 4; ++t) p[t] = _mm256_setzero_ps();
        int j = 0;
        for (; j + 8 <= k; j += 8) {
          __m256 v0 = _mm256_loadu_ps(w0 + j);
          for (int t = 0; t < nr; ++t) p[t] = _mm256_fmadd_ps(v0, _mm256_loadu_ps(x0 + (size_t)t * k + j), p[t]);
        }
        finish_col(a, r, nr, c, j, p);
      }
    }
  }
}

static void apply_rows_avx2_blocked(const apply_ctx *a, int start, int end) { apply_block(a, start, end, 0, a->n); }

/* Few rows (a decode step): the workers split the columns instead of the rows. */
typedef struct { const apply_ctx *a; int m, per; } colsplit_ctx;
static void apply_cols(void *p, int lo, int hi) {
  const colsplit_ctx *cs = (const colsplit_ctx *)p;
  int c0 = lo * cs->per, c1 = hi * cs->per < cs->a->n ? hi * cs->per : cs->a->n;
  if (c0 < c1) apply_block(cs->a, 0, cs->m, c0, c1);
}
#endif

static int g_force_scalar = 0;
static int g_blocked = 0;
void or_set_scalar_apply(int on) { g_force_scalar = on; }
void or_set_blocked(int on) { g_blocked = on; }

static void apply_tiles(void *p, int lo, int hi) {
  const apply_ctx *a = (const apply_ctx *)p;
#if defined(__x86_64__)
  if (!g_force_scalar && __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) {
    if (g_blocked)
      apply_rows_avx2_blocked(a, lo, hi);
    else
      apply_rows_avx2(a, lo, hi);
    return;
  }
#endif
  apply_rows_scalar(a, lo, hi);
}

void or_apply(const float *w, int rows, int cols, const float *x, int m, const float *bias,
              int threads, float *out) {
  apply_ctx a = {w, x, bias, out, cols, rows};
  /* count = min(threads, ceil(m/4)) workers over contiguous row ranges (tensor.rs:17-18);
   * ranges are multiples of... any split gives the same per-row results. */
  int count = threads < (m + 3) / 4 ? threads : (m + 3) / 4;
  if (count < 1) count = 1;
#if defined(__x86_64__)
  if (g_blocked && !g_force_scalar && count < threads && rows >= 64 * threads &&
      __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) {
    colsplit_ctx cs = {&a, m, 32};
    parallel((rows + 31) / 32, threads, apply_cols, &cs);
    return;
  }
#endif
  parallel(m, count, apply_tiles, &a);
}

/* src/tensor.rs:193-195 */
float or_dot(const float *a, const float *b, int n) {
  float s = -0.0f;
  for (int i = 0; i < n; ++i) s = s + a[i] * b[i];
  return s;
}

/* src/tensor.rs:132-140 */
void or_softmax(const float *x, int n, float *p) {
  float m = -INFINITY;
  for (int i = 0; i < n; ++i) m = fmaxf(m, x[i]);
  for (int i = 0; i < n; ++i) p[i] = expf(x[i] - m);
  float s = -0.0f;
  for (int i = 0; i < n; ++i) s = s + p[i];
  for (int i = 0; i < n; ++i) p[i] = p[i] / s;
}

/* src/models/openthai/model.rs:84-94 */
void or_rms(const float *x, int rows, int d, const float *w, float offset, float eps, float *y) {
  for (int r = 0; r < rows; ++r) {
    const float *a = x + (size_t)r * d;
    float scale = 1.0f / sqrtf(or_dot(a, a, d) / (float)d + eps);
    for (int j = 0; j < d; ++j) y[(size_t)r * d + j] = a[j] * scale * (offset + w[j]);
  }
}

/* src/models/openthai/model.rs:71-76 */
float or_silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

/* ------------------------------------------------------------------------- */
/* Assembled decoder                                                          */
typedef struct {
  float *attn_norm, *ffn_norm;
  float *wqkv, *bqkv; /* [(hq+2hkv)hd][d], optional bias */
  float *wo;          /* [d][hq*hd] */
  float *wi;          /* [2f][d]: gate rows then up rows */
  float *wd;          /* [d][f] */
} or_layer;

struct or_model {
  int L, d, hq, hkv, hd, f, V, ctx, threads;
  float eps;
  const or_gguf *g; /* the file the weights are decoded from (borrowed) */
  int streamed;     /* layers decoded at each use and freed after it (or_model_load_streamed) */
  const uint8_t *emb; /* raw embedding rows in the GGUF */
  uint32_t emb_kind;
  or_layer *layers;
  float *final_norm;
  float *head; /* [V][d] */
  float *cosf_, *sinf_; /* [ctx][hd] */
};

struct or_cache {
  int L, kvw, cap, len;
  float *k, *v; /* [L][cap][hkv*hd] */
};

static int set_err(char *err, int errlen, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  if (err && errlen > 0) vsnprintf(err, (size_t)errlen, fmt, ap);
  va_end(ap);
  return -1;
}

/* Decode whole blocks [lo, hi) of one tensor (each worker its own range; gguf.rs:250-336 per block). */
typedef struct {
  uint32_t kind;
  const uint8_t *data;
  uint64_t bsize, belems;
  float *out;
} decode_ctx;
static void decode_blocks(void *p, int lo, int hi) {
  const decode_ctx *c = (const decode_ctx *)p;
  or_decode(c->kind, c->data + (uint64_t)lo * c->bsize, (uint64_t)(hi - lo) * c->bsize,
            c->out + (uint64_t)lo * c->belems);
}

/* Find a tensor with dims [cols, rows] (gguf.rs order); 0 if present with that shape. */
static int find_tensor(const or_gguf *g, const char *name, uint64_t cols, uint64_t rows, uint32_t *kind,
                       const uint8_t **data, uint64_t *len, char *err, int errlen) {
  uint64_t dims[4];
  int nd;
  if (or_gguf_tensor(g, name, kind, dims, &nd, data, len)) {
    set_err(err, errlen, "missing tensor %s", name);
    return -1;
  }
  uint64_t count = 1;
  for (int i = 0; i < nd; ++i) count *= dims[i];
  if (count != cols * rows || dims[0] != cols) {
    set_err(err, errlen, "%s: unexpected shape", name);
    return -1;
  }
  return 0;
}

/* Decode a tensor with dims [cols, rows] into a fresh f32 buffer, its blocks split over `threads`
 * workers (the decode of each block does not depend on the split). */
static float *load_f32(const or_gguf *g, const char *name, uint64_t cols, uint64_t rows, int threads, char *err,
                       int errlen) {
  uint32_t kind;
  const uint8_t *data;
  uint64_t len, block, size;
  if (find_tensor(g, name, cols, rows, &kind, &data, &len, err, errlen)) return NULL;
  float *o = (float *)malloc(cols * rows * sizeof(float));
  if (!o) {
    set_err(err, errlen, "%s: out of memory", name);
    return NULL;
  }
  if (or_layout(kind, &block, &size) || len % size || len / size > 0x7fffffffULL) {
    or_decode(kind, data, len, o);
  } else {
    decode_ctx c = {kind, data, size, block, o};
    parallel((int)(len / size), threads, decode_blocks, &c);
  }
  return o;
}

static int has(const or_gguf *g, const char *name) {
  return or_gguf_tensor(g, name, NULL, NULL, NULL, NULL, NULL) == 0;
}

/* Concatenate row blocks (same per-row arithmetic as a fused matrix). */
static float *cat_rows(float *a, size_t na, float *b, size_t nb, float *c, size_t nc) {
  float *o = (float *)malloc((na + nb + nc) * sizeof(float));
  memcpy(o, a, na * sizeof(float));
  memcpy(o + na, b, nb * sizeof(float));
  if (c) memcpy(o + na + nb, c, nc * sizeof(float));
  free(a);
  free(b);
  free(c);
  return o;
}

static void free_layer(or_layer *y) {
  free(y->attn_norm); free(y->ffn_norm); free(y->wqkv); free(y->bqkv);
  free(y->wo); free(y->wi); free(y->wd);
  memset(y, 0, sizeof *y);
}

void or_model_free(or_model *m) {
  if (!m) return;
  if (m->layers)
    for (int l = 0; l < m->L; ++l) free_layer(&m->layers[l]);
  free(m->layers);
  free(m->final_norm);
  free(m->head);
  free(m->cosf_);
  free(m->sinf_);
  free(m);
}

/* Decode layer l's tensors into y (check != 0: only verify that they exist with their shapes, and
 * leave y empty).  Fused q|k|v and gate|up tensors, or their parts concatenated by rows.  0 on success;
 * on failure y holds whatever was decoded, for free_layer. */
static int load_layer(const or_model *m, int l, or_layer *y, int check, char *err, int errlen) {
  const or_gguf *g = m->g;
  int d = m->d, f = m->f, qrows = m->hq * m->hd, kvrows = m->hkv * m->hd;
  char name[128];
  memset(y, 0, sizeof *y);
#define LOAD(dst, fmt, cols, rows)                                                                         \
  do {                                                                                                     \
    snprintf(name, sizeof name, fmt, l);                                                                   \
    if (check) {                                                                                           \
      uint32_t k_;                                                                                         \
      const uint8_t *d_;                                                                                   \
      uint64_t n_;                                                                                         \
      if (find_tensor(g, name, (uint64_t)(cols), (uint64_t)(rows), &k_, &d_, &n_, err, errlen)) return -1; \
      dst = NULL;                                                                                          \
    } else if (!(dst = load_f32(g, name, (uint64_t)(cols), (uint64_t)(rows), m->threads, err, errlen))) { \
      return -1;                                                                                           \
    }                                                                                                      \
  } while (0)
  LOAD(y->attn_norm, "attn_norm.%d.weight", d, 1);
  LOAD(y->ffn_norm, "ffn_norm.%d.weight", d, 1);
  snprintf(name, sizeof name, "qkv.%d.weight", l);
  if (has(g, name)) {
    LOAD(y->wqkv, "qkv.%d.weight", d, qrows + 2 * kvrows);
    snprintf(name, sizeof name, "qkv.%d.bias", l);
    if (has(g, name)) LOAD(y->bqkv, "qkv.%d.bias", qrows + 2 * kvrows, 1);
  } else {
    float *q, *k, *v;
    LOAD(q, "q.%d.weight", d, qrows);
    LOAD(k, "k.%d.weight", d, kvrows);
    LOAD(v, "v.%d.weight", d, kvrows);
    if (!check) y->wqkv = cat_rows(q, (size_t)qrows * d, k, (size_t)kvrows * d, v, (size_t)kvrows * d);
    snprintf(name, sizeof name, "q.%d.bias", l);
    if (has(g, name)) {
      float *bq, *bk, *bv;
      LOAD(bq, "q.%d.bias", qrows, 1);
      LOAD(bk, "k.%d.bias", kvrows, 1);
      LOAD(bv, "v.%d.bias", kvrows, 1);
      if (!check) y->bqkv = cat_rows(bq, (size_t)qrows, bk, (size_t)kvrows, bv, (size_t)kvrows);
    }
  }
  LOAD(y->wo, "wo.%d.weight", qrows, d);
  snprintf(name, sizeof name, "mlp_wi.%d.weight", l);
  if (has(g, name)) {
    LOAD(y->wi, "mlp_wi.%d.weight", d, 2 * f);
  } else {
    float *ga, *up;
    LOAD(ga, "gate.%d.weight", d, f);
    LOAD(up, "up.%d.weight", d, f);
    if (!check) y->wi = cat_rows(ga, (size_t)f * d, up, (size_t)f * d, NULL, 0);
  }
  LOAD(y->wd, "mlp_wo.%d.weight", f, d);
#undef LOAD
  return 0;
}

static or_model *model_open(const or_gguf *g, int threads, int streamed, char *err, int errlen) {
  if (strcmp(or_gguf_str(g, "general.architecture"), "ggmlc") ||
      strcmp(or_gguf_str(g, "laya.model_name"), "laya-decoder")) {
    set_err(err, errlen, "not a laya-decoder GGUF");
    return NULL;
  }
  or_model *m = (or_model *)calloc(1, sizeof(*m));
  m->g = g;
  m->streamed = streamed;
  m->L = (int)or_gguf_num(g, "laya.decoder.block_count", 0);
  m->d = (int)or_gguf_num(g, "laya.decoder.embedding_length", 0);
  m->hq = (int)or_gguf_num(g, "laya.decoder.head_count", 0);
  m->hkv = (int)or_gguf_num(g, "laya.decoder.head_count_kv", 0);
  m->hd = (int)or_gguf_num(g, "laya.decoder.key_length", 0);
  m->f = (int)or_gguf_num(g, "laya.decoder.feed_forward_length", 0);
  m->V = (int)or_gguf_num(g, "laya.decoder.vocab_size", 0);
  m->ctx = (int)or_gguf_num(g, "laya.decoder.context_length", 0);
  m->eps = (float)or_gguf_num(g, "laya.decoder.layer_norm_rms_epsilon", 1e-5);
  m->threads = threads < 1 ? 1 : threads;
  if (m->L < 1 || m->d < 1 || m->hq < 1 || m->hkv < 1 || m->hq % m->hkv || m->hd < 2 ||
      m->hd % 2 || m->f < 1 || m->V < 1 || m->ctx < 1) {
    set_err(err, errlen, "invalid laya-decoder dimensions");
    or_model_free(m);
    return NULL;
  }
  int d = m->d, hd = m->hd;
  uint32_t kind;
  uint64_t dims[4];
  int nd;
  uint64_t len;
  if (or_gguf_tensor(g, "tok_emb.weight", &kind, dims, &nd, &m->emb, &len) || dims[0] != (uint64_t)d ||
      (kind != OR_F32 && kind != OR_F16)) {
    set_err(err, errlen, "tok_emb.weight must be F32/F16 [d, vocab]");
    or_model_free(m);
    return NULL;
  }
  m->emb_kind = kind;
  m->layers = (or_layer *)calloc((size_t)m->L, sizeof(or_layer));
  for (int l = 0; l < m->L; ++l)
    if (load_layer(m, l, &m->layers[l], streamed, err, errlen)) {
      or_model_free(m);
      return NULL;
    }
  if (!(m->final_norm = load_f32(g, "final_norm.weight", (uint64_t)d, 1, m->threads, err, errlen)) ||
      !(m->head = load_f32(g, "output.weight", (uint64_t)d, (uint64_t)m->V, m->threads, err, errlen)) ||
      !(m->cosf_ = load_f32(g, "cos_full", (uint64_t)hd, (uint64_t)m->ctx, m->threads, err, errlen)) ||
      !(m->sinf_ = load_f32(g, "sin_full", (uint64_t)hd, (uint64_t)m->ctx, m->threads, err, errlen))) {
    or_model_free(m);
    return NULL;
  }
  return m;
}

or_model *or_model_load(const or_gguf *g, int threads, char *err, int errlen) {
  return model_open(g, threads, 0, err, errlen);
}

or_model *or_model_load_streamed(const or_gguf *g, int threads, char *err, int errlen) {
  return model_open(g, threads, 1, err, errlen);
}

void or_model_dims(const or_model *m, int out[8]) {
  out[0] = m->L; out[1] = m->d; out[2] = m->hq; out[3] = m->hkv;
  out[4] = m->hd; out[5] = m->f; out[6] = m->V; out[7] = m->ctx;
}
void or_model_set_threads(or_model *m, int threads) { m->threads = threads < 1 ? 1 : threads; }

or_cache *or_cache_new(const or_model *m, int capacity) {
  or_cache *c = (or_cache *)calloc(1, sizeof(*c));
  c->L = m->L;
  c->kvw = m->hkv * m->hd;
  c->cap = capacity;
  c->k = (float *)calloc((size_t)m->L * capacity * c->kvw, sizeof(float));
  c->v = (float *)calloc((size_t)m->L * capacity * c->kvw, sizeof(float));
  return c;
}
or_cache *or_cache_fork(const or_cache *src, int len) {
  or_cache *c = (or_cache *)calloc(1, sizeof(*c));
  *c = *src;
  c->k = (float *)calloc((size_t)c->L * c->cap * c->kvw, sizeof(float));
  c->v = (float *)calloc((size_t)c->L * c->cap * c->kvw, sizeof(float));
  if (len > src->len) len = src->len;
  for (int l = 0; l < c->L; ++l) {
    memcpy(c->k + (size_t)l * c->cap * c->kvw, src->k + (size_t)l * c->cap * c->kvw,
           (size_t)len * c->kvw * sizeof(float));
    memcpy(c->v + (size_t)l * c->cap * c->kvw, src->v + (size_t)l * c->cap * c->kvw,
           (size_t)len * c->kvw * sizeof(float));
  }
  c->len = len;
  return c;
}
void or_cache_free(or_cache *c) {
  if (!c) return;
  free(c->k);
  free(c->v);
  free(c);
}
int or_cache_len(const or_cache *c) { return c->len; }

/* Cached K (after RoPE) and V rows [pos0, pos0 + n) of one layer, [n][hkv*hd] each. */
int or_cache_read(const or_cache *c, int layer, int pos0, int n, float *k, float *v) {
  if (layer < 0 || layer >= c->L || pos0 < 0 || n < 0 || pos0 + n > c->len) return -1;
  size_t off = ((size_t)layer * c->cap + (size_t)pos0) * c->kvw;
  memcpy(k, c->k + off, (size_t)n * c->kvw * sizeof(float));
  memcpy(v, c->v + off, (size_t)n * c->kvw * sizeof(float));
  return 0;
}

/* Table RoPE, src/tensor.rs:158-172 (rotate-half pairs (j, j+hd/2)). */
static void rope_rows(float *a, int n, int stride, int heads, int hd, int pos0, const float *cs,
                      const float *sn) {
  int half = hd / 2;
  for (int i = 0; i < n; ++i) {
    const float *c = cs + (size_t)(pos0 + i) * hd, *s = sn + (size_t)(pos0 + i) * hd;
    for (int h = 0; h < heads; ++h)
      for (int j = 0; j < half; ++j) {
        size_t p = (size_t)i * stride + (size_t)h * hd + j;
        float u = a[p], v = a[p + half];
        a[p] = u * c[j] - v * s[j];
        a[p + half] = v * c[j + half] + u * s[j + half];
      }
  }
}

/* Causal GQA attention, src/models/openthai/model.rs:276-294, generalised:
 * kh = h / (hq/hkv); s_j = dot(q_i, k_j) / sqrt(hd) for j <= pos_i; softmax; out += p_j v_j. */
typedef struct {
  const or_model *m;
  const float *q; /* [n][hq*hd] */
  const float *K, *V; /* this layer's cache rows [cap][hkv*hd] */
  float *out;     /* [n][hq*hd] */
  int n, pos0;
} attn_ctx;

static void attn_heads(void *p, int lo, int hi) {
  const attn_ctx *a = (const attn_ctx *)p;
  const or_model *m = a->m;
  int hd = m->hd, qw = m->hq * hd, kvw = m->hkv * hd, grp = m->hq / m->hkv;
  int total = a->pos0 + a->n;
  float *score = (float *)malloc((size_t)total * sizeof(float));
  float *prob = (float *)malloc((size_t)total * sizeof(float));
  float scale = sqrtf((float)hd);
  for (int h = lo; h < hi; ++h) {
    int kh = h / grp;
    for (int i = 0; i < a->n; ++i) {
      int upto = a->pos0 + i;
      const float *q = a->q + (size_t)i * qw + (size_t)h * hd;
      for (int j = 0; j <= upto; ++j)
        score[j] = or_dot(q, a->K + (size_t)j * kvw + (size_t)kh * hd, hd) / scale;
      or_softmax(score, upto + 1, prob);
      float *o = a->out + (size_t)i * qw + (size_t)h * hd;
      for (int z = 0; z < hd; ++z) o[z] = 0.0f;
      for (int j = 0; j <= upto; ++j) {
        const float *v = a->V + (size_t)j * kvw + (size_t)kh * hd;
        for (int z = 0; z < hd; ++z) o[z] = o[z] + prob[j] * v[z];
      }
    }
  }
  free(score);
  free(prob);
}

#if defined(__x86_64__)
/* attn_heads in the blocked mode: the same operations per score and per output element,
 * eight at a time.  Eight keys' dot products run in the eight lanes (each lane its own
 * sequential sum from -0.0 over the head dimension, mul then add, from a transposed copy of
 * the head's keys), and out[z] += p_j v_j[z] runs over eight z at a time in increasing j.
 * Bit-identical to attn_heads. */
__attribute__((target("avx2"))) static void attn_heads_avx2(void *p, int lo, int hi) {
  const attn_ctx *a = (const attn_ctx *)p;
  const or_model *m = a->m;
  int hd = m->hd, qw = m->hq * hd, kvw = m->hkv * hd, grp = m->hq / m->hkv;
  int total = a->pos0 + a->n;
  int tp = (total + 7) & ~7;
  float *score = (float *)malloc((size_t)tp * sizeof(float));
  float *prob = (float *)malloc((size_t)total * sizeof(float));
  float *kt = (float *)malloc((size_t)hd * tp * sizeof(float));
  float scale = sqrtf((float)hd);
  const __m256 vscale = _mm256_set1_ps(scale);
  int built = -1;
  for (int h = lo; h < hi; ++h) {
    int kh = h / grp;
    if (kh != built) {
      for (int j = 0; j < total; ++j) {
        const float *kr = a->K + (size_t)j * kvw + (size_t)kh * hd;
        for (int z = 0; z < hd; ++z) kt[(size_t)z * tp + j] = kr[z];
      }
      built = kh;
    }
    for (int i = 0; i < a->n; ++i) {
      int upto = a->pos0 + i;
      const float *q = a->q + (size_t)i * qw + (size_t)h * hd;
      int j = 0;
      for (; j + 8 <= upto + 1; j += 8) {
        __m256 s = _mm256_set1_ps(-0.0f);
        for (int z = 0; z < hd; ++z)
          s = _mm256_add_ps(s, _mm256_mul_ps(_mm256_set1_ps(q[z]), _mm256_loadu_ps(kt + (size_t)z * tp + j)));
        _mm256_storeu_ps(score + j, _mm256_div_ps(s, vscale));
      }
      for (; j <= upto; ++j) score[j] = or_dot(q, a->K + (size_t)j * kvw + (size_t)kh * hd, hd) / scale;
      or_softmax(score, upto + 1, prob);
      float *o = a->out + (size_t)i * qw + (size_t)h * hd;
      for (int z0 = 0; z0 < hd; z0 += 64) {
        int zn = hd - z0 < 64 ? hd - z0 : 64;
        if (zn == 64) {
          __m256 acc[8];
          for (int u = 0; u < 8; ++u) acc[u] = _mm256_setzero_ps();
          for (int jj = 0; jj <= upto; ++jj) {
            const float *v = a->V + (size_t)jj * kvw + (size_t)kh * hd + z0;
            __m256 pj = _mm256_set1_ps(prob[jj]);
            for (int u = 0; u < 8; ++u) acc[u] = _mm256_add_ps(acc[u], _mm256_mul_ps(pj, _mm256_loadu_ps(v + 8 * u)));
          }
          for (int u = 0; u < 8; ++u) _mm256_storeu_ps(o + z0 + 8 * u, acc[u]);
        } else {
          for (int z = z0; z < z0 + zn; ++z) o[z] = 0.0f;
          for (int jj = 0; jj <= upto; ++jj) {
            const float *v = a->V + (size_t)jj * kvw + (size_t)kh * hd;
            for (int z = z0; z < z0 + zn; ++z) o[z] = o[z] + prob[jj] * v[z];
          }
        }
      }
    }
  }
  free(kt);
  free(score);
  free(prob);
}
#endif

/* The causal GQA attention of one layer on caller-held rows (the loop of or_prefill, for timing the
 * reference's attention on a sample of query rows and for tests): q [n][hq*hd] of positions pos0..,
 * k/v [pos0 + n][hkv*hd] (already rotated), out [n][hq*hd].  src/models/openthai/model.rs:276-294. */
int or_attention(const float *q, const float *k, const float *v, int n, int pos0, int hq, int hkv, int hd,
                 int threads, float *out) {
  if (n < 1 || pos0 < 0 || hq < 1 || hkv < 1 || hq % hkv || hd < 1) return -1;
  or_model m;
  memset(&m, 0, sizeof m);
  m.hq = hq;
  m.hkv = hkv;
  m.hd = hd;
  attn_ctx ac = {&m, q, k, v, out, n, pos0};
#if defined(__x86_64__)
  if (g_blocked && !g_force_scalar && __builtin_cpu_supports("avx2"))
    parallel(hq, threads, attn_heads_avx2, &ac);
  else
#endif
    parallel(hq, threads, attn_heads, &ac);
  return 0;
}

int or_prefill(or_model *m, or_cache *c, const int32_t *ids, int n, const int32_t *gather,
               int ngather, float *hidden) {
  int d = m->d, hq = m->hq, hkv = m->hkv, hd = m->hd, f = m->f;
  int qw = hq * hd, kvw = hkv * hd, qkvw = qw + 2 * kvw;
  int pos0 = c->len;
  if (n < 1 || pos0 + n > c->cap || pos0 + n > m->ctx) return -1;
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= m->V) return -1;
  for (int i = 0; i < ngather; ++i)
    if (gather[i] < 0 || gather[i] >= n) return -1;
  size_t es = m->emb_kind == OR_F32 ? 4 : 2;
  float *x = (float *)malloc((size_t)n * d * sizeof(float));
  for (int i = 0; i < n; ++i)
    or_decode(m->emb_kind, m->emb + (size_t)ids[i] * d * es, (uint64_t)d * es, x + (size_t)i * d);
  float *h = (float *)malloc((size_t)n * d * sizeof(float));
  float *qkv = (float *)malloc((size_t)n * qkvw * sizeof(float));
  float *q = (float *)malloc((size_t)n * qw * sizeof(float));
  float *att = (float *)malloc((size_t)n * qw * sizeof(float));
  float *y = (float *)malloc((size_t)n * d * sizeof(float));
  float *gu = (float *)malloc((size_t)n * 2 * f * sizeof(float));
  float *act = (float *)malloc((size_t)n * f * sizeof(float));
  or_layer streamed_layer;
  memset(&streamed_layer, 0, sizeof streamed_layer);
  int rc = 0;
  for (int l = 0; l < m->L; ++l) {
    const or_layer *ly = &m->layers[l];
    if (m->streamed) {  /* this layer's weights only while it runs */
      free_layer(&streamed_layer);
      if (load_layer(m, l, &streamed_layer, 0, NULL, 0)) {
        rc = -1;
        break;
      }
      ly = &streamed_layer;
    }
    float *K = c->k + (size_t)l * c->cap * kvw, *V = c->v + (size_t)l * c->cap * kvw;
    or_rms(x, n, d, ly->attn_norm, 0.0f, m->eps, h);
    or_apply(ly->wqkv, qkvw, d, h, n, ly->bqkv, m->threads, qkv);
    for (int i = 0; i < n; ++i) {
      memcpy(q + (size_t)i * qw, qkv + (size_t)i * qkvw, (size_t)qw * sizeof(float));
      memcpy(K + (size_t)(pos0 + i) * kvw, qkv + (size_t)i * qkvw + qw, (size_t)kvw * sizeof(float));
      memcpy(V + (size_t)(pos0 + i) * kvw, qkv + (size_t)i * qkvw + qw + kvw,
             (size_t)kvw * sizeof(float));
    }
    rope_rows(q, n, qw, hq, hd, pos0, m->cosf_, m->sinf_);
    rope_rows(K + (size_t)pos0 * kvw, n, kvw, hkv, hd, pos0, m->cosf_, m->sinf_);
    attn_ctx ac = {m, q, K, V, att, n, pos0};
#if defined(__x86_64__)
    if (g_blocked && !g_force_scalar && __builtin_cpu_supports("avx2"))
      parallel(hq, m->threads, attn_heads_avx2, &ac);
    else
#endif
      parallel(hq, m->threads, attn_heads, &ac);
    or_apply(ly->wo, d, qw, att, n, NULL, m->threads, y);
    for (size_t i = 0; i < (size_t)n * d; ++i) x[i] = x[i] + y[i];
    or_rms(x, n, d, ly->ffn_norm, 0.0f, m->eps, h);
    or_apply(ly->wi, 2 * f, d, h, n, NULL, m->threads, gu);
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < f; ++j)
        act[(size_t)i * f + j] = or_silu(gu[(size_t)i * 2 * f + j]) * gu[(size_t)i * 2 * f + f + j];
    or_apply(ly->wd, d, f, act, n, NULL, m->threads, y);
    for (size_t i = 0; i < (size_t)n * d; ++i) x[i] = x[i] + y[i];
  }
  free_layer(&streamed_layer);
  if (rc == 0) {
    for (int i = 0; i < ngather; ++i)
      memcpy(hidden + (size_t)i * d, x + (size_t)gather[i] * d, (size_t)d * sizeof(float));
    c->len = pos0 + n;
  }
  free(x); free(h); free(qkv); free(q); free(att); free(y); free(gu); free(act);
  return rc;
}

int or_head(or_model *m, const float *hidden, int rows, const int32_t *vocab_ids, int nv,
            float *logits) {
  int d = m->d;
  float *h = (float *)malloc((size_t)rows * d * sizeof(float));
  or_rms(hidden, rows, d, m->final_norm, 0.0f, m->eps, h);
  if (!vocab_ids) {
    or_apply(m->head, m->V, d, h, rows, NULL, m->threads, logits);
  } else {
    float *w = (float *)malloc((size_t)nv * d * sizeof(float));
    for (int i = 0; i < nv; ++i) {
      if (vocab_ids[i] < 0 || vocab_ids[i] >= m->V) { free(w); free(h); return -1; }
      memcpy(w + (size_t)i * d, m->head + (size_t)vocab_ids[i] * d, (size_t)d * sizeof(float));
    }
    or_apply(w, nv, d, h, rows, NULL, m->threads, logits);
    free(w);
  }
  free(h);
  return 0;
}

int or_argmax(const float *v, int n) {
  int best = 0;
  for (int j = 1; j < n; ++j)
    if (v[j] > v[best]) best = j;
  return best;
}

void or_option_scores(const float *logits, int k, float abstain_logit, int has_abstain,
                      float temperature, float *probs, float *logprobs, float *abstain) {
  float z[257], p[257];
  int kk = k > 256 ? 256 : k;
  for (int i = 0; i < kk; ++i) z[i] = logits[i] / temperature;
  int n = kk;
  if (has_abstain) z[n++] = abstain_logit / temperature;
  or_softmax(z, n, p);
  float s = -0.0f;
  for (int i = 0; i < kk; ++i) s = s + p[i];
  if (s < 1e-12f) s = 1e-12f;
  for (int i = 0; i < kk; ++i) probs[i] = p[i] / s / 1.0f;
  if (abstain) *abstain = has_abstain ? p[kk] / 1.0f : 0.0f;
  /* final normalisation over the (single-pass) average, decision.rs:299-303 */
  float s2 = -0.0f;
  for (int i = 0; i < kk; ++i) s2 = s2 + probs[i];
  if (s2 < 1e-12f) s2 = 1e-12f;
  for (int i = 0; i < kk; ++i) probs[i] = probs[i] / s2;
  /* option log-softmax over the k option logits */
  if (logprobs) {
    float m = -INFINITY;
    for (int i = 0; i < kk; ++i) m = fmaxf(m, z[i]);
    float t = -0.0f;
    for (int i = 0; i < kk; ++i) t = t + expf(z[i] - m);
    float lse = logf(t);
    for (int i = 0; i < kk; ++i) logprobs[i] = z[i] - m - lse;
  }
}

float or_confidence(const float *p, int k, int f64) {
  if (k <= 1) return 1.0f;
  if (f64) {
    /* laya/decision.rs:159-166: x = max(p, 1e-12) in f64, e = -sum x*ln x (left to right) */
    double s = -0.0;
    for (int i = 0; i < k; ++i) {
      double x = fmax((double)p[i], 1e-12); /* f64::max: a NaN operand yields the other */
      s = s + x * log(x);
    }
    double c = 1.0 - (-s) / log((double)k);
    if (c < 0.0) c = 0.0;
    if (c > 1.0) c = 1.0;
    return (float)c;
  }
  /* openthai/decision.rs:304-313: all in f32 with logf */
  float s = -0.0f;
  for (int i = 0; i < k; ++i) {
    float x = fmaxf(p[i], 1e-12f);
    s = s + x * logf(x);
  }
  float c = 1.0f - (-s) / logf((float)k);
  if (c < 0.0f) c = 0.0f;
  if (c > 1.0f) c = 1.0f;
  return c;
}
