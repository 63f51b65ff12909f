// Kernels of the Laya encoder (src/models/laya/model.rs:301-416, src/tensor.rs:103-192) that the
// decoder path does not have: LayerNorm (with optional weight and bias, into f16 planes or f32,
// optionally gathering rows and adding a per-sequence type row), bidirectional RoPE attention
// with a local window, and the small pieces of the decision tail.  Projections and MLPs run on
// the shared MFMA GEMM (GEGLU and ReLU epilogues).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "common.h"
#include "kernels.h"
#include "wave.h"

namespace lg {
namespace {

constexpr int kT = 256;

__device__ float block_sum_ln(float v, float *red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

__device__ __forceinline__ float gelu_tanh_f(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x)));
}

// One workgroup per output row: y = (x - mean) * (1/sqrt(var + eps)) * w + b (+ add row), the
// row read once into registers (d <= 4096, d % 4 == 0).  Row r of the output reads input row
// rows[r] (rows == nullptr: r).  Output: f16 hi/lo planes (y16, y16lo) or f32 (y32).  The add
// row (f32 [3][d]) is add + sel[seq[r]] * d.
__global__ __launch_bounds__(kT) void layer_norm_kernel(const float *__restrict__ x, const int32_t *__restrict__ rows,
                                                        int d, const float *__restrict__ w, const float *__restrict__ b,
                                                        float eps, const float *__restrict__ add,
                                                        const int32_t *__restrict__ seq, const int32_t *__restrict__ sel,
                                                        _Float16 *__restrict__ y16, _Float16 *__restrict__ y16lo,
                                                        float *__restrict__ y32) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float4 *row = reinterpret_cast<const float4 *>(x + int64_t(rows ? rows[r] : r) * d);
  const int n4 = d >> 2;
  float4 v[4];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = threadIdx.x + i * kT;
    v[i] = k < n4 ? row[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  }
  const float mean = block_sum_ln(s, red) / float(d);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = threadIdx.x + i * kT;
    if (k < n4) {
      const float a = v[i].x - mean, bb = v[i].y - mean, c = v[i].z - mean, e = v[i].w - mean;
      q += (a * a + bb * bb) + (c * c + e * e);
    }
  }
  const float scale = 1.0f / sqrtf(block_sum_ln(q, red) / float(d) + eps);
  const float *addrow = add ? add + int64_t(sel[seq[r]]) * d : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = threadIdx.x + i * kT;
    if (k >= n4) continue;
    const float in[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * k + e;
      float o = (in[e] - mean) * scale * (w ? w[j] : 1.0f) + (b ? b[j] : 0.0f);
      if (addrow) o = o + addrow[j];
      const int64_t at = int64_t(r) * d + j;
      if (y32) {
        y32[at] = o;
      } else {
        const _Float16 h = _Float16(o);
        y16[at] = h;
        if (y16lo) y16lo[at] = _Float16(o - float(h));
      }
    }
  }
}

// Bidirectional attention over q|k|v rows [T][3d] (f32), head dim 64: one workgroup per (32-query
// tile of one sequence, head).  Keys j with |i - j| <= window (window < 0: the whole sequence);
// RoPE from tables [pos][64] (pairs j, j + 32) applied as Q and K tiles are staged; scores
// q.k * (1/sqrt(64)); online softmax in f32.  Output f16 planes [T][d].
constexpr int kHD = 64, kAT = 32, kHDp = kHD + 4;

__global__ __launch_bounds__(kT) void laya_attn_kernel(const float *__restrict__ qkv, int d, int window,
                                                       const float *__restrict__ cosT, const float *__restrict__ sinT,
                                                       const int32_t *__restrict__ tile_row0,
                                                       const int32_t *__restrict__ tile_pos0,
                                                       const int32_t *__restrict__ tile_n,
                                                       const int32_t *__restrict__ seq_of_tile,
                                                       const int32_t *__restrict__ seq_n,
                                                       _Float16 *__restrict__ y, _Float16 *__restrict__ ylo) {
  __shared__ __align__(16) float sQ[kAT * kHDp];
  __shared__ __align__(16) float sK[kAT * kHDp];
  __shared__ __align__(16) float sV[kAT * kHD];
  __shared__ float sP[kAT * 33];
  const int tile = blockIdx.x, h = blockIdx.y;
  const int row0 = tile_row0[tile], pos0 = tile_pos0[tile], nq = tile_n[tile];
  const int n = seq_n[seq_of_tile[tile]];
  const int srow = row0 - pos0;
  const int tid = threadIdx.x, r = tid >> 3, sub = tid & 7;
  const int ld = 3 * d;
  // stage a [32][64] tile of q (part 0) or k (part 1) rows with RoPE, rows past `cnt` zero
  auto stage_rot = [&](float *dst, int part, int t0, int cnt) {
    for (int e = tid; e < kAT * (kHD / 4); e += kT) {
      const int i = e / (kHD / 4), c4 = e % (kHD / 4);
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (i < cnt) {
        const float *src = qkv + int64_t(srow + t0 + i) * ld + part * d + h * kHD;
        v = *reinterpret_cast<const float4 *>(src + c4 * 4);
        if (cosT) {
          const int p = t0 + i, j0 = c4 * 4;
          const float4 o = *reinterpret_cast<const float4 *>(src + (j0 + kHD / 2) % kHD);
          const float *cs = cosT + int64_t(p) * kHD + j0, *sn = sinT + int64_t(p) * kHD + j0;
          const float a[4] = {v.x, v.y, v.z, v.w}, b[4] = {o.x, o.y, o.z, o.w};
          float out[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            out[k] = j0 < kHD / 2 ? a[k] * cs[k] - b[k] * sn[k] : a[k] * cs[k] + b[k] * sn[k];
          v = make_float4(out[0], out[1], out[2], out[3]);
        }
      }
      *reinterpret_cast<float4 *>(dst + i * kHDp + c4 * 4) = v;
    }
  };
  stage_rot(sQ, 0, pos0, nq);
  const int klo = window < 0 ? 0 : max(0, pos0 - window);
  const int khi = window < 0 ? n : min(n, pos0 + nq - 1 + window + 1);
  const float scale = 1.0f / sqrtf(float(kHD));
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  float m = -FLT_MAX, l = 0.0f;
  bool seen = false;
  const int qpos = pos0 + r;
  for (int k0 = klo; k0 < khi; k0 += kAT) {
    const int cnt = min(kAT, khi - k0);
    __syncthreads();
    stage_rot(sK, 1, k0, cnt);
    for (int e = tid; e < kAT * (kHD / 4); e += kT) {
      const int i = e / (kHD / 4), c4 = e % (kHD / 4);
      const float4 v = i < cnt ? *reinterpret_cast<const float4 *>(qkv + int64_t(srow + k0 + i) * ld + 2 * d + h * kHD + c4 * 4)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      *reinterpret_cast<float4 *>(sV + i * kHD + c4 * 4) = v;
    }
    __syncthreads();
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int dd = 0; dd < kHD; dd += 4) {
      const float4 q = *reinterpret_cast<const float4 *>(sQ + r * kHDp + dd);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 k = *reinterpret_cast<const float4 *>(sK + (sub + 8 * i) * kHDp + dd);
        s[i] = fmaf(q.x, k.x, s[i]);
        s[i] = fmaf(q.y, k.y, s[i]);
        s[i] = fmaf(q.z, k.z, s[i]);
        s[i] = fmaf(q.w, k.w, s[i]);
      }
    }
    bool ok[4];
    float mt = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + sub + 8 * i;
      ok[i] = sub + 8 * i < cnt && r < nq && (window < 0 || (key - qpos <= window && qpos - key <= window));
      s[i] = s[i] * scale;
      if (ok[i]) mt = fmaxf(mt, s[i]);
    }
    mt = fmaxf(mt, dpp_move<0xB1>(mt));
    mt = fmaxf(mt, dpp_move<0x4E>(mt));
    mt = fmaxf(mt, dpp_move<0x141>(mt));
    const bool any = mt > -FLT_MAX;
    const float mn = fmaxf(m, mt);
    float p[4], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = ok[i] ? expf(s[i] - mn) : 0.0f;
      ps += p[i];
    }
    ps = group8_sum(ps);
    if (any) {
      const float corr = seen ? expf(m - mn) : 0.0f;
      l = l * corr + ps;
      m = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= corr;
      seen = true;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sP[r * 33 + sub + 8 * i] = p[i];
    __syncthreads();
    for (int c = 0; c < cnt; ++c) {
      const float pc = sP[r * 33 + c];
      const float4 v0 = *reinterpret_cast<const float4 *>(sV + c * kHD + sub * 4);
      const float4 v1 = *reinterpret_cast<const float4 *>(sV + c * kHD + 32 + sub * 4);
      acc[0] = fmaf(pc, v0.x, acc[0]);
      acc[1] = fmaf(pc, v0.y, acc[1]);
      acc[2] = fmaf(pc, v0.z, acc[2]);
      acc[3] = fmaf(pc, v0.w, acc[3]);
      acc[4] = fmaf(pc, v1.x, acc[4]);
      acc[5] = fmaf(pc, v1.y, acc[5]);
      acc[6] = fmaf(pc, v1.z, acc[6]);
      acc[7] = fmaf(pc, v1.w, acc[7]);
    }
  }
  if (r >= nq) return;
  const float inv = 1.0f / l;
  const int64_t base = int64_t(row0 + r) * d + h * kHD;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int dd = (e < 4 ? 0 : 32) + sub * 4 + (e & 3);
    const float o = acc[e] * inv;
    const _Float16 hh = _Float16(o);
    y[base + dd] = hh;
    if (ylo) ylo[base + dd] = _Float16(o - float(hh));
  }
}

__global__ void gelu_inplace_kernel(float *__restrict__ x, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = gelu_tanh_f(x[i]);
}

// model.rs:392-403, one workgroup per sequence: pooled = [h[first row], top1, top1 - top2,
// entropy / ln max(k, 2), max(k, 2) / 255] from the softmax of the sequence's option logits.
__global__ __launch_bounds__(kT) void laya_act_features_kernel(const float *__restrict__ h, int d,
                                                               const int32_t *__restrict__ seq_row0,
                                                               const int32_t *__restrict__ lg_first,
                                                               const int32_t *__restrict__ lg_count,
                                                               const float *__restrict__ logits,
                                                               float *__restrict__ pooled) {
  const int sq = blockIdx.x;
  const float *row = h + int64_t(seq_row0[sq]) * d;
  float *out = pooled + int64_t(sq) * (d + 4);
  for (int j = threadIdx.x; j < d; j += kT) out[j] = row[j];
  if (threadIdx.x == 0) {
    const int k = lg_count[sq];
    const float *z = logits + lg_first[sq];
    float mx = -INFINITY;
    for (int i = 0; i < k; ++i) mx = fmaxf(mx, z[i]);
    float p[16], sum = 0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] = expf(z[i] - mx);
      sum += p[i];
    }
    float top1 = 0.0f;
    for (int i = 0; i < k; ++i) {
      p[i] = p[i] / sum;
      top1 = fmaxf(top1, p[i]);
    }
    float top2 = 0.0f, es = 0.0f;
    for (int i = 0; i < k; ++i) {
      top2 = fmaxf(top2, p[i] * (top1 - p[i]) / ((top1 - p[i]) + 1e-6f));
      es += p[i] * logf(fmaxf(p[i], 1e-9f));
    }
    const float kk = float(k > 2 ? k : 2);
    out[d] = top1;
    out[d + 1] = top1 - top2;
    out[d + 2] = -es / logf(kk);
    out[d + 3] = kk / 255.0f;
  }
}

}  // namespace

void launch_layer_norm(const float *x, const int32_t *rows, int nrows, int d, const float *w, const float *b, float eps,
                       const float *add, const int32_t *seq, const int32_t *sel, _Float16 *y16, _Float16 *y16lo,
                       float *y32, hipStream_t st) {
  LG_REQUIRE(nrows > 0 && d > 0 && d % 4 == 0 && d <= 4 * 4 * kT, "layer norm: d=%d outside 4..4096 (multiple of 4)", d);
  LG_REQUIRE((y32 != nullptr) != (y16 != nullptr), "layer norm: exactly one output form");
  LG_REQUIRE(!add || (seq && sel), "layer norm: an add row needs its selectors");
  hipLaunchKernelGGL(layer_norm_kernel, dim3(nrows), dim3(kT), 0, st, x, rows, d, w, b, eps, add, seq, sel, y16, y16lo,
                     y32);
  HIP_CHECK(hipGetLastError());
}

void launch_laya_attn(const float *qkv, int d, int hd, int window, const float *cosT, const float *sinT,
                      const int32_t *tile_row0, const int32_t *tile_pos0, const int32_t *tile_n, const int32_t *tile_seq,
                      const int32_t *seq_n, int ntiles, _Float16 *y, _Float16 *ylo, hipStream_t st) {
  LG_REQUIRE(hd == kHD, "laya attention: head_dim %d (kernel is built for 64)", hd);
  LG_REQUIRE(ntiles > 0 && d % kHD == 0 && d >= kHD, "laya attention: bad shape");
  LG_REQUIRE((cosT == nullptr) == (sinT == nullptr), "laya attention: RoPE needs both tables");
  hipLaunchKernelGGL(laya_attn_kernel, dim3(ntiles, d / kHD), dim3(kT), 0, st, qkv, d, window, cosT, sinT, tile_row0,
                     tile_pos0, tile_n, tile_seq, seq_n, y, ylo);
  HIP_CHECK(hipGetLastError());
}

void launch_gelu_inplace(float *x, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(gelu_inplace_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, x, n);
  HIP_CHECK(hipGetLastError());
}

void launch_laya_act_features(const float *h, int d, const int32_t *seq_row0, const int32_t *lg_first,
                              const int32_t *lg_count, const float *logits, int nseq, float *pooled, hipStream_t st) {
  LG_REQUIRE(nseq > 0 && d > 0, "act features: bad shape");
  hipLaunchKernelGGL(laya_act_features_kernel, dim3(nseq), dim3(kT), 0, st, h, d, seq_row0, lg_first, lg_count, logits,
                     pooled);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
