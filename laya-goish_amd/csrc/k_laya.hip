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

// Bidirectional attention over q|k|v rows [T][3d] (f32), head dim 64, on v_mfma_f32_16x16x4_f32
// (f32 operands and accumulation).  One workgroup per (32-query tile of one sequence, head), two
// waves of 16 query rows each.  Keys j with |i - j| <= window (window < 0: the whole sequence);
// RoPE from tables [pos][64] (pairs j, j + 32) applied as Q and K tiles are staged in LDS; scores
// q.k * (1/sqrt(64)); online softmax in f32.  Output f16 planes [T][d].
//   S = Q K^T per 32-key tile: lane (li = l%16, kg = l/16) supplies Q[li][16g + 4kg + c] at step
//   4g + c (a permutation of the 64-dim contraction, applied to K alike, so every operand is one
//   float4 LDS read per 4 MFMAs); D layout: lane l holds S[4kg + r][16 blk + li], r < 4.
//   Online softmax per row with 16-lane DPP reductions; P goes through LDS into the A layout;
//   O += P V with V transposed in LDS.
constexpr int kHD = 64, kAT = 32, kHDp = kHD + 4;
constexpr int kVTp = 36;  // padded row of the transposed V tile [64 dims][32 keys]
constexpr int kPp = 36;   // padded row of the P tile [16 rows][32 keys]
constexpr int kAW = 128;  // two waves

// RoPE of one float4 of a row (dims j0..j0+3) given the partner float4 (dims j0+32.. mod 64).
__device__ __forceinline__ float4 rope4(float4 v, float4 o, const float *cs, const float *sn, int j0) {
  const float a[4] = {v.x, v.y, v.z, v.w}, b[4] = {o.x, o.y, o.z, o.w};
  float out[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) out[k] = j0 < kHD / 2 ? a[k] * cs[k] - b[k] * sn[k] : a[k] * cs[k] + b[k] * sn[k];
  return make_float4(out[0], out[1], out[2], out[3]);
}

__global__ __launch_bounds__(kAW) void laya_attn_kernel(const float *__restrict__ qkv, int d, int window,
                                                        const float *__restrict__ cosT, const float *__restrict__ sinT,
                                                        const int32_t *__restrict__ tile_row0,
                                                        const int32_t *__restrict__ tile_pos0,
                                                        const int32_t *__restrict__ tile_n,
                                                        const int32_t *__restrict__ seq_of_tile,
                                                        const int32_t *__restrict__ seq_n,
                                                        _Float16 *__restrict__ y, _Float16 *__restrict__ ylo) {
  __shared__ __align__(16) float sK[kAT * kHDp];      // [32 keys][68]
  __shared__ __align__(16) float sVT[kHD * kVTp];     // [64 dims][36]
  __shared__ __align__(16) float sQ[2][16 * kHDp];    // per wave [16 rows][68]
  __shared__ __align__(16) float sP[2][16 * kPp];     // per wave [16 rows][36]
  const int tile = blockIdx.x, h = blockIdx.y;
  const int row0 = tile_row0[tile], pos0 = tile_pos0[tile], nq = tile_n[tile];
  const int n = seq_n[seq_of_tile[tile]];
  const int srow = row0 - pos0;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, kg = l >> 4;
  const int ld = 3 * d;
  const int wq = nq - 16 * w;  // this wave's valid rows (may be <= 0)
  // this wave's Q rows, rotated (rows past the tile repeat its last row and are never written)
  float *myQ = sQ[w];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = l + 64 * k, i = e >> 4, c4 = e & 15, j0 = c4 * 4;
    const int p = pos0 + min(16 * w + i, nq - 1);
    const float *src = qkv + int64_t(srow + p) * ld + h * kHD;
    float4 v = reinterpret_cast<const float4 *>(src)[c4];
    if (cosT) v = rope4(v, reinterpret_cast<const float4 *>(src)[((j0 + kHD / 2) % kHD) / 4], cosT + int64_t(p) * kHD + j0,
                        sinT + int64_t(p) * kHD + j0, j0);
    *reinterpret_cast<float4 *>(myQ + i * kHDp + j0) = v;
  }
  // key ranges: the workgroup's (staged) and this wave's (computed)
  const int klo = window < 0 ? 0 : max(0, pos0 - window);
  const int khi = window < 0 ? n : min(n, pos0 + nq + window);
  const int qlo = pos0 + 16 * w, qhi = pos0 + min(16 * w + 16, nq);  // this wave's positions [qlo, qhi)
  const int wlo = window < 0 ? 0 : max(0, qlo - window);
  const int whi = window < 0 ? n : min(n, qhi - 1 + window + 1);
  float4v acc[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) acc[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  float m[4], lsum[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -FLT_MAX;
    lsum[r] = 0.0f;
  }
  float *myP = sP[w];
  for (int k0 = (klo / kAT) * kAT; k0 < khi; k0 += kAT) {
    __syncthreads();  // previous tile's readers are done
    // stage K (rotated) and V^T for keys k0..k0+31, clamped to the sequence (masked below)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = tid + kAW * k, i = e >> 4, c4 = e & 15, j0 = c4 * 4;
      const int p = min(k0 + i, n - 1);
      const float *src = qkv + int64_t(srow + p) * ld + d + h * kHD;
      float4 kv = reinterpret_cast<const float4 *>(src)[c4];
      if (cosT) kv = rope4(kv, reinterpret_cast<const float4 *>(src)[((j0 + kHD / 2) % kHD) / 4],
                           cosT + int64_t(p) * kHD + j0, sinT + int64_t(p) * kHD + j0, j0);
      *reinterpret_cast<float4 *>(sK + i * kHDp + j0) = kv;
      const float4 vv = reinterpret_cast<const float4 *>(src + d)[c4];
      sVT[(j0 + 0) * kVTp + i] = vv.x;
      sVT[(j0 + 1) * kVTp + i] = vv.y;
      sVT[(j0 + 2) * kVTp + i] = vv.z;
      sVT[(j0 + 3) * kVTp + i] = vv.w;
    }
    __syncthreads();
    if (wq <= 0 || k0 >= whi || k0 + kAT <= wlo) continue;  // wave-uniform: nothing visible here
    float4v s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 qg = *reinterpret_cast<const float4 *>(myQ + li * kHDp + 16 * g + 4 * kg);
      const float4 ka = *reinterpret_cast<const float4 *>(sK + li * kHDp + 16 * g + 4 * kg);
      const float4 kb = *reinterpret_cast<const float4 *>(sK + (16 + li) * kHDp + 16 * g + 4 * kg);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.x, ka.x, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.x, kb.x, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.y, ka.y, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.y, kb.y, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.z, ka.z, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.z, kb.z, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.w, ka.w, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qg.w, kb.w, s1, 0, 0, 0);
    }
    const int key0 = k0 + li, key1 = key0 + 16;
    float corr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * kg + r, qpos = qlo + row;
      const bool rv = row < wq;
      const bool ok0 = rv && key0 < n && (window < 0 || (key0 - qpos <= window && qpos - key0 <= window));
      const bool ok1 = rv && key1 < n && (window < 0 || (key1 - qpos <= window && qpos - key1 <= window));
      const float a = s0[r] * 0.125f, b = s1[r] * 0.125f;
      const float mt = row_max16(fmaxf(ok0 ? a : -FLT_MAX, ok1 ? b : -FLT_MAX));
      const float mn = fmaxf(m[r], mt);
      const float p0 = ok0 ? expf(a - mn) : 0.0f, p1 = ok1 ? expf(b - mn) : 0.0f;
      const float ps = row_sum(p0 + p1);
      corr[r] = 1.0f;
      if (mt > -FLT_MAX) {
        corr[r] = m[r] > -FLT_MAX ? expf(m[r] - mn) : 0.0f;
        lsum[r] = lsum[r] * corr[r] + ps;
        m[r] = mn;
      }
      myP[row * kPp + li] = p0;
      myP[row * kPp + 16 + li] = p1;
    }
    if (__any(corr[0] != 1.0f || corr[1] != 1.0f || corr[2] != 1.0f || corr[3] != 1.0f)) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][r] *= corr[r];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float4 pa = *reinterpret_cast<const float4 *>(myP + li * kPp + 16 * u + 4 * kg);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float4 vb = *reinterpret_cast<const float4 *>(sVT + (16 * b + li) * kVTp + 16 * u + 4 * kg);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.x, vb.x, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.y, vb.y, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.z, vb.z, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.w, vb.w, acc[b], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * kg + r;
    if (row >= wq) continue;
    const float inv = 1.0f / lsum[r];
    const int64_t base = int64_t(row0 + 16 * w + row) * d + h * kHD;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float o = acc[b][r] * inv;
      const _Float16 hh = _Float16(o);
      y[base + 16 * b + li] = hh;
      if (ylo) ylo[base + 16 * b + li] = _Float16(o - float(hh));
    }
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
  hipLaunchKernelGGL(laya_attn_kernel, dim3(ntiles, d / kHD), dim3(kAW), 0, st, qkv, d, window, cosT, sinT, tile_row0,
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
