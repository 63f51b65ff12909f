// Kernels of the Laya encoder (src/models/laya/model.rs:301-416, src/tensor.rs:103-192) that the
// decoder path does not have: LayerNorm (with optional weight and bias, into f16 planes or f32,
// optionally gathering rows and adding a per-sequence type row), bidirectional RoPE attention
// with a local window, and the small pieces of the decision tail.  Projections and MLPs run on
// the shared MFMA GEMM (GEGLU and ReLU epilogues).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "common.h"
#include "kernels.h"
#include "f16split.h"
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
  // a thread's four consecutive values: 16-byte loads of w, b and the add row, one 16-byte f32 or
  // 8-byte store per f16 plane
  typedef _Float16 half4_ __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = threadIdx.x + i * kT;
    if (k >= n4) continue;
    const float in[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    const float4 w4 = w ? reinterpret_cast<const float4 *>(w)[k] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    const float4 b4 = b ? reinterpret_cast<const float4 *>(b)[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 a4 = addrow ? reinterpret_cast<const float4 *>(addrow)[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w}, av[4] = {a4.x, a4.y, a4.z, a4.w};
    float4v o;
    half4_ h4, l4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = (in[e] - mean) * scale * wv[e] + bv[e];
      if (addrow) o[e] = o[e] + av[e];
      _Float16 h, hl;
      split_f16(o[e], h, hl);
      h4[e] = h;
      l4[e] = hl;
    }
    const int64_t at = int64_t(r) * d + 4 * k;
    if (y32) {
      *reinterpret_cast<float4v *>(y32 + at) = o;
    } else {
      *reinterpret_cast<half4_ *>(y16 + at) = h4;
      if (y16lo) *reinterpret_cast<half4_ *>(y16lo + at) = l4;
    }
  }
}

constexpr int kHD = 64;

// RoPE in place on the q and k parts of q|k|v rows [T][3d] (model.rs:336-350 rotates q and k
// before attention): pairs (j, j + 32) of every 64-wide head, angle tables [pos][64].
__global__ __launch_bounds__(kT) void laya_rope_kernel(float *__restrict__ qkv, int d, const float *__restrict__ cosT,
                                                       const float *__restrict__ sinT,
                                                       const int32_t *__restrict__ tok_pos) {
  const int t = blockIdx.x;
  const int p = tok_pos[t];
  float *row = qkv + int64_t(t) * 3 * d;
  const float *cs = cosT + int64_t(p) * kHD, *sn = sinT + int64_t(p) * kHD;
  for (int e = threadIdx.x; e < d; e += kT) {  // 2 parts x (d / 64) heads x 32 pairs
    const int part = e / (d / 2), rem = e % (d / 2), hh = rem / 32, j = rem % 32;
    float *x = row + part * d + hh * kHD;
    float a, c;
    rope_pair(x[j], x[j + 32], cs[j], sn[j], cs[j + 32], sn[j + 32], a, c);  // as the wide GEMM's epilogue
    x[j] = a;
    x[j + 32] = c;
  }
}

// Bidirectional attention over q|k|v rows [T][3d] (f32, q and k already rotated), head dim 64,
// on v_mfma_f32_16x16x16_f16 with every f32 operand split into f16 hi + lo parts and three
// products per pair (lo*hi, hi*lo, hi*hi; the lo*lo term is below f32 rounding), f32
// accumulation.  One workgroup per (16 query rows of
// one sequence, head); its four waves split the visible keys into four ranges of 16-key blocks
// and merge their (m, l, O) in LDS at the end.  Keys j with |i - j| <= window (window < 0: the
// whole sequence); scores q.k * (1/sqrt(64)); online softmax in f32 (base 2).  Output f16
// planes [T][d].
//   S = Q K^T per block: lane (li = l%16, kg = l/16) supplies Q[li][16g + 4kg + c], c < 4, as the
//   A operand of k-step g (a permutation of the 64-dim contraction, applied to K alike); operands
//   come straight from the q|k|v rows as float4 loads, the next block's K and V prefetched in
//   registers.
//   D layout: lane l holds S[4kg + r][li], r < 4.  P goes through LDS into the A layout
//   (P[li][4kg + c]); O += P V with V[4kg + c][16b + li], c < 4, as the B operand.
constexpr int kPp = 20;  // padded row of a wave's P block [16 rows][16 keys]
// scores are kept as log2(e) q.k / 8 and exponentiated with the hardware exp2 (v_exp_f32,
// ~1 ulp): softmax is invariant to the base, and exp2 of a difference costs one instruction
constexpr float kScoreLog2 = 0.125f * 1.44269504088896341f;
constexpr int kOp = 68;  // padded row of a wave's partial O [16 rows][64]

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// x = hi + lo with hi = f16(x), lo = f16(x - hi): ~22 significant bits
__device__ __forceinline__ void split_hl(float4v x, half4v &hi, half4v &lo) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    _Float16 h, l;
    split_f16(x[c], h, l);
    hi[c] = h;
    lo[c] = l;
  }
}

__device__ __forceinline__ float4v mfma3(half4v ah, half4v al, half4v bh, half4v bl, float4v acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, acc, 0, 0, 0);
}

struct KVBlock {
  float4v k[4];
  float v[16];
};

__device__ __forceinline__ void laya_load_kv(KVBlock &blk, const float *__restrict__ kbase, int ld, int d, int k0,
                                             int n, int li, int kg) {
  const float *kr = kbase + int64_t(min(k0 + li, n - 1)) * ld;
#pragma unroll
  for (int g = 0; g < 4; ++g) blk.k[g] = *reinterpret_cast<const float4v *>(kr + 16 * g + 4 * kg);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float *vr = kbase + int64_t(min(k0 + 4 * kg + c, n - 1)) * ld + d;
#pragma unroll
    for (int b = 0; b < 4; ++b) blk.v[4 * b + c] = vr[16 * b + li];
  }
}

__global__ __launch_bounds__(256) void laya_attn_kernel(const float *__restrict__ qkv, int d, int window,
                                                        const int32_t *__restrict__ tile_row0,
                                                        const int32_t *__restrict__ tile_pos0,
                                                        const int32_t *__restrict__ tile_n,
                                                        const int32_t *__restrict__ seq_of_tile,
                                                        const int32_t *__restrict__ seq_n,
                                                        _Float16 *__restrict__ y, _Float16 *__restrict__ ylo) {
  __shared__ __align__(16) float sP[4][16 * kPp];
  __shared__ __align__(16) float sO[4][16 * kOp];
  __shared__ float sML[4][16][2];
  const int tile = blockIdx.x, h = blockIdx.y, z = blockIdx.z;
  const int nsub = tile_n[tile] - 16 * z;  // rows of this 16-row half of the tile
  if (nsub <= 0) return;                   // whole workgroup, before any barrier
  const int row0 = tile_row0[tile] + 16 * z, pos0 = tile_pos0[tile] + 16 * z;
  const int n = seq_n[seq_of_tile[tile]];
  const int srow = row0 - pos0;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, kg = l >> 4;
  const int ld = 3 * d;
  const float *kbase = qkv + int64_t(srow) * ld + d + h * kHD;  // key rows of the sequence
  // Q operands: row li (rows past nsub repeat the last row and are never written)
  half4v qh[4], ql[4];
  {
    const float *qr = qkv + int64_t(row0 + min(li, nsub - 1)) * ld + h * kHD;
#pragma unroll
    for (int g = 0; g < 4; ++g) split_hl(*reinterpret_cast<const float4v *>(qr + 16 * g + 4 * kg), qh[g], ql[g]);
  }
  // visible keys of the 16 rows, in 16-key blocks split over the four waves
  const int wlo = window < 0 ? 0 : max(0, pos0 - window);
  const int whi = window < 0 ? n : min(n, pos0 + nsub + window);
  const int b0 = wlo / 16, nb = (whi + 15) / 16 - b0;
  const int bw0 = b0 + (nb * w) / 4, bw1 = b0 + (nb * (w + 1)) / 4;
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
  KVBlock cur, nxt;
  if (bw0 < bw1) laya_load_kv(cur, kbase, ld, d, 16 * bw0, n, li, kg);
  for (int bi = bw0; bi < bw1; ++bi) {
    laya_load_kv(nxt, kbase, ld, d, 16 * min(bi + 1, bw1 - 1), n, li, kg);  // the last one reloads its own
    float4v s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      half4v kh, kl;
      split_hl(cur.k[g], kh, kl);
      s = mfma3(qh[g], ql[g], kh, kl, s);
    }
    const int key = 16 * bi + li;
    float corr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * kg + r, qpos = pos0 + row;
      const bool ok = row < nsub && key < n && (window < 0 || (key - qpos <= window && qpos - key <= window));
      const float a = s[r] * kScoreLog2;  // q.k / sqrt(64) in base-2 units
      const float mt = row_max16(ok ? a : -FLT_MAX);
      const float mn = fmaxf(m[r], mt);
      const float p = ok ? __builtin_amdgcn_exp2f(a - mn) : 0.0f;
      const float ps = row_sum(p);
      corr[r] = 1.0f;
      if (mt > -FLT_MAX) {
        corr[r] = m[r] == mn ? 1.0f : m[r] > -FLT_MAX ? __builtin_amdgcn_exp2f(m[r] - mn) : 0.0f;
        lsum[r] = lsum[r] * corr[r] + ps;
        m[r] = mn;
      }
      myP[row * kPp + li] = p;
    }
    if (__any(corr[0] != 1.0f || corr[1] != 1.0f || corr[2] != 1.0f || corr[3] != 1.0f)) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][r] *= corr[r];
    }
    // P moves between the lanes of this wave through its own LDS rows: the wave barriers order the
    // stores above before the read below, and this read before the next block's stores
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    half4v ph, pl;
    split_hl(*reinterpret_cast<const float4v *>(myP + li * kPp + 4 * kg), ph, pl);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      half4v vh, vl;
      split_hl(float4v{cur.v[4 * b], cur.v[4 * b + 1], cur.v[4 * b + 2], cur.v[4 * b + 3]}, vh, vl);
      acc[b] = mfma3(ph, pl, vh, vl, acc[b]);
    }
    cur = nxt;
  }
  // merge the four key ranges: O = sum_w e^(m_w - M) O_w / sum_w e^(m_w - M) l_w
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) sO[w][(4 * kg + r) * kOp + 16 * b + li] = acc[b][r];
  if (li == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sML[w][4 * kg + r][0] = m[r];
      sML[w][4 * kg + r][1] = lsum[r];
    }
  __syncthreads();
  const int row = tid >> 4, d4 = (tid & 15) * 4;
  if (row >= nsub) return;
  float M = -FLT_MAX;
#pragma unroll
  for (int v = 0; v < 4; ++v)
    if (sML[v][row][1] > 0.0f) M = fmaxf(M, sML[v][row][0]);
  float L = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (!(sML[v][row][1] > 0.0f)) continue;
    const float f = __builtin_amdgcn_exp2f(sML[v][row][0] - M);
    L += f * sML[v][row][1];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] += f * sO[v][row * kOp + d4 + e];
  }
  const float inv = 1.0f / L;
  const int64_t base = int64_t(row0 + row) * d + h * kHD + d4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    _Float16 hh, hl;
    split_f16(o[e] * inv, hh, hl);
    y[base + e] = hh;
    if (ylo) ylo[base + e] = hl;
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

void launch_laya_rope(float *qkv, int T, int d, int hd, const float *cosT, const float *sinT, const int32_t *tok_pos,
                      hipStream_t st) {
  LG_REQUIRE(hd == kHD && T > 0 && d % kHD == 0 && cosT && sinT && tok_pos, "laya rope: bad shape");
  hipLaunchKernelGGL(laya_rope_kernel, dim3(T), dim3(kT), 0, st, qkv, d, cosT, sinT, tok_pos);
  HIP_CHECK(hipGetLastError());
}

void launch_laya_attn(const float *qkv, int d, int hd, int window, const int32_t *tile_row0, const int32_t *tile_pos0,
                      const int32_t *tile_n, const int32_t *tile_seq, const int32_t *seq_n, int ntiles, _Float16 *y,
                      _Float16 *ylo, hipStream_t st) {
  LG_REQUIRE(hd == kHD, "laya attention: head_dim %d (kernel is built for 64)", hd);
  LG_REQUIRE(ntiles > 0 && d % kHD == 0 && d >= kHD, "laya attention: bad shape");
  // tiles hold at most 32 rows: two 16-row halves per tile (grid z)
  hipLaunchKernelGGL(laya_attn_kernel, dim3(ntiles, d / kHD, 2), dim3(256), 0, st, qkv, d, window, tile_row0, tile_pos0,
                     tile_n, tile_seq, seq_n, y, ylo);
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
