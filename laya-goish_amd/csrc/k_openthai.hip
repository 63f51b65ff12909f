// Kernels of the OpenThai-SystemOne text tower (src/models/openthai/model.rs:244-362) that the
// decoder path does not have: the gated DeltaNet mixer (causal conv + silu + q/k
// normalisation, the per-head recurrent scan, the gated output norm) and the sigmoid-gated
// full attention over 256-dim heads with partial RoPE.  Projections run on the shared MFMA
// GEMM; these kernels read its f32 outputs.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "common.h"
#include "kernels.h"
#include "f16split.h"
#include "wave.h"

namespace lg {
namespace {

constexpr int kLK = 128;   // linear (DeltaNet) head dim
constexpr int kHD = 256;   // full-attention head dim
constexpr int kRot = 32;   // rotary pairs per head (64 of 256 dims rotate)

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  return v;
}

__device__ __forceinline__ void store_planes(_Float16 *hi, _Float16 *lo, int64_t i, float v) {
  _Float16 h, l;
  split_f16(v, h, l);
  hi[i] = h;
  if (lo) lo[i] = l;
}

// ---------------------------------------------------------------- DeltaNet: conv + norms
// One workgroup per token.  proj row: [q|k|v raw (3*lw) | z (lw) | a (nh) | b (nh) | pad].
// Causal depthwise conv over the token and the 3 before it within its sequence (pos = index
// in the sequence; rows of one sequence are consecutive), silu, then per head
// query = q / |q| / sqrt(128), key = k / |k| (|x| = sqrt(x.x + 1e-6)), decay and beta.
// model.rs:306-318 (conv), :323-331 (scales, decay, beta).
__global__ __launch_bounds__(256) void ot_delta_prep_kernel(const float *__restrict__ proj, int ldp,
                                                            const int32_t *__restrict__ tok_pos,
                                                            const float *__restrict__ conv,
                                                            const float *__restrict__ alog,
                                                            const float *__restrict__ dt, int nh,
                                                            float *__restrict__ qk, float *__restrict__ vbuf,
                                                            float *__restrict__ gb) {
  extern __shared__ float s_x[];
  const int t = blockIdx.x;
  const int lw = nh * kLK, cd = 3 * lw;
  const int pos = tok_pos[t];
  const float *row = proj + int64_t(t) * ldp;
  for (int c = threadIdx.x; c < cd; c += 256) {
    const float4 w = reinterpret_cast<const float4 *>(conv)[c];
    float v = 0.0f;
    if (pos >= 3) v = v + row[c - 3 * int64_t(ldp)] * w.x;
    if (pos >= 2) v = v + row[c - 2 * int64_t(ldp)] * w.y;
    if (pos >= 1) v = v + row[c - int64_t(ldp)] * w.z;
    v = v + row[c] * w.w;
    s_x[c] = siluf_(v);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int vec = wv; vec < 2 * nh; vec += 4) {  // vec < nh: q of head vec; else k of head vec - nh
    const int h = vec < nh ? vec : vec - nh;
    const float *x = s_x + (vec < nh ? 0 : lw) + h * kLK;
    const float x0 = x[lane], x1 = x[lane + 64];
    const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
    float sc = 1.0f / sqrtf(ss + 1e-6f);
    if (vec < nh) sc = sc / sqrtf(128.0f);
    float *dst = qk + (int64_t(t) * nh + h) * (2 * kLK) + (vec < nh ? 0 : kLK);
    dst[lane] = x0 * sc;
    dst[lane + 64] = x1 * sc;
  }
  for (int c = threadIdx.x; c < lw; c += 256) vbuf[int64_t(t) * lw + c] = s_x[2 * lw + c];
  if (threadIdx.x < nh) {
    const int h = threadIdx.x;
    const float a = row[cd + lw + h], b = row[cd + lw + nh + h];
    const float decay = expf(-expf(alog[h]) * softplusf_(a + dt[h]));
    gb[(int64_t(t) * nh + h) * 2] = decay;
    gb[(int64_t(t) * nh + h) * 2 + 1] = sigmoidf_(b);
  }
}

// ---------------------------------------------------------------- DeltaNet: recurrent scan
// model.rs:319-358, per head a [key j][value d] = 128 x 128 state S:
//   S *= decay;  delta = (v - S^T key) * beta;  S += key delta^T;  o = S^T query.
// Columns d are independent.  A 16-lane row of a wave owns one column: lane g of the row keeps
// S[8g .. 8g+7][d] in registers, and the two sums over j are 16-lane DPP row reductions (no
// LDS round trip on the token-to-token dependency chain).  A workgroup (4 waves) owns 16
// columns of one head of one sequence: a sequence's 16 x 8 = 128 workgroups per layer run side
// by side.  Tokens go in chunks of kCh staged in LDS, double buffered: the next chunk's global
// loads are in flight while the current one is scanned.
constexpr int kCh = 16;
constexpr int kLpc = 16;                  // lanes per column
constexpr int kJpl = kLK / kLpc;          // keys per lane
constexpr int kCols = 4 * (64 / kLpc);    // columns per workgroup

// Sum over each 32-lane half of the wave, every lane receiving its half's sum: 16-lane DPP
// row sums, then the other row's sum through ds_swizzle (bitmask mode, lane ^ 16 within 32).
__device__ __forceinline__ float half_sum32(float v) {
  v = row_sum(v);
  const float other = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  return v + other;
}

template <int LPC>
__device__ __forceinline__ float column_sum(float v) {
  if constexpr (LPC == 32) return half_sum32(v);
  else return row_sum(v);
}

__global__ __launch_bounds__(256) void ot_delta_scan_kernel(const float *__restrict__ qk,
                                                            const float *__restrict__ vbuf,
                                                            const float *__restrict__ gb,
                                                            const int32_t *__restrict__ seq_row0,
                                                            const int32_t *__restrict__ seq_n, int nh,
                                                            float *__restrict__ out) {
  __shared__ float4 s_qk[2][kCh][64];  // per token: query (float4 0..31) | key (32..63)
  __shared__ float s_v[2][kCh][kCols];
  __shared__ float2 s_gb[2][kCh];
  __shared__ float s_o[kCh][kCols];
  const int sq = blockIdx.x, h = blockIdx.y, cb = blockIdx.z;
  const int row0 = seq_row0[sq], n = seq_n[sq];
  const int lw = nh * kLK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int col = (tid >> 6) * (64 / kLpc) + lane / kLpc;  // column within this block
  const int g = lane % kLpc;                              // keys j = kJpl g .. kJpl g + kJpl - 1
  const int nchunks = (n + kCh - 1) / kCh;
  static_assert(kCh * 64 == 4 * 256 && kCh * kCols <= 256 && kCh <= 64, "chunk staging layout");
  // Loads are unconditional, from the token clamped into the sequence (n >= 1 whenever a chunk
  // exists): rows past the end hold copies that the scan never reads, and no load is
  // predicated, so the next chunk's loads never wait on anything.
  float4 rq0, rq1, rq2, rq3;
  float rv;
  float2 rg;
  const int vi = tid / kCols, vc = tid % kCols;
  auto load = [&](int c) {
    const int t0 = c * kCh;
    const float4 *base = reinterpret_cast<const float4 *>(qk) + int64_t(h) * (2 * kLK / 4);
    const int q4 = tid & 63, ti = tid >> 6;
    rq0 = base[int64_t(row0 + min(t0 + ti, n - 1)) * nh * (2 * kLK / 4) + q4];
    rq1 = base[int64_t(row0 + min(t0 + ti + 4, n - 1)) * nh * (2 * kLK / 4) + q4];
    rq2 = base[int64_t(row0 + min(t0 + ti + 8, n - 1)) * nh * (2 * kLK / 4) + q4];
    rq3 = base[int64_t(row0 + min(t0 + ti + 12, n - 1)) * nh * (2 * kLK / 4) + q4];
    rv = vbuf[int64_t(row0 + min(t0 + min(vi, kCh - 1), n - 1)) * lw + h * kLK + cb * kCols + vc];
    rg = reinterpret_cast<const float2 *>(gb)[int64_t(row0 + min(t0 + (tid & (kCh - 1)), n - 1)) * nh + h];
    if (t0 + (tid & (kCh - 1)) >= n) rg = make_float2(1.0f, 0.0f);  // neutral token past the end
  };
  auto stage = [&](int b) {
    const int q4 = tid & 63, ti = tid >> 6;
    s_qk[b][ti][q4] = rq0;
    s_qk[b][ti + 4][q4] = rq1;
    s_qk[b][ti + 8][q4] = rq2;
    s_qk[b][ti + 12][q4] = rq3;
    if (vi < kCh) s_v[b][vi][vc] = rv;
    if (tid < kCh) s_gb[b][tid] = rg;
  };
  // one token's operands for this lane, read from LDS
  struct Tok {
    float k[kJpl], q[kJpl], v;
    float2 db;
  };
  auto fetch = [&](int b, int i, Tok &t) {
#pragma unroll
    for (int c = 0; c < kJpl / 4; ++c) {
      const float4 a = s_qk[b][i][32 + g * (kJpl / 4) + c], e = s_qk[b][i][g * (kJpl / 4) + c];
      t.k[4 * c] = a.x; t.k[4 * c + 1] = a.y; t.k[4 * c + 2] = a.z; t.k[4 * c + 3] = a.w;
      t.q[4 * c] = e.x; t.q[4 * c + 1] = e.y; t.q[4 * c + 2] = e.z; t.q[4 * c + 3] = e.w;
    }
    t.v = s_v[b][i][col];
    t.db = s_gb[b][i];
  };
  float S[kJpl];
#pragma unroll
  for (int j = 0; j < kJpl; ++j) S[j] = 0.0f;
  if (nchunks > 0) {
    load(0);
    stage(0);
  }
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int b = c & 1;
    if (c + 1 < nchunks) load(c + 1);
    const int cnt = min(kCh, n - c * kCh);
    // The chunk is straight-line code over all kCh tokens: staged tokens past the sequence's
    // end carry decay 1 and beta 0, which leave S exactly unchanged (S * 1 = S, S + k * 0 = S),
    // so no token needs a branch and the scheduler can issue LDS reads tokens ahead.
    float oreg[kCh];
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
      Tok t;
      fetch(b, i, t);
      float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
      for (int j = 0; j < kJpl; j += 2) {
        S[j] *= t.db.x;
        S[j + 1] *= t.db.x;
        p0 = fmaf(S[j], t.k[j], p0);
        p1 = fmaf(S[j + 1], t.k[j + 1], p1);
      }
      const float delta = (t.v - column_sum<kLpc>(p0 + p1)) * t.db.y;
      float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
      for (int j = 0; j < kJpl; j += 2) {
        S[j] = fmaf(t.k[j], delta, S[j]);
        S[j + 1] = fmaf(t.k[j + 1], delta, S[j + 1]);
        o0 = fmaf(S[j], t.q[j], o0);
        o1 = fmaf(S[j + 1], t.q[j + 1], o1);
      }
      oreg[i] = column_sum<kLpc>(o0 + o1);
    }
    if (g == 0)
#pragma unroll
      for (int i = 0; i < kCh; ++i) s_o[i][col] = oreg[i];
    __syncthreads();
    // stage the next chunk before this chunk's stores are issued, so that waiting for its loads
    // never waits for stores as well
    if (c + 1 < nchunks) stage(b ^ 1);
    for (int e = tid; e < kCh * kCols; e += 256) {
      const int i = e / kCols, cc = e % kCols;
      if (i < cnt) out[int64_t(row0 + c * kCh + i) * lw + h * kLK + cb * kCols + cc] = s_o[i][cc];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- DeltaNet: gated output norm
// model.rs:359-361: rms over each 128-dim head output (offset 0, eps 1e-6) * silu(z), written
// as f16 planes for the out_proj GEMM.  One wave per (token, head).
__global__ __launch_bounds__(256) void ot_delta_out_kernel(const float *__restrict__ o, int T, int nh,
                                                           const float *__restrict__ norm_w,
                                                           const float *__restrict__ proj, int ldp, int zcol,
                                                           _Float16 *__restrict__ y, _Float16 *__restrict__ ylo) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= T * nh) return;
  const int t = item / nh, h = item % nh, lw = nh * kLK;
  const float *x = o + int64_t(t) * lw + h * kLK;
  const float x0 = x[lane], x1 = x[lane + 64];
  const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
  const float sc = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
  const float *z = proj + int64_t(t) * ldp + zcol + h * kLK;
  const int64_t base = int64_t(t) * lw + h * kLK;
  store_planes(y, ylo, base + lane, x0 * sc * norm_w[lane] * siluf_(z[lane]));
  store_planes(y, ylo, base + lane + 64, x1 * sc * norm_w[lane + 64] * siluf_(z[lane + 64]));
}

// ---------------------------------------------------------------- full attention: q/k norm + RoPE
// model.rs:255-275: per 256-dim head, rms (offset 1: w1 = 1 + w, eps 1e-6), then rotate pairs
// (j, j + 32), j < 32, by the table angle of the token's position.  One wave per (token, head);
// heads 0..hq-1 are queries (to Qb), hq..hq+hkv-1 keys (to Kb).
__global__ __launch_bounds__(256) void ot_attn_prep_kernel(const float *__restrict__ proj, int ldp, int T,
                                                           int hq, int hkv, const int32_t *__restrict__ tok_pos,
                                                           const float *__restrict__ qn1, const float *__restrict__ kn1,
                                                           const float *__restrict__ cosT, const float *__restrict__ sinT,
                                                           float *__restrict__ Qb, float *__restrict__ Kb) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int heads = hq + hkv;
  if (item >= T * heads) return;
  const int t = item / heads, hh = item % heads;
  const bool isq = hh < hq;
  const float *src = proj + int64_t(t) * ldp + (isq ? hh * 2 * kHD : 2 * hq * kHD + (hh - hq) * kHD);
  const float *w = isq ? qn1 : kn1;
  float x[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = src[lane + 64 * e];
  const float ss = wave_sum_dpp((x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]));
  const float sc = 1.0f / sqrtf(ss / 256.0f + 1e-6f);
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = x[e] * sc * w[lane + 64 * e];
  const float partner = __shfl_xor(x[0], 32);
  const int pos = tok_pos[t];
  const float co = cosT[pos * kRot + (lane & 31)], si = sinT[pos * kRot + (lane & 31)];
  x[0] = lane < 32 ? x[0] * co - partner * si : x[0] * co + partner * si;
  float *dst = isq ? Qb + (int64_t(t) * hq + hh) * kHD : Kb + (int64_t(t) * hkv + (hh - hq)) * kHD;
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[lane + 64 * e] = x[e];
}

// ---------------------------------------------------------------- full attention
// model.rs:276-298: causal GQA (kv head h / (hq/hkv)), scores / 16, softmax, sum p v, then
// * sigmoid(gate).  One workgroup per (32-query tile of one sequence, query head); key tiles
// of 32 stream through LDS with the next tile's loads held in registers meanwhile; online
// softmax in f32.  Output: f16 planes [T][hq*256] for o_proj.
constexpr int kAT = 32;
constexpr int kHDp = kHD + 4;  // padded LDS row: 16 B shift per row

__global__ __launch_bounds__(256, 1) void ot_attn_kernel(const float *__restrict__ Qb,
                                                         const float *__restrict__ Kb,
                                                         const float *__restrict__ proj, int ldp, int hq, int hkv,
                                                         const int32_t *__restrict__ tile_row0,
                                                         const int32_t *__restrict__ tile_pos0,
                                                         const int32_t *__restrict__ tile_n,
                                                         _Float16 *__restrict__ y, _Float16 *__restrict__ ylo) {
  __shared__ __align__(16) float sQ[kAT * kHDp];  // [32][260]
  __shared__ __align__(16) float sK[kAT * kHDp];  // [32][260]
  __shared__ __align__(16) float sV[kAT * kHD];   // [32][256]
  __shared__ float sP[kAT * 33];                  // [32][33]
  const int tile = blockIdx.x, h = blockIdx.y;
  const int row0 = tile_row0[tile], pos0 = tile_pos0[tile], nq = tile_n[tile];
  const int srow = row0 - pos0;  // first row of the sequence
  const int kh = h / (hq / hkv);
  const int tid = threadIdx.x, r = tid >> 3, sub = tid & 7;
  const int qw = hq * kHD, kvw = hkv * kHD;
  for (int e = tid; e < kAT * 64; e += 256) {
    const int i = e >> 6, c4 = e & 63;
    const float4 v = i < nq ? reinterpret_cast<const float4 *>(Qb + int64_t(row0 + i) * qw + h * kHD)[c4]
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    *reinterpret_cast<float4 *>(sQ + i * kHDp + c4 * 4) = v;
  }
  const int nkeys = pos0 + nq;
  const int ntiles = (nkeys + kAT - 1) / kAT;
  float4 kr[8], vr[8];
  auto load = [&](int kt) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = tid + 256 * k, i = e >> 6, c4 = e & 63;
      const int key = kt * kAT + i;
      const bool ok = key < nkeys;
      kr[k] = ok ? reinterpret_cast<const float4 *>(Kb + int64_t(srow + key) * kvw + kh * kHD)[c4]
                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      vr[k] = ok ? reinterpret_cast<const float4 *>(proj + int64_t(srow + key) * ldp + 2 * qw + kvw + kh * kHD)[c4]
                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.0f;
  float m = -FLT_MAX, l = 0.0f;
  bool seen = false;
  const int qpos = pos0 + r;
  load(0);
  for (int kt = 0; kt < ntiles; ++kt) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = tid + 256 * k, i = e >> 6, c4 = e & 63;
      *reinterpret_cast<float4 *>(sK + i * kHDp + c4 * 4) = kr[k];
      *reinterpret_cast<float4 *>(sV + i * kHD + c4 * 4) = vr[k];
    }
    __syncthreads();
    if (kt + 1 < ntiles) load(kt + 1);
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *qrow = sQ + r * kHDp;
#pragma unroll 4
    for (int d = 0; d < kHD; d += 4) {
      const float4 q = *reinterpret_cast<const float4 *>(qrow + d);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 k = *reinterpret_cast<const float4 *>(sK + (sub + 8 * i) * kHDp + d);
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
      const int key = kt * kAT + sub + 8 * i;
      ok[i] = key <= qpos && r < nq;
      s[i] = s[i] / 16.0f;
      if (ok[i]) mt = fmaxf(mt, s[i]);
    }
    mt = group8_max(mt);
    const bool any = mt > -FLT_MAX;
    const float mn = fmaxf(m, mt);
    const float corr = seen ? expf(m - mn) : 0.0f;
    float p[4], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = ok[i] ? expf(s[i] - mn) : 0.0f;
      ps += p[i];
    }
    ps = group8_sum(ps);
    if (any) {
      l = l * corr + ps;
      m = mn;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] *= corr;
      seen = true;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sP[r * 33 + sub + 8 * i] = p[i];
    __syncthreads();
#pragma unroll 4
    for (int c = 0; c < kAT; ++c) {
      const float pc = sP[r * 33 + c];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 v = *reinterpret_cast<const float4 *>(sV + c * kHD + sub * 4 + 32 * i);
        acc[4 * i] = fmaf(pc, v.x, acc[4 * i]);
        acc[4 * i + 1] = fmaf(pc, v.y, acc[4 * i + 1]);
        acc[4 * i + 2] = fmaf(pc, v.z, acc[4 * i + 2]);
        acc[4 * i + 3] = fmaf(pc, v.w, acc[4 * i + 3]);
      }
    }
    __syncthreads();
  }
  if (r >= nq) return;
  const int t = row0 + r;
  const float inv = 1.0f / l;
  const float *gate = proj + int64_t(t) * ldp + h * 2 * kHD + kHD;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = sub * 4 + 32 * i + e;
      store_planes(y, ylo, int64_t(t) * qw + h * kHD + d, acc[4 * i + e] * inv * sigmoidf_(gate[d]));
    }
}

// ---------------------------------------------------------------- full attention on f32 MFMA
// The same attention as ot_attn_kernel on v_mfma_f32_16x16x4_f32 (f32 operands, f32
// accumulation), split over keys for parallelism.  Work item = (16 query rows of one sequence,
// a range of <= 256 keys, 4 query heads sharing one KV head): one wave per query head.
//   S = Q K^T: lane (i = l%16, kg = l/16) supplies Q[i][16g + 4kg + c] at step 4g + c: the
//   contraction order over the 256 dims is a permutation, applied to K alike, so each operand
//   is one float4 LDS read per 4 MFMAs.
//   D layout: lane l holds S[4(l/16) + r][16 blk + l%16], r < 4.
//   Online softmax per row (16-lane DPP row reductions); P goes through LDS to the A layout.
//   O += P V over keys 16u + 4kg + c (V transposed in LDS, so again one float4 per 4 MFMAs).
// Partial (m, l, O) per item and head; ot_attn_combine_kernel merges an item's key ranges.
constexpr int kQT = 16;    // query rows per item
constexpr int kKC = 256;   // keys per item
constexpr int kVTp = 36;   // padded row of the transposed V tile [256 dims][32 keys]
constexpr int kPp = 36;    // padded row of the P tile [16 rows][32 keys]

// One 32-key tile of K rows and V rows (from the projection) for 256 threads, 8 float4 each;
// keys past khi are clamped to khi - 1 (masked by the caller).
__device__ __forceinline__ void ot_load_kv(float4v (&kr)[8], float4v (&vr)[8], const float *__restrict__ Kb,
                                           const float *__restrict__ proj, int ldp, int kvw, int vcol, int kcol,
                                           int srow, int kt, int khi, int tid) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int e = tid + 256 * k, i = e >> 6, c4 = e & 63;
    const int key = min(kt * kAT + i, khi - 1);
    kr[k] = reinterpret_cast<const float4v *>(Kb + int64_t(srow + key) * kvw + kcol)[c4];
    vr[k] = reinterpret_cast<const float4v *>(proj + int64_t(srow + key) * ldp + vcol)[c4];
  }
}

__global__ __launch_bounds__(256, 1) void ot_attn_part_kernel(
    const float *__restrict__ Qb, const float *__restrict__ Kb, const float *__restrict__ proj, int ldp, int hq,
    int hkv, const int32_t *__restrict__ it_row0, const int32_t *__restrict__ it_pos0,
    const int32_t *__restrict__ it_nq, const int32_t *__restrict__ it_klo, const int32_t *__restrict__ it_khi,
    float *__restrict__ part) {
  __shared__ __align__(16) float sK[kAT * kHDp];   // [32 keys][260]
  __shared__ __align__(16) float sVT[kHD * kVTp];  // [256 dims][36]
  __shared__ __align__(16) float sP[4][kQT * kPp]; // per wave [16 rows][36]
  __shared__ __align__(16) float sQ[4][kQT * kHDp]; // per wave [16 rows][260]
  const int item = blockIdx.x;
  const int row0 = it_row0[item], pos0 = it_pos0[item], nq = it_nq[item];
  const int klo = it_klo[item], khi = it_khi[item];
  const int srow = row0 - pos0;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int h = blockIdx.y * 4 + w;
  const int kh = (blockIdx.y * 4) / (hq / hkv);
  const int qw = hq * kHD, kvw = hkv * kHD;
  const int li = l & 15, kg = l >> 4;
  // this wave's Q rows into LDS (rows past nq repeat row nq - 1 and are never written out)
  float *myQ = sQ[w];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int e = l + 64 * k, i = e >> 6, c4 = e & 63;
    *reinterpret_cast<float4 *>(myQ + i * kHDp + c4 * 4) =
        reinterpret_cast<const float4 *>(Qb + int64_t(row0 + min(i, nq - 1)) * qw + h * kHD)[c4];
  }
  float4v acc_o[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) acc_o[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  float m[4], lsum[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -FLT_MAX;
    lsum[r] = 0.0f;
  }
  const int kt0 = klo / kAT, kt1 = (khi + kAT - 1) / kAT;
  float4v kr[8], vr[8];
  ot_load_kv(kr, vr, Kb, proj, ldp, kvw, 2 * qw + kvw + kh * kHD, kh * kHD, srow, kt0, khi, tid);
  float *myP = sP[w];
  for (int kt = kt0; kt < kt1; ++kt) {
    __syncthreads();  // previous tile's readers are done
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = tid + 256 * k, i = e >> 6, c4 = e & 63;
      *reinterpret_cast<float4v *>(sK + i * kHDp + c4 * 4) = kr[k];
      sVT[(c4 * 4 + 0) * kVTp + i] = vr[k][0];
      sVT[(c4 * 4 + 1) * kVTp + i] = vr[k][1];
      sVT[(c4 * 4 + 2) * kVTp + i] = vr[k][2];
      sVT[(c4 * 4 + 3) * kVTp + i] = vr[k][3];
    }
    __syncthreads();
    // next tile's loads, unconditional (the last iteration reloads its own tile)
    ot_load_kv(kr, vr, Kb, proj, ldp, kvw, 2 * qw + kvw + kh * kHD, kh * kHD, srow, min(kt + 1, kt1 - 1), khi, tid);
    // S = Q K^T, two 16x16 blocks of keys
    float4v s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 16; ++g) {
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
    // scale, mask, online softmax; lane holds rows 4 kg + r, keys li and 16 + li
    const int key0 = kt * kAT + li, key1 = key0 + 16;
    float corr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * kg + r, qpos = pos0 + row;
      const bool ok0 = key0 >= klo && key0 < khi && key0 <= qpos && row < nq;
      const bool ok1 = key1 >= klo && key1 < khi && key1 <= qpos && row < nq;
      const float a = s0[r] / 16.0f, b = s1[r] / 16.0f;
      float mt = fmaxf(ok0 ? a : -FLT_MAX, ok1 ? b : -FLT_MAX);
      mt = row_max16(mt);
      const float mn = fmaxf(m[r], mt);
      const bool any = mt > -FLT_MAX;
      const float p0 = ok0 ? expf(a - mn) : 0.0f, p1 = ok1 ? expf(b - mn) : 0.0f;
      const float ps = row_sum(p0 + p1);
      corr[r] = 1.0f;
      if (any) {
        corr[r] = m[r] > -FLT_MAX ? expf(m[r] - mn) : 0.0f;
        lsum[r] = lsum[r] * corr[r] + ps;
        m[r] = mn;
      }
      myP[row * kPp + li] = p0;
      myP[row * kPp + 16 + li] = p1;
    }
    // rescale the running output only when some row's maximum moved (a wave-uniform branch:
    // the accumulators stay in place otherwise)
    if (__any(corr[0] != 1.0f || corr[1] != 1.0f || corr[2] != 1.0f || corr[3] != 1.0f)) {
#pragma unroll
      for (int b = 0; b < 16; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc_o[b][r] *= corr[r];
    }
    // O += P V: A = P[li][16u + 4kg + c], B = V[16u + 4kg + c][16b + li]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float4 pa = *reinterpret_cast<const float4 *>(myP + li * kPp + 16 * u + 4 * kg);
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const float4 vb = *reinterpret_cast<const float4 *>(sVT + (16 * b + li) * kVTp + 16 * u + 4 * kg);
        acc_o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.x, vb.x, acc_o[b], 0, 0, 0);
        acc_o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.y, vb.y, acc_o[b], 0, 0, 0);
        acc_o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.z, vb.z, acc_o[b], 0, 0, 0);
        acc_o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.w, vb.w, acc_o[b], 0, 0, 0);
      }
    }
  }
  // partial: [item][head][16 rows][256] O, then [item][head][16][2] (m, l)
  float *po = part + (int64_t(item) * hq + h) * (kQT * kHD + 2 * kQT);
#pragma unroll
  for (int b = 0; b < 16; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) po[(4 * kg + r) * kHD + 16 * b + li] = acc_o[b][r];
  if (li == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      po[kQT * kHD + 2 * (4 * kg + r)] = m[r];
      po[kQT * kHD + 2 * (4 * kg + r) + 1] = lsum[r];
    }
}

// Merge the key-range partials of one 16-row query tile and head: O = sum_s e^(m_s - M) O_s /
// sum_s e^(m_s - M) l_s, then * sigmoid(gate) -> f16 planes.  256 threads: 16 rows x 16 dims
// groups of 16.
__global__ __launch_bounds__(256) void ot_attn_combine_kernel(const float *__restrict__ part, const float *__restrict__ proj,
                                                              int ldp, int hq, const int32_t *__restrict__ cb_row0,
                                                              const int32_t *__restrict__ cb_nq,
                                                              const int32_t *__restrict__ cb_first,
                                                              const int32_t *__restrict__ cb_n, _Float16 *__restrict__ y,
                                                              _Float16 *__restrict__ ylo) {
  const int tile = blockIdx.x, h = blockIdx.y;
  const int row0 = cb_row0[tile], nq = cb_nq[tile], first = cb_first[tile], ns = cb_n[tile];
  const int r = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 16;
  if (r >= nq) return;
  const int64_t stride = int64_t(hq) * (kQT * kHD + 2 * kQT);
  const float *p0 = part + int64_t(first) * stride + int64_t(h) * (kQT * kHD + 2 * kQT);
  float M = -FLT_MAX;
  for (int s = 0; s < ns; ++s) {
    const float *ml = p0 + s * stride + kQT * kHD + 2 * r;
    if (ml[1] > 0.0f) M = fmaxf(M, ml[0]);
  }
  float L = 0.0f, o[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) o[e] = 0.0f;
  for (int s = 0; s < ns; ++s) {
    const float *ps = p0 + s * stride;
    const float *ml = ps + kQT * kHD + 2 * r;
    if (!(ml[1] > 0.0f)) continue;
    const float f = expf(ml[0] - M);
    L += f * ml[1];
    const float4 *src = reinterpret_cast<const float4 *>(ps + r * kHD + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 v = src[e];
      o[4 * e] += f * v.x;
      o[4 * e + 1] += f * v.y;
      o[4 * e + 2] += f * v.z;
      o[4 * e + 3] += f * v.w;
    }
  }
  const float inv = 1.0f / L;
  const int t = row0 + r;
  const float *gate = proj + int64_t(t) * ldp + h * 2 * kHD + kHD;
  const int qw = hq * kHD;
#pragma unroll
  for (int e = 0; e < 16; ++e)
    store_planes(y, ylo, int64_t(t) * qw + h * kHD + d0 + e, o[e] * inv * sigmoidf_(gate[d0 + e]));
}

}  // namespace

void launch_ot_delta_prep(const float *proj, int ldp, int T, const int32_t *tok_pos, const float *conv,
                          const float *alog, const float *dt, int nh, float *qk, float *vbuf, float *gb,
                          hipStream_t st) {
  LG_REQUIRE(T > 0 && nh > 0 && nh <= 32, "delta prep: bad shape T=%d nh=%d", T, nh);
  LG_REQUIRE(ldp % 4 == 0 && ldp >= 3 * nh * kLK + nh * kLK + 2 * nh, "delta prep: projection row %d too short", ldp);
  const size_t lds = size_t(3) * nh * kLK * sizeof(float);
  hipLaunchKernelGGL(ot_delta_prep_kernel, dim3(T), dim3(256), lds, st, proj, ldp, tok_pos, conv, alog, dt, nh,
                     qk, vbuf, gb);
  HIP_CHECK(hipGetLastError());
}

void launch_ot_delta_scan(const float *qk, const float *vbuf, const float *gb, const int32_t *seq_row0,
                          const int32_t *seq_n, int nseq, int nh, float *out, hipStream_t st) {
  LG_REQUIRE(nseq > 0 && nh > 0 && nh <= 65535, "delta scan: bad shape nseq=%d nh=%d", nseq, nh);
  hipLaunchKernelGGL(ot_delta_scan_kernel, dim3(nseq, nh, kLK / kCols), dim3(256), 0, st, qk, vbuf, gb, seq_row0,
                     seq_n, nh, out);
  HIP_CHECK(hipGetLastError());
}

void launch_ot_delta_out(const float *o, int T, int nh, const float *norm_w, const float *proj, int ldp, int zcol,
                         _Float16 *y, _Float16 *ylo, hipStream_t st) {
  LG_REQUIRE(T > 0 && nh > 0 && zcol + nh * kLK <= ldp, "delta out: bad shape");
  const int64_t items = int64_t(T) * nh;
  hipLaunchKernelGGL(ot_delta_out_kernel, dim3(unsigned((items + 3) / 4)), dim3(256), 0, st, o, T, nh, norm_w, proj,
                     ldp, zcol, y, ylo);
  HIP_CHECK(hipGetLastError());
}

void launch_ot_attn_prep(const float *proj, int ldp, int T, int hq, int hkv, const int32_t *tok_pos,
                         const float *qn1, const float *kn1, const float *cosT, const float *sinT, float *Qb,
                         float *Kb, hipStream_t st) {
  LG_REQUIRE(T > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "attn prep: bad heads %d/%d", hq, hkv);
  LG_REQUIRE(ldp >= (2 * hq + 2 * hkv) * kHD, "attn prep: projection row %d too short", ldp);
  const int64_t items = int64_t(T) * (hq + hkv);
  hipLaunchKernelGGL(ot_attn_prep_kernel, dim3(unsigned((items + 3) / 4)), dim3(256), 0, st, proj, ldp, T, hq, hkv,
                     tok_pos, qn1, kn1, cosT, sinT, Qb, Kb);
  HIP_CHECK(hipGetLastError());
}

void launch_ot_attn(const float *Qb, const float *Kb, const float *proj, int ldp, int hq, int hkv,
                    const int32_t *tile_row0, const int32_t *tile_pos0, const int32_t *tile_n, int ntiles,
                    _Float16 *y, _Float16 *ylo, hipStream_t st) {
  LG_REQUIRE(ntiles > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "attn: bad shape");
  LG_REQUIRE(ldp % 4 == 0 && ldp >= (2 * hq + 2 * hkv) * kHD, "attn: projection row %d too short", ldp);
  hipLaunchKernelGGL(ot_attn_kernel, dim3(ntiles, hq), dim3(256), 0, st, Qb, Kb, proj, ldp, hq, hkv, tile_row0,
                     tile_pos0, tile_n, y, ylo);
  HIP_CHECK(hipGetLastError());
}

int64_t ot_attn_part_floats(int nitems, int hq) { return int64_t(nitems) * hq * (kQT * kHD + 2 * kQT); }

void launch_ot_attn_mfma(const float *Qb, const float *Kb, const float *proj, int ldp, int hq, int hkv,
                         const int32_t *it_row0, const int32_t *it_pos0, const int32_t *it_nq, const int32_t *it_klo,
                         const int32_t *it_khi, int nitems, const int32_t *cb_row0, const int32_t *cb_nq,
                         const int32_t *cb_first, const int32_t *cb_n, int ncomb, float *part, _Float16 *y,
                         _Float16 *ylo, hipStream_t st) {
  LG_REQUIRE(nitems > 0 && ncomb > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (hq / hkv) % 4 == 0,
             "attn: MFMA path needs groups of 4 query heads per KV head (heads %d/%d)", hq, hkv);
  LG_REQUIRE(ldp % 4 == 0 && ldp >= (2 * hq + 2 * hkv) * kHD, "attn: projection row %d too short", ldp);
  launch_timed(ot_attn_part_kernel, dim3(nitems, hq / 4), dim3(256), 0, st, Qb, Kb, proj, ldp, hq, hkv, it_row0,
               it_pos0, it_nq, it_klo, it_khi, part);
  HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(ot_attn_combine_kernel, dim3(ncomb, hq), dim3(256), 0, st, part, proj, ldp, hq, cb_row0, cb_nq,
                     cb_first, cb_n, y, ylo);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
