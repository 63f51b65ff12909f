// Kernels of the OpenThai-SystemOne text tower (src/models/openthai/model.rs:244-362) that the
// decoder path does not have: the gated DeltaNet mixer (causal conv + silu + q/k
// normalisation, the per-head recurrent scan, the gated output norm) and the sigmoid-gated
// full attention over 256-dim heads with partial RoPE.  Projections run on the shared MFMA
// GEMM; these kernels read its f32 outputs.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "common.h"
#include "kernels.h"
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
  const _Float16 h = _Float16(v);
  hi[i] = h;
  if (lo) lo[i] = _Float16(v - float(h));
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
// Columns d are independent, so one workgroup owns 32 columns of one head of one sequence:
// lane = (column, j-group of 16 keys); each lane keeps its 16 x 1 slice of S in registers and
// the two sums over j are 8-lane DPP reductions.  Tokens go in chunks of kCh staged in LDS,
// double buffered: the next chunk's loads are in flight while the current one is scanned.
constexpr int kCh = 16;
constexpr int kCols = 32;

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
  const int col = (tid >> 6) * 8 + (lane >> 3);  // column within this block, 0..31
  const int g = lane & 7;                        // keys j = 16 g .. 16 g + 15
  const int nchunks = (n + kCh - 1) / kCh;
  float4 rq[kCh * 64 / 256];
  float rv[kCh * kCols / 256];
  float2 rg = make_float2(0.0f, 0.0f);
  auto load = [&](int c) {
    const int t0 = c * kCh;
#pragma unroll
    for (int k = 0; k < kCh * 64 / 256; ++k) {
      const int e = tid + 256 * k, i = e >> 6, q4 = e & 63;
      rq[k] = t0 + i < n ? reinterpret_cast<const float4 *>(qk + (int64_t(row0 + t0 + i) * nh + h) * (2 * kLK))[q4]
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < kCh * kCols / 256; ++k) {
      const int e = tid + 256 * k, i = e / kCols, cc = e % kCols;
      rv[k] = t0 + i < n ? vbuf[int64_t(row0 + t0 + i) * lw + h * kLK + cb * kCols + cc] : 0.0f;
    }
    if (tid < kCh)
      rg = t0 + tid < n ? reinterpret_cast<const float2 *>(gb)[int64_t(row0 + t0 + tid) * nh + h]
                        : make_float2(0.0f, 0.0f);
  };
  auto stage = [&](int b) {
#pragma unroll
    for (int k = 0; k < kCh * 64 / 256; ++k) {
      const int e = tid + 256 * k;
      s_qk[b][e >> 6][e & 63] = rq[k];
    }
#pragma unroll
    for (int k = 0; k < kCh * kCols / 256; ++k) {
      const int e = tid + 256 * k;
      s_v[b][e / kCols][e % kCols] = rv[k];
    }
    if (tid < kCh) s_gb[b][tid] = rg;
  };
  float S[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) S[j] = 0.0f;
  if (nchunks > 0) {
    load(0);
    stage(0);
  }
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int b = c & 1;
    if (c + 1 < nchunks) load(c + 1);
    const int cnt = min(kCh, n - c * kCh);
    for (int i = 0; i < cnt; ++i) {
      const float2 db = s_gb[b][i];
      float kk[16], qq[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 a = s_qk[b][i][32 + g * 4 + q], e = s_qk[b][i][g * 4 + q];
        kk[4 * q] = a.x; kk[4 * q + 1] = a.y; kk[4 * q + 2] = a.z; kk[4 * q + 3] = a.w;
        qq[4 * q] = e.x; qq[4 * q + 1] = e.y; qq[4 * q + 2] = e.z; qq[4 * q + 3] = e.w;
      }
      const float vd = s_v[b][i][col];
      float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        S[j] *= db.x;
        S[j + 1] *= db.x;
        p0 = fmaf(S[j], kk[j], p0);
        p1 = fmaf(S[j + 1], kk[j + 1], p1);
      }
      const float delta = (vd - group8_sum(p0 + p1)) * db.y;
      float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        S[j] = fmaf(kk[j], delta, S[j]);
        S[j + 1] = fmaf(kk[j + 1], delta, S[j + 1]);
        o0 = fmaf(S[j], qq[j], o0);
        o1 = fmaf(S[j + 1], qq[j + 1], o1);
      }
      const float o = group8_sum(o0 + o1);
      if (g == 0) s_o[i][col] = o;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kCh * kCols / 256; ++k) {
      const int e = tid + 256 * k, i = e / kCols, cc = e % kCols;
      if (i < cnt) out[int64_t(row0 + c * kCh + i) * lw + h * kLK + cb * kCols + cc] = s_o[i][cc];
    }
    if (c + 1 < nchunks) stage(b ^ 1);
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

}  // namespace lg
