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
// query = q / |q| / sqrt(128), key = k / |k| (|x| = sqrt(x.x + 1e-6)), log-decay and beta.
// model.rs:306-318 (conv), :323-331 (scales, decay, beta).
constexpr int kPrepThreads = 512;
__global__ __launch_bounds__(kPrepThreads) void ot_delta_prep_kernel(const float *__restrict__ proj, int ldp, int T,
                                                            const int32_t *__restrict__ tok_pos,
                                                            const float *__restrict__ conv,
                                                            const float *__restrict__ alog,
                                                            const float *__restrict__ dt, int nh,
                                                            float *__restrict__ qk, float *__restrict__ vbuf,
                                                            float *__restrict__ gb) {
  extern __shared__ float s_x[];
  // consecutive workgroups go to the 8 XCDs in turn: XCD x takes tokens x * per .. + per - 1, so the three
  // rows before a token that its conv reads were read by the XCD's previous tokens and sit in its L2 (the
  // grid is 8 * per workgroups; those past T have no token)
  const int per = int(gridDim.x) >> 3, t = int(blockIdx.x & 7) * per + int(blockIdx.x >> 3);
  if (t >= T) return;
  const int lw = nh * kLK, cd = 3 * lw;
  const int pos = tok_pos[t];
  const float *row = proj + int64_t(t) * ldp;
  const int h_ab = min(int(threadIdx.x), nh - 1);
  const float a = row[cd + lw + h_ab], b = row[cd + lw + nh + h_ab];
  // four channels a thread: one 16-byte load per tap row and four of taps (conv is [channel][4 taps]); a
  // thread's loads for three rounds of 4 * kPrepThreads channels (every channel of a 16-head layer) are
  // issued before any of them is used (a round past the row clamped into it: its results are not stored).
  // q and k channels go to LDS for their norms, v channels straight out to vbuf.
  const float4v zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int kR = 3;
  for (int c0 = 4 * int(threadIdx.x); c0 < cd; c0 += kR * 4 * kPrepThreads) {
    float4v x[kR][4];
    float4 w[kR][4];
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int c = min(c0 + j * 4 * kPrepThreads, cd - 4);
      x[j][0] = *reinterpret_cast<const float4v *>(row + c);
      x[j][1] = pos >= 1 ? *reinterpret_cast<const float4v *>(row + c - int64_t(ldp)) : zero4;
      x[j][2] = pos >= 2 ? *reinterpret_cast<const float4v *>(row + c - 2 * int64_t(ldp)) : zero4;
      x[j][3] = pos >= 3 ? *reinterpret_cast<const float4v *>(row + c - 3 * int64_t(ldp)) : zero4;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[j][e] = reinterpret_cast<const float4 *>(conv)[c + e];
    }
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int c = c0 + j * 4 * kPrepThreads;
      if (c >= cd) break;
      float4v o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = 0.0f;
        if (pos >= 3) v = v + x[j][3][e] * w[j][e].x;
        if (pos >= 2) v = v + x[j][2][e] * w[j][e].y;
        if (pos >= 1) v = v + x[j][1][e] * w[j][e].z;
        v = v + x[j][0][e] * w[j][e].w;
        o[e] = siluf_(v);
      }
      if (c < 2 * lw) *reinterpret_cast<float4v *>(s_x + c) = o;
      else *reinterpret_cast<float4v *>(vbuf + int64_t(t) * lw + (c - 2 * lw)) = o;
    }
  }
  __syncthreads();
  // per-head norms, four vectors of a wave at a time (vec < nh: q of head vec; else k of head vec - nh)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int v0 = wv; v0 < 2 * nh; v0 += 4 * (kPrepThreads / 64)) {
    float x0[4], x1[4], ss[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int vec = min(v0 + i * (kPrepThreads / 64), 2 * nh - 1);
      x0[i] = s_x[vec * kLK + lane];
      x1[i] = s_x[vec * kLK + lane + 64];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) ss[i] = wave_sum_dpp(x0[i] * x0[i] + x1[i] * x1[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int vec = v0 + i * (kPrepThreads / 64);
      if (vec >= 2 * nh) break;
      const int h = vec < nh ? vec : vec - nh;
      float sc = 1.0f / sqrtf(ss[i] + 1e-6f);
      if (vec < nh) sc = sc / sqrtf(128.0f);
      float *dst = qk + (int64_t(t) * nh + h) * (2 * kLK) + (vec < nh ? 0 : kLK);
      dst[lane] = x0[i] * sc;
      dst[lane + 64] = x1[i] * sc;
    }
  }
  if (threadIdx.x < nh) {
    const int h = threadIdx.x;
    // the log of the decay a_t = exp(-exp(A_log) softplus(a + dt)); the chunked scan takes exp of sums of these
    gb[(int64_t(t) * nh + h) * 2] = -expf(alog[h]) * softplusf_(a + dt[h]);
    gb[(int64_t(t) * nh + h) * 2 + 1] = sigmoidf_(b);
  }
}

// ---------------------------------------------------------------- DeltaNet: chunked scan
// model.rs:319-358, per head a [key j][value d] = 128 x 128 state S, token by token:
//   S *= a_t;  delta_t = (v_t - S^T k_t) * beta_t;  S += k_t delta_t^T;  o_t = S^T q_t.
// Taken here over chunks of kDC tokens in the chunk's WY form (the same mathematics, another rounding
// order).  With S0 the state entering a chunk and gam_t = sum_{r <= t} log a_r inside it:
//   (I + A) X = [diag(beta) V | diag(beta e^gam) K],   A_ts = beta_t e^(gam_t - gam_s) (k_t . k_s), s < t
//   X = [U | W];   Delta = U - W S0                    (the rows delta_t of the token loop)
//   O = diag(e^gam) Q S0 + P Delta,                    P_ts = e^(gam_t - gam_s) (q_t . k_s), s <= t
//   S = e^gam_last S0 + K^T diag(e^(gam_last - gam)) Delta.
// ot_delta_chunk_kernel builds A and P and solves for X by forward substitution, every chunk of every
// head at once; ot_delta_state_kernel walks a sequence's chunks in order, carrying S.  Products on
// v_mfma_f32_16x16x4_f32 (f32 operands and accumulation); gam is summed in f64, so each decay factor
// e^(gam_t - gam_s) is exp of a difference that is exact to f32 rounding.  Tokens past a sequence's end
// carry beta 0 and log-decay 0 (with zero k, q, v in the chunk kernel), which leave S unchanged.
constexpr int kDC = 32;   // tokens per chunk
constexpr int kDP = 132;  // LDS row stride (floats) of a chunk's [kDC][128] operands
constexpr int kDA = 36;   // LDS row stride of A
// one (chunk, head) record of the workspace, floats: U [kDC][128], W [kDC][128], P [kDC][kDC],
// e^gam_t [kDC], e^(gam_last - gam_t) [kDC]
constexpr int kOffU = 0, kOffW = kDC * kLK, kOffP = 2 * kDC * kLK, kOffE = kOffP + kDC * kDC;
constexpr int kOffL = kOffE + kDC, kChunkFloats = kOffL + kDC;
// a chunk's record: sequences own consecutive slots, chunk c of sequence sq (first batch row row0)
// in slot sq + row0 / kDC + c; fewer than nseq + T / kDC + 1 slots in all
__device__ __forceinline__ int64_t ot_chunk_slot(int sq, int row0, int c) { return int64_t(sq) + row0 / kDC + c; }

__global__ __launch_bounds__(256) void ot_delta_chunk_kernel(const float *__restrict__ qk,
                                                             const float *__restrict__ vbuf,
                                                             const float *__restrict__ gb,
                                                             const int32_t *__restrict__ seq_row0,
                                                             const int32_t *__restrict__ seq_n, int nh,
                                                             float *__restrict__ ws) {
  __shared__ __align__(16) float sK[kDC * kDP], sQ[kDC * kDP], sV[kDC * kDP];
  __shared__ __align__(16) float sA[kDC * kDA];
  __shared__ float sB[kDC], sBE[kDC];
  __shared__ double sGam[kDC];
  const int c = blockIdx.x, h = blockIdx.y, sq = blockIdx.z;
  const int row0 = seq_row0[sq], n = seq_n[sq], t0 = c * kDC;
  if (t0 >= n) return;  // the grid covers the longest sequence's chunks
  const int m = min(kDC, n - t0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, kg = lane >> 4;
  const int lw = nh * kLK;
  float *rec = ws + (ot_chunk_slot(sq, row0, c) * nh + h) * kChunkFloats;
  // the chunk's q, k, v rows (rows past m zero); loads from the row clamped into the chunk, unpredicated
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int idx = tid + 256 * e, i = idx >> 5, c4 = idx & 31;
    const int64_t r = row0 + t0 + min(i, m - 1);
    const float4 *qrow = reinterpret_cast<const float4 *>(qk + (r * nh + h) * (2 * kLK));
    float4 qv = qrow[c4], kv = qrow[32 + c4], vv = reinterpret_cast<const float4 *>(vbuf + r * lw + h * kLK)[c4];
    if (i >= m) qv = kv = vv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    *reinterpret_cast<float4 *>(sQ + i * kDP + 4 * c4) = qv;
    *reinterpret_cast<float4 *>(sK + i * kDP + 4 * c4) = kv;
    *reinterpret_cast<float4 *>(sV + i * kDP + 4 * c4) = vv;
  }
  if (tid < kDC) {
    // a log-decay below -1e4 (a decay that is 0 in f32) is held at -1e4 so that differences stay finite
    const float2 v = reinterpret_cast<const float2 *>(gb)[(row0 + t0 + min(tid, m - 1)) * int64_t(nh) + h];
    sB[tid] = tid < m ? v.y : 0.0f;
    sBE[tid] = tid < m ? (v.x < -1e4f ? -1e4f : v.x) : 0.0f;  // the log-decay, until the sums below
  }
  __syncthreads();
  if (tid == 0) {  // gam in f64, token after token
    double gam = 0.0;
    for (int i = 0; i < kDC; ++i) {
      gam += double(sBE[i]);
      sGam[i] = gam;
      sBE[i] = sB[i] * expf(float(gam));
    }
  }
  __syncthreads();
  // K K^T and Q K^T, 32 x 32: wave w takes the 16 x 16 block (rows 16 (w / 2), columns 16 (w % 2)); the
  // 128-deep contraction in the order j = 16 g + 4 kg + component, the same for both operands
  {
    const int bt = w >> 1, bs = w & 1;
    float4v kk = {0.0f, 0.0f, 0.0f, 0.0f}, qq = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const float4 ka = *reinterpret_cast<const float4 *>(sK + (16 * bt + li) * kDP + 16 * g + 4 * kg);
      const float4 qa = *reinterpret_cast<const float4 *>(sQ + (16 * bt + li) * kDP + 16 * g + 4 * kg);
      const float4 kb = *reinterpret_cast<const float4 *>(sK + (16 * bs + li) * kDP + 16 * g + 4 * kg);
      kk = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, kb.x, kk, 0, 0, 0);
      qq = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.x, kb.x, qq, 0, 0, 0);
      kk = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, kb.y, kk, 0, 0, 0);
      qq = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.y, kb.y, qq, 0, 0, 0);
      kk = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, kb.z, kk, 0, 0, 0);
      qq = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.z, kb.z, qq, 0, 0, 0);
      kk = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, kb.w, kk, 0, 0, 0);
      qq = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.w, kb.w, qq, 0, 0, 0);
    }
    // lane: rows t = 16 bt + 4 kg + r, column s = 16 bs + li
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * bt + 4 * kg + r, s = 16 * bs + li;
      const float dec = s <= t ? expf(float(sGam[t] - sGam[s])) : 0.0f;
      sA[t * kDA + s] = s < t ? sB[t] * dec * kk[r] : 0.0f;
      rec[kOffP + t * kDC + s] = s <= t ? dec * qq[r] : 0.0f;
    }
  }
  if (tid < kDC) {
    rec[kOffE + tid] = expf(float(sGam[tid]));
    rec[kOffL + tid] = expf(float(sGam[kDC - 1] - sGam[tid]));
  }
  __syncthreads();
  // forward substitution, one column of X = [U | W] per thread: x_t = rhs_t - sum_{s < t} A_ts x_s, s ascending
  {
    const bool isU = tid < kLK;
    const int cc = tid & (kLK - 1);
    float x[kDC];
#pragma unroll
    for (int t = 0; t < kDC; ++t) {
      float acc = isU ? sB[t] * sV[t * kDP + cc] : sBE[t] * sK[t * kDP + cc];
#pragma unroll
      for (int s = 0; s < t; ++s) acc = fmaf(-sA[t * kDA + s], x[s], acc);
      x[t] = acc;
    }
    float *dst = rec + (isU ? kOffU : kOffW) + cc;
#pragma unroll
    for (int t = 0; t < kDC; ++t) dst[t * kLK] = x[t];
  }
}

// One workgroup per (16 value columns, head, sequence), four compute waves and one memory wave.
// S[:, 16 cb .. 16 cb + 16) lives in the compute waves' MFMA accumulators, wave w < 4 holding key rows
// 32 w .. 32 w + 31 (two 16 x 16 blocks; lane: rows 32 w + 16 b + 4 kg + r, column li).  Per chunk c,
// two barriers:
//   1. each compute wave's share of W S0 (its 32 key rows; its S accumulators serve as the B operand
//      directly, the contraction taken as j = 32 w + 16 b + 4 kg + r), then of Q S0, whose MFMAs run
//      on while the wave waits at the barrier;
//   2. Delta = U - (sum of the four shares of W S0, fixed order); waves 0 and 1 meanwhile form the O rows
//      of chunk c - 1 in LDS: P Delta (MFMA) + e^gam (sum of its Q S0 shares);
//   3. the Q S0 shares of chunk c; S = e^gam_last S + K^T (e^(gam_last - gam) Delta).
// Only W S0 -> Delta -> S is on the chunk-to-chunk path.  The compute waves load W and Q (two chunks
// ahead, into one of two register sets in the A-operand layout of step 1) and nothing else; wave 4
// loads K, P, U and the decay factors into the LDS set of the chunk (double-buffered by parity; K rows
// with their 16-float column groups XOR-swizzled by row, so the K^T operand reads fall in distinct
// banks) and stores the O rows, as whole 2 KB blocks of out[head][column block][T][16].  A wave's
// loads and stores wait in one counter, so kept out of the compute waves, the stores' acknowledgements
// never hold up a chunk.
struct OtPre {
  float4v W[2][2], Q[2][2];
};
constexpr int kStateThreads = 320;
// dynamic LDS of ot_delta_state_kernel, floats: K [2][kDC][128], P [2][kDC][kDC], U [kDC][16],
// e^gam [2][kDC], e^(gam_last - gam) [2][kDC], Delta [2][kDC][16], W S0 and Q S0 shares [4][kDC][16]
// each, O [kDC][16]
constexpr int kSK = 0, kSP = kSK + 2 * kDC * kLK, kSU = kSP + 2 * kDC * kDC, kSE = kSU + kDC * 16;
constexpr int kSL = kSE + 2 * kDC, kSD = kSL + 2 * kDC, kSPW = kSD + 2 * kDC * 16, kSPQ = kSPW + 4 * kDC * 16;
constexpr int kSO = kSPQ + 4 * kDC * 16, kStateLdsFloats = kSO + kDC * 16;

__device__ __forceinline__ int ot_kswz(int row, int col) { return row * kLK + (col ^ ((row & 3) << 4)); }

__global__ __launch_bounds__(kStateThreads, 1) void ot_delta_state_kernel(const float *__restrict__ qk,
                                                                         const float *__restrict__ ws,
                                                                         const int32_t *__restrict__ seq_row0,
                                                                         const int32_t *__restrict__ seq_n, int nh,
                                                                         int T, float *__restrict__ out) {
  extern __shared__ float4v smem_v[];
  float *smem = reinterpret_cast<float *>(smem_v);
  float *sK[2] = {smem + kSK, smem + kSK + kDC * kLK}, *sP[2] = {smem + kSP, smem + kSP + kDC * kDC};
  float *sE[2] = {smem + kSE, smem + kSE + kDC}, *sL[2] = {smem + kSL, smem + kSL + kDC};
  float *sD[2] = {smem + kSD, smem + kSD + kDC * 16};
  float *sU = smem + kSU, *sO = smem + kSO;
  auto sPW = [&](int w) { return smem + kSPW + w * kDC * 16; };
  auto sPQ = [&](int w) { return smem + kSPQ + w * kDC * 16; };
  // grid (heads, column blocks, sequences): consecutive workgroups go to the 8 XCDs in turn, so with
  // x = head the eight column blocks of a head share one XCD and its L2 (each reads the whole chunk's W,
  // Q and K)
  const int h = blockIdx.x, cb = blockIdx.y, sq = blockIdx.z;
  const int row0 = seq_row0[sq], n = seq_n[sq];
  const int nch = (n + kDC - 1) / kDC;
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, kg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the role branches are scalar
  auto record = [&](int c) { return ws + (ot_chunk_slot(sq, row0, c) * nh + h) * kChunkFloats; };

  if (w == 4) {
    // ---- memory wave: stage chunk c (between the second barrier of chunk c - 1 and the first of
    // chunk c, when nothing reads its LDS set or U), store the O rows of chunk c - 2, load chunk c + 1
    float4v rK[16], rP[4], rU[2];
    float rE = 0.0f, rL = 0.0f;
    auto load = [&](int c) {
      const float *rec = record(c);
      const int t0 = c * kDC, m = min(kDC, n - t0);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int idx = lane + 64 * e, i = idx >> 5, c4 = idx & 31;
        const int64_t r = row0 + t0 + min(i, m - 1);
        rK[e] = reinterpret_cast<const float4v *>(qk + (r * nh + h) * (2 * kLK) + kLK)[c4];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) rP[e] = reinterpret_cast<const float4v *>(rec + kOffP)[lane + 64 * e];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int idx = lane + 64 * e;
        rU[e] = *reinterpret_cast<const float4v *>(rec + kOffU + (idx >> 2) * kLK + cb * 16 + 4 * (idx & 3));
      }
      rE = rec[kOffE + (lane & (kDC - 1))];
      rL = rec[kOffL + (lane & (kDC - 1))];
    };
    auto stage = [&](int X) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int idx = lane + 64 * e, i = idx >> 5, c4 = idx & 31;
        *reinterpret_cast<float4v *>(sK[X] + ot_kswz(i, 4 * c4)) = rK[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) reinterpret_cast<float4v *>(sP[X])[lane + 64 * e] = rP[e];
#pragma unroll
      for (int e = 0; e < 2; ++e) reinterpret_cast<float4v *>(sU)[lane + 64 * e] = rU[e];
      if (lane < kDC) {
        sE[X][lane] = rE;
        sL[X][lane] = rL;
      }
    };
    auto store_o = [&](int cc) {
      const int t0 = cc * kDC, m = min(kDC, n - t0);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int idx = lane + 64 * e, t = idx >> 2;
        if (t < m)
          *reinterpret_cast<float4v *>(out + ((int64_t(h) * (kLK / 16) + cb) * T + row0 + t0 + t) * 16 + 4 * (idx & 3)) =
              reinterpret_cast<const float4v *>(sO)[idx];
      }
    };
    if (nch > 0) load(0);
    for (int c = 0; c < nch; ++c) {
      stage(c & 1);
      if (c >= 2) store_o(c - 2);
      if (c + 1 < nch) load(c + 1);
      __syncthreads();
      __syncthreads();
    }
    __syncthreads();
    if (nch >= 2) store_o(nch - 2);
    __syncthreads();
    __syncthreads();
    if (nch >= 1) store_o(nch - 1);
    return;
  }

  // ---- compute waves
  auto load = [&](int c, OtPre &p) {
    const float *rec = record(c);
    const int t0 = c * kDC, m = min(kDC, n - t0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int t = 16 * tb + li, j = 32 * w + 16 * b + 4 * kg;
        p.W[tb][b] = *reinterpret_cast<const float4v *>(rec + kOffW + t * kLK + j);
        const int64_t r = row0 + t0 + min(t, m - 1);
        p.Q[tb][b] = *reinterpret_cast<const float4v *>(qk + (r * nh + h) * (2 * kLK) + j);
      }
  };
  // O rows t = 16 w + 4 kg + r (column li) of chunk cc from LDS set Y: P Delta over the chunk's tokens
  // s = 4 q + kg (P is zero above its diagonal), then + e^gam_t (sum of the Q S0 shares), into sO
  auto emit_o = [&](int Y) {
    float4v po = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < kDC / 4; ++q) {
      const int si = 4 * q + kg;
      po = __builtin_amdgcn_mfma_f32_16x16x4f32(sP[Y][(16 * w + li) * kDC + si], sD[Y][si * 16 + li], po, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * w + 4 * kg + r, e = t * 16 + li;
      const float qs = ((sPQ(0)[e] + sPQ(1)[e]) + sPQ(2)[e]) + sPQ(3)[e];
      sO[e] = fmaf(sE[Y][t], qs, po[r]);
    }
  };
  float4v S[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) S[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  // chunk c from cur, which then takes chunk c + 2
  auto body = [&](int c, OtPre &cur) {
    const int X = c & 1;
    float4v aW[2][2], aQ[2][2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        aW[tb][b] = cur.W[tb][b];
        aQ[tb][b] = cur.Q[tb][b];
      }
    if (c + 2 < nch) load(c + 2, cur);
    // 1. W S0 (two independent chains), then Q S0
    float4v dw[2], dq[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) dw[tb] = dq[tb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) dw[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(aW[tb][b][r], S[b][r], dw[tb], 0, 0, 0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) sPW(w)[(16 * tb + 4 * kg + r) * 16 + li] = dw[tb][r];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) dq[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(aQ[tb][b][r], S[b][r], dq[tb], 0, 0, 0);
    __syncthreads();
    // 2. Delta: entries e = tid and tid + 256 (t = e / 16, d = e % 16)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = tid + 256 * k;
      const float ws0 = ((sPW(0)[e] + sPW(1)[e]) + sPW(2)[e]) + sPW(3)[e];
      sD[X][e] = sU[e] - ws0;
    }
    if (c > 0 && w < 2) emit_o(X ^ 1);
    __syncthreads();
    // 3. this chunk's Q S0 shares; S = e^gam_last S + K^T Delta_scaled over the tokens t = 4 s + kg
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) sPQ(w)[(16 * tb + 4 * kg + r) * 16 + li] = dq[tb][r];
    const float gl = sE[X][kDC - 1];
#pragma unroll
    for (int b = 0; b < 2; ++b) S[b] = S[b] * gl;
#pragma unroll
    for (int s = 0; s < kDC / 4; ++s) {
      const int t = 4 * s + kg;
      const float dsc = sL[X][t] * sD[X][t * 16 + li];
#pragma unroll
      for (int b = 0; b < 2; ++b)
        S[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(sK[X][ot_kswz(t, 32 * w + 16 * b + li)], dsc, S[b], 0, 0, 0);
    }
  };
  OtPre pa, pb;
  if (nch > 0) load(0, pa);
  if (nch > 1) load(1, pb);
  for (int c = 0; c < nch; c += 2) {
    body(c, pa);
    if (c + 1 < nch) body(c + 1, pb);
  }
  __syncthreads();  // the last chunk's Q S0 shares; the memory wave then stores chunk nch - 2's O
  __syncthreads();
  if (nch > 0 && w < 2) emit_o((nch - 1) & 1);
  __syncthreads();
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
  // o is [head][column block of 16][T][16] (the scan's layout)
  const float *x = o + (int64_t(h) * (kLK / 16) * T + t) * 16;
  const float x0 = x[(lane >> 4) * int64_t(T) * 16 + (lane & 15)], x1 = x[((lane >> 4) + 4) * int64_t(T) * 16 + (lane & 15)];
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
constexpr int kPp = 36;    // padded row of the P tile [16 rows][32 keys]

// One 32-key tile of K rows and V rows (from the projection) for 256 threads, 8 float4 each; keys past khi
// are clamped to khi - 1 (masked by the caller).  K: kr[2 j + u] holds dims 8 o + 4 u .. + 3 of key i, with
// (i, o) = ((tid + 256 j) / 32, (tid + 256 j) % 32); V: vr[u] holds dims 4 (tid % 64) .. + 3 of key
// 8 (tid / 64) + u.  So a thread stages 8 consecutive dims of a K row, and 8 consecutive keys of each of 4
// rows of the transposed V tile, as 16-byte groups.
__device__ __forceinline__ void ot_load_kv(float4v (&kr)[8], float4v (&vr)[8], const float *__restrict__ Kb,
                                           const float *__restrict__ proj, int ldp, int kvw, int vcol, int kcol,
                                           int srow, int kt, int khi, int tid) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = tid + 256 * j, i = e >> 5, o = e & 31;
    const int key = min(kt * kAT + i, khi - 1);
    const float4v *kp = reinterpret_cast<const float4v *>(Kb + int64_t(srow + key) * kvw + kcol + 8 * o);
    kr[2 * j] = kp[0];
    kr[2 * j + 1] = kp[1];
  }
  const int oc = tid >> 6, c4 = tid & 63;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int key = min(kt * kAT + 8 * oc + u, khi - 1);
    vr[u] = reinterpret_cast<const float4v *>(proj + int64_t(srow + key) * ldp + vcol)[c4];
  }
}

// The products on v_mfma_f32_16x16x32_f16 with every f32 operand split into f16 hi + lo (hi = f16(x),
// lo = f16(x - hi)) and three products per pair (lo.hi, hi.lo, hi.hi; ~22 significant bits, f32
// accumulation): Q split once into registers, each K and V tile split as it is staged, P as it is read
// back.  LDS (dynamic): K hi and lo [32 keys][kKh], the transposed V tile hi and lo [256 dims][kVh], and each
// wave's f32 P tile [16 rows][kPp].
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
constexpr int kKh = kHD + 8;  // halves a staged K row (16 bytes of padding)
constexpr int kVh = kAT + 8;  // halves a staged V^T row
constexpr int kAttnLdsBytes = 2 * (2 * kAT * kKh + 2 * kHD * kVh) + 4 * 4 * kQT * kPp;

__device__ __forceinline__ void split8(float4v a, float4v b, half8v &hi, half8v &lo) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    _Float16 h, l;
    split_f16(a[c], h, l);
    hi[c] = h;
    lo[c] = l;
    split_f16(b[c], h, l);
    hi[4 + c] = h;
    lo[4 + c] = l;
  }
}

__device__ __forceinline__ float4v mfma3h(half8v ah, half8v al, half8v bh, half8v bl, float4v acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
}

__global__ __launch_bounds__(256, 1) void ot_attn_part_kernel(
    const float *__restrict__ Qb, const float *__restrict__ Kb, const float *__restrict__ proj, int ldp, int hq,
    int hkv, const int32_t *__restrict__ it_row0, const int32_t *__restrict__ it_pos0,
    const int32_t *__restrict__ it_nq, const int32_t *__restrict__ it_klo, const int32_t *__restrict__ it_khi,
    float *__restrict__ part) {
  extern __shared__ float4v attn_smem[];
  _Float16 *sKh = reinterpret_cast<_Float16 *>(attn_smem), *sKl = sKh + kAT * kKh;
  _Float16 *sVh = sKl + kAT * kKh, *sVl = sVh + kHD * kVh;
  float *sP = reinterpret_cast<float *>(sVl + kHD * kVh);  // [4 waves][16 rows][kPp]
  const int item = blockIdx.x;
  const int row0 = it_row0[item], pos0 = it_pos0[item], nq = it_nq[item];
  const int klo = it_klo[item], khi = it_khi[item];
  const int srow = row0 - pos0;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int h = blockIdx.y * 4 + w;
  const int kh = (blockIdx.y * 4) / (hq / hkv);
  const int qw = hq * kHD, kvw = hkv * kHD;
  const int li = l & 15, kg = l >> 4;
  // this wave's Q rows as A operands: row li (rows past nq repeat row nq - 1 and are never written out),
  // dims 32 s + 8 kg .. + 7 of k-step s
  half8v qh[8], ql[8];
  {
    const float *qr = Qb + int64_t(row0 + min(li, nq - 1)) * qw + h * kHD;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      split8(*reinterpret_cast<const float4v *>(qr + 32 * st + 8 * kg),
             *reinterpret_cast<const float4v *>(qr + 32 * st + 8 * kg + 4), qh[st], ql[st]);
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
  float *myP = sP + w * (kQT * kPp);
  for (int kt = kt0; kt < kt1; ++kt) {
    __syncthreads();  // previous tile's readers are done
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = tid + 256 * j, i = e >> 5, o = e & 31;
      half8v h8, l8;
      split8(kr[2 * j], kr[2 * j + 1], h8, l8);
      *reinterpret_cast<half8v *>(sKh + i * kKh + 8 * o) = h8;
      *reinterpret_cast<half8v *>(sKl + i * kKh + 8 * o) = l8;
    }
    {
      const int oc = tid >> 6, c4 = tid & 63;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        half8v h8, l8;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          _Float16 hh, ll;
          split_f16(vr[u][c], hh, ll);
          h8[u] = hh;
          l8[u] = ll;
        }
        *reinterpret_cast<half8v *>(sVh + (4 * c4 + c) * kVh + 8 * oc) = h8;
        *reinterpret_cast<half8v *>(sVl + (4 * c4 + c) * kVh + 8 * oc) = l8;
      }
    }
    __syncthreads();
    // next tile's loads, unconditional (the last iteration reloads its own tile)
    ot_load_kv(kr, vr, Kb, proj, ldp, kvw, 2 * qw + kvw + kh * kHD, kh * kHD, srow, min(kt + 1, kt1 - 1), khi, tid);
    // S = Q K^T, two 16x16 blocks of keys: B = K[16 kb + li][32 s + 8 kg .. + 7]
    float4v s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int o0 = li * kKh + 32 * st + 8 * kg, o1 = (16 + li) * kKh + 32 * st + 8 * kg;
      s0 = mfma3h(qh[st], ql[st], *reinterpret_cast<const half8v *>(sKh + o0), *reinterpret_cast<const half8v *>(sKl + o0),
                  s0);
      s1 = mfma3h(qh[st], ql[st], *reinterpret_cast<const half8v *>(sKh + o1), *reinterpret_cast<const half8v *>(sKl + o1),
                  s1);
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
    // O += P V over the tile's 32 keys in one k-step: A = P[li][8 kg .. + 7], B = V[8 kg .. + 7][16 b + li]
    {
      half8v ph, pl;
      split8(*reinterpret_cast<const float4v *>(myP + li * kPp + 8 * kg),
             *reinterpret_cast<const float4v *>(myP + li * kPp + 8 * kg + 4), ph, pl);
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const int o = (16 * b + li) * kVh + 8 * kg;
        acc_o[b] = mfma3h(ph, pl, *reinterpret_cast<const half8v *>(sVh + o), *reinterpret_cast<const half8v *>(sVl + o),
                          acc_o[b]);
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
  // partials in groups of 4 whose loads issue together (entries past ns read partial ns - 1 and are
  // skipped); the merge itself runs in partial order
  constexpr int G = 4;
  float M = -FLT_MAX;
  for (int s0 = 0; s0 < ns; s0 += G) {
    float2 ml[G];
#pragma unroll
    for (int u = 0; u < G; ++u)
      ml[u] = *reinterpret_cast<const float2 *>(p0 + min(s0 + u, ns - 1) * stride + kQT * kHD + 2 * r);
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (s0 + u < ns && ml[u].y > 0.0f) M = fmaxf(M, ml[u].x);
  }
  float L = 0.0f;
  float4v o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < ns; s0 += G) {
    float2 ml[G];
    float4v v[G][4];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const float *ps = p0 + min(s0 + u, ns - 1) * stride;
      ml[u] = *reinterpret_cast<const float2 *>(ps + kQT * kHD + 2 * r);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[u][e] = reinterpret_cast<const float4v *>(ps + r * kHD + d0)[e];
    }
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (!(s0 + u < ns && ml[u].y > 0.0f)) continue;
      const float f = expf(ml[u].x - M);
      L += f * ml[u].y;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int c = 0; c < 4; ++c) o[e][c] += f * v[u][e][c];
    }
  }
  const float inv = 1.0f / L;
  const int t = row0 + r;
  const float4v *gate = reinterpret_cast<const float4v *>(proj + int64_t(t) * ldp + h * 2 * kHD + kHD + d0);
  const int qw = hq * kHD;
  typedef _Float16 half8v_ __attribute__((ext_vector_type(8)));
  half8v_ hi[2], lo[2];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float4v g = gate[e];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      _Float16 hh, ll;
      split_f16(o[e][c] * inv * sigmoidf_(g[c]), hh, ll);
      hi[e >> 1][4 * (e & 1) + c] = hh;
      lo[e >> 1][4 * (e & 1) + c] = ll;
    }
  }
  const int64_t at = int64_t(t) * qw + h * kHD + d0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    reinterpret_cast<half8v_ *>(y + at)[k] = hi[k];
    if (ylo) reinterpret_cast<half8v_ *>(ylo + at)[k] = lo[k];
  }
}

}  // namespace

void launch_ot_delta_prep(const float *proj, int ldp, int T, const int32_t *tok_pos, const float *conv,
                          const float *alog, const float *dt, int nh, float *qk, float *vbuf, float *gb,
                          hipStream_t st) {
  LG_REQUIRE(T > 0 && nh > 0 && nh <= 32, "delta prep: bad shape T=%d nh=%d", T, nh);
  LG_REQUIRE(ldp % 4 == 0 && ldp >= 3 * nh * kLK + nh * kLK + 2 * nh, "delta prep: projection row %d too short", ldp);
  const size_t lds = size_t(2) * nh * kLK * sizeof(float);  // the q and k rows of one token
  const int per = (T + 7) / 8;
  hipLaunchKernelGGL(ot_delta_prep_kernel, dim3(8 * per), dim3(kPrepThreads), lds, st, proj, ldp, T, tok_pos, conv, alog, dt, nh,
                     qk, vbuf, gb);
  HIP_CHECK(hipGetLastError());
}

size_t ot_delta_chunk_floats(int T, int nseq, int nh) { return size_t(nseq + T / kDC + 1) * nh * kChunkFloats; }

void launch_ot_delta_scan(const float *qk, const float *vbuf, const float *gb, const int32_t *seq_row0,
                          const int32_t *seq_n, int nseq, int T, int max_n, int nh, float *chunk_ws, float *out,
                          hipStream_t st) {
  LG_REQUIRE(nseq > 0 && nseq <= 65535 && nh > 0 && nh <= 65535, "delta scan: bad shape nseq=%d nh=%d", nseq, nh);
  LG_REQUIRE(max_n > 0 && max_n <= T && chunk_ws, "delta scan: no tokens or no chunk workspace");
  const int maxch = (max_n + kDC - 1) / kDC;
  hipLaunchKernelGGL(ot_delta_chunk_kernel, dim3(maxch, nh, nseq), dim3(256), 0, st, qk, vbuf, gb, seq_row0, seq_n,
                     nh, chunk_ws);
  HIP_CHECK(hipGetLastError());
  const size_t lds = size_t(kStateLdsFloats) * sizeof(float);
  grant_lds(reinterpret_cast<const void *>(&ot_delta_state_kernel), lds);
  hipLaunchKernelGGL(ot_delta_state_kernel, dim3(nh, kLK / 16, nseq), dim3(kStateThreads), lds, st, qk, chunk_ws,
                     seq_row0, seq_n, nh, T, out);
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
  grant_lds(reinterpret_cast<const void *>(&ot_attn_part_kernel), size_t(kAttnLdsBytes));
  launch_timed(ot_attn_part_kernel, dim3(nitems, hq / 4), dim3(256), size_t(kAttnLdsBytes), st, Qb, Kb, proj, ldp, hq,
               hkv, it_row0, it_pos0, it_nq, it_klo, it_khi, part);
  HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(ot_attn_combine_kernel, dim3(ncomb, hq), dim3(256), 0, st, part, proj, ldp, hq, cb_row0, cb_nq,
                     cb_first, cb_n, y, ylo);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
