// Decode GEMV (one token): y = x . W^T with dequantisation fused into the weight stream.
//
// HBM-bound: every weight byte is read once, 16 bytes per lane per load, coalesced along
// the row.  The input vector is staged once per workgroup in LDS ("planes" layout: plane i
// holds elements 4i..4i+3 of every 16-element chunk, so a wave's b128 reads are
// conflict-free), optionally through a fused RMSNorm.  Each wave owns whole rows and
// reduces them with cross-lane shuffles; the epilogue adds bias / residual or applies SwiGLU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"
#include "kernels.h"
#include "quant.h"
#include "wave.h"

namespace lg {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_dpp(v); }

// Stage x (times the RMSNorm weight when norm_w is set) into LDS and return the RMSNorm factor
// 1/sqrt(mean(x^2) + eps) (1 without a norm), which the caller applies to its finished row sums:
// y = inv * sum_k W[n][k] * (x[k] * w[k]).  Layout: for chunk size E (elements per lane load),
// float4 index (i * nchunk + c) holds elements c*E + 4i .. c*E + 4i + 3.  This form serves K
// beyond the register prologue of gemv_kernel (two float4 of x per thread per round trip).
template <int E>
__device__ float stage_x(const float *__restrict__ x, int K, const float *__restrict__ norm_w,
                         float eps, float4 *xs, float *red) {
  constexpr int B = 2;
  const int t = threadIdx.x, nq = K / 4, nchunk = K / E;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 *w4 = reinterpret_cast<const float4 *>(norm_w);
  float ss = 0.0f;
  for (int q0 = 0; q0 < nq; q0 += B * kThreads) {
    float4 v[B], w[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int q = q0 + j * kThreads + t;
      v[j] = q < nq ? x4[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (norm_w) w[j] = q < nq ? w4[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int q = q0 + j * kThreads + t;
      if (q >= nq) continue;
      if (norm_w) {
        ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
        v[j].x *= w[j].x;
        v[j].y *= w[j].y;
        v[j].z *= w[j].z;
        v[j].w *= w[j].w;
      }
      const int c = q / (E / 4), i = q % (E / 4);
      xs[i * nchunk + c] = v[j];
    }
  }
  if (norm_w) {
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
  }
  __syncthreads();
  if (!norm_w) return 1.0f;
  const float tot = red[0] + red[1] + red[2] + red[3];
  return 1.0f / sqrtf(tot / float(K) + eps);
}

// Elements per lane load for each kind (x staging chunk size).
template <uint32_t KIND>
constexpr int chunk_elems() { return KIND == LG_F16 ? 8 : 16; }

// Scale of chunk ch of row n (Q8_0: per 32-element block, Q6_K: per 16), as stored: the load is
// kept apart from its f16 -> f32 conversion so that no load waits on an earlier one.
template <uint32_t KIND>
__device__ __forceinline__ uint32_t chunk_scale_bits(const DevMatrix &W, int64_t n, int ch) {
  if constexpr (KIND == LG_Q8_0)
    return static_cast<const uint16_t *>(W.s)[n * (W.cols / 32) + ch / 2];
  else if constexpr (KIND == LG_Q6_K) return static_cast<const uint32_t *>(W.s)[n * (W.cols / 16) + ch];
  else return 0u;
}

template <uint32_t KIND>
__device__ __forceinline__ float scale_value(uint32_t bits) {
  if constexpr (KIND == LG_Q8_0)  // hardware f16 -> f32: exact for every finite scale and infinity
    return float(__builtin_bit_cast(_Float16, uint16_t(bits)));
  else return __builtin_bit_cast(float, bits);
}

// x (and the RMSNorm weight) for up to XQ float4 per thread, loaded before the weight stream so
// that the LDS stage waits only for these (vector loads return in issue order).
template <int XQ>
__device__ __forceinline__ void load_x_regs(const float *__restrict__ x, const float *__restrict__ norm_w, int nq,
                                            float4 (&v)[XQ], float4 (&w)[XQ]) {
  // clamped indices instead of predicated loads: no branch separates a load from its use, and
  // entries past nq are never stored (store_x_regs)
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll
  for (int j = 0; j < XQ; ++j) v[j] = x4[min(j * kThreads + int(threadIdx.x), nq - 1)];
  if (norm_w) {
    const float4 *w4 = reinterpret_cast<const float4 *>(norm_w);
#pragma unroll
    for (int j = 0; j < XQ; ++j) w[j] = w4[min(j * kThreads + int(threadIdx.x), nq - 1)];
  }
}

// Store the registers of load_x_regs into the LDS planes layout of stage_x and return the
// RMSNorm factor (1 without a norm).  Ends with a workgroup barrier.
template <int E, int XQ>
__device__ float store_x_regs(const float4 (&v)[XQ], const float4 (&w)[XQ], bool norm, int K, float eps,
                              float4 *xs, float *red) {
  const int t = threadIdx.x, nq = K / 4, nchunk = K / E;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < XQ; ++j) {
    const int q = j * kThreads + t;
    if (q >= nq) continue;
    float4 u = v[j];
    if (norm) {
      ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
      u.x *= w[j].x;
      u.y *= w[j].y;
      u.z *= w[j].z;
      u.w *= w[j].w;
    }
    xs[(q % (E / 4)) * nchunk + q / (E / 4)] = u;
  }
  if (norm) {
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
  }
  __syncthreads();
  if (!norm) return 1.0f;
  return 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / float(K) + eps);
}

// Each wave owns R outputs (RPO weight rows each: 2 for SwiGLU's gate|up).  Issue order: the
// input vector x (L2-resident, small), then every weight load of the chunk group, chunk-major so
// the dot products below consume loads in the order they return; the x stage into LDS waits
// only for x.  Chunk c of a lane covers chunk index g*64*CPL + c*64 + lane.
template <uint32_t KIND, int EPI, int R, int CPL, bool BIGK>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const float *__restrict__ x, DevMatrix W,
                                                        float *__restrict__ y,
                                                        const float *__restrict__ bias,
                                                        const float *__restrict__ norm_w, float eps,
                                                        int outputs) {
  extern __shared__ float4 xs[];
  __shared__ float red[4];
  constexpr int E = chunk_elems<KIND>();
  constexpr int RPO = EPI == int(Epi::SWIGLU) ? 2 : 1;
  constexpr int NR = R * RPO;
  typedef uint32_t wvec __attribute__((ext_vector_type(4 * NR * CPL)));
  typedef uint32_t svec __attribute__((ext_vector_type(NR * CPL)));
  typedef float avec __attribute__((ext_vector_type(NR)));
  const int K = W.cols, nchunk = K / E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * (kThreads / 64) + wave) * R;
  const int f = W.rows / 2;
  const uint4 *q = static_cast<const uint4 *>(W.q);
  const int64_t row_chunks = int64_t(K) * (KIND == LG_F16 ? 2 : 1) / 16;  // uint4 per weight row
  // without BIGK one chunk group covers K (K <= 64*CPL*E <= 1024*CPL), so x fits in XQ = CPL
  // prologue registers per thread; BIGK stages x into LDS after the first group's weight loads
  constexpr int XQ = BIGK ? 1 : CPL;
  float4 xr[XQ], nr[XQ];
  if constexpr (!BIGK) load_x_regs(x, norm_w, K / 4, xr, nr);
  // the epilogue's other operand (the residual row for ADD, the bias for F32) loaded with x, ahead of
  // the weights, so the store at the end waits on no further memory round trip; the index is kept in
  // a vector register so each lane issues the (uniform) load itself
  float ep[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int oi = min(o0 + r, outputs - 1);
    asm volatile("" : "+v"(oi));
    ep[r] = 0.0f;
    if constexpr (EPI == int(Epi::ADD)) ep[r] = y[oi];
    else if constexpr (EPI == int(Epi::F32)) ep[r] = bias ? bias[oi] : 0.0f;
  }
  wvec w;
  svec sc;
  avec acc;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  const int ngroups = (nchunk + 64 * CPL - 1) / (64 * CPL);
  float inv = 1.0f;
  for (int g = 0; g < ngroups; ++g) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = g * 64 * CPL + c * 64 + lane;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int o = min(o0 + r / RPO, outputs - 1);  // clamped rows are never stored
        const int64_t n = (r % RPO) ? f + o : o;
        const int i = c * NR + r;
        const int chc = min(ch, nchunk - 1);  // lanes past the row load a valid chunk and skip it below
        const uint4 v = q[n * row_chunks + chc];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        sc[i] = chunk_scale_bits<KIND>(W, n, chc);
      }
    }
    if (g == 0) {  // every wave reaches this barrier
      if constexpr (BIGK) inv = stage_x<E>(x, K, norm_w, eps, xs, red);
      else inv = store_x_regs<E, XQ>(xr, nr, norm_w != nullptr, K, eps, xs, red);
    }
    // each x chunk is read from LDS once and used for all NR rows of the wave
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = g * 64 * CPL + c * 64 + lane;
      if (ch < nchunk) {
        float4 xv[E / 4];
#pragma unroll
        for (int p = 0; p < E / 4; ++p) xv[p] = xs[p * nchunk + ch];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int i = c * NR + r;
          const uint32_t wd[4] = {w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
          float d0 = 0.0f, d1 = 0.0f;  // two FMA chains
          if constexpr (KIND == LG_F16) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const _Float16 *h0 = reinterpret_cast<const _Float16 *>(&wd[2 * p]);
              const _Float16 *h1 = reinterpret_cast<const _Float16 *>(&wd[2 * p + 1]);
              d0 = fmaf(float(h0[0]), xv[p].x, d0);
              d1 = fmaf(float(h0[1]), xv[p].y, d1);
              d0 = fmaf(float(h1[0]), xv[p].z, d0);
              d1 = fmaf(float(h1[1]), xv[p].w, d1);
            }
            acc[r] += d0 + d1;
          } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const uint32_t word = wd[p];
              d0 = fmaf(float(int8_t(word)), xv[p].x, d0);
              d1 = fmaf(float(int8_t(word >> 8)), xv[p].y, d1);
              d0 = fmaf(float(int8_t(word >> 16)), xv[p].z, d0);
              d1 = fmaf(float(int8_t(word >> 24)), xv[p].w, d1);
            }
            acc[r] = fmaf(scale_value<KIND>(sc[i]), d0 + d1, acc[r]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = o0 + r;
    if (EPI == int(Epi::SWIGLU)) {
      const float gsum = wave_sum(acc[r * 2]) * inv;
      const float usum = wave_sum(acc[r * 2 + 1]) * inv;
      if (lane == 0 && o < outputs) y[o] = silu(gsum) * usum;
    } else {
      const float v = wave_sum(acc[r]) * inv;
      if (lane == 0 && o < outputs) {
        if (EPI == int(Epi::ADD)) y[o] = ep[r] + v;
        else y[o] = v + ep[r];
      }
    }
  }
}

// ---------------------------------------------------------------- Q4_K
// Q4_K rows as repacked (quant.h): nibble bytes [rows][K/2], byte (k/64)*32 + k%32 holding element k in
// its low nibble when k%64 < 32 and in its high nibble otherwise, and float2 (A, B) = (d*sc, dmin*m)
// per 32-element sub-block, w = A*q - B (src/gguf.rs:281-307).  A lane's 16-byte word w of a row
// covers group g = w/2 of 64 elements, half h = w%2: its low nibbles are elements 64g + 16h + 0..15 (of
// sub-block 2g), its high nibbles elements 64g + 32 + 16h + 0..15 (of sub-block 2g + 1).  Over those 16
// elements of each sub-block the lane adds  A * sum(x*q) - B * sum(x)  (two f32 FMA chains over the
// nibbles, then two FMAs per sub-block against the staged chunk sums of x); the other half of each
// sub-block is the neighbouring lane's word.

// The register prologue's x (times the RMSNorm weight) into the E = 16 planes layout of stage_x, and the
// sum of each 16-element chunk of the staged values into xsum[K/16] (four float4 of a chunk sit in four
// consecutive lanes: a quad DPP sum, the same order for every chunk).  Ends with a workgroup barrier and
// returns the RMSNorm factor (1 without a norm).
template <int XQ>
__device__ float store_x_regs_sums(const float4 (&v)[XQ], const float4 (&w)[XQ], bool norm, int K, float eps,
                                   float4 *xs, float *xsum, float *red) {
  const int t = threadIdx.x, nq = K / 4, nchunk = K / 16;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < XQ; ++j) {
    const int q = j * kThreads + t;  // quads of lanes are whole chunks, inside or past K together
    const bool in = q < nq;
    float4 u = in ? v[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (norm) {
      ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
      if (in) {
        u.x *= w[j].x;
        u.y *= w[j].y;
        u.z *= w[j].z;
        u.w *= w[j].w;
      }
    }
    float s = ((u.x + u.y) + u.z) + u.w;
    s += dpp_move<0xB1>(s);
    s += dpp_move<0x4E>(s);
    if (in) {
      xs[(q % 4) * nchunk + q / 4] = u;
      if ((q & 3) == 0) xsum[q / 4] = s;
    }
  }
  if (norm) {
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
  }
  __syncthreads();
  if (!norm) return 1.0f;
  return 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / float(K) + eps);
}

// stage_x<16> with the chunk sums of store_x_regs_sums, for K beyond the register prologue.
__device__ float stage_x_sums(const float *__restrict__ x, int K, const float *__restrict__ norm_w, float eps,
                              float4 *xs, float *xsum, float *red) {
  constexpr int B = 2;
  const int t = threadIdx.x, nq = K / 4, nchunk = K / 16;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 *w4 = reinterpret_cast<const float4 *>(norm_w);
  float ss = 0.0f;
  for (int q0 = 0; q0 < nq; q0 += B * kThreads) {
    float4 v[B], w[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int q = min(q0 + j * kThreads + t, nq - 1);
      v[j] = x4[q];
      if (norm_w) w[j] = w4[q];
    }
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int q = q0 + j * kThreads + t;
      const bool in = q < nq;
      float4 u = in ? v[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (norm_w) {
        ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
        if (in) {
          u.x *= w[j].x;
          u.y *= w[j].y;
          u.z *= w[j].z;
          u.w *= w[j].w;
        }
      }
      float s = ((u.x + u.y) + u.z) + u.w;
      s += dpp_move<0xB1>(s);
      s += dpp_move<0x4E>(s);
      if (in) {
        xs[(q % 4) * nchunk + q / 4] = u;
        if ((q & 3) == 0) xsum[q / 4] = s;
      }
    }
  }
  if (norm_w) {
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
  }
  __syncthreads();
  if (!norm_w) return 1.0f;
  return 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / float(K) + eps);
}

// Dot of the 16 nibbles of one half of word `wd` (low nibbles when HI is false) with the 16 staged x
// values xv[0..3] (float4 p holds elements 4p..4p+3 of the range), two FMA chains.
template <bool HI>
__device__ __forceinline__ float q4_dot16(const uint32_t (&wd)[4], const float4 (&xv)[4]) {
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t n = (HI ? wd[p] >> 4 : wd[p]) & 0x0F0F0F0Fu;  // byte e holds the nibble of element 4p + e
    d0 = fmaf(float(n & 0xFFu), xv[p].x, d0);
    d1 = fmaf(float((n >> 8) & 0xFFu), xv[p].y, d1);
    d0 = fmaf(float((n >> 16) & 0xFFu), xv[p].z, d0);
    d1 = fmaf(float(n >> 24), xv[p].w, d1);
  }
  return d0 + d1;
}

// Each wave owns R outputs (RPO rows each: 2 for SwiGLU's gate|up), as gemv_kernel; the weight words
// of a chunk group and their (A, B) pairs (one float4: both sub-blocks of the word) are loaded before
// the x stage waits for anything.  Word c of a lane is index g*64*CPL + c*64 + lane of the row.
template <int EPI, int R, int CPL, bool BIGK>
__global__ __launch_bounds__(kThreads) void gemv_q4k_kernel(const float *__restrict__ x, DevMatrix W,
                                                            float *__restrict__ y, const float *__restrict__ bias,
                                                            const float *__restrict__ norm_w, float eps,
                                                            int outputs) {
  extern __shared__ float4 xs[];
  __shared__ float red[4];
  constexpr int RPO = EPI == int(Epi::SWIGLU) ? 2 : 1;
  constexpr int NR = R * RPO;
  typedef uint32_t wvec __attribute__((ext_vector_type(4 * NR * CPL)));
  typedef float avec __attribute__((ext_vector_type(NR)));
  const int K = W.cols, nwords = K / 32, nc16 = K / 16;
  float *xsum = reinterpret_cast<float *>(xs + K / 4);  // K/16 chunk sums after the x planes
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * (kThreads / 64) + wave) * R;
  const int f = W.rows / 2;
  const uint4 *q = static_cast<const uint4 *>(W.q);
  const float4 *ab = static_cast<const float4 *>(W.s);  // (A, B) of sub-blocks 2g and 2g + 1
  constexpr int XQ = BIGK ? 1 : CPL * 2;  // float4 of x per thread without BIGK: K <= 2048 * CPL
  float4 xr[XQ], nr[XQ];
  if constexpr (!BIGK) load_x_regs(x, norm_w, K / 4, xr, nr);
  float ep[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int oi = min(o0 + r, outputs - 1);
    asm volatile("" : "+v"(oi));
    ep[r] = 0.0f;
    if constexpr (EPI == int(Epi::ADD)) ep[r] = y[oi];
    else if constexpr (EPI == int(Epi::F32)) ep[r] = bias ? bias[oi] : 0.0f;
  }
  wvec w;
  float4 sab[NR * CPL];
  avec acc;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  const int ngroups = (nwords + 64 * CPL - 1) / (64 * CPL);
  float inv = 1.0f;
  for (int g = 0; g < ngroups; ++g) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int wi = min(g * 64 * CPL + c * 64 + lane, nwords - 1);  // past the row: a valid word, skipped
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int o = min(o0 + r / RPO, outputs - 1);  // clamped rows are never stored
        const int64_t n = (r % RPO) ? f + o : o;
        const int i = c * NR + r;
        const uint4 v = q[n * nwords + wi];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        sab[i] = ab[n * (nwords / 2) + wi / 2];
      }
    }
    if (g == 0) {  // every wave reaches this barrier
      if constexpr (BIGK) inv = stage_x_sums(x, K, norm_w, eps, xs, xsum, red);
      else inv = store_x_regs_sums<XQ>(xr, nr, norm_w != nullptr, K, eps, xs, xsum, red);
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int wi = g * 64 * CPL + c * 64 + lane;
      if (wi < nwords) {
        const int c0 = (wi >> 1) * 4 + (wi & 1), c1 = c0 + 2;  // 16-element chunks of the two halves
        float4 xl[4], xh[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          xl[p] = xs[p * nc16 + c0];
          xh[p] = xs[p * nc16 + c1];
        }
        const float s0 = xsum[c0], s1 = xsum[c1];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int i = c * NR + r;
          const uint32_t wd[4] = {w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
          const float dl = q4_dot16<false>(wd, xl), dh = q4_dot16<true>(wd, xh);
          float a = acc[r];
          a = fmaf(sab[i].x, dl, a);
          a = fmaf(-sab[i].y, s0, a);
          a = fmaf(sab[i].z, dh, a);
          a = fmaf(-sab[i].w, s1, a);
          acc[r] = a;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = o0 + r;
    if (EPI == int(Epi::SWIGLU)) {
      const float gsum = wave_sum(acc[r * 2]) * inv;
      const float usum = wave_sum(acc[r * 2 + 1]) * inv;
      if (lane == 0 && o < outputs) y[o] = silu(gsum) * usum;
    } else {
      const float v = wave_sum(acc[r]) * inv;
      if (lane == 0 && o < outputs) {
        if (EPI == int(Epi::ADD)) y[o] = ep[r] + v;
        else y[o] = v + ep[r];
      }
    }
  }
}

// Generic fallback (F32 and anything else): per-element decode, still one wave per row.
__device__ float weight_at_gemv(const DevMatrix &W, int64_t n, int64_t k) {
  const int64_t cols = W.cols;
  switch (W.kind) {
    case LG_F32: return static_cast<const float *>(W.q)[n * cols + k];
    case LG_Q4_K: {
      const uint8_t byte = static_cast<const uint8_t *>(W.q)[n * (cols / 2) + (k / 64) * 32 + (k % 32)];
      const uint32_t nib = (k % 64) >= 32 ? (byte >> 4) : (byte & 15u);
      const float2 ab = static_cast<const float2 *>(W.s)[n * (cols / 32) + k / 32];
      return kq4_weight(ab.x, nib, ab.y);
    }
  }
  return 0.0f;
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemv_generic_kernel(const float *__restrict__ x, DevMatrix W,
                                                                float *__restrict__ y,
                                                                const float *__restrict__ bias,
                                                                const float *__restrict__ norm_w,
                                                                float eps, int outputs) {
  extern __shared__ float4 xs[];
  __shared__ float red[4];
  const float inv = stage_x<4>(x, W.cols, norm_w, eps, xs, red);  // E = 4: plain order
  const float *xf = reinterpret_cast<const float *>(xs);
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (o >= outputs) return;
  auto rowdot = [&](int n) {
    float s = 0.0f;
    for (int k = lane; k < W.cols; k += 64) s += weight_at_gemv(W, n, k) * xf[k];
    return wave_sum(s) * inv;
  };
  if (EPI == int(Epi::SWIGLU)) {
    const float g = rowdot(o), u = rowdot(W.rows / 2 + o);
    if (lane == 0) y[o] = silu(g) * u;
  } else {
    const float v = rowdot(o);
    if (lane == 0) {
      if (EPI == int(Epi::ADD)) y[o] += v;
      else y[o] = v + (bias ? bias[o] : 0.0f);
    }
  }
}

// Largest LDS block a workgroup may take on the current device (160 KiB on gfx950).
size_t lds_limit() {
  static std::once_flag once;
  static int bytes = 0;
  std::call_once(once, [] {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    HIP_CHECK(hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
  });
  return size_t(bytes);
}

// Launch with `lds` bytes of dynamic LDS.
template <typename F, typename... Args>
void launch_lds(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
  grant_lds(reinterpret_cast<const void *>(kernel), lds);
  launch_timed(kernel, grid, block, lds, st, args...);
}

template <uint32_t KIND, int EPI, int R, int CPL>
void launch_rc(const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w, float eps,
               int outputs, hipStream_t st) {
  const int per_block = (kThreads / 64) * R;
  const dim3 grid((outputs + per_block - 1) / per_block), block(kThreads);
  const size_t lds = size_t(W.cols) * sizeof(float);
  const bool bigk = W.cols / chunk_elems<KIND>() > 64 * CPL;
  if (bigk)
    launch_lds(gemv_kernel<KIND, EPI, R, CPL, true>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
  else
    launch_lds(gemv_kernel<KIND, EPI, R, CPL, false>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
}

template <uint32_t KIND, int EPI, int R>
void launch_r(int cpl, const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w,
              float eps, int outputs, hipStream_t st) {
  switch (cpl) {
    case 2: launch_rc<KIND, EPI, R, 2>(x, W, y, bias, norm_w, eps, outputs, st); break;
    case 4: launch_rc<KIND, EPI, R, 4>(x, W, y, bias, norm_w, eps, outputs, st); break;
    default: launch_rc<KIND, EPI, R, 8>(x, W, y, bias, norm_w, eps, outputs, st); break;
  }
}

template <uint32_t KIND, int EPI>
void launch_e(const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w, float eps,
              hipStream_t st) {
  const int outputs = EPI == int(Epi::SWIGLU) ? W.rows / 2 : W.rows;
  const int nchunk = W.cols / chunk_elems<KIND>();
  const int cpl = nchunk <= 128 ? 2 : nchunk <= 256 ? 4 : 8;
  // rows per wave: as many as keep >= 512 workgroups (two per CU) in the grid; rows longer than one
  // chunk group (BIGK) take at least two from 2048 outputs (7B down projection, Q6_K, K 18944: 25.5 ->
  // 21.0 us; the d2048 shapes keep the rule, measured best at each)
  int r = outputs >= 4 * 4 * 512 ? 4 : outputs >= 4 * 2 * 512 ? 2 : 1;
  if (nchunk > 64 * cpl && r == 1 && outputs >= 2048) r = 2;
  switch (r) {
    case 4: launch_r<KIND, EPI, 4>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
    case 2: launch_r<KIND, EPI, 2>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
    default: launch_r<KIND, EPI, 1>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
  }
}

// Q4_K: two words per lane and chunk group (four past 4096 columns), at most eight words' registers
// (weights and scale pairs) per lane; rows per wave measured at the 7B decode shapes (K 3584): one
// for SwiGLU's gate|up (two: 7% slower), two from 2048 outputs (o, q|k: 5% faster than one).
template <int EPI, int R, int CPL>
void launch_q4k_rc(const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w, float eps,
                   int outputs, hipStream_t st) {
  static_assert(R * (EPI == int(Epi::SWIGLU) ? 2 : 1) * CPL <= 8, "Q4_K GEMV register budget");
  const int per_block = (kThreads / 64) * R;
  const dim3 grid((outputs + per_block - 1) / per_block), block(kThreads);
  const size_t lds = size_t(W.cols) * sizeof(float) + size_t(W.cols / 16) * sizeof(float);
  if (W.cols / 32 > 64 * CPL)
    launch_lds(gemv_q4k_kernel<EPI, R, CPL, true>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
  else
    launch_lds(gemv_q4k_kernel<EPI, R, CPL, false>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
}

template <int EPI>
void launch_q4k_e(const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w, float eps,
                  hipStream_t st) {
  const bool glu = EPI == int(Epi::SWIGLU);
  const int outputs = glu ? W.rows / 2 : W.rows;
  const bool wide = W.cols / 32 > 128;
  int r = glu ? 1 : outputs >= 4 * 4 * 1024 ? 4 : outputs >= 2048 ? 2 : 1;
  if (wide) r = std::min(r, 2);
  if (wide) {
    if constexpr (EPI != int(Epi::SWIGLU)) {
      if (r == 2) return launch_q4k_rc<EPI, 2, 4>(x, W, y, bias, norm_w, eps, outputs, st);
    }
    return launch_q4k_rc<EPI, 1, 4>(x, W, y, bias, norm_w, eps, outputs, st);
  }
  if constexpr (EPI != int(Epi::SWIGLU)) {
    if (r == 4) return launch_q4k_rc<EPI, 4, 2>(x, W, y, bias, norm_w, eps, outputs, st);
  }
  if (r == 2) return launch_q4k_rc<EPI, 2, 2>(x, W, y, bias, norm_w, eps, outputs, st);
  return launch_q4k_rc<EPI, 1, 2>(x, W, y, bias, norm_w, eps, outputs, st);
}

template <uint32_t KIND>
void launch_gemv_kind(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                      const float *norm_w, float eps, hipStream_t st) {
  switch (epi) {
    case Epi::F32: launch_e<KIND, 0>(x, W, y, bias, norm_w, eps, st); break;
    case Epi::ADD: launch_e<KIND, 1>(x, W, y, bias, norm_w, eps, st); break;
    case Epi::SWIGLU: launch_e<KIND, 3>(x, W, y, bias, norm_w, eps, st); break;
    default: fail(LG_ERR_UNSUPPORTED, "gemv: f16 epilogue not supported");
  }
}

}  // namespace

// Raise `kernel`'s dynamic LDS limit on the current device to `lds` bytes when it passes the 64 KiB
// every kernel may take without asking.  The size granted so far is kept per (device, kernel) under
// a lock: engines on other threads launch the same kernels, and every GEMV instance has the same
// parameter list, so a counter per launcher template would be shared between kernels.
void grant_lds(const void *kernel, size_t lds) {
  if (lds <= 64 * 1024) return;
  static std::mutex mu;
  static std::map<std::pair<int, const void *>, size_t> granted;
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  size_t &g = granted[{dev, kernel}];
  if (lds > g) {
    HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    g = lds;
  }
}

void launch_gemv(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                 const float *norm_w, float eps, hipStream_t st) {
  LG_REQUIRE(W.rows > 0 && W.cols > 0, "gemv: empty matrix");
  LG_REQUIRE(W.cols % 16 == 0, "gemv: K=%d must be a multiple of 16", W.cols);
  LG_REQUIRE(size_t(W.cols) * 4 + 64 <= lds_limit(), "gemv: K=%d exceeds the %zu-byte LDS stage", W.cols, lds_limit());
  if (epi == Epi::SWIGLU) LG_REQUIRE(W.rows % 2 == 0, "gemv: gate|up needs an even row count");
  switch (W.kind) {
    case LG_Q8_0: launch_gemv_kind<LG_Q8_0>(x, W, epi, y, bias, norm_w, eps, st); break;
    case LG_Q6_K: launch_gemv_kind<LG_Q6_K>(x, W, epi, y, bias, norm_w, eps, st); break;
    case LG_F16: launch_gemv_kind<LG_F16>(x, W, epi, y, bias, norm_w, eps, st); break;
    case LG_Q4_K:
      LG_REQUIRE(W.cols % 256 == 0, "gemv: Q4_K rows of %d columns (whole 256-element super-blocks)", W.cols);
      LG_REQUIRE(size_t(W.cols) * 4 + size_t(W.cols / 16) * 4 + 64 <= lds_limit(),
                 "gemv: K=%d exceeds the %zu-byte LDS stage", W.cols, lds_limit());
      switch (epi) {
        case Epi::F32: launch_q4k_e<0>(x, W, y, bias, norm_w, eps, st); break;
        case Epi::ADD: launch_q4k_e<1>(x, W, y, bias, norm_w, eps, st); break;
        case Epi::SWIGLU: launch_q4k_e<3>(x, W, y, bias, norm_w, eps, st); break;
        default: fail(LG_ERR_UNSUPPORTED, "gemv: f16 epilogue not supported");
      }
      break;
    default: {
      const int outputs = epi == Epi::SWIGLU ? W.rows / 2 : W.rows;
      const dim3 grid((outputs + 3) / 4), block(kThreads);
      const size_t lds = size_t(W.cols) * sizeof(float);
      switch (epi) {
        case Epi::F32:
          launch_lds(gemv_generic_kernel<0>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        case Epi::ADD:
          launch_lds(gemv_generic_kernel<1>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        case Epi::SWIGLU:
          launch_lds(gemv_generic_kernel<3>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        default: fail(LG_ERR_UNSUPPORTED, "gemv: f16 epilogue not supported");
      }
    }
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
