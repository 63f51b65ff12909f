// Decode GEMV (one token): y = x . W^T with dequantisation fused into the weight stream.
//
// HBM-bound: every weight byte is read once, 16 bytes per lane per load, coalesced along
// the row.  The input vector is staged once per workgroup in LDS ("planes" layout: plane i
// holds elements 4i..4i+3 of every 16-element chunk, so a wave's b128 reads are
// conflict-free), optionally through a fused RMSNorm.  Each wave owns whole rows and
// reduces them with cross-lane shuffles; the epilogue adds bias / residual or applies SwiGLU.
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels.h"
#include "quant.h"

namespace lg {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Stage x (optionally RMS-normalised) into LDS.  Layout: for chunk size E (elements per
// lane load), float4 index (i * nchunk + c) holds elements c*E + 4i .. c*E + 4i + 3.
template <int E>
__device__ void stage_x(const float *__restrict__ x, int K, const float *__restrict__ norm_w,
                        float eps, float4 *xs, float *red) {
  const int t = threadIdx.x;
  float inv = 1.0f;
  if (norm_w) {
    float ss = 0.0f;
    for (int k = t; k < K; k += kThreads) ss += x[k] * x[k];
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    inv = 1.0f / sqrtf(tot / float(K) + eps);
  }
  const int nchunk = K / E;
  for (int q = t; q < K / 4; q += kThreads) {
    const int c = q / (E / 4), i = q % (E / 4);
    float4 v = reinterpret_cast<const float4 *>(x)[q];
    if (norm_w) {
      const float4 w = reinterpret_cast<const float4 *>(norm_w)[q];
      v.x = v.x * inv * w.x;
      v.y = v.y * inv * w.y;
      v.z = v.z * inv * w.z;
      v.w = v.w * inv * w.w;
    }
    xs[i * nchunk + c] = v;
  }
  __syncthreads();
}

__device__ __forceinline__ float dot16_i8(uint4 c, const float4 *xs, int plane_stride, int ch) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 xv = xs[i * plane_stride + ch];
    const uint32_t word = w[i];
    s += float(int8_t(word)) * xv.x;
    s += float(int8_t(word >> 8)) * xv.y;
    s += float(int8_t(word >> 16)) * xv.z;
    s += float(int8_t(word >> 24)) * xv.w;
  }
  return s;
}

__device__ __forceinline__ float dot8_f16(uint4 c, const float4 *xs, int plane_stride, int ch) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 xv = xs[i * plane_stride + ch];
    const _Float16 *h0 = reinterpret_cast<const _Float16 *>(&w[2 * i]);
    const _Float16 *h1 = reinterpret_cast<const _Float16 *>(&w[2 * i + 1]);
    s += float(h0[0]) * xv.x;
    s += float(h0[1]) * xv.y;
    s += float(h1[0]) * xv.z;
    s += float(h1[1]) * xv.w;
  }
  return s;
}

// Elements per lane load for each kind (x staging chunk size).
template <uint32_t KIND>
constexpr int chunk_elems() { return KIND == LG_F16 ? 8 : 16; }

// Scale of chunk ch of row n (Q8_0: per 32-element block, Q6_K: per 16).
template <uint32_t KIND>
__device__ __forceinline__ float chunk_scale(const DevMatrix &W, int64_t n, int ch) {
  if constexpr (KIND == LG_Q8_0)  // hardware f16 -> f32: exact for every finite scale and infinity
    return float(static_cast<const _Float16 *>(W.s)[n * (W.cols / 32) + ch / 2]);
  else if constexpr (KIND == LG_Q6_K) return static_cast<const float *>(W.s)[n * (W.cols / 16) + ch];
  else return 1.0f;
}

// Each wave owns R outputs (RPO weight rows each: 2 for SwiGLU's gate|up).  All weight loads of
// a chunk group are issued before the input vector is staged, so the x/RMSNorm prologue
// overlaps the HBM reads.  Chunk c of a lane covers chunk index g*64*CPL + c*64 + lane.
template <uint32_t KIND, int EPI, int R, int CPL>
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
  typedef float svec __attribute__((ext_vector_type(NR * CPL)));
  typedef float avec __attribute__((ext_vector_type(NR)));
  const int K = W.cols, nchunk = K / E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * (kThreads / 64) + wave) * R;
  const int f = W.rows / 2;
  const uint4 *q = static_cast<const uint4 *>(W.q);
  const int64_t row_chunks = int64_t(K) * (KIND == LG_F16 ? 2 : 1) / 16;  // uint4 per weight row
  wvec w;
  svec sc;
  avec acc;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  const int ngroups = (nchunk + 64 * CPL - 1) / (64 * CPL);
  for (int g = 0; g < ngroups; ++g) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int o = min(o0 + r / RPO, outputs - 1);  // clamped rows are never stored
      const int64_t n = (r % RPO) ? f + o : o;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = g * 64 * CPL + c * 64 + lane;
        const int i = r * CPL + c;
        uint4 v = make_uint4(0, 0, 0, 0);
        float s = 0.0f;
        if (ch < nchunk) {
          v = q[n * row_chunks + ch];
          s = chunk_scale<KIND>(W, n, ch);
        }
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        sc[i] = s;
      }
    }
    if (g == 0) stage_x<E>(x, K, norm_w, eps, xs, red);  // every wave reaches this barrier
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
          const int i = r * CPL + c;
          const uint32_t wd[4] = {w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
          float d = 0.0f;
          if constexpr (KIND == LG_F16) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const _Float16 *h0 = reinterpret_cast<const _Float16 *>(&wd[2 * p]);
              const _Float16 *h1 = reinterpret_cast<const _Float16 *>(&wd[2 * p + 1]);
              d += float(h0[0]) * xv[p].x + float(h0[1]) * xv[p].y + float(h1[0]) * xv[p].z +
                   float(h1[1]) * xv[p].w;
            }
            acc[r] += d;
          } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const uint32_t word = wd[p];
              d += float(int8_t(word)) * xv[p].x + float(int8_t(word >> 8)) * xv[p].y +
                   float(int8_t(word >> 16)) * xv[p].z + float(int8_t(word >> 24)) * xv[p].w;
            }
            acc[r] += sc[i] * d;
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = o0 + r;
    if (EPI == int(Epi::SWIGLU)) {
      const float gsum = wave_sum(acc[r * 2]);
      const float usum = wave_sum(acc[r * 2 + 1]);
      if (lane == 0 && o < outputs) y[o] = silu(gsum) * usum;
    } else {
      const float v = wave_sum(acc[r]);
      if (lane == 0 && o < outputs) {
        if (EPI == int(Epi::ADD)) y[o] += v;
        else y[o] = v + (bias ? bias[o] : 0.0f);
      }
    }
  }
}

// Generic fallback (Q4_K and anything else): per-element decode, still one wave per row.
__device__ float weight_at_gemv(const DevMatrix &W, int64_t n, int64_t k) {
  const int64_t cols = W.cols;
  switch (W.kind) {
    case LG_F32: return static_cast<const float *>(W.q)[n * cols + k];
    case LG_Q4_K: {
      const uint8_t byte = static_cast<const uint8_t *>(W.q)[n * (cols / 2) + (k / 64) * 32 + (k % 32)];
      const uint32_t nib = (k % 64) >= 32 ? (byte >> 4) : (byte & 15u);
      const float2 ab = static_cast<const float2 *>(W.s)[n * (cols / 32) + k / 32];
      return ab.x * float(nib) - ab.y;
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
  stage_x<4>(x, W.cols, norm_w, eps, xs, red);  // E = 4: plain order
  const float *xf = reinterpret_cast<const float *>(xs);
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (o >= outputs) return;
  auto rowdot = [&](int n) {
    float s = 0.0f;
    for (int k = lane; k < W.cols; k += 64) s += weight_at_gemv(W, n, k) * xf[k];
    return wave_sum(s);
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

template <uint32_t KIND, int EPI, int R, int CPL>
void launch_rc(const float *x, const DevMatrix &W, float *y, const float *bias, const float *norm_w, float eps,
               int outputs, hipStream_t st) {
  const int per_block = (kThreads / 64) * R;
  const dim3 grid((outputs + per_block - 1) / per_block), block(kThreads);
  const size_t lds = size_t(W.cols) * sizeof(float);
  hipLaunchKernelGGL((gemv_kernel<KIND, EPI, R, CPL>), grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
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
  // rows per wave: as many as keep >= 512 workgroups (two per CU) in the grid
  const int r = outputs >= 4 * 4 * 512 ? 4 : outputs >= 4 * 2 * 512 ? 2 : 1;
  switch (r) {
    case 4: launch_r<KIND, EPI, 4>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
    case 2: launch_r<KIND, EPI, 2>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
    default: launch_r<KIND, EPI, 1>(cpl, x, W, y, bias, norm_w, eps, outputs, st); break;
  }
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

void launch_gemv(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                 const float *norm_w, float eps, hipStream_t st) {
  LG_REQUIRE(W.rows > 0 && W.cols > 0, "gemv: empty matrix");
  LG_REQUIRE(W.cols % 16 == 0, "gemv: K=%d must be a multiple of 16", W.cols);
  LG_REQUIRE(size_t(W.cols) * 4 <= 64 * 1024, "gemv: K=%d exceeds the 64 KiB LDS stage", W.cols);
  if (epi == Epi::SWIGLU) LG_REQUIRE(W.rows % 2 == 0, "gemv: gate|up needs an even row count");
  switch (W.kind) {
    case LG_Q8_0: launch_gemv_kind<LG_Q8_0>(x, W, epi, y, bias, norm_w, eps, st); break;
    case LG_Q6_K: launch_gemv_kind<LG_Q6_K>(x, W, epi, y, bias, norm_w, eps, st); break;
    case LG_F16: launch_gemv_kind<LG_F16>(x, W, epi, y, bias, norm_w, eps, st); break;
    default: {
      const int outputs = epi == Epi::SWIGLU ? W.rows / 2 : W.rows;
      const dim3 grid((outputs + 3) / 4), block(kThreads);
      const size_t lds = size_t(W.cols) * sizeof(float);
      switch (epi) {
        case Epi::F32:
          hipLaunchKernelGGL(gemv_generic_kernel<0>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        case Epi::ADD:
          hipLaunchKernelGGL(gemv_generic_kernel<1>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        case Epi::SWIGLU:
          hipLaunchKernelGGL(gemv_generic_kernel<3>, grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
          break;
        default: fail(LG_ERR_UNSUPPORTED, "gemv: f16 epilogue not supported");
      }
    }
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
