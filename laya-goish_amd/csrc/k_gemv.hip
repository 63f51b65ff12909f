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
constexpr int kUnroll = 4;

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

// Partial dot product of weight row n with the staged x, this lane's chunks.
template <uint32_t KIND>
__device__ __forceinline__ float row_partial(const DevMatrix &W, int n, const float4 *xs, int lane) {
  const int K = W.cols;
  float acc = 0.0f;
  if constexpr (KIND == LG_Q8_0 || KIND == LG_Q6_K) {
    const int nchunk = K / 16;
    const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const int8_t *>(W.q) + int64_t(n) * K);
    for (int base = 0; base < nchunk; base += 64 * kUnroll) {
      uint4 c[kUnroll];
      float d[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int ch = base + u * 64 + lane;
        if (ch < nchunk) {
          c[u] = q[ch];
          if constexpr (KIND == LG_Q8_0)
            d[u] = half_bits(static_cast<const uint16_t *>(W.s)[int64_t(n) * (K / 32) + ch / 2]);
          else
            d[u] = static_cast<const float *>(W.s)[int64_t(n) * (K / 16) + ch];
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int ch = base + u * 64 + lane;
        if (ch < nchunk) acc += d[u] * dot16_i8(c[u], xs, nchunk, ch);
      }
    }
  } else if constexpr (KIND == LG_F16) {
    const int nchunk = K / 8;
    const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const _Float16 *>(W.q) + int64_t(n) * K);
    for (int base = 0; base < nchunk; base += 64 * kUnroll) {
      uint4 c[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int ch = base + u * 64 + lane;
        if (ch < nchunk) c[u] = q[ch];
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int ch = base + u * 64 + lane;
        if (ch < nchunk) acc += dot8_f16(c[u], xs, nchunk, ch);
      }
    }
  }
  return acc;
}

// Elements per lane load for each kind (x staging chunk size).
template <uint32_t KIND>
constexpr int chunk_elems() { return KIND == LG_F16 ? 8 : 16; }

template <uint32_t KIND, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const float *__restrict__ x, DevMatrix W,
                                                        float *__restrict__ y,
                                                        const float *__restrict__ bias,
                                                        const float *__restrict__ norm_w, float eps,
                                                        int outputs) {
  extern __shared__ float4 xs[];
  __shared__ float red[4];
  constexpr int E = chunk_elems<KIND>();
  stage_x<E>(x, W.cols, norm_w, eps, xs, red);
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (o >= outputs) return;
  if (EPI == int(Epi::SWIGLU)) {
    const int f = W.rows / 2;
    const float g = wave_sum(row_partial<KIND>(W, o, xs, lane));
    const float u = wave_sum(row_partial<KIND>(W, f + o, xs, lane));
    if (lane == 0) y[o] = silu(g) * u;
  } else {
    const float v = wave_sum(row_partial<KIND>(W, o, xs, lane));
    if (lane == 0) {
      if (EPI == int(Epi::ADD)) y[o] += v;
      else y[o] = v + (bias ? bias[o] : 0.0f);
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

template <uint32_t KIND>
void launch_gemv_kind(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                      const float *norm_w, float eps, hipStream_t st) {
  const int outputs = epi == Epi::SWIGLU ? W.rows / 2 : W.rows;
  const dim3 grid((outputs + 3) / 4), block(kThreads);
  const size_t lds = size_t(W.cols) * sizeof(float);
  switch (epi) {
    case Epi::F32:
      hipLaunchKernelGGL((gemv_kernel<KIND, 0>), grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
      break;
    case Epi::ADD:
      hipLaunchKernelGGL((gemv_kernel<KIND, 1>), grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
      break;
    case Epi::SWIGLU:
      hipLaunchKernelGGL((gemv_kernel<KIND, 3>), grid, block, lds, st, x, W, y, bias, norm_w, eps, outputs);
      break;
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
