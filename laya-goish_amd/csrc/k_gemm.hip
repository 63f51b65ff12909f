// Prefill GEMM for gfx950: C = A . W^T, A = activations (f16, [M][K] row-major),
// W = quantised/F16 weights dequantised to f16 in LDS, f32 accumulation on MFMA
// v_mfma_f32_32x32x16_f16, epilogue fused (bias, residual add, SwiGLU, f16 store).
//
// Tile 128 x 128 x 64, 256 threads = 4 wave64s in a 2 x 2 arrangement, each wave a
// 64 x 64 sub-tile = 2 x 2 MFMA blocks of 32 x 32.  Global loads for the next K tile are
// issued before the MFMAs of the current one (register double buffering).
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels.h"
#include "quant.h"

namespace lg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;  // LDS row stride (halves): 144 B keeps 16-lane b128 reads conflict-free

__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

// ---------------------------------------------------------------- B tile loaders
// Each loader fetches its share of a BN x BK weight tile into registers (fetch) and later
// dequantises into LDS rows (store).  `wrow` is the weight row for local row r.
template <uint32_t KIND>
struct BLoad;

template <>
struct BLoad<LG_F16> {
  uint4 v[4];
  __device__ void fetch(const DevMatrix &W, const int *wrow, int k0, int t) {
    const _Float16 *q = static_cast<const _Float16 *>(W.q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = t / 8 + 32 * i, c = (t % 8) * 8;
      v[i] = *reinterpret_cast<const uint4 *>(q + int64_t(wrow[i]) * W.cols + k0 + c);
    }
  }
  __device__ void store(_Float16 *Bs, int t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = t / 8 + 32 * i, c = (t % 8) * 8;
      *reinterpret_cast<uint4 *>(Bs + r * LDK + c) = v[i];
    }
  }
  __device__ static int row_of(int t, int i) { return t / 8 + 32 * i; }
  static constexpr int kRows = 4;
};

template <>
struct BLoad<LG_Q8_0> {
  uint4 c0, c1;
  uint32_t sb;
  __device__ void fetch(const DevMatrix &W, const int *wrow, int k0, int t) {
    const int part = t % 2;
    const int8_t *q = static_cast<const int8_t *>(W.q) + int64_t(wrow[0]) * W.cols + k0 + part * 32;
    c0 = *reinterpret_cast<const uint4 *>(q);
    c1 = *reinterpret_cast<const uint4 *>(q + 16);
    sb = static_cast<const uint16_t *>(W.s)[int64_t(wrow[0]) * (W.cols / 32) + k0 / 32 + part];
  }
  __device__ static void cvt16(uint4 c, _Float16 d, _Float16 *dst) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    half8 o0, o1;
    // f16(d) * code is the round-to-nearest f16 of the exact product (d*code is exact in f32)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = w[j / 4];
      o0[j] = _Float16(int8_t(word >> (8 * (j % 4)))) * d;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = w[2 + j / 4];
      o1[j] = _Float16(int8_t(word >> (8 * (j % 4)))) * d;
    }
    *reinterpret_cast<half8 *>(dst) = o0;
    *reinterpret_cast<half8 *>(dst + 8) = o1;
  }
  __device__ void store(_Float16 *Bs, int t) {
    const int r = t / 2, part = t % 2;
    const _Float16 d = __builtin_bit_cast(_Float16, uint16_t(sb));
    cvt16(c0, d, Bs + r * LDK + part * 32);
    cvt16(c1, d, Bs + r * LDK + part * 32 + 16);
  }
  __device__ static int row_of(int t, int) { return t / 2; }
  static constexpr int kRows = 1;
};

template <>
struct BLoad<LG_Q4_K> {
  uint4 c;
  float2 s0, s1;
  __device__ void fetch(const DevMatrix &W, const int *wrow, int k0, int t) {
    const int part = t % 2;
    const uint8_t *q = static_cast<const uint8_t *>(W.q) + int64_t(wrow[0]) * (W.cols / 2) + k0 / 2 + part * 16;
    c = *reinterpret_cast<const uint4 *>(q);
    const float2 *s = static_cast<const float2 *>(W.s) + int64_t(wrow[0]) * (W.cols / 32) + k0 / 32;
    s0 = s[0];
    s1 = s[1];
  }
  __device__ void store(_Float16 *Bs, int t) {
    const int r = t / 2, part = t % 2;
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    half8 lo0, lo1, hi0, hi1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t byte = (w[j / 4] >> (8 * (j % 4))) & 0xffu;
      const float l = s0.x * float(byte & 15u) - s0.y;
      const float h = s1.x * float(byte >> 4) - s1.y;
      if (j < 8) { lo0[j] = _Float16(l); hi0[j] = _Float16(h); }
      else { lo1[j - 8] = _Float16(l); hi1[j - 8] = _Float16(h); }
    }
    _Float16 *row = Bs + r * LDK;
    *reinterpret_cast<half8 *>(row + part * 16) = lo0;
    *reinterpret_cast<half8 *>(row + part * 16 + 8) = lo1;
    *reinterpret_cast<half8 *>(row + 32 + part * 16) = hi0;
    *reinterpret_cast<half8 *>(row + 32 + part * 16 + 8) = hi1;
  }
  __device__ static int row_of(int t, int) { return t / 2; }
  static constexpr int kRows = 1;
};

template <>
struct BLoad<LG_Q6_K> {
  uint4 c0, c1;
  float a0, a1;
  __device__ void fetch(const DevMatrix &W, const int *wrow, int k0, int t) {
    const int part = t % 2;
    const int8_t *q = static_cast<const int8_t *>(W.q) + int64_t(wrow[0]) * W.cols + k0 + part * 32;
    c0 = *reinterpret_cast<const uint4 *>(q);
    c1 = *reinterpret_cast<const uint4 *>(q + 16);
    const float *s = static_cast<const float *>(W.s) + int64_t(wrow[0]) * (W.cols / 16) + (k0 + part * 32) / 16;
    a0 = s[0];
    a1 = s[1];
  }
  __device__ static void cvt16(uint4 c, float a, _Float16 *dst) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    half8 o0, o1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float v = a * float(int8_t(w[j / 4] >> (8 * (j % 4))));
      if (j < 8) o0[j] = _Float16(v); else o1[j - 8] = _Float16(v);
    }
    *reinterpret_cast<half8 *>(dst) = o0;
    *reinterpret_cast<half8 *>(dst + 8) = o1;
  }
  __device__ void store(_Float16 *Bs, int t) {
    const int r = t / 2, part = t % 2;
    cvt16(c0, a0, Bs + r * LDK + part * 32);
    cvt16(c1, a1, Bs + r * LDK + part * 32 + 16);
  }
  __device__ static int row_of(int t, int) { return t / 2; }
  static constexpr int kRows = 1;
};

// Tile order: the hardware hands consecutive workgroups to the 8 XCDs round-robin; give
// each XCD a contiguous range of tiles, and inside it walk groups of 8 M-tiles so that the
// concurrently running tiles of one XCD share A rows and weight rows through its L2.
__device__ __forceinline__ void tile_coords(int bid, int nblk, int MT, int NT, int &mt, int &nt) {
  int t = bid;
  if ((nblk & 7) == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
  constexpr int GM = 8;
  const int group = t / (GM * NT);
  const int first = group * GM;
  const int gm = min(MT - first, GM);
  const int in = t - group * GM * NT;
  mt = first + in % gm;
  nt = in / gm;
}

template <uint32_t KIND, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const _Float16 *__restrict__ A, int M, int K,
                                                   DevMatrix W, float *__restrict__ C,
                                                   _Float16 *__restrict__ C16, int ldc,
                                                   const float *__restrict__ bias, int MT, int NT,
                                                   int ffn) {
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int mt, nt;
  tile_coords(blockIdx.x, gridDim.x, MT, NT, mt, nt);
  const int m0 = mt * BM;

  // weight rows this thread loads
  using BL = BLoad<KIND>;
  int wrow[BL::kRows];
#pragma unroll
  for (int i = 0; i < BL::kRows; ++i) {
    const int r = BL::row_of(t, i);
    if (EPI == int(Epi::SWIGLU)) {
      // local row r: wave column r/64, MFMA block (r/32)&1 (0 gate, 1 up), lane r&31
      wrow[i] = ((r >> 5) & 1) * ffn + nt * 64 + (r >> 6) * 32 + (r & 31);
    } else {
      wrow[i] = nt * BN + r;
    }
  }
  // activation rows this thread loads (clamped; rows >= M are never stored)
  const _Float16 *arow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = min(m0 + t / 8 + 32 * i, M - 1);
    arow[i] = A + int64_t(r) * K + (t % 8) * 8;
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  uint4 av[4];
  BL bl;
#pragma unroll
  for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const uint4 *>(arow[i]);
  bl.fetch(W, wrow, 0, t);

  const int nk = K / BK;
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4 *>(As + (t / 8 + 32 * i) * LDK + (t % 8) * 8) = av[i];
    bl.store(Bs, t);
    __syncthreads();
    if (kt + 1 < nk) {
      const int k1 = (kt + 1) * BK;
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const uint4 *>(arow[i] + k1);
      bl.fetch(W, wrow, k1, t);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int kc = kk * 16 + (lane >> 5) * 8;
      const half8 a0 = *reinterpret_cast<const half8 *>(As + (wm * 64 + (lane & 31)) * LDK + kc);
      const half8 a1 = *reinterpret_cast<const half8 *>(As + (wm * 64 + 32 + (lane & 31)) * LDK + kc);
      const half8 b0 = *reinterpret_cast<const half8 *>(Bs + (wn * 64 + (lane & 31)) * LDK + kc);
      const half8 b1 = *reinterpret_cast<const half8 *>(Bs + (wn * 64 + 32 + (lane & 31)) * LDK + kc);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, acc[1][1], 0, 0, 0);
    }
  }

  // epilogue: acc[i][j] register r -> row (r/4)*8 + (lane/32)*4 + r%4, column lane%32
  const int col_in = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= M) continue;
      if (EPI == int(Epi::SWIGLU)) {
        const int col = nt * 64 + wn * 32 + col_in;
        C16[int64_t(row) * ldc + col] = _Float16(silu(acc[i][0][r]) * acc[i][1][r]);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = nt * BN + wn * 64 + j * 32 + col_in;
          float v = acc[i][j][r];
          if (EPI == int(Epi::F32)) {
            if (bias) v += bias[col];
            C[int64_t(row) * ldc + col] = v;
          } else if (EPI == int(Epi::ADD)) {
            C[int64_t(row) * ldc + col] += v;
          } else {
            if (bias) v += bias[col];
            C16[int64_t(row) * ldc + col] = _Float16(v);
          }
        }
      }
    }
  }
}

template <uint32_t KIND>
void launch_kind(const _Float16 *A, int M, const DevMatrix &W, Epi epi, float *C, _Float16 *C16,
                 int ldc, const float *bias, int MT, int NT, hipStream_t st) {
  const dim3 grid(MT * NT), block(256);
  const int K = W.cols, ffn = W.rows / 2;
  switch (epi) {
    case Epi::F32:
      hipLaunchKernelGGL((gemm_kernel<KIND, 0>), grid, block, 0, st, A, M, K, W, C, C16, ldc, bias, MT, NT, ffn);
      break;
    case Epi::ADD:
      hipLaunchKernelGGL((gemm_kernel<KIND, 1>), grid, block, 0, st, A, M, K, W, C, C16, ldc, bias, MT, NT, ffn);
      break;
    case Epi::F16:
      hipLaunchKernelGGL((gemm_kernel<KIND, 2>), grid, block, 0, st, A, M, K, W, C, C16, ldc, bias, MT, NT, ffn);
      break;
    case Epi::SWIGLU:
      hipLaunchKernelGGL((gemm_kernel<KIND, 3>), grid, block, 0, st, A, M, K, W, C, C16, ldc, bias, MT, NT, ffn);
      break;
  }
}

// ---------------------------------------------------------------- generic f32 GEMM
__device__ float weight_at(const DevMatrix &W, int64_t n, int64_t k) {
  const int64_t cols = W.cols;
  switch (W.kind) {
    case LG_F32: return static_cast<const float *>(W.q)[n * cols + k];
    case LG_F16: return half_bits(static_cast<const uint16_t *>(W.q)[n * cols + k]);
    case LG_Q8_0:
      return half_bits(static_cast<const uint16_t *>(W.s)[n * (cols / 32) + k / 32]) *
             float(static_cast<const int8_t *>(W.q)[n * cols + k]);
    case LG_Q4_K: {
      const uint8_t byte = static_cast<const uint8_t *>(W.q)[n * (cols / 2) + (k / 64) * 32 + (k % 32)];
      const uint32_t nib = (k % 64) >= 32 ? (byte >> 4) : (byte & 15u);
      const float2 ab = static_cast<const float2 *>(W.s)[n * (cols / 32) + k / 32];
      return ab.x * float(nib) - ab.y;
    }
    case LG_Q6_K:
      return static_cast<const float *>(W.s)[n * (cols / 16) + k / 16] *
             float(static_cast<const int8_t *>(W.q)[n * cols + k]);
  }
  return 0.0f;
}

// One wave per (row m, column n) pair group: lanes split K, wave-reduce.
__global__ __launch_bounds__(256) void gemm_generic_kernel(const float *__restrict__ X, int M,
                                                           DevMatrix W,
                                                           const float *__restrict__ bias,
                                                           float *__restrict__ Y) {
  const int lane = threadIdx.x & 63;
  const int64_t pair = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int N = W.rows, K = W.cols;
  if (pair >= int64_t(M) * N) return;
  const int m = int(pair / N), n = int(pair % N);
  float s = 0.0f;
  for (int k = lane; k < K; k += 64) s += X[int64_t(m) * K + k] * weight_at(W, n, k);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) Y[int64_t(m) * N + n] = s + (bias ? bias[n] : 0.0f);
}

}  // namespace

void launch_gemm(const _Float16 *A, int M, const DevMatrix &W, Epi epi, float *C, _Float16 *C16,
                 int ldc, const float *bias, hipStream_t st) {
  LG_REQUIRE(M > 0, "gemm: empty activation");
  if (W.cols % BK != 0)
    fail(LG_ERR_UNSUPPORTED, "gemm: K=%d is not a multiple of %d", W.cols, BK);
  if (W.kind == LG_Q4_K || W.kind == LG_Q6_K)
    LG_REQUIRE(W.cols % 256 == 0, "gemm: K-quant rows must be whole super-blocks");
  int NT;
  if (epi == Epi::SWIGLU) {
    if (W.rows % 128 != 0) fail(LG_ERR_UNSUPPORTED, "gemm: gate|up rows %d not a multiple of 128", W.rows);
    NT = (W.rows / 2) / 64;
    LG_REQUIRE(C16 != nullptr && ldc >= W.rows / 2, "gemm: SwiGLU output needs ldc >= ffn");
  } else {
    if (W.rows % BN != 0) fail(LG_ERR_UNSUPPORTED, "gemm: N=%d is not a multiple of %d", W.rows, BN);
    NT = W.rows / BN;
    LG_REQUIRE(ldc >= W.rows, "gemm: ldc %d < N %d", ldc, W.rows);
    LG_REQUIRE(epi == Epi::F16 ? C16 != nullptr : C != nullptr, "gemm: missing output");
  }
  const int MT = (M + BM - 1) / BM;
  LG_REQUIRE(int64_t(MT) * NT < (1ll << 31), "gemm: grid too large");
  switch (W.kind) {
    case LG_F16: launch_kind<LG_F16>(A, M, W, epi, C, C16, ldc, bias, MT, NT, st); break;
    case LG_Q8_0: launch_kind<LG_Q8_0>(A, M, W, epi, C, C16, ldc, bias, MT, NT, st); break;
    case LG_Q4_K: launch_kind<LG_Q4_K>(A, M, W, epi, C, C16, ldc, bias, MT, NT, st); break;
    case LG_Q6_K: launch_kind<LG_Q6_K>(A, M, W, epi, C, C16, ldc, bias, MT, NT, st); break;
    default: fail(LG_ERR_UNSUPPORTED, "gemm: no MFMA path for GGML type %u", W.kind);
  }
  HIP_CHECK(hipGetLastError());
}

void launch_gemm_generic(const float *X, int M, const DevMatrix &W, const float *bias, float *Y,
                         hipStream_t st) {
  const int64_t pairs = int64_t(M) * W.rows;
  LG_REQUIRE(M > 0 && pairs > 0, "gemm: empty problem");
  LG_REQUIRE(pairs / 4 < (1ll << 31), "gemm: problem too large");
  hipLaunchKernelGGL(gemm_generic_kernel, dim3(unsigned((pairs + 3) / 4)), dim3(256), 0, st, X, M, W,
                     bias, Y);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
