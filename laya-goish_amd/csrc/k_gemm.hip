// Prefill GEMM entry points and the generic f32 GEMM; the tile kernels are in gemm_tiles.h.
#include "gemm_tiles.h"

namespace lg {
namespace {

// Per-kind, per-mode tile configuration: <MODE, BK, HM, HN, STAGES> (workgroup tile 32 HM x 32 HN).
template <uint32_t KIND>
void launch_kind(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                 _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st, const _Float16 *ks) {
  // Chosen by sweeps at the 35,840-token Q8_0/F16 and 32,768-token Q4_K/Q6_K 7B prefill
  // shapes; a 256-wide N tile falls back to 128 when it does not divide the output width.
  if (!Alo) {
    if (launch_cfg<KIND, FAST, 64, 8, 8, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
    if (launch_cfg<KIND, FAST, 64, 4, 4, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
  } else if (launch_gemm_wide(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st, ks)) {
    return;
  } else if (KIND == LG_Q4_K && needs_ksum(W)) {
    if (launch_gemm_q4_exact(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st, ks)) return;
  } else if constexpr (KIND == LG_Q8_0) {
    if (launch_gemm_q8_exact(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
  } else if constexpr (KIND == LG_F16) {
    // fewer 128 x 128 tiles than CUs (short prefills, narrow outputs): 64 x 128 tiles, twice
    // the workgroups, and 128-deep K steps when K allows (half the load round trips of these
    // latency-bound launches); the per-element K order is the same, so the results are too
    const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
    const int outN = glu ? W.rows / 2 : W.rows;
    const int64_t tiles = int64_t((M + 127) / 128) * (outN / (glu ? 64 : 128));
    // few 64 x 64 tiles (a short request): 32 x 32 tiles (32 x 64 weight rows for gate|up) over two LDS
    // stages, four times the workgroups and a quarter of each K step's LDS traffic per workgroup (C1's
    // 144-token request 0.49-0.51 -> 0.40 ms; 128-deep K steps with one stage 0.41-0.43, 64-deep 0.45)
    if (int64_t((M + 63) / 64) * (outN / 64) < 128 && W.cols % 128 == 0 &&
        (glu ? launch_cfg<KIND, SPLIT, 128, 1, 2, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)
             : launch_cfg<KIND, SPLIT, 128, 1, 1, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)))
      return;
    // a few hundred rows over a deep K (narrow outputs, K >= 2048): 32 x 64 tiles over two LDS stages, four
    // times the workgroups of 64 x 128 (480 rows, N 1024: K 2048 27.6 -> 14.0 us, K 3584 47.1 -> 22.2 us)
    if (!glu && int64_t((M + 63) / 64) * (outN / 128) < 128 && W.cols >= 2048 && W.cols % 128 == 0 &&
        launch_cfg<KIND, SPLIT, 128, 1, 2, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st))
      return;
    // a handful of 64 x 128 tiles (a few dozen rows, narrow outputs): 64 x 64 tiles, twice again
    if (!glu && (M + 63) / 64 * (outN / 128) < 64 && W.cols % 128 == 0 &&
        launch_cfg<KIND, SPLIT, 128, 2, 2, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st))
      return;
    if (tiles < 256 && W.cols % 128 == 0 &&
        launch_cfg<KIND, SPLIT, 128, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st))
      return;
    if (tiles < 256 && launch_cfg<KIND, SPLIT, 64, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
    if (launch_cfg<KIND, SPLIT, 64, 4, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
  } else {
    // short launches, as the exact Q8_0 and Q4_K tiles (a 144-token request on two layers of the Q4_K/Q6_K
    // 7B shape 2.43 -> 1.77 ms, 560 tokens 2.75 -> 2.17 ms, 1024 tokens 3.29 -> 3.21 ms).  Q4_K weights
    // are dequantised in 64-deep steps of 32-element chunks, so their tiles are at least 128 columns wide.
    {
      const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
      const int outN = glu ? W.rows / 2 : W.rows;
      const bool few64 = int64_t((M + 63) / 64) * (outN / 64) < 128;
      const bool few128 = int64_t((M + 127) / 128) * (outN / 128) < 192;
      if constexpr (KIND == LG_Q4_K) {
        if (few64 && launch_cfg<KIND, SPLIT3, 64, 1, 4, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
        if (few128 && launch_cfg<KIND, SPLIT3, 64, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
      } else if (W.cols % 128 == 0) {
        if (few64 && (glu ? launch_cfg<KIND, SPLIT3, 128, 1, 2, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)
                          : launch_cfg<KIND, SPLIT3, 128, 1, 1, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)))
          return;
        if (few128 && launch_cfg<KIND, SPLIT3, 128, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
      }
    }
    if (launch_cfg<KIND, SPLIT3, 64, 4, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)) return;
  }
  fail(LG_ERR_UNSUPPORTED, "gemm: no tile configuration for N=%d", W.rows);
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
      return kq4_weight(ab.x, nib, ab.y);
    }
    case LG_Q6_K:
      return static_cast<const float *>(W.s)[n * (cols / 16) + k / 16] *
             float(static_cast<const int8_t *>(W.q)[n * cols + k]);
  }
  return 0.0f;
}

// One wave per (row m, column n) pair: lanes split K, wave-reduce.
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

bool gemm_small_rope_takes(int M, const DevMatrix &W, int hd) {
  return M > 0 && (W.kind == LG_F16 || W.kind == LG_Q8_0) && (hd == 64 || hd == 128) && W.rows % hd == 0 &&
         W.cols % 128 == 0 && int64_t((M + 63) / 64) * (W.rows / 64) < 128;
}

bool launch_gemm_small_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                            const RopeKvOut &ro, hipStream_t st) {
  if (!gemm_small_rope_takes(M, W, ro.hd) || !Alo) return false;
  if (W.kind == LG_Q8_0) return launch_gemm_q8_small_rope(A, Alo, M, W, bias, ro, st);
  const bool ok = launch_cfg_rope<LG_F16, SPLIT, 128, 1, 2>(A, Alo, M, W, bias, ro, st);
  if (ok) HIP_CHECK(hipGetLastError());
  return ok;
}

void launch_gemm(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W, Epi epi, float *C,
                 _Float16 *C16, _Float16 *C16_lo, int ldc, const float *bias, hipStream_t st, const _Float16 *ks) {
  LG_REQUIRE(M > 0, "gemm: empty activation");
  LG_REQUIRE(!A_lo || !needs_ksum(W) || ks, "gemm: an exact Q4_K launch needs its activation's chunk sums");
  if (W.cols % 64 != 0) fail(LG_ERR_UNSUPPORTED, "gemm: K=%d is not a multiple of 64", W.cols);
  if (W.kind == LG_Q4_K || W.kind == LG_Q6_K)
    LG_REQUIRE(W.cols % 256 == 0, "gemm: K-quant rows must be whole super-blocks");
  if (epi == Epi::SWIGLU || epi == Epi::GEGLU) {
    if (W.rows % 128 != 0) fail(LG_ERR_UNSUPPORTED, "gemm: gate|up rows %d not a multiple of 128", W.rows);
    LG_REQUIRE(C16 != nullptr && ldc >= W.rows / 2, "gemm: gated output needs ldc >= ffn");
  } else {
    if (W.rows % 128 != 0) fail(LG_ERR_UNSUPPORTED, "gemm: N=%d is not a multiple of 128", W.rows);
    LG_REQUIRE(ldc >= W.rows, "gemm: ldc %d < N %d", ldc, W.rows);
    LG_REQUIRE(epi == Epi::F16 || epi == Epi::RELU16 ? C16 != nullptr : C != nullptr, "gemm: missing output");
  }
  switch (W.kind) {
    case LG_F16: launch_kind<LG_F16>(A, A_lo, M, W, epi, C, C16, C16_lo, ldc, bias, st, ks); break;
    case LG_Q8_0: launch_kind<LG_Q8_0>(A, A_lo, M, W, epi, C, C16, C16_lo, ldc, bias, st, ks); break;
    case LG_Q4_K: launch_kind<LG_Q4_K>(A, A_lo, M, W, epi, C, C16, C16_lo, ldc, bias, st, ks); break;
    case LG_Q6_K: launch_kind<LG_Q6_K>(A, A_lo, M, W, epi, C, C16, C16_lo, ldc, bias, st, ks); break;
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
